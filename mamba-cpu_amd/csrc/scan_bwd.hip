// Selective-scan backward on gfx950.
//
// Reverse-mode of the forward recurrence, following the analytic formulas of
// bwd_row_body (reference csrc/selective_scan.cpp:168-248):
//   g    = gh + dy_t C_t            (gh = dLoss/dh_t carried backwards)
//   dC_t += dy_t h_t ;  dB_t += g dt_t u_t
//   ga   = g h_{t-1} exp(dt_t A) ;  dA += ga dt_t
//   ddt  = <ga, A> + u_t <g, B_t> ;  du_t = dy_t D + dt_t <g, B_t>
//   ddelta_t = ddt * sigmoid(delta_t + bias) if softplus ; gh = g exp(dt_t A)
// with dy_t = dout_t z_t s(z_t) and dz_t = dout_t y_t s(z_t)(1 + z_t(1 - s(z_t))).
//
// Instead of the reference's per-thread copy of every state (L * dstate floats
// per row), time is walked backwards in 16-step blocks: each block restarts
// from the checkpointed state at its start (written by the forward kernel),
// recomputes its 16 states and decay factors in registers, then runs the
// reverse recurrence. Sums over states use DPP row reduce-scatters; dB/dC sums
// over channels use permlane swaps inside a wave, then LDS across the
// workgroup's 4 waves, then one partial per workgroup that a separate kernel
// reduces in a fixed order (deterministic, no atomics). dA/dD/ddelta_bias are
// per-(batch, channel) partials reduced over the batch the same way.
#include "scan_common.h"

namespace mcpu {

template <typename Tx, int SPL, bool HAS_Z>
__global__ void __launch_bounds__(kScanThreads) scan_bwd_kernel(const ScanParams p) {
  constexpr int NW = 16 * SPL;
  __shared__ float lds_dB[kScanWaves][kScanBlockT][NW];
  __shared__ float lds_dC[kScanWaves][kScanBlockT][NW];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane >> 4, j = lane & 15;
  const RowCtx rc = scan_row_ctx(p, wave, r);
  const int64_t N = p.dstate, L = p.seqlen;
  const int64_t row = rc.b * p.dim + rc.d;
  const int64_t cblk = blockIdx.x % p.nblk_c;

  float Av[SPL], A2[SPL], gh[SPL], dA_acc[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int n = j + 16 * s;
    Av[s] = n < N ? p.A[rc.d * N + n] : 0.f;
    A2[s] = Av[s] * kLog2e;
    gh[s] = (n < N && p.dlast_state != nullptr) ? p.dlast_state[row * N + n] : 0.f;
    dA_acc[s] = 0.f;
  }
  const float Dd = p.D ? p.D[rc.d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[rc.d] : 0.f;
  const int64_t ubase = rc.b * p.su[0] + rc.d * p.su[1];
  const int64_t dbase = rc.b * p.sdl[0] + rc.d * p.sdl[1];
  const int64_t zbase = rc.b * p.sz[0] + rc.d * p.sz[1];
  const int64_t obase = rc.b * p.sdo[0] + rc.d * p.sdo[1];
  const float* Bbase = p.B + rc.b * p.sB[0] + rc.g * p.sB[1];
  const float* Cbase = p.C + rc.b * p.sC[0] + rc.g * p.sC[1];
  const float* ck = p.ckpt + row * p.nblk * N;
  const int64_t part_base = ((rc.b * p.ngroups + rc.g) * p.nblk_c + cblk) * L;
  float dD_acc = 0.f, dbias_acc = 0.f;

  for (int64_t k = p.nblk - 1; k >= 0; --k) {
    const int64_t t0 = k * kScanBlockT;
    const int64_t t = t0 + j;
    const bool tv = t < L;
    const int nvalid = static_cast<int>(L - t0 < kScanBlockT ? L - t0 : kScanBlockT);
    const float uu = tv ? ld<Tx>(p.u, ubase + t * p.su[2]) : 0.f;
    const float dl = tv ? ld<Tx>(p.delta, dbase + t * p.sdl[2]) : 0.f;
    const float go = (tv && p.dout != nullptr) ? ld<Tx>(p.dout, obase + t * p.sdo[2]) : 0.f;
    const float zz = (HAS_Z && tv) ? ld<Tx>(p.z, zbase + t * p.sz[2]) : 0.f;

    float Bv[kScanBlockT][SPL], Cv[kScanBlockT][SPL], h0[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      const int n = j + 16 * s;
      h0[s] = n < N ? ck[k * N + n] : 0.f;
#pragma unroll
      for (int i = 0; i < kScanBlockT; ++i) {
        const bool ok = i < nvalid && n < N;
        Bv[i][s] = ok ? Bbase[(t0 + i) * p.sB[2] + n] : 0.f;
        Cv[i][s] = ok ? Cbase[(t0 + i) * p.sC[2] + n] : 0.f;
      }
    }

    const float pre = dl + bias;
    const float dt = p.softplus ? softplus(pre) : pre;
    const float dtu = dt * uu;

    // Forward recompute of the block's states and decay factors.
    float hs[kScanBlockT][SPL], as[kScanBlockT][SPL], pacc[kScanBlockT];
    {
      float hc[SPL];
#pragma unroll
      for (int s = 0; s < SPL; ++s) hc[s] = h0[s];
      static_for<kScanBlockT>([&](auto I) {
        constexpr int i = decltype(I)::value;
        if (i < nvalid) {
          const float dti = row_bcast<i>(dt);
          const float dtui = row_bcast<i>(dtu);
          float acc = 0.f;
#pragma unroll
          for (int s = 0; s < SPL; ++s) {
            const float a = fast_exp2(dti * A2[s]);
            hc[s] = fmaf(a, hc[s], dtui * Bv[i][s]);
            hs[i][s] = hc[s];
            as[i][s] = a;
            if (HAS_Z) acc = fmaf(hc[s], Cv[i][s], acc);
          }
          pacc[i] = acc;
        } else {
#pragma unroll
          for (int s = 0; s < SPL; ++s) hs[i][s] = as[i][s] = 0.f;
          pacc[i] = 0.f;
        }
      });
    }

    // Output gating: dy_t and dz_t for the step this lane owns.
    float dy = go, dzv = 0.f;
    if (HAS_Z) {
      float y = row_reduce_scatter16(pacc, j);
      if (p.D != nullptr) y = fmaf(Dd, uu, y);
      const float sg = sigmoid(zz);
      dzv = go * y * sg * (1.f + zz * (1.f - sg));
      dy = go * zz * sg;
    }

    // Reverse recurrence over the block.
    float r1[kScanBlockT], r2[kScanBlockT], dBc[SPL][kScanBlockT], dCc[SPL][kScanBlockT];
    static_for<kScanBlockT>([&](auto I) {
      constexpr int i = kScanBlockT - 1 - decltype(I)::value;
      if (i < nvalid) {
        const float dyi = row_bcast<i>(dy);
        const float dti = row_bcast<i>(dt);
        const float dtui = row_bcast<i>(dtu);
        float acc1 = 0.f, acc2 = 0.f;
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
          const float g = fmaf(dyi, Cv[i][s], gh[s]);
          dCc[s][i] = dyi * hs[i][s];
          const float hp = i > 0 ? hs[i > 0 ? i - 1 : 0][s] : h0[s];
          const float ga = g * hp * as[i][s];
          dA_acc[s] = fmaf(ga, dti, dA_acc[s]);
          acc1 = fmaf(ga, Av[s], acc1);
          acc2 = fmaf(g, Bv[i][s], acc2);
          dBc[s][i] = g * dtui;
          gh[s] = g * as[i][s];
        }
        r1[i] = acc1;
        r2[i] = acc2;
      } else {
        r1[i] = r2[i] = 0.f;
#pragma unroll
        for (int s = 0; s < SPL; ++s) dBc[s][i] = dCc[s][i] = 0.f;
      }
    });

    const float R1 = row_reduce_scatter16(r1, j);  // <ga, A> for step t
    const float R2 = row_reduce_scatter16(r2, j);  // <g, B_t> for step t
    if (tv) {
      float ddt = fmaf(uu, R2, R1);
      const float duv = fmaf(dy, Dd, dt * R2);
      if (p.softplus) ddt *= sigmoid(pre);
      if (rc.active) {
        st<Tx>(p.du, row * L + t, duv);
        st<Tx>(p.ddelta, row * L + t, ddt);
        if (HAS_Z) st<Tx>(p.dz, row * L + t, dzv);
      }
      dD_acc = fmaf(dy, uu, dD_acc);
      dbias_acc += ddt;
    }

    // dB/dC: sum over the workgroup's channels.
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      if (!rc.active) {
#pragma unroll
        for (int i = 0; i < kScanBlockT; ++i) dBc[s][i] = dCc[s][i] = 0.f;
      }
      float yB[4], yC[4];
      wave_rows_reduce_scatter(dBc[s], yB);
      wave_rows_reduce_scatter(dCc[s], yC);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        lds_dB[wave][4 * r + q][j + 16 * s] = yB[q];
        lds_dC[wave][4 * r + q][j + 16 * s] = yC[q];
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < kScanBlockT * NW; idx += kScanThreads) {
      const int tt = idx / NW, n = idx % NW;
      if (n < N && tt < nvalid) {
        float sb = 0.f, sc = 0.f;
#pragma unroll
        for (int w = 0; w < kScanWaves; ++w) {
          sb += lds_dB[w][tt][n];
          sc += lds_dC[w][tt][n];
        }
        p.dB_part[(part_base + t0 + tt) * N + n] = sb;
        p.dC_part[(part_base + t0 + tt) * N + n] = sc;
      }
    }
    __syncthreads();
  }

  if (rc.active) {
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      if (j + 16 * s < N) p.dA_part[row * N + j + 16 * s] = dA_acc[s];
  }
  dD_acc = row_allreduce16(dD_acc);
  dbias_acc = row_allreduce16(dbias_acc);
  if (rc.active && j == 0) {
    p.dD_part[row] = dD_acc;
    p.dbias_part[row] = dbias_acc;
  }
}

// dB/dC: out[b, g, t, n] = sum over channel blocks of part[b, g, cblk, t, n].
__global__ void __launch_bounds__(256) reduce_bc_kernel(const float* __restrict__ part,
                                                        float* __restrict__ out, int64_t slices,
                                                        int64_t nblk_c, int64_t per_slice) {
  const int64_t total = slices * per_slice;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += 256ll * gridDim.x) {
    const int64_t sl = i / per_slice, e = i % per_slice;
    const float* src = part + sl * nblk_c * per_slice + e;
    float acc = 0.f;
    for (int64_t c = 0; c < nblk_c; ++c) acc += src[c * per_slice];
    out[i] = acc;
  }
}

// out[e] = sum over batch of part[b, e].
__global__ void __launch_bounds__(256) reduce_batch_kernel(const float* __restrict__ part,
                                                           float* __restrict__ out, int64_t batch,
                                                           int64_t per_batch) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < per_batch; i += 256ll * gridDim.x) {
    float acc = 0.f;
    for (int64_t b = 0; b < batch; ++b) acc += part[b * per_batch + i];
    out[i] = acc;
  }
}

template <typename Tx, int SPL>
static hipError_t launch_bwd_z(const ScanParams& p, hipStream_t stream) {
  const int64_t blocks = p.batch * p.ngroups * p.nblk_c;
  if (p.z != nullptr)
    hipLaunchKernelGGL((scan_bwd_kernel<Tx, SPL, true>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kScanThreads), 0, stream, p);
  else
    hipLaunchKernelGGL((scan_bwd_kernel<Tx, SPL, false>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kScanThreads), 0, stream, p);
  return hipGetLastError();
}

template <typename Tx>
static hipError_t launch_bwd_spl(const ScanParams& p, hipStream_t stream) {
  if (p.dstate <= 16) return launch_bwd_z<Tx, 1>(p, stream);
  if (p.dstate <= 32) return launch_bwd_z<Tx, 2>(p, stream);
  return launch_bwd_z<Tx, 4>(p, stream);
}

hipError_t scan_bwd_launch(const ScanParams& p, int dtype, hipStream_t stream) {
  switch (dtype) {
    case MCPU_F32: return launch_bwd_spl<float>(p, stream);
    case MCPU_BF16: return launch_bwd_spl<bf16>(p, stream);
    default: return launch_bwd_spl<f16>(p, stream);
  }
}

static unsigned grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65535 * 16) g = 65535 * 16;
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

hipError_t scan_reduce_bc_launch(const float* part, float* out, int64_t slices, int64_t nblk_c,
                                 int64_t per_slice, hipStream_t stream) {
  hipLaunchKernelGGL(reduce_bc_kernel, dim3(grid_for(slices * per_slice)), dim3(256), 0, stream,
                     part, out, slices, nblk_c, per_slice);
  return hipGetLastError();
}

hipError_t scan_reduce_batch_launch(const float* part, float* out, int64_t batch,
                                    int64_t per_batch, hipStream_t stream) {
  hipLaunchKernelGGL(reduce_batch_kernel, dim3(grid_for(per_batch)), dim3(256), 0, stream, part,
                     out, batch, per_batch);
  return hipGetLastError();
}

}  // namespace mcpu
