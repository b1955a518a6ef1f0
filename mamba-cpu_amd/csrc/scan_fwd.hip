// Selective-scan forward on gfx950.
//
// Computes, per (batch, channel) row and for t = 0 .. L-1 (the recurrence of
// fwd_row_body, reference csrc/selective_scan.cpp:120-145):
//   dt_t  = softplus?(delta_t + delta_bias)
//   h_t   = exp(dt_t * A) * h_{t-1} + dt_t * u_t * B_t
//   out_t = (<h_t, C_t> + D * u_t) * silu(z_t)
// One state per lane (see scan_common.h); exp is v_exp_f32 on A * log2(e).
// The <h_t, C_t> contraction over the 16 state lanes of a row is done for all
// 16 steps of a block at once with a DPP reduce-scatter, which leaves y_t in
// the lane that owns step t. Optional outputs: the final state, and the state
// at the start of every 16-step block (checkpoints for the backward pass).
#include "scan_common.h"

namespace mcpu {

template <typename Tx, int SPL, bool HAS_Z, bool WRITE_OUT>
__global__ void __launch_bounds__(kScanThreads) scan_fwd_kernel(const ScanParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane >> 4, j = lane & 15;
  const RowCtx rc = scan_row_ctx(p, wave, r);
  const int64_t N = p.dstate, L = p.seqlen;
  const int64_t row = rc.b * p.dim + rc.d;

  float A2[SPL], h[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int n = j + 16 * s;
    A2[s] = n < N ? p.A[rc.d * N + n] * kLog2e : 0.f;
    h[s] = 0.f;
  }
  const float Dd = p.D ? p.D[rc.d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[rc.d] : 0.f;
  const int64_t ubase = rc.b * p.su[0] + rc.d * p.su[1];
  const int64_t dbase = rc.b * p.sdl[0] + rc.d * p.sdl[1];
  const int64_t zbase = rc.b * p.sz[0] + rc.d * p.sz[1];
  const float* Bbase = p.B + rc.b * p.sB[0] + rc.g * p.sB[1];
  const float* Cbase = p.C + rc.b * p.sC[0] + rc.g * p.sC[1];
  float* ck = p.ckpt ? p.ckpt + row * p.nblk * N : nullptr;

  for (int64_t k = 0; k < p.nblk; ++k) {
    const int64_t t0 = k * kScanBlockT;
    if (ck != nullptr && rc.active) {
#pragma unroll
      for (int s = 0; s < SPL; ++s)
        if (j + 16 * s < N) ck[k * N + j + 16 * s] = h[s];
    }
    const int64_t t = t0 + j;
    const bool tv = t < L;
    const float uu = tv ? ld<Tx>(p.u, ubase + t * p.su[2]) : 0.f;
    const float dl = tv ? ld<Tx>(p.delta, dbase + t * p.sdl[2]) : 0.f;
    float zz = 0.f;
    if (HAS_Z && WRITE_OUT) zz = tv ? ld<Tx>(p.z, zbase + t * p.sz[2]) : 0.f;
    const int nvalid = static_cast<int>(L - t0 < kScanBlockT ? L - t0 : kScanBlockT);

    float Bv[kScanBlockT][SPL], Cv[kScanBlockT][SPL];
#pragma unroll
    for (int i = 0; i < kScanBlockT; ++i) {
#pragma unroll
      for (int s = 0; s < SPL; ++s) {
        const int n = j + 16 * s;
        const bool ok = i < nvalid && n < N;
        Bv[i][s] = ok ? Bbase[(t0 + i) * p.sB[2] + n] : 0.f;
        Cv[i][s] = (WRITE_OUT && ok) ? Cbase[(t0 + i) * p.sC[2] + n] : 0.f;
      }
    }

    float dt = dl + bias;
    if (p.softplus) dt = softplus(dt);
    const float dtu = dt * uu;

    float pacc[kScanBlockT];
    auto step = [&](auto I) {
      constexpr int i = decltype(I)::value;
      const float dti = row_bcast<i>(dt);
      const float dtui = row_bcast<i>(dtu);
      float acc = 0.f;
#pragma unroll
      for (int s = 0; s < SPL; ++s) {
        const float a = fast_exp2(dti * A2[s]);
        h[s] = fmaf(a, h[s], dtui * Bv[i][s]);
        if (WRITE_OUT) acc = fmaf(h[s], Cv[i][s], acc);
      }
      pacc[i] = acc;
    };
    if (nvalid == kScanBlockT) {
      static_for<kScanBlockT>(step);
    } else {
      static_for<kScanBlockT>([&](auto I) {
        if (decltype(I)::value < nvalid) step(I);
        else pacc[decltype(I)::value] = 0.f;
      });
    }

    if (WRITE_OUT) {
      float y = row_reduce_scatter16(pacc, j);
      if (tv && rc.active) {
        if (p.D != nullptr) y = fmaf(Dd, uu, y);
        if (HAS_Z) y *= zz * sigmoid(zz);
        st<Tx>(p.out, row * L + t, y);
      }
    }
  }
  if (p.last_state != nullptr && rc.active) {
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      if (j + 16 * s < N) p.last_state[row * N + j + 16 * s] = h[s];
  }
}

template <typename Tx, int SPL, bool HAS_Z, bool WRITE_OUT>
static hipError_t launch_fwd(const ScanParams& p, hipStream_t stream) {
  const int64_t blocks = p.batch * p.ngroups * p.nblk_c;
  hipLaunchKernelGGL((scan_fwd_kernel<Tx, SPL, HAS_Z, WRITE_OUT>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kScanThreads), 0, stream, p);
  return hipGetLastError();
}

template <typename Tx, int SPL>
static hipError_t dispatch_fwd_flags(const ScanParams& p, bool write_out, hipStream_t stream) {
  if (!write_out) return launch_fwd<Tx, SPL, false, false>(p, stream);
  if (p.z != nullptr) return launch_fwd<Tx, SPL, true, true>(p, stream);
  return launch_fwd<Tx, SPL, false, true>(p, stream);
}

template <typename Tx>
static hipError_t dispatch_fwd_spl(const ScanParams& p, bool write_out, hipStream_t stream) {
  if (p.dstate <= 16) return dispatch_fwd_flags<Tx, 1>(p, write_out, stream);
  if (p.dstate <= 32) return dispatch_fwd_flags<Tx, 2>(p, write_out, stream);
  return dispatch_fwd_flags<Tx, 4>(p, write_out, stream);
}

// Launches the forward kernel. write_out = false computes states only
// (checkpoints and/or last_state), skipping C, z and the outputs.
hipError_t scan_fwd_launch(const ScanParams& p, int dtype, bool write_out, hipStream_t stream) {
  switch (dtype) {
    case MCPU_F32: return dispatch_fwd_spl<float>(p, write_out, stream);
    case MCPU_BF16: return dispatch_fwd_spl<bf16>(p, write_out, stream);
    default: return dispatch_fwd_spl<f16>(p, write_out, stream);
  }
}

}  // namespace mcpu
