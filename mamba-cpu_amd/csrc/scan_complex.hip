// Selective scan with complex A on gfx950: forward and backward.
//
// mamba_ssm's complex-A recurrence (its selective_scan_ref; the reference
// rejects complex A, src/mamba_cpu/ops/selective_scan_interface.py:160-161):
//   a_t = exp(dt_t A) = exp(dt_t Re A) (cos(dt_t Im A) + i sin(dt_t Im A))
//   h_t = a_t h_{t-1} + dt_t u_t B_t        (complex state and B_t)
//   y_t = 2 Re(sum_n h_t C_t) + D u_t ;  out_t = y_t silu(z_t)
// with dt, D and z as in the real scan. Lane layout and staging are the real
// kernels' (scan_common.h): 4 channels x 16 state lanes per wave, 16-step
// blocks, the next block's operands prefetched into double-buffered LDS. B
// and C arrive as (re, im) float pairs and are parked as two real tiles. The
// rotation angle is taken in revolutions, fract(dt Im A / 2 pi), the input
// v_sin_f32 / v_cos_f32 expect.
//
// Backward, by the chain rule on real and imaginary parts (a complex gradient
// holds dLoss/dRe + i dLoss/dIm, torch's convention), for t = L-1 .. 0 with
// gh = dLoss/dh_t carried backwards:
//   g   = gh + 2 dy conj(C_t) ;  dC_t = 2 dy conj(h_t) ;  dB_t = g dt u
//   gh' = g conj(a_t) ;  q = gh' conj(h_{t-1}) ;  dA += dt q
//   ddt = sum_n Re(q conj(A)) + u sum_n Re(g conj(B_t))
//   du  = dy D + dt sum_n Re(g conj(B_t))
// Each block restarts from the forward's checkpointed state. dB/dC are
// summed over the wave's channel rows (permlane swaps), over the workgroup's
// waves (LDS) into one partial per workgroup, and the partials are summed in a
// fixed order by the backward's reduce launch.
//
// Above 32 states the states are cut into slices of 32 that the grid scans
// side by side (scan_slice), as for real A: the forward's slices write their
// shares of 2 Re(sum_n h C) (PART), which scan_fwd_finish_kernel adds with D
// u and the gate; the backward's slices write their shares of
// sum_n Re(q conj(A)) and sum_n Re(g conj(B)) (SLICED), from which
// scan_bwd_finish_kernel forms du, ddelta, dz and the dD / ddelta_bias
// partials. All other outputs are per state and land in place.
#include "scan_common.h"

namespace mcpu {

constexpr int kCWaves = 4;
constexpr float kInv2Pi = 0.15915494309189535f;

// a = exp(dt A) from x2 = dt Re(A) log2(e) and rev = dt Im(A) / (2 pi).
__device__ __forceinline__ void cexp_step(float x2, float rev, float& ar, float& ai) {
  const float mag = fast_exp2(x2);
  const float f = __builtin_amdgcn_fractf(rev);
  ar = mag * __builtin_amdgcn_cosf(f);
  ai = mag * __builtin_amdgcn_sinf(f);
}

// WRITE_OUT = false: states only (checkpoints and/or last_state), no C, z or
// outputs. PART: a state slice's share of y into p.ypart (no D, no gate).
template <typename Tx, int SPL, bool HAS_Z, bool WRITE_OUT, bool PART>
__global__ void __launch_bounds__(64 * kCWaves) scan_cfwd_kernel(const ScanParams p) {
  constexpr int W = kCWaves;
  constexpr int CH = 4 * W;
  constexpr int NW = 16 * SPL;
  constexpr int T = kScanBlockT;
  using BC = BCStage<W, SPL>;
  // [buffer][u, delta, z][channel][step]
  __shared__ __align__(16) float s_x[2][3][CH][T];
  // [buffer][re, im][state][step]
  __shared__ __align__(16) float s_B[2][2][NW][kBCPad];
  __shared__ __align__(16) float s_C[2][2][NW][kBCPad];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane >> 4, j = lane & 15;
  const int c_local = wave * kScanRowsPerWave + r;
  const SliceCtx sc = scan_slice(p);
  const RowCtx rc = scan_row_ctx<W>(p, sc.bx, wave, r);
  // This slice's states, n0 .. n0 + N - 1 of the NS per row.
  const int64_t N = sc.N, NS = p.nstride, n0 = sc.n0, L = p.seqlen, nb = p.nblk;
  const int64_t row = rc.b * p.dim + rc.d;

  float Ar2[SPL], Air[SPL], hr[SPL], hi[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int n = j + 16 * s;
    const bool ok = n < N;
    Ar2[s] = ok ? p.A[2 * (rc.d * NS + n0 + n)] * kLog2e : 0.f;
    Air[s] = ok ? p.A[2 * (rc.d * NS + n0 + n) + 1] * kInv2Pi : 0.f;
    hr[s] = hi[s] = 0.f;
  }
  const float Dd = p.D ? p.D[rc.d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[rc.d] : 0.f;
  // Checkpoints (batch, dim, nblk, NS, 2): the state at each block start.
  float* ck = p.ckpt ? p.ckpt + (row * nb * NS + n0) * 2 : nullptr;
  const int64_t crow = rc.d - (rc.g * p.dpg + rc.cl0);
  char* const out0 = static_cast<char*>(p.out) +
      static_cast<int64_t>(sizeof(Tx)) * (rc.b * p.sout[0] + (rc.g * p.dpg + rc.cl0) * p.sout[1]);
  const int64_t out_ts = static_cast<int64_t>(sizeof(Tx)) * p.sout[2];
  const uint32_t out_off = static_cast<uint32_t>(sizeof(Tx) * (crow * p.sout[1] + j * p.sout[2]));

  XStage<W> xu, xd, xz;
  xu.template init<Tx>(tid, p.u, p.su, p, rc, 0);
  xd.template init<Tx>(tid, p.delta, p.sdl, p, rc, 0);
  if (HAS_Z && WRITE_OUT) xz.template init<Tx>(tid, p.z, p.sz, p, rc, 0);
  const float* Brow = p.B + rc.b * p.sB[0] + rc.g * p.sB[1] + n0 * p.sB[3];
  const float* Crow = p.C + rc.b * p.sC[0] + rc.g * p.sC[1] + n0 * p.sC[3];
  BC tbr, tbi, tcr, tci;
  tbr.init(tid, Brow, p.sB, N, 0, true);
  tbi.init(tid, Brow + 1, p.sB, N, 0, true);
  if (WRITE_OUT) {
    tcr.init(tid, Crow, p.sC, N, 0, true);
    tci.init(tid, Crow + 1, p.sC, N, 0, true);
  }
  const int64_t t_full = L - L % T;

  uint32_t nu = 0u, nd = 0u, nz = 0u;  // raw bits, widened at the park
  float nBr[BC::PER_THREAD], nBi[BC::PER_THREAD], nCr[BC::PER_THREAD], nCi[BC::PER_THREAD];
  // Loads the block at t0 and moves the cursors one block on, except from the
  // last block (`last`), which re-reads itself: no load is conditional.
  auto fetch = [&](int64_t t0, bool last) {
    if (t0 < t_full) {
      nu = xu.template load<Tx>();
      nd = xd.template load<Tx>();
      if (HAS_Z && WRITE_OUT) nz = xz.template load<Tx>();
      tbr.load(nBr);
      tbi.load(nBi);
      if (WRITE_OUT) {
        tcr.load(nCr);
        tci.load(nCi);
      }
    } else {
      nu = xu.template load_guarded<Tx>(t0, L);
      nd = xd.template load_guarded<Tx>(t0, L);
      if (HAS_Z && WRITE_OUT) nz = xz.template load_guarded<Tx>(t0, L);
      tbr.load_guarded(t0, L, nBr);
      tbi.load_guarded(t0, L, nBi);
      if (WRITE_OUT) {
        tcr.load_guarded(t0, L, nCr);
        tci.load_guarded(t0, L, nCi);
      }
    }
    xu.advance_unless(1, last);
    xd.advance_unless(1, last);
    if (HAS_Z && WRITE_OUT) xz.advance_unless(1, last);
    tbr.advance_unless(1, last);
    tbi.advance_unless(1, last);
    if (WRITE_OUT) {
      tcr.advance_unless(1, last);
      tci.advance_unless(1, last);
    }
  };
  auto park = [&](int buf) {
    (&s_x[buf][0][0][0])[xu.slot] = raw_f32<Tx>(nu);
    (&s_x[buf][1][0][0])[xd.slot] = raw_f32<Tx>(nd);
    if (HAS_Z && WRITE_OUT) (&s_x[buf][2][0][0])[xz.slot] = raw_f32<Tx>(nz);
    tbr.park(s_B[buf][0], nBr);
    tbi.park(s_B[buf][1], nBi);
    if (WRITE_OUT) {
      tcr.park(s_C[buf][0], nCr);
      tci.park(s_C[buf][1], nCi);
    }
  };

  if (nb > 0) {
    fetch(0, nb <= 1);
    park(0);
  }
  __syncthreads();
  __builtin_amdgcn_s_waitcnt(0);
  if (ck != nullptr && rc.active && nb > 0) {
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      if (j + 16 * s < N) {
        ck[2 * (j + 16 * s)] = 0.f;
        ck[2 * (j + 16 * s) + 1] = 0.f;
      }
  }

  for (int64_t k = 0; k < nb; ++k) {
    const int buf = static_cast<int>(k & 1);
    const int64_t t0 = k * T;
    fetch(k + 1 < nb ? t0 + T : t0, k + 2 >= nb);

    const bool tv = t0 + j < L;
    const float uu = s_x[buf][0][c_local][j];
    const float dl = s_x[buf][1][c_local][j];
    const float zz = (HAS_Z && WRITE_OUT) ? s_x[buf][2][c_local][j] : 0.f;
    const int nvalid = static_cast<int>(L - t0 < T ? L - t0 : T);

    float Br[SPL][T], Bi[SPL][T], Cr[SPL][T], Ci[SPL][T];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      read_bc_row(s_B[buf][0], j + 16 * s, Br[s]);
      read_bc_row(s_B[buf][1], j + 16 * s, Bi[s]);
      if (WRITE_OUT) {
        read_bc_row(s_C[buf][0], j + 16 * s, Cr[s]);
        read_bc_row(s_C[buf][1], j + 16 * s, Ci[s]);
      }
    }
    float dt = dl + bias;
    if (p.softplus) dt = softplus(dt);
    const float dtu = dt * uu;

    float pacc[T];
    auto step = [&](auto I) {
      constexpr int i = decltype(I)::value;
      const float dti = row_bcast<i>(dt);
      const float dtui = row_bcast<i>(dtu);
      float acc = 0.f;
#pragma unroll
      for (int s = 0; s < SPL; ++s) {
        float ar, ai;
        cexp_step(dti * Ar2[s], dti * Air[s], ar, ai);
        const float nr = fmaf(ar, hr[s], fmaf(-ai, hi[s], dtui * Br[s][i]));
        const float ni = fmaf(ar, hi[s], fmaf(ai, hr[s], dtui * Bi[s][i]));
        hr[s] = nr;
        hi[s] = ni;
        if (WRITE_OUT) acc = fmaf(nr, Cr[s][i], fmaf(-ni, Ci[s][i], acc));
      }
      pacc[i] = acc;
    };
    if (nvalid == T) {
      static_for<T>(step);
    } else {
      static_for<T>([&](auto I) {
        if (decltype(I)::value < nvalid) step(I);
        else pacc[decltype(I)::value] = 0.f;
      });
    }

    float y = 0.f, yg = 0.f;
    if (WRITE_OUT) {
      y = 2.f * row_reduce_scatter16(pacc, j);
      if (!PART && p.D != nullptr) y = fmaf(Dd, uu, y);
      yg = (HAS_Z && !PART) ? y * (zz * sigmoid(zz)) : y;
    }

    park(buf ^ 1);  // in the last iteration a harmless copy into the idle buffer

    if (WRITE_OUT && tv && rc.active) {
      if constexpr (PART) p.ypart[((sc.sl * p.batch + rc.b) * p.dim + rc.d) * L + t0 + j] = y;
      else buf_st<Tx>(wave_rsrc(out0 + t0 * out_ts), out_off, yg);
    }
    if (ck != nullptr && rc.active && k + 1 < nb) {
#pragma unroll
      for (int s = 0; s < SPL; ++s)
        if (j + 16 * s < N) {
          float* c = ck + ((k + 1) * NS + j + 16 * s) * 2;
          c[0] = hr[s];
          c[1] = hi[s];
        }
    }
    __syncthreads();
  }
  if (p.last_state != nullptr && rc.active) {
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      if (j + 16 * s < N) {
        p.last_state[(row * NS + n0 + j + 16 * s) * 2] = hr[s];
        p.last_state[(row * NS + n0 + j + 16 * s) * 2 + 1] = hi[s];
      }
  }
}

// SLICED: one state slice, which writes its sum_n Re(q conj(A)) and
// sum_n Re(g conj(B)) shares (rpart) in place of du, ddelta, dz and the dD /
// ddelta_bias partials.
template <typename Tx, int W, int SPL, bool HAS_Z, bool SLICED>
__global__ void __launch_bounds__(64 * W) scan_cbwd_kernel(const ScanParams p) {
  constexpr int CH = 4 * W;
  constexpr int NW = 16 * SPL;
  constexpr int T = kScanBlockT;
  using BC = BCStage<W, SPL>;
  // [buffer][u, delta, dout, z][channel][step]
  __shared__ __align__(16) float s_x[2][4][CH][T];
  __shared__ __align__(16) float s_B[2][2][NW][kBCPad];
  __shared__ __align__(16) float s_C[2][2][NW][kBCPad];
  // [buffer][dB re, dB im, dC re, dC im][wave][step][state]: per-wave channel
  // sums awaiting the cross-wave sum.
  __shared__ float s_red[2][4][W][T][NW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane >> 4, j = lane & 15;
  const int c_local = wave * kScanRowsPerWave + r;
  const SliceCtx sc = scan_slice(p);
  const RowCtx rc = scan_row_ctx<W>(p, sc.bx, wave, r);
  // This slice's states, n0 .. n0 + N - 1 of the NS per row of A,
  // dlast_state, the checkpoints and the dA/dB/dC layouts.
  const int64_t N = sc.N, NS = p.nstride, n0 = sc.n0, L = p.seqlen, nb = p.nblk;
  const int64_t row = rc.b * p.dim + rc.d;
  const int64_t kl = nb - 1;
  const int64_t t_last = kl * T;

  float Ar[SPL], Ai[SPL], Ar2[SPL], Air[SPL], ghr[SPL], ghi[SPL], dAr[SPL], dAi[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int n = j + 16 * s;
    const bool ok = n < N;
    Ar[s] = ok ? p.A[2 * (rc.d * NS + n0 + n)] : 0.f;
    Ai[s] = ok ? p.A[2 * (rc.d * NS + n0 + n) + 1] : 0.f;
    Ar2[s] = Ar[s] * kLog2e;
    Air[s] = Ai[s] * kInv2Pi;
    ghr[s] = (ok && p.dlast_state != nullptr) ? p.dlast_state[(row * NS + n0 + n) * 2] : 0.f;
    ghi[s] = (ok && p.dlast_state != nullptr) ? p.dlast_state[(row * NS + n0 + n) * 2 + 1] : 0.f;
    dAr[s] = dAi[s] = 0.f;
  }
  const float Dd = p.D ? p.D[rc.d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[rc.d] : 0.f;
  const bool has_D = p.D != nullptr;
  const bool softplus_on = p.softplus != 0;
  const bool has_dout = p.dout != nullptr;
  float dD_acc = 0.f, dbias_acc = 0.f;

  XStage<W> xu, xd, xo, xz;
  xu.template init<Tx>(tid, p.u, p.su, p, rc, t_last);
  xd.template init<Tx>(tid, p.delta, p.sdl, p, rc, t_last);
  xo.template init<Tx>(tid, has_dout ? p.dout : p.u, p.sdo, p, rc, t_last);
  if (HAS_Z) xz.template init<Tx>(tid, p.z, p.sz, p, rc, t_last);
  const float* Brow = p.B + rc.b * p.sB[0] + rc.g * p.sB[1] + n0 * p.sB[3];
  const float* Crow = p.C + rc.b * p.sC[0] + rc.g * p.sC[1] + n0 * p.sC[3];
  BC tbr, tbi, tcr, tci;
  tbr.init(tid, Brow, p.sB, N, t_last, true);
  tbi.init(tid, Brow + 1, p.sB, N, t_last, true);
  tcr.init(tid, Crow, p.sC, N, t_last, true);
  tci.init(tid, Crow + 1, p.sC, N, t_last, true);

  const int64_t row0 = rc.b * p.dim + rc.g * p.dpg + rc.cl0;
  const int64_t crow = rc.d - (rc.g * p.dpg + rc.cl0);
  // Checkpointed state pair of lane j, state j + 16 s, of the current block.
  const char* ck_base = reinterpret_cast<const char*>(p.ckpt + ((row0 * nb + kl) * NS + n0) * 2);
  const uint32_t ck_off = static_cast<uint32_t>(sizeof(float) * (crow * nb * NS * 2 + 2 * j));
  uint32_t ck_lane[SPL];
  bool ck_ok[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    ck_ok[s] = j + 16 * s < N;
    ck_lane[s] = ck_ok[s] ? ck_off + 128 * s : ck_off - 8 * j;
  }
  constexpr int64_t esz = sizeof(Tx);
  const int64_t cl = rc.g * p.dpg + rc.cl0;
  char* o_du = static_cast<char*>(p.du) + esz * (rc.b * p.sdu[0] + cl * p.sdu[1] + t_last * p.sdu[2]);
  char* o_dd = static_cast<char*>(p.ddelta) + esz * (rc.b * p.sdd[0] + cl * p.sdd[1] + t_last * p.sdd[2]);
  char* o_dz = HAS_Z ? static_cast<char*>(p.dz) + esz * (rc.b * p.sdz[0] + cl * p.sdz[1] + t_last * p.sdz[2])
                     : nullptr;
  const uint32_t off_du = static_cast<uint32_t>(esz * (crow * p.sdu[1] + j * p.sdu[2]));
  const uint32_t off_dd = static_cast<uint32_t>(esz * (crow * p.sdd[1] + j * p.sdd[2]));
  const uint32_t off_dz = HAS_Z ? static_cast<uint32_t>(esz * (crow * p.sdz[1] + j * p.sdz[2])) : 0u;

  // Cross-wave dB/dC outputs of this thread: element e = (array, step, state);
  // T * NW is a multiple of 64 * W, so the array is uniform over a wave.
  // Partials are (batch, ngroups, nblk_c, seqlen, NS, 2).
  constexpr int NOUT = 4 * T * NW / (64 * W);
  const int64_t part_row = ((rc.b * p.ngroups + rc.g) * p.nblk_c + rc.cblk) * L + t_last;
  char* o_part[NOUT];
  uint32_t o_poff[NOUT];
  int o_red[NOUT], o_t[NOUT];
  bool o_ok[NOUT];
#pragma unroll
  for (int q = 0; q < NOUT; ++q) {
    const int e = tid + q * 64 * W;
    const int arr = __builtin_amdgcn_readfirstlane(e / (T * NW));
    const int tt = (e % (T * NW)) / NW, n = e % NW;
    o_t[q] = tt;
    o_red[q] = (arr * W * T + tt) * NW + n;
    o_ok[q] = n < N;
    o_part[q] = reinterpret_cast<char*>((arr < 2 ? p.dB_part : p.dC_part) + (part_row * NS + n0) * 2);
    o_poff[q] = static_cast<uint32_t>(sizeof(float) * ((tt * NS + n) * 2 + (arr & 1)));
  }

  uint32_t nu = 0u, nd = 0u, no = 0u, nz = 0u;  // raw bits, widened at the park
  float nBr[BC::PER_THREAD], nBi[BC::PER_THREAD], nCr[BC::PER_THREAD], nCi[BC::PER_THREAD];
  float nh0r[SPL], nh0i[SPL];
  // Loads the operands of the block at t0 (full unless GUARD) and moves every
  // cursor one block back, except from block 0 (`stay`): no load is
  // conditional, and nothing consumes a prefetched value before park().
  auto fetch = [&](auto GUARD, int64_t t0, bool stay) {
    if constexpr (decltype(GUARD)::value) {
      nu = xu.template load_guarded<Tx>(t0, L);
      nd = xd.template load_guarded<Tx>(t0, L);
      no = xo.template load_guarded<Tx>(t0, L);
      if (HAS_Z) nz = xz.template load_guarded<Tx>(t0, L);
      tbr.load_guarded(t0, L, nBr);
      tbi.load_guarded(t0, L, nBi);
      tcr.load_guarded(t0, L, nCr);
      tci.load_guarded(t0, L, nCi);
    } else {
      nu = xu.template load<Tx>();
      nd = xd.template load<Tx>();
      no = xo.template load<Tx>();
      if (HAS_Z) nz = xz.template load<Tx>();
      tbr.load(nBr);
      tbi.load(nBi);
      tcr.load(nCr);
      tci.load(nCi);
    }
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      nh0r[s] = buf_ld<float>(wave_rsrc(ck_base), ck_lane[s]);
      nh0i[s] = buf_ld<float>(wave_rsrc(ck_base), ck_lane[s] + 4);
    }
    xu.advance_unless(-1, stay);
    xd.advance_unless(-1, stay);
    xo.advance_unless(-1, stay);
    if (HAS_Z) xz.advance_unless(-1, stay);
    tbr.advance_unless(-1, stay);
    tbi.advance_unless(-1, stay);
    tcr.advance_unless(-1, stay);
    tci.advance_unless(-1, stay);
    ck_base -= stay ? 0 : sizeof(float) * NS * 2;
  };
  auto park = [&](int buf) {
    (&s_x[buf][0][0][0])[xu.slot] = raw_f32<Tx>(nu);
    (&s_x[buf][1][0][0])[xd.slot] = raw_f32<Tx>(nd);
    (&s_x[buf][2][0][0])[xo.slot] = has_dout ? raw_f32<Tx>(no) : 0.f;
    if (HAS_Z) (&s_x[buf][3][0][0])[xz.slot] = raw_f32<Tx>(nz);
    tbr.park(s_B[buf][0], nBr);
    tbi.park(s_B[buf][1], nBi);
    tcr.park(s_C[buf][0], nCr);
    tci.park(s_C[buf][1], nCi);
  };

  float h0r[SPL], h0i[SPL];
  fetch(std::true_type{}, t_last, kl == 0);
  park(static_cast<int>(kl & 1));
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    h0r[s] = ck_ok[s] ? nh0r[s] : 0.f;
    h0i[s] = ck_ok[s] ? nh0i[s] : 0.f;
  }
  __syncthreads();
  __builtin_amdgcn_s_waitcnt(0);

  auto block = [&](auto FULL, int64_t k, int nvalid) {
    constexpr bool full = decltype(FULL)::value;
    const int buf = static_cast<int>(k & 1);
    const int64_t t0 = k * T;
    if (k > 0) fetch(std::false_type{}, t0 - T, k - 1 <= 0);
    else fetch(std::integral_constant<bool, !full>{}, t0, true);
    auto valid = [&](int i) { return full || i < nvalid; };

    const bool tv = full || j < nvalid;
    const float uu = s_x[buf][0][c_local][j];
    const float dl = s_x[buf][1][c_local][j];
    const float go = s_x[buf][2][c_local][j];
    const float zz = HAS_Z ? s_x[buf][3][c_local][j] : 0.f;

    float Br[SPL][T], Bi[SPL][T], Cr[SPL][T], Ci[SPL][T];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      read_bc_row(s_B[buf][0], j + 16 * s, Br[s]);
      read_bc_row(s_B[buf][1], j + 16 * s, Bi[s]);
      read_bc_row(s_C[buf][0], j + 16 * s, Cr[s]);
      read_bc_row(s_C[buf][1], j + 16 * s, Ci[s]);
    }
    const float pre = dl + bias;
    float dt = pre, sg_pre = 1.f;
    if (softplus_on) dt = softplus_sigmoid(pre, sg_pre);
    const float dtu = dt * uu;

    // Forward recompute of the block's states and decay factors.
    float hsr[SPL][T], hsi[SPL][T], asr[SPL][T], asi[SPL][T], pacc[T];
    {
      float cr[SPL], ci[SPL];
#pragma unroll
      for (int s = 0; s < SPL; ++s) {
        cr[s] = h0r[s];
        ci[s] = h0i[s];
      }
      static_for<T>([&](auto I) {
        constexpr int i = decltype(I)::value;
        if (valid(i)) {
          const float dti = row_bcast<i>(dt);
          const float dtui = row_bcast<i>(dtu);
          float acc = 0.f;
#pragma unroll
          for (int s = 0; s < SPL; ++s) {
            float ar, ai;
            cexp_step(dti * Ar2[s], dti * Air[s], ar, ai);
            const float nr = fmaf(ar, cr[s], fmaf(-ai, ci[s], dtui * Br[s][i]));
            const float ni = fmaf(ar, ci[s], fmaf(ai, cr[s], dtui * Bi[s][i]));
            cr[s] = nr;
            ci[s] = ni;
            hsr[s][i] = nr;
            hsi[s][i] = ni;
            asr[s][i] = ar;
            asi[s][i] = ai;
            if (HAS_Z && !SLICED) acc = fmaf(nr, Cr[s][i], fmaf(-ni, Ci[s][i], acc));
          }
          pacc[i] = acc;
        } else {
#pragma unroll
          for (int s = 0; s < SPL; ++s) hsr[s][i] = hsi[s][i] = asr[s][i] = asi[s][i] = 0.f;
          pacc[i] = 0.f;
        }
      });
    }

    // Output gating: dy_t and dz_t for the step this lane owns (a slice sees
    // only its share of y: dz is formed by the finish kernel from ysave).
    float dy = go, dzv = 0.f;
    if (HAS_Z) {
      const float sg = sigmoid(zz);
      if constexpr (!SLICED) {
        float y = 2.f * row_reduce_scatter16(pacc, j);
        if (has_D) y = fmaf(Dd, uu, y);
        dzv = go * y * sg * (1.f + zz * (1.f - sg));
      }
      dy = go * zz * sg;
    }

    // Padding rows (channels past the slice end) add nothing to dB/dC: their
    // dy and dt u are zero in the terms dC = 2 dy conj(h), dB = g dt u.
    const float dy_b = rc.active ? dy : 0.f;
    const float dtu_b = rc.active ? dtu : 0.f;
    // Reverse recurrence over the block. The dB/dC terms of steps 15..8 are
    // summed over the wave's 4 channel rows and parked for the cross-wave sum
    // as soon as step 8 is done, those of 7..0 at the end, which halves the
    // registers they hold.
    constexpr int TH = T / 2;
    float r1[T], r2[T], dBr[SPL][T], dBi[SPL][T], dCr[SPL][T], dCi[SPL][T];
    auto flush = [&](auto LO) {
      constexpr int i0 = decltype(LO)::value;
#pragma unroll
      for (int s = 0; s < SPL; ++s) {
        float xs[4][TH];
#pragma unroll
        for (int i = 0; i < TH; ++i) {
          xs[0][i] = dBr[s][i0 + i];
          xs[1][i] = dBi[s][i0 + i];
          xs[2][i] = dCr[s][i0 + i];
          xs[3][i] = dCi[s][i0 + i];
        }

#pragma unroll
        for (int a = 0; a < 4; ++a) {
          float y2[2];
          wave_rows_reduce_scatter8(xs[a], y2);
          s_red[buf][a][wave][i0 + 2 * r][j + 16 * s] = y2[0];
          s_red[buf][a][wave][i0 + 2 * r + 1][j + 16 * s] = y2[1];
        }
      }
    };
    static_for<T>([&](auto I) {
      constexpr int i = T - 1 - decltype(I)::value;
      if (valid(i)) {
        const float dy2 = 2.f * row_bcast<i>(dy_b);
        const float dti = row_bcast<i>(dt);
        const float dtui = row_bcast<i>(dtu_b);
        float acc1 = 0.f, acc2 = 0.f;
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
          const float gr = fmaf(dy2, Cr[s][i], ghr[s]);
          const float gi = fmaf(-dy2, Ci[s][i], ghi[s]);
          dCr[s][i] = dy2 * hsr[s][i];
          dCi[s][i] = -dy2 * hsi[s][i];
          dBr[s][i] = dtui * gr;
          dBi[s][i] = dtui * gi;
          acc2 = fmaf(gr, Br[s][i], fmaf(gi, Bi[s][i], acc2));
          const float ar = asr[s][i], ai = asi[s][i];
          const float nr = fmaf(gr, ar, gi * ai);   // g conj(a)
          const float ni = fmaf(gi, ar, -gr * ai);
          ghr[s] = nr;
          ghi[s] = ni;
          const float hpr = i > 0 ? hsr[s][i > 0 ? i - 1 : 0] : h0r[s];
          const float hpi = i > 0 ? hsi[s][i > 0 ? i - 1 : 0] : h0i[s];
          const float qr = fmaf(nr, hpr, ni * hpi);  // gh conj(h_{t-1})
          const float qi = fmaf(ni, hpr, -nr * hpi);
          dAr[s] = fmaf(dti, qr, dAr[s]);
          dAi[s] = fmaf(dti, qi, dAi[s]);
          acc1 = fmaf(qr, Ar[s], fmaf(qi, Ai[s], acc1));
        }
        r1[i] = acc1;
        r2[i] = acc2;
      } else {
        r1[i] = r2[i] = 0.f;
#pragma unroll
        for (int s = 0; s < SPL; ++s) dBr[s][i] = dBi[s][i] = dCr[s][i] = dCi[s][i] = 0.f;
      }
      if constexpr (i == TH) flush(std::integral_constant<int, TH>{});
      if constexpr (i == 0) flush(std::integral_constant<int, 0>{});
    });

    const float R1 = row_reduce_scatter16(r1, j);  // sum_n Re(q conj(A)) for step t
    const float R2 = row_reduce_scatter16(r2, j);  // sum_n Re(g conj(B_t)) for step t
    float ddt = fmaf(uu, R2, R1);
    const float duv = fmaf(dy, Dd, dt * R2);
    if (softplus_on) ddt *= sg_pre;
    if (tv) {
      dD_acc = fmaf(dy, uu, dD_acc);
      dbias_acc += ddt;
    }

    park(buf ^ 1);  // from block 0 a harmless copy into the idle buffer
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      h0r[s] = ck_ok[s] ? nh0r[s] : 0.f;
      h0i[s] = ck_ok[s] ? nh0i[s] : 0.f;
    }
    if (tv && rc.active) {
      if constexpr (SLICED) {
        const int64_t at = ((sc.sl * p.batch + rc.b) * p.dim + rc.d) * L + t0 + j;
        p.rpart[at] = R1;
        p.rpart[p.nslices * p.batch * p.dim * L + at] = R2;
      } else {
        buf_st<Tx>(wave_rsrc(o_du), off_du, duv);
        buf_st<Tx>(wave_rsrc(o_dd), off_dd, ddt);
        if (HAS_Z) buf_st<Tx>(wave_rsrc(o_dz), off_dz, dzv);
      }
    }
    o_du -= T * esz * p.sdu[2];
    o_dd -= T * esz * p.sdd[2];
    if (HAS_Z) o_dz -= T * esz * p.sdz[2];
    __syncthreads();

    // Cross-wave sum of this block's dB/dC and the workgroup's partial.
#pragma unroll
    for (int q = 0; q < NOUT; ++q) {
      if (o_ok[q] && (full || o_t[q] < nvalid)) {
        const float* src = &s_red[buf][0][0][0][0] + o_red[q];
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) acc += src[w * T * NW];
        buf_st<float>(wave_rsrc(o_part[q]), o_poff[q], acc);
      }
      o_part[q] -= sizeof(float) * T * NS * 2;
    }
  };

  const int nlast = static_cast<int>(L - t_last < T ? L - t_last : T);
  if (nlast == T) block(std::true_type{}, kl, T);
  else block(std::false_type{}, kl, nlast);
  for (int64_t k = kl - 1; k >= 0; --k) block(std::true_type{}, k, T);

  if (rc.active) {
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      if (j + 16 * s < N) {
        p.dA_part[(row * NS + n0 + j + 16 * s) * 2] = dAr[s];
        p.dA_part[(row * NS + n0 + j + 16 * s) * 2 + 1] = dAi[s];
      }
  }
  if constexpr (SLICED) return;
  dD_acc = row_allreduce16(dD_acc);
  dbias_acc = row_allreduce16(dbias_acc);
  if (rc.active && j == 0) {
    p.dD_part[row] = dD_acc;
    p.dbias_part[row] = dbias_acc;
  }
}

// A sliced forward (p.nslices > 1) writes the slices' shares of y when
// p.ypart is set; the caller then runs the finish kernel.
template <typename Tx, int SPL>
static hipError_t launch_cfwd(const ScanParams& p, bool write_out, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.batch * p.ngroups * p.nblk_c * p.nslices));
  const dim3 block(64 * kCWaves);
  if (!write_out)
    hipLaunchKernelGGL((scan_cfwd_kernel<Tx, SPL, false, false, false>), grid, block, 0, stream, p);
  else if (p.ypart != nullptr)
    hipLaunchKernelGGL((scan_cfwd_kernel<Tx, SPL, false, true, true>), grid, block, 0, stream, p);
  else if (p.z != nullptr)
    hipLaunchKernelGGL((scan_cfwd_kernel<Tx, SPL, true, true, false>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((scan_cfwd_kernel<Tx, SPL, false, true, false>), grid, block, 0, stream, p);
  return hipGetLastError();
}

// Sliced backwards (p.rpart set) run 32-state slices: only SPL 2 has a
// sliced form.
template <typename Tx, int W, int SPL>
static hipError_t launch_cbwd(const ScanParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.batch * p.ngroups * p.nblk_c * p.nslices));
  const dim3 block(64 * W);
  if constexpr (SPL == 2) {
    if (p.rpart != nullptr) {
      if (p.z != nullptr)
        hipLaunchKernelGGL((scan_cbwd_kernel<Tx, W, SPL, true, true>), grid, block, 0, stream, p);
      else
        hipLaunchKernelGGL((scan_cbwd_kernel<Tx, W, SPL, false, true>), grid, block, 0, stream, p);
      return hipGetLastError();
    }
  }
  if (p.z != nullptr)
    hipLaunchKernelGGL((scan_cbwd_kernel<Tx, W, SPL, true, false>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((scan_cbwd_kernel<Tx, W, SPL, false, false>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <typename Tx>
static hipError_t cfwd_spl(const ScanParams& p, bool write_out, hipStream_t stream) {
  if (p.dstate <= 16) return launch_cfwd<Tx, 1>(p, write_out, stream);
  return launch_cfwd<Tx, 2>(p, write_out, stream);
}

// 4-wave workgroups for the backward too: 8 waves halve the dB/dC partials
// but their LDS leaves one workgroup per CU, and the kernel ran 25 % slower.
template <typename Tx>
static hipError_t cbwd_spl(const ScanParams& p, hipStream_t stream) {
  if (p.dstate <= 16) return launch_cbwd<Tx, kCWaves, 1>(p, stream);
  return launch_cbwd<Tx, kCWaves, 2>(p, stream);
}

int scan_complex_waves() { return kCWaves; }

// Complex-A forward (p.nblk_c for scan_complex_waves(), one time chunk).
hipError_t scan_cfwd_launch(const ScanParams& p, int dtype, bool write_out, hipStream_t stream) {
  switch (dtype) {
    case MCPU_F32: return cfwd_spl<float>(p, write_out, stream);
    case MCPU_BF16: return cfwd_spl<bf16>(p, write_out, stream);
    default: return cfwd_spl<f16>(p, write_out, stream);
  }
}

// Complex-A backward (p.ckpt filled by the forward, partial buffers set).
hipError_t scan_cbwd_launch(const ScanParams& p, int dtype, hipStream_t stream) {
  switch (dtype) {
    case MCPU_F32: return cbwd_spl<float>(p, stream);
    case MCPU_BF16: return cbwd_spl<bf16>(p, stream);
    default: return cbwd_spl<f16>(p, stream);
  }
}

}  // namespace mcpu
