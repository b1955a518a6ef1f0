// Selective-scan forward on gfx950.
//
// Computes, per (batch, channel) row and for t = 0 .. L-1 (the recurrence of
// fwd_row_body, reference csrc/selective_scan.cpp:120-145):
//   dt_t  = softplus?(delta_t + delta_bias)
//   h_t   = exp(dt_t * A) * h_{t-1} + dt_t * u_t * B_t
//   y_t   = <h_t, C_t> + D * u_t ;  out_t = y_t * silu(z_t)
// One state per lane (see scan_common.h); exp is v_exp_f32 on A * log2(e).
// The <h_t, C_t> contraction over the 16 state lanes of a row is done for all
// 16 steps of a block at once with a DPP reduce-scatter, which leaves y_t in
// the lane that owns step t. Operands of block k+1 are fetched while block k
// computes (double-buffered LDS). Optional outputs: the final state, the state
// at the start of every block (checkpoints for the backward), and y before the
// z gate (lets the backward skip recomputing it).
//
// Precision of long runs: v_exp_f32 is correctly rounded for about 95 % of
// arguments and otherwise mostly one ulp low (mean error -0.04 ulp, measured
// over [-8, 0]), so a slowly decaying state carried through hundreds of
// serial steps drifts low by that bias times the step count. Time-chunked
// float32 runs (CORR) therefore carry each 16-step block's start state with
// one exponential of the block's summed step instead of the product of its
// 16 per-step factors: h_end += (exp(A sum dt) - prod a) h_start. At batch 1,
// dim 1536, seqlen 2048 with A = -U(0, 1) that takes the largest output error
// against float64 from 5.4e-4 to 2.0e-4 (the reference's kernels: 2.6e-4);
// it costs one multiply per state-step (about 10 % of the forward), which
// unchunked runs (rows that fill the GPU, typically short or fast-decaying)
// do not pay, nor do 16-bit inputs, whose outputs are rounded far more
// coarsely than that drift.
//
// Time chunks (when there are too few rows to fill the GPU): a summary pass
// scans every chunk but the last from a zero state and records the state at
// its end and its sum of dt; the main pass then starts chunk c from
//   h = fold over c' < c of  exp(A * sum_dt[c']) * h + h_end[c']
// (the recurrence is affine in h, and the decay over a chunk is the product of
// the per-step decays, exp(A * sum of dt)).
#include "scan_common.h"

namespace mcpu {

constexpr int kFwdWaves = 4;

// MODE: outputs (out, optional ysave / ckpt / last_state), states only
// (ckpt / last_state), the chunk summaries of the chunked scan, or a state
// slice's share of y (ypart; optional ckpt / last_state).
enum FwdMode { kFwdOut = 0, kFwdStates = 1, kFwdSummary = 2, kFwdPart = 3 };

template <typename Tx, int SPL, bool HAS_Z, int MODE, bool CORR>
__global__ void __launch_bounds__(64 * kFwdWaves) scan_fwd_kernel(const ScanParams p) {
  constexpr bool WRITE_OUT = MODE == kFwdOut || MODE == kFwdPart;
  constexpr int W = kFwdWaves;
  constexpr int CH = 4 * W;
  constexpr int NW = 16 * SPL;
  using BC = BCStage<W, SPL>;
  // [buffer][u, delta, z][channel][step]
  __shared__ __align__(16) float s_x[2][3][CH][kScanBlockT];
  __shared__ __align__(16) float s_B[2][NW][kBCPad];
  __shared__ __align__(16) float s_C[2][NW][kBCPad];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane >> 4, j = lane & 15;
  const int c_local = wave * kScanRowsPerWave + r;
  const SliceCtx sc = scan_slice(p);
  const int64_t chunk = sc.bx % p.nchunk;
  // The summary pass has nothing to record for the last chunk.
  if (MODE == kFwdSummary && chunk == p.nchunk - 1) return;
  const RowCtx rc = scan_row_ctx<W>(p, sc.bx / p.nchunk, wave, r);
  // This slice's states, n0 .. n0 + N - 1 of the NS per row of A, the
  // checkpoints, the last state and the chunk summaries.
  const int64_t N = sc.N, NS = p.nstride, n0 = sc.n0, L = p.seqlen;
  const int64_t row = rc.b * p.dim + rc.d;
  // Block indices as uniform 32-bit values: the host's 32-bit tile-offset
  // check keeps seqlen under 2^32 / (element size * channels per tile), so
  // they stay far below 2^31, and the loop's tests on them become scalar
  // compares (the scalar unit has no signed 64-bit compare).
  // This chunk's blocks: [kb0, kb1).
  const int kb0 = __builtin_amdgcn_readfirstlane(static_cast<int>(chunk * p.chunk_blocks));
  const int kb1 = __builtin_amdgcn_readfirstlane(
      static_cast<int>(kb0 + p.chunk_blocks < p.nblk ? kb0 + p.chunk_blocks : p.nblk));

  float A2[SPL], h[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int n = j + 16 * s;
    A2[s] = n < N ? p.A[rc.d * NS + n0 + n] * kLog2e : 0.f;
    h[s] = 0.f;
  }
  if (MODE != kFwdSummary && chunk > 0) {
    // Carry the state over the chunks before this one.
    fold_summaries<SPL>(h, A2, p.sum_h + row * p.nchunk * NS + n0, p.sum_dt + row * p.nchunk, 0, chunk, 1, j,
                        N, NS);
  }
  const float Dd = p.D ? p.D[rc.d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[rc.d] : 0.f;
  float* ck = (MODE != kFwdSummary && p.ckpt) ? p.ckpt + row * p.nblk * NS + n0 : nullptr;
  // Per-step outputs and checkpoints as a uniform base (the workgroup's first
  // row, moved one block at a time) plus a fixed 32-bit per-lane offset.
  const int64_t row0 = rc.b * p.dim + rc.g * p.dpg + rc.cl0;
  const int64_t crow = rc.d - (rc.g * p.dpg + rc.cl0);
  const uint32_t o_off = static_cast<uint32_t>(sizeof(Tx) * (crow * L + j));  // ysave (contiguous)
  // out: strides p.sout, uniform base per block + per-lane offset.
  char* const out0 = static_cast<char*>(p.out) +
      static_cast<int64_t>(sizeof(Tx)) * (rc.b * p.sout[0] + (rc.g * p.dpg + rc.cl0) * p.sout[1]);
  const int64_t out_ts = static_cast<int64_t>(sizeof(Tx)) * p.sout[2];
  const uint32_t out_off = static_cast<uint32_t>(sizeof(Tx) * (crow * p.sout[1] + j * p.sout[2]));
  const uint32_t ck_off = static_cast<uint32_t>(sizeof(float) * (crow * p.nblk * NS + j));
  float dts = 0.f;  // sum of dt over this lane's steps (summary pass)

  const int64_t tb0 = static_cast<int64_t>(kb0) * kScanBlockT;
  XStage<W> xu, xd, xz;
  xu.template init<Tx>(tid, p.u, p.su, p, rc, tb0);
  xd.template init<Tx>(tid, p.delta, p.sdl, p, rc, tb0);
  if (HAS_Z && WRITE_OUT) xz.template init<Tx>(tid, p.z, p.sz, p, rc, tb0);
  BC tb, tc;
  tb.init(tid, p.B + rc.b * p.sB[0] + rc.g * p.sB[1] + n0 * p.sB[3], p.sB, N, tb0);
  if (WRITE_OUT) tc.init(tid, p.C + rc.b * p.sC[0] + rc.g * p.sC[1] + n0 * p.sC[3], p.sC, N, tb0);
  // Only the last block can extend past the sequence end.
  const int64_t t_full = L - L % kScanBlockT;

  // Registers holding the next block's operands between fetch and park.
  uint32_t nu = 0u, nd = 0u, nz = 0u;  // raw bits, widened at the park
  float nB[BC::PER_THREAD], nC[BC::PER_THREAD];
  // Loads the block at t0 and moves the cursors to the next block, except
  // from the chunk's last block (`last`), where they stay: the loop fetches
  // in every iteration, the last one re-reading its own block, so no load or
  // park is ever conditional.
  auto fetch = [&](auto GUARD, int64_t t0, bool last) {
    if (!decltype(GUARD)::value || t0 < t_full) {
      nu = xu.template load<Tx>();
      nd = xd.template load<Tx>();
      if (HAS_Z && WRITE_OUT) nz = xz.template load<Tx>();
      tb.load(nB);
      if (WRITE_OUT) tc.load(nC);
    } else {
      nu = xu.template load_guarded<Tx>(t0, L);
      nd = xd.template load_guarded<Tx>(t0, L);
      if (HAS_Z && WRITE_OUT) nz = xz.template load_guarded<Tx>(t0, L);
      tb.load_guarded(t0, L, nB);
      if (WRITE_OUT) tc.load_guarded(t0, L, nC);
    }
    xu.advance_unless(1, last);
    xd.advance_unless(1, last);
    if (HAS_Z && WRITE_OUT) xz.advance_unless(1, last);
    tb.advance_unless(1, last);
    if (WRITE_OUT) tc.advance_unless(1, last);
  };
  auto park = [&](int buf) {
    (&s_x[buf][0][0][0])[xu.slot] = raw_f32<Tx>(nu);
    (&s_x[buf][1][0][0])[xd.slot] = raw_f32<Tx>(nd);
    if (HAS_Z && WRITE_OUT) (&s_x[buf][2][0][0])[xz.slot] = raw_f32<Tx>(nz);
    tb.park(s_B[buf], nB);
    if (WRITE_OUT) tc.park(s_C[buf], nC);
  };

  if (kb0 < kb1) {
    fetch(std::true_type{}, tb0, kb0 + 1 >= kb1);
    park(static_cast<int>(kb0 & 1));
  }
  __syncthreads();
  // Retire every load issued so far. Otherwise the loop's first use of a
  // value loaded above (bias, D, A) makes the compiler wait for all memory
  // operations at the top of every block, which would also wait for the
  // prefetch of the next block.
  __builtin_amdgcn_s_waitcnt(0);
  if (ck != nullptr && rc.active && kb0 < kb1) {
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      if (j + 16 * s < N) ck[kb0 * NS + j + 16 * s] = h[s];
  }

  // Per block: prefetch the next block, compute this one, park the prefetch,
  // then store. Stores come last so that waiting for the prefetched loads
  // never waits for this block's stores as well. Only the chunk's last block
  // can be partial, so every fetch but the one of that block is unguarded:
  // the loop runs the blocks before the last two with plain fetches, then
  // the last two with guarded ones.
  auto block = [&](auto GUARD, int k) {
    const int buf = static_cast<int>(k & 1);
    const int64_t t0 = static_cast<int64_t>(k) * kScanBlockT;
    const bool has_next = k + 1 < kb1;
    fetch(GUARD, has_next ? t0 + kScanBlockT : t0, k + 2 >= kb1);

    const int64_t t = t0 + j;
    const int nvalid = static_cast<int>(L - t0 < kScanBlockT ? L - t0 : kScanBlockT);
    // This lane's step exists; unguarded blocks are always whole.
    const bool tv = !decltype(GUARD)::value || j < nvalid;
    const float uu = s_x[buf][0][c_local][j];
    const float dl = s_x[buf][1][c_local][j];
    const float zz = (HAS_Z && WRITE_OUT) ? s_x[buf][2][c_local][j] : 0.f;

    float Bv[SPL][kScanBlockT], Cv[SPL][kScanBlockT];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      read_bc_row(s_B[buf], j + 16 * s, Bv[s]);
      if (WRITE_OUT) read_bc_row(s_C[buf], j + 16 * s, Cv[s]);
    }

    float dt = dl + bias;
    if (p.softplus) dt = softplus(dt);
    const float dtu = dt * uu;
    if (MODE == kFwdSummary && tv) dts += dt;

    float pacc[kScanBlockT];
    // CORR: the block's start state and the product of its decay factors.
    // The summary pass needs only each block's end state, so its blocks run
    // from a zero state instead and the start state's decay is added at the
    // end: the same sum without the per-step product. (The states-only mode
    // keeps the product form, so that its checkpoints are bit-identical to
    // those of the output mode.)
    constexpr bool LOCAL = CORR && MODE == kFwdSummary;
    float hstart[SPL], prod[SPL];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      hstart[s] = h[s];
      prod[s] = 1.f;
      if (LOCAL) h[s] = 0.f;
    }
    auto step = [&](auto I) {
      constexpr int i = decltype(I)::value;
      const float dti = row_bcast<i>(dt);
      const float dtui = row_bcast<i>(dtu);
      float acc = 0.f;
#pragma unroll
      for (int s = 0; s < SPL; ++s) {
        const float a = fast_exp2(dti * A2[s]);
        h[s] = fmaf(a, h[s], dtui * Bv[s][i]);
        if (CORR && !LOCAL) prod[s] *= a;
        if (WRITE_OUT) acc = fmaf(h[s], Cv[s][i], acc);
      }
      pacc[i] = acc;
    };
    if (!decltype(GUARD)::value || nvalid == kScanBlockT) {
      static_for<kScanBlockT>(step);
    } else {
      static_for<kScanBlockT>([&](auto I) {
        if (decltype(I)::value < nvalid) step(I);
        else pacc[decltype(I)::value] = 0.f;
      });
    }

    if (CORR) {
      // The start state decays by exp(A * the block's summed step).
      const float bdt = row_allreduce16(j < nvalid ? dt : 0.f);
#pragma unroll
      for (int s = 0; s < SPL; ++s)
        h[s] = fmaf(LOCAL ? fast_exp2(A2[s] * bdt) : fast_exp2(A2[s] * bdt) - prod[s], hstart[s], h[s]);
    }
    float y = 0.f, yg = 0.f;
    if (WRITE_OUT) {
      y = row_reduce_scatter16(pacc, j);
      if (p.D != nullptr) y = fmaf(Dd, uu, y);
      yg = HAS_Z ? y * (zz * sigmoid(zz)) : y;
    }

    park(buf ^ 1);  // in the last iteration a harmless copy into the idle buffer

    if (WRITE_OUT && tv && rc.active) {
      if constexpr (MODE == kFwdPart) {
        // A state slice: its share of y, summed with the others (and D u
        // added, the gate applied) by scan_fwd_finish_kernel.
        p.ypart[((sc.sl * p.batch + rc.b) * p.dim + rc.d) * L + t] = y;
      } else {
        const int64_t o_pos = (row0 * L + t0) * static_cast<int64_t>(sizeof(Tx));
        if (p.ysave != nullptr) buf_st<Tx>(wave_rsrc(static_cast<char*>(p.ysave) + o_pos), o_off, y);
        buf_st<Tx>(wave_rsrc(out0 + t0 * out_ts), out_off, yg);
      }
    }
    if (ck != nullptr && rc.active && k + 1 < kb1) {
#pragma unroll
      for (int s = 0; s < SPL; ++s)
        if (j + 16 * s < N)
          buf_st<float>(wave_rsrc(p.ckpt + (row0 * p.nblk + k + 1) * NS + n0), ck_off + 64 * s, h[s]);
    }
    __syncthreads();
  };
  const int kg = kb1 - 2 > kb0 ? kb1 - 2 : kb0;  // first block whose fetch may be guarded
  for (int k = kb0; k < kg; ++k) block(std::false_type{}, k);
  for (int k = kg; k < kb1; ++k) block(std::true_type{}, k);
  if (MODE == kFwdSummary) {
    dts = row_allreduce16(dts);
    if (rc.active) {
#pragma unroll
      for (int s = 0; s < SPL; ++s)
        if (j + 16 * s < N) p.sum_h[(row * p.nchunk + chunk) * NS + n0 + j + 16 * s] = h[s];
      if (j == 0) p.sum_dt[row * p.nchunk + chunk] = dts;
    }
  } else if (p.last_state != nullptr && rc.active && kb1 == p.nblk) {
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      if (j + 16 * s < N) p.last_state[row * NS + n0 + j + 16 * s] = h[s];
  }
}

// A sliced forward's outputs, per (batch, channel, step): y = the slices'
// shares + D u, ysave = y, out = y silu(z) (or y), with the arithmetic of the
// unsliced kernel's epilogue.
template <typename Tx, bool HAS_Z>
__global__ void __launch_bounds__(256) scan_fwd_finish_kernel(const ScanParams p) {
  const int64_t L = p.seqlen, n = p.batch * p.dim * L;
  const int64_t i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= n) return;
  const int64_t t = i % L, row = i / L, d = row % p.dim, b = row / p.dim;
  float y = 0.f;
  for (int64_t s = 0; s < p.nslices; ++s) y += p.ypart[s * n + i];
  if (p.D != nullptr) y = fmaf(p.D[d], ld<Tx>(p.u, b * p.su[0] + d * p.su[1] + t * p.su[2]), y);
  if (p.ysave != nullptr) st<Tx>(p.ysave, i, y);
  float o = y;
  if (HAS_Z) {
    const float zz = ld<Tx>(p.z, b * p.sz[0] + d * p.sz[1] + t * p.sz[2]);
    o = y * (zz * sigmoid(zz));
  }
  if (p.out != nullptr) st<Tx>(p.out, b * p.sout[0] + d * p.sout[1] + t * p.sout[2], o);
}

template <typename Tx, int SPL, bool HAS_Z, int MODE>
static hipError_t launch_fwd(const ScanParams& p, hipStream_t stream) {
  const int64_t blocks = p.batch * p.ngroups * p.nblk_c * p.nchunk * p.nslices;
  if (std::is_same_v<Tx, float> && p.nchunk > 1)
    hipLaunchKernelGGL((scan_fwd_kernel<Tx, SPL, HAS_Z, MODE, true>), dim3(static_cast<unsigned>(blocks)),
                       dim3(64 * kFwdWaves), 0, stream, p);
  else
    hipLaunchKernelGGL((scan_fwd_kernel<Tx, SPL, HAS_Z, MODE, false>), dim3(static_cast<unsigned>(blocks)),
                       dim3(64 * kFwdWaves), 0, stream, p);
  return hipGetLastError();
}

template <typename Tx, int SPL>
static hipError_t dispatch_fwd_flags(const ScanParams& p, bool write_out, hipStream_t stream) {
  if (p.nchunk > 1) {
    if (hipError_t e = launch_fwd<Tx, SPL, false, kFwdSummary>(p, stream)) return e;
  }
  if (!write_out) return launch_fwd<Tx, SPL, false, kFwdStates>(p, stream);
  if (p.ypart != nullptr) return launch_fwd<Tx, SPL, false, kFwdPart>(p, stream);
  if (p.z != nullptr) return launch_fwd<Tx, SPL, true, kFwdOut>(p, stream);
  return launch_fwd<Tx, SPL, false, kFwdOut>(p, stream);
}

template <typename Tx>
static hipError_t dispatch_fwd_spl(const ScanParams& p, bool write_out, hipStream_t stream) {
  if (p.dstate <= 16) return dispatch_fwd_flags<Tx, 1>(p, write_out, stream);
  if (p.dstate <= 32) return dispatch_fwd_flags<Tx, 2>(p, write_out, stream);
  return dispatch_fwd_flags<Tx, 4>(p, write_out, stream);
}

// Sliced (p.nslices > 1, p.ypart set when write_out): the slices' kernels
// without D and the gate, then the outputs from their shares.
template <typename Tx>
static hipError_t dispatch_fwd_sliced(const ScanParams& p, bool write_out, hipStream_t stream) {
  if (!write_out) return dispatch_fwd_spl<Tx>(p, false, stream);
  ScanParams ps = p;
  ps.D = nullptr;
  ps.z = nullptr;
  ps.ysave = nullptr;
  if (hipError_t e = dispatch_fwd_spl<Tx>(ps, true, stream)) return e;
  const int64_t n = p.batch * p.dim * p.seqlen;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  if (p.z != nullptr) hipLaunchKernelGGL((scan_fwd_finish_kernel<Tx, true>), grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL((scan_fwd_finish_kernel<Tx, false>), grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

int scan_fwd_waves() { return kFwdWaves; }

// The outputs of a sliced forward from its slices' shares of y (p.ypart),
// with D u, ysave and the gate: the complex-A forward's finish.
hipError_t scan_fwd_finish_launch(const ScanParams& p, int dtype, hipStream_t stream) {
  const int64_t n = p.batch * p.dim * p.seqlen;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  const bool z = p.z != nullptr;
  switch (dtype) {
    case MCPU_F32:
      if (z) hipLaunchKernelGGL((scan_fwd_finish_kernel<float, true>), grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL((scan_fwd_finish_kernel<float, false>), grid, dim3(256), 0, stream, p);
      break;
    case MCPU_BF16:
      if (z) hipLaunchKernelGGL((scan_fwd_finish_kernel<bf16, true>), grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL((scan_fwd_finish_kernel<bf16, false>), grid, dim3(256), 0, stream, p);
      break;
    default:
      if (z) hipLaunchKernelGGL((scan_fwd_finish_kernel<f16, true>), grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL((scan_fwd_finish_kernel<f16, false>), grid, dim3(256), 0, stream, p);
      break;
  }
  return hipGetLastError();
}

// Time chunks for a forward with these parameters (p.nblk_c set for
// scan_fwd_waves()): enough chunks to give the GPU's 256 compute units about
// five workgroups each (the kernel's occupancy), and chunks of at most 64
// 16-step blocks, at least two blocks per chunk. Measured: batch 1, dim 1536,
// seqlen 2048 fp32 runs fastest at 13 chunks (40 us against 44 us at 11);
// batch 1, dim 5120, seqlen 16384 bf16 at 16-24 chunks (0.73 ms against
// 0.83 ms at 4), although the summary pass then covers 15/16 of the sequence.
// Short sequences over at least half the GPU's compute units are not cut: the
// summary pass costs more than the parallelism gains there (dim 1536 fp32
// with z: batch 4 x 256 steps 21.9 us unchunked against 29.0 us in 4 chunks,
// batch 4 x 1024 68.1 against 72.7, batch 2 x 512 29.9 against 31.2; but
// batch 2 x 1024 54.3 against 49.3, so 128-255 workgroups keep chunks beyond
// 32 blocks). Sets p.nchunk / p.chunk_blocks; nchunk == 1 when the rows alone
// fill the GPU.
void scan_fwd_chunks(ScanParams& p) {
  const int64_t wgs = p.batch * p.ngroups * p.nblk_c * p.nslices;
  const bool short_rows = (wgs >= 256 && p.nblk <= 64) || (wgs >= 128 && p.nblk <= 32);
  int64_t n = 1;
  if (wgs > 0 && wgs < 512 && p.nblk >= 4 && !short_rows) {
    n = (1280 + wgs - 1) / wgs;
    if (n < p.nblk / 64) n = p.nblk / 64;
    if (n > p.nblk / 2) n = p.nblk / 2;
  }
  p.chunk_blocks = n > 1 ? (p.nblk + n - 1) / n : (p.nblk > 0 ? p.nblk : 1);
  p.nchunk = n > 1 ? (p.nblk + p.chunk_blocks - 1) / p.chunk_blocks : 1;
}

// Launches the forward kernel (p.nblk_c must be computed for scan_fwd_waves()).
// write_out = false computes states only (checkpoints and/or last_state),
// skipping C, z and the outputs.
hipError_t scan_fwd_launch(const ScanParams& p, int dtype, bool write_out, hipStream_t stream) {
  if (p.nslices > 1) {
    switch (dtype) {
      case MCPU_F32: return dispatch_fwd_sliced<float>(p, write_out, stream);
      case MCPU_BF16: return dispatch_fwd_sliced<bf16>(p, write_out, stream);
      default: return dispatch_fwd_sliced<f16>(p, write_out, stream);
    }
  }
  switch (dtype) {
    case MCPU_F32: return dispatch_fwd_spl<float>(p, write_out, stream);
    case MCPU_BF16: return dispatch_fwd_spl<bf16>(p, write_out, stream);
    default: return dispatch_fwd_spl<f16>(p, write_out, stream);
  }
}

}  // namespace mcpu
