// Selective-scan backward on gfx950.
//
// Reverse-mode of the forward recurrence, following the analytic formulas of
// bwd_row_body (reference csrc/selective_scan.cpp:168-248):
//   g    = gh + dy_t C_t            (gh = dLoss/dh_t carried backwards)
//   dC_t += dy_t h_t ;  dB_t += g dt_t u_t
//   gh'  = g exp(dt_t A) ;  ga = gh' h_{t-1} ;  dA += ga dt_t
//   ddt  = <ga, A> + u_t <g, B_t> ;  du_t = dy_t D + dt_t <g, B_t>
//   ddelta_t = ddt * sigmoid(delta_t + bias) if softplus ; gh = gh'
// with dy_t = dout_t z_t s(z_t) and dz_t = dout_t y_t s(z_t)(1 + z_t(1 - s(z_t))).
//
// Instead of the reference's per-thread copy of every state (L * dstate floats
// per row), time is walked backwards in 16-step blocks: each block restarts
// from the checkpointed state at its start (written by the forward kernel),
// recomputes its 16 states and decay factors in registers, then runs the
// reverse recurrence. y_t comes from the forward's saved copy when one is
// given, otherwise from a recomputed <h_t, C_t>. Sums over states use DPP row
// reduce-scatters; dB/dC sums over channels use permlane swaps inside a wave,
// then LDS across the workgroup's W waves, then one partial per workgroup that
// a separate kernel reduces in a fixed order (deterministic, no atomics).
// dA/dD/ddelta_bias are per-(batch, channel) partials reduced over the batch
// the same way. Operands of the next (earlier) block are fetched while the
// current block computes.
#include "scan_common.h"

namespace mcpu {

// SLICED: one state slice of a sliced backward, which writes its <ga, A> and
// <g, B> shares (rpart) in place of du, ddelta, dz, dD and ddelta_bias.
template <typename Tx, int W, int SPL, bool HAS_Z, bool HAS_Y, bool SLICED>
__global__ void __launch_bounds__(64 * W) scan_bwd_kernel(const ScanParams p) {
  constexpr int CH = 4 * W;
  constexpr int NW = 16 * SPL;
  constexpr int T = kScanBlockT;
  using BC = BCStage<W, SPL>;
  // [buffer][u, delta, dout, z, y][channel][step]
  __shared__ __align__(16) float s_x[2][5][CH][T];
  __shared__ __align__(16) float s_B[2][NW][kBCPad];
  __shared__ __align__(16) float s_C[2][NW][kBCPad];
  // [buffer][dB, dC][wave][step][state]: per-wave channel sums awaiting the
  // cross-wave sum.
  __shared__ float s_red[2][2][W][T][NW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane >> 4, j = lane & 15;
  const int c_local = wave * kScanRowsPerWave + r;
  // Time chunk of this workgroup: blocks [kb0, kb1), walked from kb1 - 1 down.
  const SliceCtx sc = scan_slice(p);
  const int64_t chunk = sc.bx % p.nchunk;
  const RowCtx rc = scan_row_ctx<W>(p, sc.bx / p.nchunk, wave, r);
  // This slice's states, n0 .. n0 + N - 1 of the NS per row of A, dlast_state,
  // the checkpoints, the chunk summaries and the dA/dB/dC layouts.
  const int64_t N = sc.N, NS = p.nstride, n0 = sc.n0, L = p.seqlen;
  const int64_t row = rc.b * p.dim + rc.d;
  // Block indices as uniform 32-bit values: the host's 32-bit tile-offset
  // check keeps seqlen under 2^32 / (element size * channels per tile), so
  // they stay far below 2^31, and the loop's tests on them become scalar
  // compares (the scalar unit has no signed 64-bit compare).
  const int kb0 = __builtin_amdgcn_readfirstlane(static_cast<int>(chunk * p.chunk_blocks));
  const int kb1 = __builtin_amdgcn_readfirstlane(
      static_cast<int>(kb0 + p.chunk_blocks < p.nblk ? kb0 + p.chunk_blocks : p.nblk));
  const int kl = kb1 - 1;  // the chunk's last block
  const int64_t t_last = static_cast<int64_t>(kl) * T;
  // Row of the per-(chunk, batch, channel) partials of dA, dD, ddelta_bias.
  const int64_t prow = (chunk * p.batch + rc.b) * p.dim + rc.d;

  float Av[SPL], A2[SPL], gh[SPL], dA_acc[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int n = j + 16 * s;
    Av[s] = n < N ? p.A[rc.d * NS + n0 + n] : 0.f;
    A2[s] = Av[s] * kLog2e;
    gh[s] = (n < N && p.dlast_state != nullptr) ? p.dlast_state[row * NS + n0 + n] : 0.f;
    dA_acc[s] = 0.f;
  }
  if (chunk < p.nchunk - 1) {
    // Carry the adjoint state over the summary units after this chunk:
    // through unit u it maps gh to exp(A * sum_dt[u]) * gh + sum_h[u]
    // (sum_h[u] = the adjoint at u's start from a zero adjoint at its end).
    const int64_t last_unit = (chunk + 1) * p.sum_per_chunk;
    fold_summaries<SPL>(gh, A2, p.sum_h + row * p.nsum * NS + n0, p.sum_dt + row * p.nsum, p.nsum - 1,
                        p.nsum - last_unit, -1, j, N, NS);
  }
  const float Dd = p.D ? p.D[rc.d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[rc.d] : 0.f;
  const bool has_D = p.D != nullptr;
  const bool softplus_on = p.softplus != 0;
  float dD_acc = 0.f, dbias_acc = 0.f;

  // Staging cursors, all positioned on the last block and walked backwards.
  XStage<W> xu, xd, xo, xz, xy;
  xu.template init<Tx>(tid, p.u, p.su, p, rc, t_last);
  xd.template init<Tx>(tid, p.delta, p.sdl, p, rc, t_last);
  const bool has_dout = p.dout != nullptr;
  xo.template init<Tx>(tid, has_dout ? p.dout : p.u, p.sdo, p, rc, t_last);
  if (HAS_Z) xz.template init<Tx>(tid, p.z, p.sz, p, rc, t_last);
  const int64_t sy[3] = {p.dim * L, L, 1};
  if (HAS_Y) xy.template init<Tx>(tid, p.ysave, sy, p, rc, t_last);
  BC tb, tc;
  tb.init(tid, p.B + rc.b * p.sB[0] + rc.g * p.sB[1] + n0 * p.sB[3], p.sB, N, t_last);
  tc.init(tid, p.C + rc.b * p.sC[0] + rc.g * p.sC[1] + n0 * p.sC[3], p.sC, N, t_last);

  // Rows of the workgroup: uniform first row + per-lane offsets (rows past the
  // slice end use the last channel for loads and store nothing).
  const int64_t row0 = rc.b * p.dim + rc.g * p.dpg + rc.cl0;
  const int64_t crow = rc.d - (rc.g * p.dpg + rc.cl0);  // this lane's row within the workgroup
  // Checkpointed state lane j of the current block.
  const char* ck_base = reinterpret_cast<const char*>(p.ckpt + (row0 * p.nblk + kl) * NS + n0);
  const uint32_t ck_off = static_cast<uint32_t>(sizeof(float) * (crow * p.nblk * NS + j));
  // Per-lane outputs at step t0 + j of the current block, each with its own
  // strides: a uniform base (the workgroup's first channel at t0, moved one
  // block back per block) plus a fixed per-lane offset.
  constexpr int64_t esz = sizeof(Tx);
  const int64_t cl = rc.g * p.dpg + rc.cl0;
  char* o_du = static_cast<char*>(p.du) + esz * (rc.b * p.sdu[0] + cl * p.sdu[1] + t_last * p.sdu[2]);
  char* o_dd = static_cast<char*>(p.ddelta) + esz * (rc.b * p.sdd[0] + cl * p.sdd[1] + t_last * p.sdd[2]);
  char* o_dz = HAS_Z ? static_cast<char*>(p.dz) + esz * (rc.b * p.sdz[0] + cl * p.sdz[1] + t_last * p.sdz[2])
                     : nullptr;
  const uint32_t off_du = static_cast<uint32_t>(esz * (crow * p.sdu[1] + j * p.sdu[2]));
  const uint32_t off_dd = static_cast<uint32_t>(esz * (crow * p.sdd[1] + j * p.sdd[2]));
  const uint32_t off_dz = HAS_Z ? static_cast<uint32_t>(esz * (crow * p.sdz[1] + j * p.sdz[2])) : 0u;

  // Cross-wave dB/dC outputs of this thread: element e = (array, step, state).
  // T * NW is a multiple of 64, so the array is uniform over a wave.
  constexpr int NOUT = (2 * T * NW + 64 * W - 1) / (64 * W);
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
    o_red[q] = (arr * W * T + tt) * NW + n;  // index of (arr, wave 0, tt, n) in s_red[buf]
    o_ok[q] = e < 2 * T * NW && n < N;
    o_part[q] = reinterpret_cast<char*>((arr == 0 ? p.dB_part : p.dC_part) + part_row * NS + n0);
    o_poff[q] = static_cast<uint32_t>(sizeof(float) * (tt * NS + n));
  }

  uint32_t nu = 0u, nd = 0u, no = 0u, nz = 0u, ny = 0u;  // raw bits, widened at the park
  float nB[BC::PER_THREAD], nC[BC::PER_THREAD];
  float nh0[SPL];
  // Checkpointed state lanes past dstate load lane 0's entry and read as 0.
  uint32_t ck_lane[SPL];
  bool ck_ok[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    ck_ok[s] = j + 16 * s < N;
    ck_lane[s] = ck_ok[s] ? ck_off + 64 * s : ck_off - sizeof(float) * j;
  }
  // Loads the operands of the block at t0 (full unless GUARD) and moves every
  // cursor one block back, except from block 0 (`stay`). Every iteration
  // fetches, block 0 re-reading itself, and nothing consumes a prefetched
  // value before park(), so no load is conditional and the loads are only
  // waited for at the park.
  auto fetch = [&](auto GUARD, int64_t t0, bool stay) {
    if constexpr (decltype(GUARD)::value) {
      nu = xu.template load_guarded<Tx>(t0, L);
      nd = xd.template load_guarded<Tx>(t0, L);
      no = xo.template load_guarded<Tx>(t0, L);
      if (HAS_Z) nz = xz.template load_guarded<Tx>(t0, L);
      if (HAS_Y) ny = xy.template load_guarded<Tx>(t0, L);
      tb.load_guarded(t0, L, nB);
      tc.load_guarded(t0, L, nC);
    } else {
      nu = xu.template load<Tx>();
      nd = xd.template load<Tx>();
      no = xo.template load<Tx>();
      if (HAS_Z) nz = xz.template load<Tx>();
      if (HAS_Y) ny = xy.template load<Tx>();
      tb.load(nB);
      tc.load(nC);
    }
#pragma unroll
    for (int s = 0; s < SPL; ++s) nh0[s] = buf_ld<float>(wave_rsrc(ck_base), ck_lane[s]);
    xu.advance_unless(-1, stay);
    xd.advance_unless(-1, stay);
    xo.advance_unless(-1, stay);
    if (HAS_Z) xz.advance_unless(-1, stay);
    if (HAS_Y) xy.advance_unless(-1, stay);
    tb.advance_unless(-1, stay);
    tc.advance_unless(-1, stay);
    ck_base -= stay ? 0 : sizeof(float) * NS;
  };
  auto park = [&](int buf) {
    (&s_x[buf][0][0][0])[xu.slot] = raw_f32<Tx>(nu);
    (&s_x[buf][1][0][0])[xd.slot] = raw_f32<Tx>(nd);
    (&s_x[buf][2][0][0])[xo.slot] = has_dout ? raw_f32<Tx>(no) : 0.f;
    if (HAS_Z) (&s_x[buf][3][0][0])[xz.slot] = raw_f32<Tx>(nz);
    if (HAS_Y) (&s_x[buf][4][0][0])[xy.slot] = raw_f32<Tx>(ny);
    tb.park(s_B[buf], nB);
    tc.park(s_C[buf], nC);
  };

  float h0[SPL];
  if (kb0 < kb1) {
    fetch(std::true_type{}, t_last, kl == kb0);
    park(static_cast<int>(kl & 1));
#pragma unroll
    for (int s = 0; s < SPL; ++s) h0[s] = ck_ok[s] ? nh0[s] : 0.f;
  }
  __syncthreads();
  // Retire every load issued so far, so the loop never has to wait for the
  // prefetch of the next block on behalf of a value loaded above.
  __builtin_amdgcn_s_waitcnt(0);

  // One block; FULL = all 16 steps exist (every block but possibly the last).
  auto block = [&](auto FULL, int k, int nvalid) {
    constexpr bool full = decltype(FULL)::value;
    const int buf = static_cast<int>(k & 1);
    const int64_t t0 = static_cast<int64_t>(k) * T;
    // The block before this one (always full), or this block again from the
    // chunk's first block (guarded like this block).
    // Full blocks load at the cursor either way (block k - 1, or block k
    // again from the chunk's first block, where the cursor stayed), so one
    // branch-free fetch covers both.
    if constexpr (full) {
      fetch(std::false_type{}, t0 - T, k - 1 <= kb0);
    } else {
      if (k > kb0) fetch(std::false_type{}, t0 - T, k - 1 <= kb0);
      else fetch(std::true_type{}, t0, true);
    }
    auto valid = [&](int i) { return full || i < nvalid; };
    // Wave priority: raised for the recompute and the reverse pass, lowered
    // for the block's tail (reductions, park, stores), so a wave that reaches
    // its tail first yields the vector ALU to the waves still in their
    // bodies and the workgroup arrives at the barrier closer together
    // (measured 3-4 % faster at batch 8, dim 1536, seqlen 1024).
    __builtin_amdgcn_s_setprio(2);

    const bool tv = full || j < nvalid;
    const float uu = s_x[buf][0][c_local][j];
    const float dl = s_x[buf][1][c_local][j];
    const float go = s_x[buf][2][c_local][j];
    const float zz = HAS_Z ? s_x[buf][3][c_local][j] : 0.f;

    float Bv[SPL][T], Cv[SPL][T];
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      read_bc_row(s_B[buf], j + 16 * s, Bv[s]);
      read_bc_row(s_C[buf], j + 16 * s, Cv[s]);
    }

    const float pre = dl + bias;
    float dt = pre, sg_pre = 1.f;
    if (softplus_on) dt = softplus_sigmoid(pre, sg_pre);
    const float dtu = dt * uu;
    // The reverse pass broadcasts its own copies of dt and dt*u: the compiler
    // folds a DPP broadcast into its multiplies only when they follow it
    // closely, so one broadcast shared by the recompute and the reverse pass
    // (which identical values would be merged into) costs a move per step.
    // Rows past the slice end contribute nothing to dB/dC: their dy and
    // dt*u read as zero in the reverse pass.
    const float dt_r = dt + 0.0f, dtu_r = rc.active ? dtu + 0.0f : 0.f;

    // Forward recompute of the block's states and decay factors.
    float hs[SPL][T], as[SPL][T], pacc[T];
    {
      float hc[SPL];
#pragma unroll
      for (int s = 0; s < SPL; ++s) hc[s] = h0[s];
      static_for<T>([&](auto I) {
        constexpr int i = decltype(I)::value;
        if (valid(i)) {
          const float dti = row_bcast<i>(dt);
          const float dtui = row_bcast<i>(dtu);
          float acc = 0.f;
#pragma unroll
          for (int s = 0; s < SPL; ++s) {
            const float a = fast_exp2(dti * A2[s]);
            hc[s] = fmaf(a, hc[s], dtui * Bv[s][i]);
            hs[s][i] = hc[s];
            as[s][i] = a;
            if (HAS_Z && !HAS_Y) acc = fmaf(hc[s], Cv[s][i], acc);
          }
          pacc[i] = acc;
        } else {
#pragma unroll
          for (int s = 0; s < SPL; ++s) hs[s][i] = as[s][i] = 0.f;
          pacc[i] = 0.f;
        }
      });
    }

    // Output gating: dy_t and dz_t for the step this lane owns.
    float dy = rc.active ? go : 0.f, dzv = 0.f;
    if (HAS_Z) {
      float y;
      if (HAS_Y) {
        y = s_x[buf][4][c_local][j];
      } else {
        y = row_reduce_scatter16(pacc, j);
        if (has_D) y = fmaf(Dd, uu, y);
      }
      const float sg = sigmoid(zz);
      dzv = go * y * sg * (1.f + zz * (1.f - sg));
      dy = rc.active ? go * zz * sg : 0.f;
    }

    // Reverse recurrence over the block.
    float r1[T], r2[T], dBc[SPL][T], dCc[SPL][T];
    static_for<T>([&](auto I) {
      constexpr int i = T - 1 - decltype(I)::value;
      if (valid(i)) {
        // dt, dt*u and dy of step i from its owner lane: fused into the
        // instructions that consume them (DPP row broadcasts).
        const float dyi = row_bcast<i>(dy);
        float acc1 = 0.f, acc2 = 0.f;
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
          const float g = fmac_bcast<i>(gh[s], dy, Cv[s][i]);
          dCc[s][i] = dyi * hs[s][i];
          const float hp = i > 0 ? hs[s][i > 0 ? i - 1 : 0] : h0[s];
          gh[s] = g * as[s][i];
          const float ga = gh[s] * hp;
          dA_acc[s] = fmac_bcast<i>(dA_acc[s], dt_r, ga);
          acc1 = fmaf(ga, Av[s], acc1);
          acc2 = fmaf(g, Bv[s][i], acc2);
          dBc[s][i] = mul_bcast<i>(dtu_r, g);
        }
        r1[i] = acc1;
        r2[i] = acc2;
      } else {
        r1[i] = r2[i] = 0.f;
#pragma unroll
        for (int s = 0; s < SPL; ++s) dBc[s][i] = dCc[s][i] = 0.f;
      }
    });

    __builtin_amdgcn_s_setprio(0);
    const float R1 = row_reduce_scatter16(r1, j);  // <ga, A> for step t
    const float R2 = row_reduce_scatter16(r2, j);  // <g, B_t> for step t
    float ddt = fmaf(uu, R2, R1);
    const float duv = fmaf(dy, Dd, dt * R2);
    if (softplus_on) ddt *= sg_pre;
    if (tv) {
      dD_acc = fmaf(dy, uu, dD_acc);
      dbias_acc += ddt;
    }

    // dB/dC: sum over the wave's 4 channels, park for the cross-wave sum.
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      float yB[4], yC[4];
      wave_rows_reduce_scatter(dBc[s], yB);
      wave_rows_reduce_scatter(dCc[s], yC);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        s_red[buf][0][wave][4 * r + q][j + 16 * s] = yB[q];
        s_red[buf][1][wave][4 * r + q][j + 16 * s] = yC[q];
      }
    }
    park(buf ^ 1);  // from the chunk's first block a harmless copy into the idle buffer
    // The next block's checkpointed state, taken here: the empty asm keeps
    // the select (and the wait for its load) ahead of this block's stores.
    // Left to the compiler it sinks to the next block's first use, past the
    // stores, and its wait then covers the stores' completion as well.
#pragma unroll
    for (int s = 0; s < SPL; ++s) {
      h0[s] = ck_ok[s] ? nh0[s] : 0.f;
      asm volatile("" : "+v"(h0[s]));
    }
    // Stores after the park, so waiting for the prefetch never waits for them.
    if (tv && rc.active) {
      if constexpr (SLICED) {
        // A state slice: its <ga, A> and <g, B> shares, from which
        // scan_bwd_finish_kernel forms du, ddelta, dz, dD and ddelta_bias.
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
      o_part[q] -= sizeof(float) * T * NS;
    }
  };

  if (kb0 < kb1) {
    const int nlast = static_cast<int>(L - t_last < T ? L - t_last : T);
    if (nlast == T) block(std::true_type{}, kl, T);
    else block(std::false_type{}, kl, nlast);
  }
  for (int k = kl - 1; k >= kb0; --k) block(std::true_type{}, k, T);

  if (rc.active) {
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      if (j + 16 * s < N) p.dA_part[prow * NS + n0 + j + 16 * s] = dA_acc[s];
  }
  dD_acc = row_allreduce16(dD_acc);
  dbias_acc = row_allreduce16(dbias_acc);
  if (rc.active && j == 0 && !SLICED) {  // a sliced backward forms them in its finish kernel
    p.dD_part[prow] = dD_acc;
    p.dbias_part[prow] = dbias_acc;
  }
}

// A sliced backward's per-step gradients, one wave per (batch, channel) row,
// its lanes walking the steps: R1 = the slices' <ga, A> shares summed, R2 =
// their <g, B_t>; with dt, dy and dz from the row's inputs as the unsliced
// kernel forms them,
//   ddelta = (R1 + u R2) softplus'(pre), du = dy D + dt R2,
//   dz = dout y s(z) (1 + z (1 - s(z))),
// and the row's sums dD = sum dy u and ddelta_bias = sum ddelta into the
// per-(batch, channel) partials.
template <typename Tx, bool HAS_Z>
__global__ void __launch_bounds__(256) scan_bwd_finish_kernel(const ScanParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = blockIdx.x * 4ll + (threadIdx.x >> 6);
  if (row >= p.batch * p.dim) return;  // the whole wave
  const int64_t d = row % p.dim, b = row / p.dim, L = p.seqlen, n = p.batch * p.dim * L;
  const float Dd = p.D ? p.D[d] : 0.f;
  const float bias = p.delta_bias ? p.delta_bias[d] : 0.f;
  float dD = 0.f, dbias = 0.f;
  for (int64_t t = lane; t < L; t += 64) {
    const int64_t i = row * L + t;
    float R1 = 0.f, R2 = 0.f;
    for (int64_t s = 0; s < p.nslices; ++s) {
      R1 += p.rpart[s * n + i];
      R2 += p.rpart[(p.nslices + s) * n + i];
    }
    const float uu = ld<Tx>(p.u, b * p.su[0] + d * p.su[1] + t * p.su[2]);
    const float dl = ld<Tx>(p.delta, b * p.sdl[0] + d * p.sdl[1] + t * p.sdl[2]);
    const float go = p.dout ? ld<Tx>(p.dout, b * p.sdo[0] + d * p.sdo[1] + t * p.sdo[2]) : 0.f;
    const float pre = dl + bias;
    float dt = pre, sg_pre = 1.f;
    if (p.softplus) dt = softplus_sigmoid(pre, sg_pre);
    float dy = go;
    if (HAS_Z) {
      const float zz = ld<Tx>(p.z, b * p.sz[0] + d * p.sz[1] + t * p.sz[2]);
      const float y = ld<Tx>(p.ysave, i);
      const float sg = sigmoid(zz);
      st<Tx>(p.dz, b * p.sdz[0] + d * p.sdz[1] + t * p.sdz[2], go * y * sg * (1.f + zz * (1.f - sg)));
      dy = go * zz * sg;
    }
    float ddt = fmaf(uu, R2, R1);
    const float duv = fmaf(dy, Dd, dt * R2);
    if (p.softplus) ddt *= sg_pre;
    dD = fmaf(dy, uu, dD);
    dbias += ddt;
    st<Tx>(p.du, b * p.sdu[0] + d * p.sdu[1] + t * p.sdu[2], duv);
    st<Tx>(p.ddelta, b * p.sdd[0] + d * p.sdd[1] + t * p.sdd[2], ddt);
  }
  dD = row_allreduce16(dD);
  dD = swap_sum<16>(dD, dD);
  dD = swap_sum<32>(dD, dD);
  dbias = row_allreduce16(dbias);
  dbias = swap_sum<16>(dbias, dbias);
  dbias = swap_sum<32>(dbias, dbias);
  if (lane == 0) {
    p.dD_part[row] = dD;
    p.dbias_part[row] = dbias;
  }
}

hipError_t scan_bwd_finish_launch(const ScanParams& p, int dtype, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((p.batch * p.dim + 3) / 4));
  const bool z = p.z != nullptr;
  switch (dtype) {
    case MCPU_F32:
      if (z) hipLaunchKernelGGL((scan_bwd_finish_kernel<float, true>), grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL((scan_bwd_finish_kernel<float, false>), grid, dim3(256), 0, stream, p);
      break;
    case MCPU_BF16:
      if (z) hipLaunchKernelGGL((scan_bwd_finish_kernel<bf16, true>), grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL((scan_bwd_finish_kernel<bf16, false>), grid, dim3(256), 0, stream, p);
      break;
    default:
      if (z) hipLaunchKernelGGL((scan_bwd_finish_kernel<f16, true>), grid, dim3(256), 0, stream, p);
      else hipLaunchKernelGGL((scan_bwd_finish_kernel<f16, false>), grid, dim3(256), 0, stream, p);
      break;
  }
  return hipGetLastError();
}

// Adjoint summaries of a time-chunked backward. For every summary unit u
// after the first chunk, runs the adjoint recurrence g = gh + dy_t C_t,
// gh = g exp(dt_t A) backwards over the unit from gh = 0 at its end and
// records gh at the unit's start (sum_h) and the unit's sum of dt (sum_dt).
// The recurrence is affine in gh, so the backward kernel rebuilds the adjoint
// entering chunk c from these and dlast_state alone. Needs only delta, dout,
// z and C: no states, no B. Units are finer than chunks so that this pass,
// which skips the first chunk, still fills the GPU.
template <typename Tx, int SPL, bool HAS_Z>
__global__ void __launch_bounds__(64 * kScanSumWaves) scan_bwd_summary_kernel(const ScanParams p) {
  constexpr int W = kScanSumWaves;
  constexpr int CH = 4 * W;
  constexpr int NW = 16 * SPL;
  constexpr int T = kScanBlockT;
  using BC = BCStage<W, SPL>;
  __shared__ __align__(16) float s_x[2][3][CH][T];  // delta, dout, z
  __shared__ __align__(16) float s_C[2][NW][kBCPad];

  const SliceCtx sc = scan_slice(p);
  const int64_t unit = sc.bx % p.nsum;
  if (unit < p.sum_per_chunk) return;  // the first chunk's units feed no carry
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r = lane >> 4, j = lane & 15;
  const int c_local = wave * kScanRowsPerWave + r;
  const RowCtx rc = scan_row_ctx<W>(p, sc.bx / p.nsum, wave, r);
  const int64_t N = sc.N, NS = p.nstride, n0 = sc.n0, L = p.seqlen;
  const int64_t row = rc.b * p.dim + rc.d;
  const int kb0 = __builtin_amdgcn_readfirstlane(static_cast<int>(unit * p.sum_blocks));
  const int kb1 = __builtin_amdgcn_readfirstlane(
      static_cast<int>(kb0 + p.sum_blocks < p.nblk ? kb0 + p.sum_blocks : p.nblk));
  const int kl = kb1 - 1;
  const int64_t t_last = static_cast<int64_t>(kl) * T;

  float A2[SPL], gh[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int n = j + 16 * s;
    A2[s] = n < N ? p.A[rc.d * NS + n0 + n] * kLog2e : 0.f;
    gh[s] = 0.f;
  }
  const float bias = p.delta_bias ? p.delta_bias[rc.d] : 0.f;
  const bool softplus_on = p.softplus != 0;
  const bool has_dout = p.dout != nullptr;
  float dts = 0.f;

  XStage<W> xd, xo, xz;
  xd.template init<Tx>(tid, p.delta, p.sdl, p, rc, t_last);
  xo.template init<Tx>(tid, has_dout ? p.dout : p.delta, p.sdo, p, rc, t_last);
  if (HAS_Z) xz.template init<Tx>(tid, p.z, p.sz, p, rc, t_last);
  BC tc;
  tc.init(tid, p.C + rc.b * p.sC[0] + rc.g * p.sC[1] + n0 * p.sC[3], p.sC, N, t_last);

  uint32_t nd = 0u, no = 0u, nz = 0u;  // raw bits, widened at the park
  float nC[BC::PER_THREAD];
  auto fetch = [&](auto GUARD, int64_t t0, bool stay) {
    if constexpr (decltype(GUARD)::value) {
      nd = xd.template load_guarded<Tx>(t0, L);
      no = xo.template load_guarded<Tx>(t0, L);
      if (HAS_Z) nz = xz.template load_guarded<Tx>(t0, L);
      tc.load_guarded(t0, L, nC);
    } else {
      nd = xd.template load<Tx>();
      no = xo.template load<Tx>();
      if (HAS_Z) nz = xz.template load<Tx>();
      tc.load(nC);
    }
    xd.advance_unless(-1, stay);
    xo.advance_unless(-1, stay);
    if (HAS_Z) xz.advance_unless(-1, stay);
    tc.advance_unless(-1, stay);
  };
  auto park = [&](int buf) {
    (&s_x[buf][0][0][0])[xd.slot] = raw_f32<Tx>(nd);
    (&s_x[buf][1][0][0])[xo.slot] = has_dout ? raw_f32<Tx>(no) : 0.f;
    if (HAS_Z) (&s_x[buf][2][0][0])[xz.slot] = raw_f32<Tx>(nz);
    tc.park(s_C[buf], nC);
  };

  fetch(std::true_type{}, t_last, kl == kb0);
  park(static_cast<int>(kl & 1));
  __syncthreads();
  __builtin_amdgcn_s_waitcnt(0);

  auto block = [&](auto FULL, int k, int nvalid) {
    constexpr bool full = decltype(FULL)::value;
    const int buf = static_cast<int>(k & 1);
    const int64_t t0 = static_cast<int64_t>(k) * T;
    // Full blocks load at the cursor either way (block k - 1, or block k
    // again from the chunk's first block, where the cursor stayed), so one
    // branch-free fetch covers both.
    if constexpr (full) {
      fetch(std::false_type{}, t0 - T, k - 1 <= kb0);
    } else {
      if (k > kb0) fetch(std::false_type{}, t0 - T, k - 1 <= kb0);
      else fetch(std::true_type{}, t0, true);
    }
    const float dl = s_x[buf][0][c_local][j];
    const float go = s_x[buf][1][c_local][j];
    const float zz = HAS_Z ? s_x[buf][2][c_local][j] : 0.f;
    float Cv[SPL][T];
#pragma unroll
    for (int s = 0; s < SPL; ++s) read_bc_row(s_C[buf], j + 16 * s, Cv[s]);
    float dt = dl + bias;
    if (softplus_on) dt = softplus(dt);
    float dy = go;
    if (HAS_Z) dy = go * zz * sigmoid(zz);
    if (full || j < nvalid) dts += dt;
    static_for<T>([&](auto I) {
      constexpr int i = T - 1 - decltype(I)::value;
      if (full || i < nvalid) {
        const float dti = row_bcast<i>(dt);
        const float dyi = row_bcast<i>(dy);
#pragma unroll
        for (int s = 0; s < SPL; ++s) {
          const float a = fast_exp2(dti * A2[s]);
          gh[s] = fmaf(dyi, Cv[s][i], gh[s]) * a;
        }
      }
    });
    park(buf ^ 1);
    __syncthreads();
  };

  const int nlast = static_cast<int>(L - t_last < T ? L - t_last : T);
  if (nlast == T) block(std::true_type{}, kl, T);
  else block(std::false_type{}, kl, nlast);
  for (int k = kl - 1; k >= kb0; --k) block(std::true_type{}, k, T);

  dts = row_allreduce16(dts);
  if (rc.active) {
#pragma unroll
    for (int s = 0; s < SPL; ++s)
      if (j + 16 * s < N) p.sum_h[(row * p.nsum + unit) * NS + n0 + j + 16 * s] = gh[s];
    if (j == 0) p.sum_dt[row * p.nsum + unit] = dts;
  }
}

// All reductions of one backward in one launch, as a grid-stride loop over the
// concatenation of
//   dB, dC:  out[s, e] = sum over channel blocks c of part[s, c, e]  (four
//            elements per item when the slice size allows, else one)
//   dA, dD, ddelta_bias:  out[e] = sum over the batch of part[b, e]
// Every element is summed in the fixed order c = 0, 1, ... or b = 0, 1, ...
// (deterministic, no atomics). A job with part == nullptr is absent.
struct ReduceJob {
  const float* part;
  float* out;
  int64_t outer;   // slices (dB/dC) or 1 (batch reductions)
  int64_t nsum;    // terms per element: channel blocks or batch
  int64_t per;     // elements per slice
  int64_t items;   // work items of this job
  int vec;         // 4: float4 items, 1: scalar items
};
struct ReduceJobs {
  ReduceJob job[5];
  int njobs;
};

// The terms are loaded 32 (then 16) at a time, so a launch that has about
// one wave per SIMD waits for one or two memory round trips per item instead
// of a load-add chain, and added in the same fixed order c = 0, 1, ...
template <int U, typename V, typename Ld, typename Add>
__device__ __forceinline__ void sum_terms(int64_t& c, int64_t nsum, Ld ld, Add add) {
  for (; c + U <= nsum; c += U) {
    V v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ld(c + u);
#pragma unroll
    for (int u = 0; u < U; ++u) add(v[u]);
  }
}

__device__ __forceinline__ void reduce_item(const ReduceJob& j, int64_t i) {
  if (j.vec == 4) {
    const int64_t per4 = j.per / 4;
    const int64_t sl = i / per4, e = (i % per4) * 4;
    const float* src = j.part + sl * j.nsum * j.per + e;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    auto ld = [&](int64_t c) { return *reinterpret_cast<const float4*>(src + c * j.per); };
    auto add = [&](const float4 v) {
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    };
    int64_t c = 0;
    sum_terms<32, float4>(c, j.nsum, ld, add);
    sum_terms<16, float4>(c, j.nsum, ld, add);
    for (; c < j.nsum; ++c) add(ld(c));
    *reinterpret_cast<float4*>(j.out + sl * j.per + e) = acc;
  } else {
    const int64_t sl = i / j.per, e = i % j.per;
    const float* src = j.part + sl * j.nsum * j.per + e;
    float acc = 0.f;
    auto ld = [&](int64_t c) { return src[c * j.per]; };
    auto add = [&](const float v) { acc += v; };
    int64_t c = 0;
    sum_terms<32, float>(c, j.nsum, ld, add);
    sum_terms<16, float>(c, j.nsum, ld, add);
    for (; c < j.nsum; ++c) add(ld(c));
    j.out[sl * j.per + e] = acc;
  }
}

__global__ void __launch_bounds__(256) reduce_jobs_kernel(const ReduceJobs jobs, int64_t total) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += 256ll * gridDim.x) {
    int64_t k = i;
    for (int q = 0; q < jobs.njobs; ++q) {
      if (k < jobs.job[q].items) {
        reduce_item(jobs.job[q], k);
        break;
      }
      k -= jobs.job[q].items;
    }
  }
}

template <typename Tx, int W, int SPL, bool SLICED>
static hipError_t launch_bwd_zys(const ScanParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.batch * p.ngroups * p.nblk_c * p.nchunk * p.nslices));
  const dim3 block(64 * W);
  if (p.z != nullptr && p.ysave != nullptr)
    hipLaunchKernelGGL((scan_bwd_kernel<Tx, W, SPL, true, true, SLICED>), grid, block, 0, stream, p);
  else if (p.z != nullptr)
    hipLaunchKernelGGL((scan_bwd_kernel<Tx, W, SPL, true, false, SLICED>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((scan_bwd_kernel<Tx, W, SPL, false, false, SLICED>), grid, block, 0, stream, p);
  return hipGetLastError();
}

// Sliced backwards (p.rpart set) run 16-state slices, so only SPL 1 has a
// sliced form.
template <typename Tx, int W, int SPL>
static hipError_t launch_bwd_zy(const ScanParams& p, hipStream_t stream) {
  if constexpr (SPL == 1)
    if (p.rpart != nullptr) return launch_bwd_zys<Tx, W, SPL, true>(p, stream);
  return launch_bwd_zys<Tx, W, SPL, false>(p, stream);
}

// Wider workgroups (8 or 12 waves) only for dstate <= 16, where their LDS fits.
template <typename Tx>
static hipError_t launch_bwd_w(const ScanParams& p, int waves, hipStream_t stream) {
  if (p.dstate <= 16) {
    if (waves == 12) return launch_bwd_zy<Tx, 12, 1>(p, stream);
    if (waves == 8) return launch_bwd_zy<Tx, 8, 1>(p, stream);
    return launch_bwd_zy<Tx, 4, 1>(p, stream);
  }
  if (p.dstate <= 32) return launch_bwd_zy<Tx, 4, 2>(p, stream);
  return launch_bwd_zy<Tx, 4, 4>(p, stream);
}

// Waves per backward workgroup. More waves mean fewer dB/dC partials to
// reduce; the choice keeps enough workgroups to fill the GPU's 256 compute
// units in whole rounds.
int scan_bwd_waves(int64_t batch, int64_t ngroups, int64_t dpg, int64_t dstate) {
  if (dstate > 16) return 4;  // keeps the per-workgroup LDS small
  const int64_t slices = batch * ngroups;
  for (int w : {12, 8}) {
    const int64_t wgs = slices * ((dpg + 4 * w - 1) / (4 * w));
    const int64_t pad = slices * ((dpg + 4 * w - 1) / (4 * w)) * 4 * w - slices * dpg;
    if (wgs >= 256 && wgs % 256 == 0 && pad == 0) return w;
  }
  // Time-chunked shapes with many channels per slice: 8 waves halve the
  // per-channel-block dB/dC partials (measured: batch 1, dim 5120, seqlen
  // 16384 bf16 is 3 % faster than with 4 waves; 16 waves, one workgroup per
  // CU, are 10 % slower again).
  if (dpg >= 4096 && dpg % 32 == 0) return 8;
  return 4;
}

template <typename Tx, int SPL>
static hipError_t launch_bwd_summary(const ScanParams& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.batch * p.ngroups * p.nblk_c * p.nsum * p.nslices));
  const dim3 block(64 * kScanSumWaves);
  if (p.z != nullptr)
    hipLaunchKernelGGL((scan_bwd_summary_kernel<Tx, SPL, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((scan_bwd_summary_kernel<Tx, SPL, false>), grid, block, 0, stream, p);
  return hipGetLastError();
}

template <typename Tx>
static hipError_t launch_bwd_summary_spl(const ScanParams& p, hipStream_t stream) {
  if (p.dstate <= 16) return launch_bwd_summary<Tx, 1>(p, stream);
  if (p.dstate <= 32) return launch_bwd_summary<Tx, 2>(p, stream);
  return launch_bwd_summary<Tx, 4>(p, stream);
}

// Adjoint summaries of a chunked backward (p.nchunk > 1, p.nblk_c for
// kScanSumWaves waves, p.sum_h / p.sum_dt set).
hipError_t scan_bwd_summary_launch(const ScanParams& p, int dtype, hipStream_t stream) {
  switch (dtype) {
    case MCPU_F32: return launch_bwd_summary_spl<float>(p, stream);
    case MCPU_BF16: return launch_bwd_summary_spl<bf16>(p, stream);
    default: return launch_bwd_summary_spl<f16>(p, stream);
  }
}

hipError_t scan_bwd_launch(const ScanParams& p, int dtype, int waves, hipStream_t stream) {
  switch (dtype) {
    case MCPU_F32: return launch_bwd_w<float>(p, waves, stream);
    case MCPU_BF16: return launch_bwd_w<bf16>(p, waves, stream);
    default: return launch_bwd_w<f16>(p, waves, stream);
  }
}

static unsigned grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65535 * 16) g = 65535 * 16;
  return static_cast<unsigned>(g < 1 ? 1 : g);
}

// Sums up to five partial arrays in one launch: out[s, e] = sum over c of
// part[s, c, e] (outer slices s, nsum terms c, per elements e), each in the
// fixed order c = 0, 1, ... Entries with part == nullptr are skipped.
hipError_t partial_sums_launch(const PartialSum* sums, int n, hipStream_t stream) {
  ReduceJobs jobs{};
  int64_t total = 0;
  for (int i = 0; i < n && jobs.njobs < 5; ++i) {
    const PartialSum& ps = sums[i];
    if (ps.part == nullptr || ps.outer * ps.per == 0) continue;
    ReduceJob& j = jobs.job[jobs.njobs++];
    j.part = ps.part;
    j.out = ps.out;
    j.outer = ps.outer;
    j.nsum = ps.nsum;
    j.per = ps.per;
    const bool aligned = reinterpret_cast<uintptr_t>(ps.part) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(ps.out) % 16 == 0;
    j.vec = ps.per % 4 == 0 && aligned ? 4 : 1;
    j.items = ps.outer * ps.per / j.vec;
    total += j.items;
  }
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(reduce_jobs_kernel, dim3(grid_for(total)), dim3(256), 0, stream, jobs, total);
  return hipGetLastError();
}

// Sums the backward's partials: dB/dC over channel blocks (`slices` slices of
// `per_slice` elements, `nblk_c` blocks each; skipped when dB_part is null),
// and dA / dD / ddelta_bias over the batch (each skipped when its part is null).
hipError_t scan_reduce_launch(const float* dB_part, float* dB, const float* dC_part, float* dC,
                              int64_t slices, int64_t nblk_c, int64_t per_slice,
                              const float* dA_part, float* dA, int64_t nA, const float* dD_part,
                              float* dD, const float* dbias_part, float* dbias, int64_t dim,
                              int64_t batch, hipStream_t stream) {
  ReduceJobs jobs{};
  int64_t total = 0;
  auto add = [&](const float* part, float* out, int64_t outer, int64_t nsum, int64_t per) {
    if (part == nullptr || outer * per == 0) return;
    ReduceJob& j = jobs.job[jobs.njobs++];
    j.part = part;
    j.out = out;
    j.outer = outer;
    j.nsum = nsum;
    j.per = per;
    const bool aligned = reinterpret_cast<uintptr_t>(part) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(out) % 16 == 0;
    j.vec = per % 4 == 0 && aligned ? 4 : 1;
    j.items = outer * per / j.vec;
    total += j.items;
  };
  add(dB_part, dB, slices, nblk_c, per_slice);
  add(dC_part, dC, slices, nblk_c, per_slice);
  add(dA_part, dA, 1, batch, nA);
  add(dD_part, dD, 1, batch, dim);
  add(dbias_part, dbias, 1, batch, dim);
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(reduce_jobs_kernel, dim3(grid_for(total)), dim3(256), 0, stream, jobs, total);
  return hipGetLastError();
}

}  // namespace mcpu
