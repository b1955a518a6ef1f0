// Mamba-2 SSD scan (mamba_ssm's mamba_chunk_scan_combined) on gfx950, in
// 64-step chunks with the chunk-local contractions on the matrix cores
// (v_mfma_f32_16x16x4_f32, float32 in and out; the storage type is widened
// when a tile is staged in LDS).
//
// Per batch row b and head h (group g), with a_t = dt_t A and, inside a
// chunk, cs_t = a_0 + ... + a_t (so cs <= 0 and decays are exp of differences):
//   forward
//     F1  S_c  = sum_s exp(cs_L - cs_s) dt_s x_s B_s^T          (chunk-end state from 0)
//     F2  H_c  = exp(cs_L(c-1)) H_{c-1} + S_{c-1}               (state entering chunk c)
//     F3  Y    = (C B^T o M) (dt x) + diag(exp(cs)) C H_c^T + D x,  M[t][s] = exp(cs_t - cs_s) [s <= t]
//         out  = Y silu(z)
//   backward (dY the gradient of Y, dH_c^out that of the state leaving chunk c)
//     K1  intra-chunk: dG = dY (dt x)^T, dCB = dG o M, d(dt x) += (CB o M)^T dY,
//         dC += dCB B, dB += dCB^T C, dcs from dG o G, and the seed
//         E_c = (diag(exp(cs)) C)^T dY of dL/dH_c
//     K2  dH^out_c = dH^in_{c+1} ; dH^in_c = exp(cs_L) dH^out_c + E_c (reverse over
//         chunks); dcs_L += <dH^out_c, exp(cs_L) H_c>
//     K3  state terms: d(dt x) += B~ dH^out^T, dC += diag(exp(cs)) dY H_c,
//         dB += diag(w) (dt x) dH^out (B~ = diag(w) B, w_s = exp(cs_L - cs_s)),
//         their dcs terms, then da = suffix sums of dcs, ddt, dx and the
//         per-chunk partials of dA, dD, ddt_bias
//     a fixed-order reduce sums dB/dC over a group's heads and the partials.
// Chunks past the sequence end are padded with dt = 0 (no decay, no input).
#include "mcpu_common.h"
#include "scan_common.h"
#include "ssd_params.h"

namespace mcpu {

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int Q = kSsdQ;
constexpr int QP = Q + 4;          // padded row lengths of the LDS tiles
constexpr int XP = kSsdMaxP + 4;
constexpr int NP = kSsdMaxN + 4;
constexpr int kThreads = 256;

// acc[j] += A(16 x K) B(K x 16 columns 16 j ..) for column tiles j < nt
// (uniform), operands float32 in LDS: A(i, k) = a[i ai + k ak] (a at the
// strip's first row), B(k, c) = b[k bk + c bj]. In each
// v_mfma_f32_16x16x4_f32 lane l supplies A(l % 16, k + l / 16) and
// B(k + l / 16, l % 16); lane l ends holding D(4 (l / 16) + e, l % 16) in
// acc[j][e].
template <int NT>
__device__ __forceinline__ void mma_strip(v4f (&acc)[NT], int nt, const float* a, int ai, int ak,
                                          const float* b, int bk, int bj, int K) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, q = lane >> 4;
  const float* pa = a + r * ai + q * ak;
  const float* pb = b + q * bk + r * bj;
  for (int k = 0; k < K; k += 4) {
    const float av = pa[k * ak];
#pragma unroll
    for (int j = 0; j < NT; ++j)
      if (j < nt) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, pb[k * bk + 16 * j * bj], acc[j], 0, 0, 0);
  }
}

template <int NT>
__device__ __forceinline__ void zero(v4f (&acc)[NT]) {
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
}

// Inclusive prefix sum over the 64 lanes of a wave (lane 0 first).
__device__ __forceinline__ float wave_prefix_sum(float v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave as a float pair hi + lo:
// each addition keeps its rounding error (Knuth's TwoSum) in lo, so a
// difference (hi_t - hi_s) + (lo_t - lo_s) is accurate relative to itself
// rather than to the size of the running sums.
__device__ __forceinline__ void wave_prefix_sum2(float v, float& hi, float& lo) {
  const int lane = threadIdx.x & 63;
  hi = v;
  lo = 0.f;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float oh = __shfl_up(hi, d, 64), ol = __shfl_up(lo, d, 64);
    if (lane >= d) {
      const float sum = hi + oh;
      const float bv = sum - hi;
      const float err = (hi - (sum - bv)) + (oh - bv);
      hi = sum;
      lo = (lo + ol) + err;
    }
  }
}

// exp(cs_t - cs_s) from the float pairs of the running sums.
__device__ __forceinline__ float seg_exp(const float* cs, const float* lo, int t, int s) {
  return fast_exp((cs[t] - cs[s]) + (lo[t] - lo[s]));
}

// Inclusive suffix sum over the 64 lanes of a wave (lane 63 first).
__device__ __forceinline__ float wave_suffix_sum(float v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float o = __shfl_down(v, d, 64);
    if (lane + d < 64) v += o;
  }
  return v;
}

// Sum over the 64 lanes of a wave, in a fixed order, in every lane.
__device__ __forceinline__ float wave_total(float v) {
  v = row_allreduce16(v);
  v = swap_sum<32>(v, v);
  return swap_sum<16>(v, v);
}

// The effective step of (b, t, h) and, when grad, d(step)/d(raw dt): the
// softplus derivative, zero where the clamp is active. 0 past the sequence.
__device__ __forceinline__ float ssd_step(const SsdParams& p, int64_t b, int64_t t, int64_t h, float* grad) {
  if (t >= p.seqlen) {
    if (grad) *grad = 0.f;
    return 0.f;
  }
  const float pre = p.dt[(b * p.seqlen + t) * p.nheads + h] + (p.dt_bias ? p.dt_bias[h] : 0.f);
  float sg = 1.f;
  float st = pre;
  if (p.softplus) st = softplus_sigmoid(pre, sg);
  if (p.clamp) {
    const bool inside = st >= p.dt_lo && st <= p.dt_hi;
    st = fminf(fmaxf(st, p.dt_lo), p.dt_hi);
    if (!inside) sg = 0.f;
  }
  if (grad) *grad = sg;
  return st;
}

// Chunk row (b, h, c) of the cs / step arrays.
__device__ __forceinline__ int64_t chunk_row(const SsdParams& p, int64_t b, int64_t h, int64_t c) {
  return ((b * p.nheads + h) * p.nchunks + c) * Q;
}

// Offset of the (b, c, h) state block in states / dstates.
__device__ __forceinline__ int64_t state_block(const SsdParams& p, int64_t b, int64_t c, int64_t h) {
  return ((b * p.nchunks + c) * p.nheads + h) * p.headdim * p.dstate;
}

}  // namespace

// F1: steps and running decays of the chunk (saved for F3 and the backward),
// and the chunk-end state S(p, n) = sum_s exp(cs_L - cs_s) dt_s x_s(p) B_s(n).
// Grid (nchunks, nheads, batch); wave w computes state rows p in [16 w, 16 w + 16).
template <typename Tx>
__global__ void __launch_bounds__(kThreads) ssd_chunk_state_kernel(const SsdParams p) {
  __shared__ float s_x[Q][XP];
  __shared__ float s_B[Q][NP];
  __shared__ float s_cs[Q], s_csl[Q], s_dt[Q];
  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t g = h / (H / G);
  const int64_t t0 = c * Q;
  if (wave == 0) {
    const float st = ssd_step(p, b, t0 + lane, h, nullptr);
    float cs, csl;
    wave_prefix_sum2(st * p.A[h], cs, csl);
    s_cs[lane] = cs;
    s_csl[lane] = csl;
    s_dt[lane] = st;
    const int64_t row = chunk_row(p, b, h, c);
    p.cs[row + lane] = cs;
    p.cs_lo[row + lane] = csl;
    p.step[row + lane] = st;
  }
  __syncthreads();
  for (int e = tid; e < Q * P; e += kThreads) {
    const int t = e / P, pp = e % P;
    const float v = t0 + t < L ? ld<Tx>(p.x, ((b * L + t0 + t) * H + h) * P + pp) : 0.f;
    s_x[t][pp] = v * s_dt[t] * seg_exp(s_cs, s_csl, Q - 1, t);
  }
  for (int e = tid; e < Q * N; e += kThreads) {
    const int t = e / N, n = e % N;
    s_B[t][n] = t0 + t < L ? ld<Tx>(p.B, ((b * L + t0 + t) * G + g) * N + n) : 0.f;
  }
  __syncthreads();
  if (16 * wave < P) {
    v4f acc[kSsdMaxN / 16];
    zero(acc);
    mma_strip(acc, static_cast<int>(N / 16), &s_x[0][16 * wave], 1, XP, &s_B[0][0], NP, 1, Q);
    const int r = lane & 15, q = lane >> 4;
    float* dst = p.states + state_block(p, b, c, h);
#pragma unroll
    for (int j = 0; j < kSsdMaxN / 16; ++j)
      if (j < N / 16)
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(16 * wave + 4 * q + e) * N + 16 * j + r] = acc[j][e];
  }
}

// F2: walks the chunks in order, replacing each chunk-end state by the state
// entering the chunk, H_c = exp(cs_L(c-1)) H_{c-1} + S_{c-1} (H_0 = the
// initial state or 0), and writes the final state. One thread per state
// element; grid (nslices, nheads, batch).
__global__ void __launch_bounds__(kThreads) ssd_state_pass_kernel(const SsdParams p) {
  const int64_t PN = p.headdim * p.dstate, H = p.nheads;
  const int64_t e = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  const int64_t h = blockIdx.y, b = blockIdx.z;
  if (e >= PN) return;
  float run = p.init ? p.init[(b * H + h) * PN + e] : 0.f;
  float* st = p.states + state_block(p, b, 0, h) + e;
  const int64_t cstride = H * PN;
  const float* csl = p.cs + chunk_row(p, b, h, 0) + (Q - 1);
  for (int64_t c = 0; c < p.nchunks; ++c) {
    const float s = st[c * cstride];
    const float d = fast_exp(csl[c * Q]);
    st[c * cstride] = run;
    run = fmaf(d, run, s);
  }
  if (p.final_states) p.final_states[(b * H + h) * PN + e] = run;
}

// F3: the chunk's outputs, Y = (C B^T o M) (dt x) + diag(exp(cs)) C H^T + D x,
// out = Y silu(z) (and Y itself into ysave when the backward needs it).
// Grid (nchunks, nheads, batch); wave w computes rows t in [16 w, 16 w + 16).
template <typename Tx, bool HAS_Z>
__global__ void __launch_bounds__(kThreads) ssd_chunk_scan_kernel(const SsdParams p) {
  __shared__ float s_C[Q][NP];
  __shared__ float s_BH[Q][NP];     // B (Q x N), then the entering state H (P x N)
  __shared__ float s_G[Q][QP];
  __shared__ float s_X[Q][XP];      // dt x
  __shared__ float s_cs[Q], s_csl[Q], s_dt[Q];
  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t g = h / (H / G);
  const int64_t t0 = c * Q;
  const int64_t row = chunk_row(p, b, h, c);
  if (tid < Q) {
    s_cs[tid] = p.cs[row + tid];
    s_csl[tid] = p.cs_lo[row + tid];
    s_dt[tid] = p.step[row + tid];
  }
  for (int e = tid; e < Q * N; e += kThreads) {
    const int t = e / N, n = e % N;
    const bool ok = t0 + t < L;
    const int64_t at = ((b * L + t0 + t) * G + g) * N + n;
    s_C[t][n] = ok ? ld<Tx>(p.C, at) : 0.f;
    s_BH[t][n] = ok ? ld<Tx>(p.B, at) : 0.f;
  }
  __syncthreads();
  {
    v4f cb[Q / 16];
    zero(cb);
    mma_strip(cb, Q / 16, &s_C[16 * wave][0], NP, 1, &s_BH[0][0], 1, NP, static_cast<int>(N));
#pragma unroll
    for (int j = 0; j < Q / 16; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * wave + 4 * q + e, s = 16 * j + r;
        s_G[t][s] = s <= t ? cb[j][e] * seg_exp(s_cs, s_csl, t, s) : 0.f;
      }
  }
  __syncthreads();
  for (int e = tid; e < Q * P; e += kThreads) {
    const int t = e / P, pp = e % P;
    s_X[t][pp] = t0 + t < L ? ld<Tx>(p.x, ((b * L + t0 + t) * H + h) * P + pp) * s_dt[t] : 0.f;
  }
  const float* hin = p.states + state_block(p, b, c, h);
  for (int e = tid; e < P * N; e += kThreads) s_BH[e / N][e % N] = hin[e];
  __syncthreads();
  v4f y1[kSsdMaxP / 16], y2[kSsdMaxP / 16];
  zero(y1);
  zero(y2);
  const int np = static_cast<int>(P / 16);
  mma_strip(y1, np, &s_G[16 * wave][0], QP, 1, &s_X[0][0], XP, 1, Q);
  mma_strip(y2, np, &s_C[16 * wave][0], NP, 1, &s_BH[0][0], 1, NP, static_cast<int>(N));
#pragma unroll
  for (int j = 0; j < kSsdMaxP / 16; ++j) {
    if (j >= np) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * wave + 4 * q + e;
      const int64_t pp = 16 * j + r;
      if (t0 + t >= L) continue;
      const int64_t at = ((b * L + t0 + t) * H + h) * P + pp;
      float y = y1[j][e] + fast_exp(s_cs[t]) * y2[j][e];
      if (p.D) y = fmaf(p.D[h * P + pp], ld<Tx>(p.x, at), y);
      if (HAS_Z) {
        if (p.ysave) st<Tx>(p.ysave, at, y);
        const float zz = ld<Tx>(p.z, at);
        y *= zz * sigmoid(zz);
      }
      st<Tx>(p.out, at, y);
    }
  }
}

// dY = dout silu(z) (dout without z) at x-layout index `at`; also dz there.
template <typename Tx, bool HAS_Z>
__device__ __forceinline__ float ssd_dy(const SsdParams& p, int64_t at, bool write_dz) {
  const float go = ld<Tx>(p.dout, at);
  if (!HAS_Z) return go;
  const float zz = ld<Tx>(p.z, at);
  const float sg = sigmoid(zz);
  if (write_dz) {
    const float y = ld<Tx>(p.ysave, at);
    st<Tx>(p.dz, at, go * y * sg * (1.f + zz * (1.f - sg)));
  }
  return go * zz * sg;
}

// K1: intra-chunk gradients and the seed E_c of dL/dH_c. Grid (nchunks,
// nheads, batch); wave w owns rows [16 w, 16 w + 16) of every Q-row product.
template <typename Tx, bool HAS_Z>
__global__ void __launch_bounds__(kThreads) ssd_bwd_intra_kernel(const SsdParams p) {
  __shared__ float s_C[Q][NP];
  __shared__ float s_B[Q][NP];
  __shared__ float s_X[Q][XP];      // dt x
  __shared__ float s_dY[Q][XP];
  __shared__ float s_G[Q][QP];      // G = C B^T o M
  __shared__ float s_dCB[Q][QP];
  __shared__ float s_colp[16][Q];   // column sums of dG o G, per (wave, lane quarter)
  __shared__ float s_cs[Q], s_csl[Q], s_dt[Q];
  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t g = h / (H / G);
  const int64_t t0 = c * Q;
  const int64_t row = chunk_row(p, b, h, c);
  if (tid < Q) {
    s_cs[tid] = p.cs[row + tid];
    s_csl[tid] = p.cs_lo[row + tid];
    s_dt[tid] = p.step[row + tid];
  }
  __syncthreads();
  for (int e = tid; e < Q * N; e += kThreads) {
    const int t = e / N, n = e % N;
    const bool ok = t0 + t < L;
    const int64_t at = ((b * L + t0 + t) * G + g) * N + n;
    s_C[t][n] = ok ? ld<Tx>(p.C, at) : 0.f;
    s_B[t][n] = ok ? ld<Tx>(p.B, at) : 0.f;
  }
  for (int e = tid; e < Q * P; e += kThreads) {
    const int t = e / P, pp = e % P;
    const bool ok = t0 + t < L;
    const int64_t at = ((b * L + t0 + t) * H + h) * P + pp;
    s_X[t][pp] = ok ? ld<Tx>(p.x, at) * s_dt[t] : 0.f;
    s_dY[t][pp] = ok ? ssd_dy<Tx, HAS_Z>(p, at, true) : 0.f;
  }
  __syncthreads();
  // CB = C B^T and dG = dY (dt x)^T, rows t of this wave, all columns s.
  v4f cb[Q / 16], dg[Q / 16];
  zero(cb);
  zero(dg);
  mma_strip(cb, Q / 16, &s_C[16 * wave][0], NP, 1, &s_B[0][0], 1, NP, static_cast<int>(N));
  mma_strip(dg, Q / 16, &s_dY[16 * wave][0], XP, 1, &s_X[0][0], 1, XP, static_cast<int>(P));
  // G = CB o M, dCB = dG o M, R = dG o G: row sums of R in the wave, column
  // sums through LDS; both in a fixed order.
  float rowsum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < Q / 16; ++j) {
    float colsum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * wave + 4 * q + e, s = 16 * j + r;
      const float m = s <= t ? seg_exp(s_cs, s_csl, t, s) : 0.f;
      const float gv = cb[j][e] * m, dcb = dg[j][e] * m;
      const float rv = dg[j][e] * gv;
      cb[j][e] = gv;
      dg[j][e] = dcb;
      rowsum[e] += rv;
      colsum += rv;
    }
    s_colp[4 * wave + q][16 * j + r] = colsum;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) rowsum[e] = row_allreduce16(rowsum[e]);
  __syncthreads();
  // dcs_intra[t] = sum_s R[t][s] - sum_s R[s][t]; lane r == e of quarter q holds row t.
  {
    float mine = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (r == e) mine = rowsum[e];
    if (r < 4) {
      const int t = 16 * wave + 4 * q + r;
      float col = 0.f;
      for (int k = 0; k < 16; ++k) col += s_colp[k][t];
      p.dcs[row + t] = mine - col;
    }
  }
#pragma unroll
  for (int j = 0; j < Q / 16; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * wave + 4 * q + e, s = 16 * j + r;
      s_G[t][s] = cb[j][e];
      s_dCB[t][s] = dg[j][e];
    }
  __syncthreads();
  const int np = static_cast<int>(P / 16), nn = static_cast<int>(N / 16);
  {
    // d(dt x)[s][p] += sum_t G[t][s] dY[t][p]: rows s of this wave.
    v4f dx[kSsdMaxP / 16];
    zero(dx);
    mma_strip(dx, np, &s_G[0][16 * wave], 1, QP, &s_dY[0][0], XP, 1, Q);
#pragma unroll
    for (int j = 0; j < kSsdMaxP / 16; ++j) {
      if (j >= np) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int s = 16 * wave + 4 * q + e;
        if (t0 + s < L) p.dxt[((b * L + t0 + s) * H + h) * P + 16 * j + r] = dx[j][e];
      }
    }
  }
  {
    // dC[t][n] = sum_s dCB[t][s] B[s][n] ; dB[s][n] = sum_t dCB[t][s] C[t][n].
    v4f dcv[kSsdMaxN / 16], dbv[kSsdMaxN / 16];
    zero(dcv);
    zero(dbv);
    mma_strip(dcv, nn, &s_dCB[16 * wave][0], QP, 1, &s_B[0][0], NP, 1, Q);
    mma_strip(dbv, nn, &s_dCB[0][16 * wave], 1, QP, &s_C[0][0], NP, 1, Q);
#pragma unroll
    for (int j = 0; j < kSsdMaxN / 16; ++j) {
      if (j >= nn) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * wave + 4 * q + e;
        if (t0 + t >= L) continue;
        const int64_t at = ((b * L + t0 + t) * H + h) * N + 16 * j + r;
        p.dC_head[at] = dcv[j][e];
        p.dB_head[at] = dbv[j][e];
      }
    }
  }
  __syncthreads();
  // E_c[n][p] = sum_t exp(cs_t) C[t][n] dY[t][p], stored like a state (p, n).
  for (int e = tid; e < Q * N; e += kThreads) s_C[e / N][e % N] *= fast_exp(s_cs[e / N]);
  __syncthreads();
  float* dst = p.dstates + state_block(p, b, c, h);
  for (int strip = wave; strip < N / 16; strip += 4) {
    v4f ev[kSsdMaxP / 16];
    zero(ev);
    mma_strip(ev, np, &s_C[0][16 * strip], 1, NP, &s_dY[0][0], XP, 1, Q);
#pragma unroll
    for (int j = 0; j < kSsdMaxP / 16; ++j) {
      if (j >= np) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[(16 * j + r) * N + 16 * strip + 4 * q + e] = ev[j][e];
    }
  }
}

// K2: walks the chunks from the last: dH^out_c (gradient of the state leaving
// chunk c) replaces E_c in dstates, dH^in_c = exp(cs_L) dH^out_c + E_c
// carries on, and <dH^out_c, exp(cs_L) H_c> (this slice's share of dL/dcs_L)
// goes to dcsL. The gradient of the initial state is what is left after
// chunk 0. Grid (nslices, nheads, batch).
__global__ void __launch_bounds__(kThreads) ssd_bwd_pass_kernel(const SsdParams p) {
  __shared__ float s_part[kThreads / 64];
  const int64_t PN = p.headdim * p.dstate, H = p.nheads;
  const int64_t e = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool ok = e < PN;
  float run = (ok && p.dfinal) ? p.dfinal[(b * H + h) * PN + e] : 0.f;
  const int64_t base = state_block(p, b, 0, h) + (ok ? e : 0);
  const int64_t cstride = H * PN;
  const float* csl = p.cs + chunk_row(p, b, h, 0) + (Q - 1);
  for (int64_t c = p.nchunks - 1; c >= 0; --c) {
    const float ec = ok ? p.dstates[base + c * cstride] : 0.f;
    const float hin = ok ? p.states[base + c * cstride] : 0.f;
    const float d = fast_exp(csl[c * Q]);
    if (ok) p.dstates[base + c * cstride] = run;
    const float part = wave_total(run * d * hin);
    if (lane == 0) s_part[wave] = part;
    __syncthreads();
    if (threadIdx.x == 0)
      p.dcsL[(chunk_row(p, b, h, 0) / Q + c) * p.nslices + blockIdx.x] =
          (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    __syncthreads();
    run = fmaf(d, run, ec);
  }
  if (ok && p.dinit) p.dinit[(b * H + h) * PN + e] = run;
}

// K3: the state terms and the combine. Grid (nchunks, nheads, batch); wave w
// owns rows [16 w, 16 w + 16) of every Q-row product.
template <typename Tx, bool HAS_Z>
__global__ void __launch_bounds__(kThreads) ssd_bwd_state_kernel(const SsdParams p) {
  __shared__ float s_X[Q][XP];      // dt x
  __shared__ float s_dY[Q][XP];
  __shared__ float s_dH[kSsdMaxP][NP];
  __shared__ float s_H[kSsdMaxP][NP];
  __shared__ float s_Bt[Q][NP];     // exp(cs_L - cs_s) B
  __shared__ float s_dcs[Q];
  __shared__ float s_tot[4];
  __shared__ float s_dD[16][kSsdMaxP];
  __shared__ float s_cs[Q], s_csl[Q], s_dt[Q];
  __shared__ float s_w[Q];          // exp(cs_L - cs_s)
  const int64_t c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t g = h / (H / G);
  const int64_t t0 = c * Q;
  const int64_t row = chunk_row(p, b, h, c);
  if (tid < Q) {
    s_cs[tid] = p.cs[row + tid];
    s_csl[tid] = p.cs_lo[row + tid];
    s_dt[tid] = p.step[row + tid];
  }
  __syncthreads();
  if (tid < Q) s_w[tid] = seg_exp(s_cs, s_csl, Q - 1, tid);
  for (int e = tid; e < Q * P; e += kThreads) {
    const int t = e / P, pp = e % P;
    const bool ok = t0 + t < L;
    const int64_t at = ((b * L + t0 + t) * H + h) * P + pp;
    s_X[t][pp] = ok ? ld<Tx>(p.x, at) * s_dt[t] : 0.f;
    s_dY[t][pp] = ok ? ssd_dy<Tx, HAS_Z>(p, at, false) : 0.f;
  }
  const int64_t sb = state_block(p, b, c, h);
  for (int e = tid; e < P * N; e += kThreads) {
    s_dH[e / N][e % N] = p.dstates[sb + e];
    s_H[e / N][e % N] = p.states[sb + e];
  }
  __syncthreads();
  for (int e = tid; e < Q * N; e += kThreads) {
    const int t = e / N, n = e % N;
    s_Bt[t][n] = t0 + t < L ? ld<Tx>(p.B, ((b * L + t0 + t) * G + g) * N + n) * s_w[t] : 0.f;
  }
  __syncthreads();
  const int np = static_cast<int>(P / 16), nn = static_cast<int>(N / 16);
  // T = (dt x) dH^out (rows s), dYH = dY H (rows t): both Q x N.
  v4f tv[kSsdMaxN / 16], yh[kSsdMaxN / 16];
  zero(tv);
  zero(yh);
  mma_strip(tv, nn, &s_X[16 * wave][0], XP, 1, &s_dH[0][0], NP, 1, static_cast<int>(P));
  mma_strip(yh, nn, &s_dY[16 * wave][0], XP, 1, &s_H[0][0], NP, 1, static_cast<int>(P));
  float a_row[4] = {0.f, 0.f, 0.f, 0.f};  // sum_n C dC_state
  float b_row[4] = {0.f, 0.f, 0.f, 0.f};  // sum_n B~ T
#pragma unroll
  for (int j = 0; j < kSsdMaxN / 16; ++j) {
    if (j >= nn) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * wave + 4 * q + e;
      const int64_t n = 16 * j + r;
      const float bt = s_Bt[t][n];
      b_row[e] = fmaf(bt, tv[j][e], b_row[e]);
      if (t0 + t >= L) continue;
      const float ecs = fast_exp(s_cs[t]);
      const float dcs_state = ecs * yh[j][e];
      const int64_t at = ((b * L + t0 + t) * H + h) * N + n;
      a_row[e] = fmaf(ld<Tx>(p.C, ((b * L + t0 + t) * G + g) * N + n), dcs_state, a_row[e]);
      p.dC_head[at] += dcs_state;
      p.dB_head[at] += s_w[t] * tv[j][e];
    }
  }
  // d(dt x) state part: B~ dH^out^T (rows s, columns p).
  v4f dxs[kSsdMaxP / 16];
  zero(dxs);
  mma_strip(dxs, np, &s_Bt[16 * wave][0], NP, 1, &s_dH[0][0], 1, NP, static_cast<int>(N));
  float c_row[4] = {0.f, 0.f, 0.f, 0.f};  // sum_p d(dt x) x
  float dD_col[kSsdMaxP / 16];
#pragma unroll
  for (int j = 0; j < kSsdMaxP / 16; ++j) {
    dD_col[j] = 0.f;
    if (j >= np) continue;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * wave + 4 * q + e;
      if (t0 + t >= L) continue;
      const int64_t pp = 16 * j + r;
      const int64_t at = ((b * L + t0 + t) * H + h) * P + pp;
      const float dxt = p.dxt[at] + dxs[j][e];
      const float xv = ld<Tx>(p.x, at);
      const float dy = s_dY[t][pp];
      c_row[e] = fmaf(dxt, xv, c_row[e]);
      dD_col[j] = fmaf(dy, xv, dD_col[j]);
      float dxv = dxt * s_dt[t];
      if (p.D) dxv = fmaf(p.D[h * P + pp], dy, dxv);
      st<Tx>(p.dx, at, dxv);
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a_row[e] = row_allreduce16(a_row[e]);
    b_row[e] = row_allreduce16(b_row[e]);
    c_row[e] = row_allreduce16(c_row[e]);
  }
#pragma unroll
  for (int j = 0; j < kSsdMaxP / 16; ++j)
    if (j < np) s_dD[4 * wave + q][16 * j + r] = dD_col[j];
  // sum over the chunk of sum_n B~ T (the cs_L term), in a fixed order
  float bsum = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) bsum += b_row[e];  // this quarter's 4 rows, every lane of the row alike
  bsum = (r == 0) ? bsum : 0.f;
  bsum = wave_total(bsum);
  if (lane == 0) s_tot[wave] = bsum;
  // dcs (without the cs_L terms) for the 4 rows this lane quarter holds
  if (r < 4) {
    float av = 0.f, bv = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (r == e) {
        av = a_row[e];
        bv = b_row[e];
      }
    const int t = 16 * wave + 4 * q + r;
    s_dcs[t] = p.dcs[row + t] + av - bv;
  }
  __syncthreads();
  float c_mine = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (r == e) c_mine = c_row[e];
  if (wave == 0) {
    // add the cs_L terms, then da = suffix sums of dcs over the chunk
    float v = s_dcs[lane];
    if (lane == Q - 1) {
      float l = (s_tot[0] + s_tot[1]) + (s_tot[2] + s_tot[3]);
      const float* dl = p.dcsL + (chunk_row(p, b, h, 0) / Q + c) * p.nslices;
      for (int64_t k = 0; k < p.nslices; ++k) l += dl[k];
      v += l;
    }
    const float da = wave_suffix_sum(v);
    s_dcs[lane] = da;
  }
  __syncthreads();
  // dstep = sum_p d(dt x) x + da A, then through softplus / clamp / bias.
  float ddt_raw = 0.f, dA_term = 0.f;
  if (r < 4) {
    const int t = 16 * wave + 4 * q + r;
    if (t0 + t < L) {
      float gfac;
      ssd_step(p, b, t0 + t, h, &gfac);
      const float da = s_dcs[t];
      const float dstep = fmaf(da, p.A[h], c_mine);
      ddt_raw = dstep * gfac;
      dA_term = da * s_dt[t];
      p.ddt[(b * L + t0 + t) * H + h] = ddt_raw;
    }
  }
  // per-chunk partials: dA, ddt_bias (wave sums, then the 4 waves), dD (columns)
  const float wa = wave_total(dA_term), wb = wave_total(ddt_raw);
  __syncthreads();
  if (lane == 0) {
    s_dcs[wave] = wa;
    s_dcs[4 + wave] = wb;
  }
  __syncthreads();
  const int64_t prt = (b * p.nchunks + c) * H + h;
  if (tid == 0) {
    p.dA_part[prt] = (s_dcs[0] + s_dcs[1]) + (s_dcs[2] + s_dcs[3]);
    p.dbias_part[prt] = (s_dcs[4] + s_dcs[5]) + (s_dcs[6] + s_dcs[7]);
  }
  if (tid < P) {
    float v = 0.f;
    for (int k = 0; k < 16; ++k) v += s_dD[k][tid];
    p.dD_part[prt * P + tid] = v;
  }
}

namespace {

template <typename Tx>
hipError_t fwd_t(const SsdParams& p, hipStream_t st) {
  const dim3 chunks(static_cast<unsigned>(p.nchunks), static_cast<unsigned>(p.nheads),
                    static_cast<unsigned>(p.batch));
  hipLaunchKernelGGL(ssd_chunk_state_kernel<Tx>, chunks, dim3(kThreads), 0, st, p);
  if (hipError_t e = hipGetLastError()) return e;
  const dim3 slices(static_cast<unsigned>(p.nslices), static_cast<unsigned>(p.nheads),
                    static_cast<unsigned>(p.batch));
  hipLaunchKernelGGL(ssd_state_pass_kernel, slices, dim3(kThreads), 0, st, p);
  if (hipError_t e = hipGetLastError()) return e;
  if (p.z) hipLaunchKernelGGL((ssd_chunk_scan_kernel<Tx, true>), chunks, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL((ssd_chunk_scan_kernel<Tx, false>), chunks, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <typename Tx>
hipError_t bwd_t(const SsdParams& p, hipStream_t st) {
  const dim3 chunks(static_cast<unsigned>(p.nchunks), static_cast<unsigned>(p.nheads),
                    static_cast<unsigned>(p.batch));
  const dim3 slices(static_cast<unsigned>(p.nslices), static_cast<unsigned>(p.nheads),
                    static_cast<unsigned>(p.batch));
  if (p.z) hipLaunchKernelGGL((ssd_bwd_intra_kernel<Tx, true>), chunks, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL((ssd_bwd_intra_kernel<Tx, false>), chunks, dim3(kThreads), 0, st, p);
  if (hipError_t e = hipGetLastError()) return e;
  hipLaunchKernelGGL(ssd_bwd_pass_kernel, slices, dim3(kThreads), 0, st, p);
  if (hipError_t e = hipGetLastError()) return e;
  if (p.z) hipLaunchKernelGGL((ssd_bwd_state_kernel<Tx, true>), chunks, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL((ssd_bwd_state_kernel<Tx, false>), chunks, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

}  // namespace

hipError_t ssd_fwd_launch(const SsdParams& p, int dtype, hipStream_t st) {
  switch (dtype) {
    case MCPU_F32: return fwd_t<float>(p, st);
    case MCPU_BF16: return fwd_t<bf16>(p, st);
    default: return fwd_t<f16>(p, st);
  }
}

hipError_t ssd_bwd_launch(const SsdParams& p, int dtype, hipStream_t st) {
  switch (dtype) {
    case MCPU_F32: return bwd_t<float>(p, st);
    case MCPU_BF16: return bwd_t<bf16>(p, st);
    default: return bwd_t<f16>(p, st);
  }
}

}  // namespace mcpu
