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
//     K1  the seed E_c = (diag(exp(cs)) C)^T dY of dL/dH_c from the chunk's own outputs
//     K2  dH^out_c = dH^in_{c+1} ; dH^in_c = exp(cs_L) dH^out_c + E_c (reverse over
//         chunks); dcs_L += <dH^out_c, exp(cs_L) H_c>
//     K3  per chunk: dG = dY (dt x)^T, dCB = dG o M, d(dt x) = (CB o M)^T dY
//         + B~ dH^out^T, dC = dCB B + diag(exp(cs)) dY H_c, dB = dCB^T C +
//         diag(w) (dt x) dH^out (B~ = diag(w) B, w_s = exp(cs_L - cs_s)), dcs
//         from all of them, da = suffix sums of dcs, then ddt, dx, dz and the
//         per-chunk partials of dA, dD, ddt_bias
//     a fixed-order reduce sums dB/dC over the head blocks of a group and the
//     partials.
// The chunk kernels (F1, F3, K1, K3) give a workgroup one chunk of `hb` heads
// of one group: B, C and C B^T are staged and formed once and each head reuses
// them; K3 keeps dB and dC of the block's heads in matrix-core accumulators.
// Chunks past the sequence end are padded with dt = 0 (no decay, no input).
#include "mcpu_common.h"
#include "scan_common.h"
#include "ssd_params.h"

namespace mcpu {

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int Q = kSsdQ;
constexpr int QP = Q + 4;          // padded row lengths of the LDS tiles (16-byte multiples)
constexpr int XP = kSsdMaxP + 4;
constexpr int NP = kSsdMaxN + 4;
constexpr int kThreads = 256;

__device__ __forceinline__ v4f mfma4(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// acc[j] += A(16 x K) B(K x 16 columns 16 j ..) for column tiles j < NTC,
// operands float32 in LDS: A(i, k) = a[i ai + k ak] (a at the strip's first
// row), times `as` when SCALE (the lane's own row factor), B(k, c) = b[k bk +
// c bj]. K is a multiple of 16: four k-steps of operands are read before
// their products issue (and no more, to bound the registers). In each
// v_mfma_f32_16x16x4_f32 lane l supplies A(l % 16, k + l / 16) and B(k + l /
// 16, l % 16); lane l ends holding D(4 (l / 16) + e, l % 16) in acc[j][e].
template <int NTC, int NT, bool SCALE>
__device__ __forceinline__ void mma_n(v4f (&acc)[NT], const float* a, int ai, int ak, const float* b, int bk, int bj,
                                      int K, float as) {
  const int lane = threadIdx.x & 63;
  const int r = lane & 15, q = lane >> 4;
  const float* pa = a + r * ai + q * ak;
  const float* pb = b + q * bk + r * bj;
#pragma clang loop unroll(disable)
  for (int k0 = 0; k0 < K; k0 += 16) {
    float av[4], bv[4][NTC];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      av[u] = pa[(k0 + 4 * u) * ak];
      if (SCALE) av[u] *= as;
#pragma unroll
      for (int j = 0; j < NTC; ++j) bv[u][j] = pb[(k0 + 4 * u) * bk + 16 * j * bj];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int j = 0; j < NTC; ++j) acc[j] = mfma4(av[u], bv[u][j], acc[j]);
  }
}

// mma_n for a tile count nt (uniform, 1 <= nt <= NT) known only at run time:
// one branch picks the compile-time variant, so the products of a k-step
// issue back to back.
template <int NT, bool SCALE = false>
__device__ __forceinline__ void mma(v4f (&acc)[NT], int nt, const float* a, int ai, int ak, const float* b, int bk,
                                    int bj, int K, float as = 1.f) {
  static_assert(NT >= 1 && NT <= 8, "tile count");
  if (nt <= 0) return;
  switch (nt) {
    case 1: mma_n<1, NT, SCALE>(acc, a, ai, ak, b, bk, bj, K, as); break;
    case 2: if constexpr (NT >= 2) mma_n<2, NT, SCALE>(acc, a, ai, ak, b, bk, bj, K, as); break;
    case 3: if constexpr (NT >= 3) mma_n<3, NT, SCALE>(acc, a, ai, ak, b, bk, bj, K, as); break;
    case 4: if constexpr (NT >= 4) mma_n<4, NT, SCALE>(acc, a, ai, ak, b, bk, bj, K, as); break;
    case 5: if constexpr (NT >= 5) mma_n<5, NT, SCALE>(acc, a, ai, ak, b, bk, bj, K, as); break;
    case 6: if constexpr (NT >= 6) mma_n<6, NT, SCALE>(acc, a, ai, ak, b, bk, bj, K, as); break;
    case 7: if constexpr (NT >= 7) mma_n<7, NT, SCALE>(acc, a, ai, ak, b, bk, bj, K, as); break;
    default: if constexpr (NT >= 8) mma_n<8, NT, SCALE>(acc, a, ai, ak, b, bk, bj, K, as); break;
  }
}

template <int NT>
__device__ __forceinline__ void zero(v4f (&acc)[NT]) {
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
}

// ---- four consecutive storage elements <-> float4 (16-byte aligned float32,
// 8-byte aligned 16-bit types) ----
// As loaded: float4 for float32, the raw 16-bit pairs otherwise. Prefetched
// tiles stay raw in registers and are widened where they are parked in LDS:
// widening next to the load would make the wave wait for the load there.
template <typename Tx> struct Raw4 { using type = uint2; };
template <> struct Raw4<float> { using type = float4; };
template <typename Tx> using raw4 = typename Raw4<Tx>::type;

template <typename Tx> __device__ __forceinline__ raw4<Tx> ld_raw(const Tx* p) {
  return *reinterpret_cast<const raw4<Tx>*>(p);
}
template <typename Tx> __device__ __forceinline__ raw4<Tx> raw_zero() { return make_uint2(0u, 0u); }
template <> __device__ __forceinline__ float4 raw_zero<float>() { return make_float4(0.f, 0.f, 0.f, 0.f); }
template <typename Tx> __device__ __forceinline__ float4 widen(raw4<Tx> u);
template <> __device__ __forceinline__ float4 widen<float>(float4 u) { return u; }
template <> __device__ __forceinline__ float4 widen<bf16>(uint2 u) {
  return make_float4(__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xffff0000u),
                     __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xffff0000u));
}
template <> __device__ __forceinline__ float4 widen<f16>(uint2 u) {
  auto h = [](uint32_t bits) { return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(bits))); };
  return make_float4(h(u.x & 0xffff), h(u.x >> 16), h(u.y & 0xffff), h(u.y >> 16));
}
template <typename Tx> __device__ __forceinline__ void st4(Tx* p, float4 v);
template <> __device__ __forceinline__ void st4<float>(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
template <> __device__ __forceinline__ void st4<bf16>(bf16* p, float4 v) {
  *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
}
template <> __device__ __forceinline__ void st4<f16>(f16* p, float4 v) {
  auto b = [](float f) { return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<f16>(f))); };
  *reinterpret_cast<uint2*>(p) = make_uint2(b(v.x) | (b(v.y) << 16), b(v.z) | (b(v.w) << 16));
}

__device__ __forceinline__ float4 scale4(float4 v, float s) { return make_float4(v.x * s, v.y * s, v.z * s, v.w * s); }

// The row of float4 number v of a tile with nv float4 per row: floor((v +
// 0.5) / nv) in float32 is exact for the tile sizes here (v < 2^11, nv <= 32:
// the quotient is at least 0.5 / nv away from an integer).
__device__ __forceinline__ int tile_row(int v, float inv_nv) {
  return static_cast<int>((static_cast<float>(v) + 0.5f) * inv_nv);
}

// The backward chunk kernel runs 8 waves: two per 16-row strip, splitting
// each product's column tiles.
constexpr int kThreads3 = 512;

// float4 per thread of the staged tiles: (64 x dstate) and (headdim x
// dstate) tiles, (64 x headdim) tiles and (headdim x 64-state half) tiles,
// for a workgroup of TPB threads.
template <int TPB = kThreads> constexpr int vec_n() { return Q * kSsdMaxN / 4 / TPB; }
template <int TPB = kThreads> constexpr int vec_x() { return Q * kSsdMaxP / 4 / TPB; }
constexpr int kVecN = vec_n();
constexpr int kVecX = vec_x();

// Registers x = rows r < nrows, columns c < ncols (multiple of 4) of
// src[r rs + c], four elements per entry, rows from nvalid on zero; thread
// tid holds entry number tid + k TPB of the row-major tile. The loads are
// issued here and waited for where the registers are used.
template <typename Tx, int V, int TPB = kThreads>
__device__ __forceinline__ void tile_load(raw4<Tx> (&x)[V], const Tx* src, int64_t rs, int nrows, int nvalid,
                                          int ncols) {
  const int nv = ncols >> 2, total = nrows * nv;
  const float inv = 1.0f / static_cast<float>(nv);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int v = threadIdx.x + k * TPB;
    x[k] = raw_zero<Tx>();
    if (v < total) {
      const int r = tile_row(v, inv);
      if (r < nvalid) x[k] = ld_raw<Tx>(src + r * rs + ((v - r * nv) << 2));
    }
  }
}

// LDS tile s (rows of ld floats) from registers filled by tile_load with the
// same nrows / ncols, widened to float32, times scale[r] when given.
template <typename Tx, int V, int TPB = kThreads>
__device__ __forceinline__ void tile_store(float* s, int ld, const raw4<Tx> (&x)[V], int nrows, int ncols,
                                           const float* scale = nullptr) {
  const int nv = ncols >> 2, total = nrows * nv;
  const float inv = 1.0f / static_cast<float>(nv);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int v = threadIdx.x + k * TPB;
    if (v < total) {
      const int r = tile_row(v, inv);
      const int c = (v - r * nv) << 2;
      const float4 f = widen<Tx>(x[k]);
      *reinterpret_cast<float4*>(s + r * ld + c) = scale ? scale4(f, scale[r]) : f;
    }
  }
}

// The same with entry k times sc[k].
template <typename Tx, int V, int TPB = kThreads>
__device__ __forceinline__ void tile_store_scaled(float* s, int ld, const raw4<Tx> (&x)[V], int nrows, int ncols,
                                                  const float (&sc)[V]) {
  const int nv = ncols >> 2, total = nrows * nv;
  const float inv = 1.0f / static_cast<float>(nv);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int v = threadIdx.x + k * TPB;
    if (v < total) {
      const int r = tile_row(v, inv);
      *reinterpret_cast<float4*>(s + r * ld + ((v - r * nv) << 2)) = scale4(widen<Tx>(x[k]), sc[k]);
    }
  }
}

// tile_load then tile_store.
template <typename Tx, int V, int TPB = kThreads>
__device__ __forceinline__ void stage(float* s, int ld, const Tx* src, int64_t rs, int nrows, int nvalid, int ncols,
                                      const float* scale = nullptr) {
  raw4<Tx> x[V];
  tile_load<Tx, V, TPB>(x, src, rs, nrows, nvalid, ncols);
  tile_store<Tx, V, TPB>(s, ld, x, nrows, ncols, scale);
}

// The dout, z and ysave tiles of one head's chunk (x layout from `off`, z and
// ysave only when HAS_Z and, for ysave, want_y), for a workgroup of TPB threads.
template <typename Tx, bool HAS_Z, int TPB = kThreads>
struct DyTiles {
  static constexpr int V = vec_x<TPB>();
  raw4<Tx> go[V], zz[V], yy[V];

  __device__ __forceinline__ void load(const SsdParams& p, int64_t off, int64_t rs, int nvalid, int ncols,
                                       bool want_y) {
    tile_load<Tx, V, TPB>(go, static_cast<const Tx*>(p.dout) + off, rs, Q, nvalid, ncols);
    if (HAS_Z) {
      tile_load<Tx, V, TPB>(zz, static_cast<const Tx*>(p.z) + off, rs, Q, nvalid, ncols);
      if (want_y) tile_load<Tx, V, TPB>(yy, static_cast<const Tx*>(p.ysave) + off, rs, Q, nvalid, ncols);
    }
  }

  // LDS tile of dY = dout silu(z) (dout without z), times scale[r] when
  // given; dz = dout y silu'(z) written to rows below nvalid when write_dz.
  __device__ __forceinline__ void store(float* s, int ld, const SsdParams& p, int64_t off, int64_t rs, int nvalid,
                                        int ncols, bool write_dz, const float* scale = nullptr) const {
    const int nv = ncols >> 2, total = Q * nv;
    const float inv = 1.0f / static_cast<float>(nv);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int v = threadIdx.x + k * TPB;
      if (v >= total) continue;
      const int r = tile_row(v, inv);
      const int c = (v - r * nv) << 2;
      float4 dz = make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 dy = dy_of(k, write_dz ? &dz : nullptr);
      if (HAS_Z && write_dz && r < nvalid) st4<Tx>(static_cast<Tx*>(p.dz) + off + r * rs + c, dz);
      *reinterpret_cast<float4*>(s + r * ld + c) = scale ? scale4(dy, scale[r]) : dy;
    }
  }

  // The same LDS tile (no dz) with float4 number k scaled by sc[k].
  __device__ __forceinline__ void store_scaled(float* s, int ld, int ncols, const float (&sc)[V]) const {
    const int nv = ncols >> 2, total = Q * nv;
    const float inv = 1.0f / static_cast<float>(nv);
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const int v = threadIdx.x + k * TPB;
      if (v >= total) continue;
      const int r = tile_row(v, inv);
      *reinterpret_cast<float4*>(s + r * ld + ((v - r * nv) << 2)) = scale4(dy_of(k, nullptr), sc[k]);
    }
  }

  // dY of float4 number k, and dz into *dzp when given (HAS_Z).
  __device__ __forceinline__ float4 dy_of(int k, float4* dzp) const {
    const float4 g4 = widen<Tx>(go[k]);
    if (!HAS_Z) return g4;
    const float4 z4 = widen<Tx>(zz[k]);
    const float gx[4] = {g4.x, g4.y, g4.z, g4.w}, zx[4] = {z4.x, z4.y, z4.z, z4.w};
    float d[4], sg[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      sg[u] = sigmoid(zx[u]);
      d[u] = gx[u] * zx[u] * sg[u];
    }
    if (dzp) {
      const float4 y4 = widen<Tx>(yy[k]);
      const float yv[4] = {y4.x, y4.y, y4.z, y4.w};
      float dzv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) dzv[u] = gx[u] * yv[u] * sg[u] * (1.f + zx[u] * (1.f - sg[u]));
      *dzp = make_float4(dzv[0], dzv[1], dzv[2], dzv[3]);
    }
    return make_float4(d[0], d[1], d[2], d[3]);
  }
};

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

// The effective step for dt + dt_bias = pre and, when grad, d(step)/d(raw
// dt): the softplus derivative, zero where the clamp to [dt_lo, dt_hi] is
// active. The clamp always applies, as in mamba_ssm (its default (0, inf)
// makes a negative raw step 0), and keeps a NaN step NaN, as torch.clamp does.
__device__ __forceinline__ float step_of(const SsdParams& p, float pre, float* grad) {
  float sg = 1.f;
  float st = pre;
  if (p.softplus) st = softplus_sigmoid(pre, sg);
  const bool inside = st >= p.dt_lo && st <= p.dt_hi;
  st = st < p.dt_lo ? p.dt_lo : (st > p.dt_hi ? p.dt_hi : st);
  if (!inside) sg = 0.f;
  if (grad) *grad = sg;
  return st;
}
// The same for (b, t, h); 0 past the sequence.
__device__ __forceinline__ float ssd_step(const SsdParams& p, int64_t b, int64_t t, int64_t h, float* grad) {
  if (t >= p.seqlen) {
    if (grad) *grad = 0.f;
    return 0.f;
  }
  return step_of(p, p.dt[(b * p.seqlen + t) * p.nheads + h] + (p.dt_bias ? p.dt_bias[h] : 0.f), grad);
}

// Chunk row (b, h, c) of the cs / step arrays.
__device__ __forceinline__ int64_t chunk_row(const SsdParams& p, int64_t b, int64_t h, int64_t c) {
  return ((b * p.nheads + h) * p.nchunks + c) * Q;
}

// Offset of the (b, c, h) state block in states / dstates.
__device__ __forceinline__ int64_t state_block(const SsdParams& p, int64_t b, int64_t c, int64_t h) {
  return ((b * p.nchunks + c) * p.nheads + h) * p.headdim * p.dstate;
}

// Steps of the chunk that exist.
__device__ __forceinline__ int chunk_steps(const SsdParams& p, int64_t t0) {
  return static_cast<int>(p.seqlen - t0 < Q ? p.seqlen - t0 : Q);
}

// Packed sequences. Kernels built with SEQ read p.seq_idx; without it every
// helper below folds to a constant (one sequence, id 0).
//
// Id of step t of batch row b: 0 before the first step (the initial state's
// id); steps past the sequence (a chunk's padding) take the last step's id.
template <bool SEQ>
__device__ __forceinline__ int32_t seq_of(const SsdParams& p, int64_t b, int64_t t) {
  if constexpr (!SEQ) return 0;
  if (t < 0) return 0;
  return p.seq_idx[b * p.seqlen + (t < p.seqlen ? t : p.seqlen - 1)];
}

// Ids do not decrease, so the steps of a chunk that share an id form a run.
// For the wave whose lane l stands for step t0 + l: the first step (in the
// chunk) of lane l's run.
template <bool SEQ>
__device__ __forceinline__ int run_first(const SsdParams& p, int64_t b, int64_t t0, int lane) {
  if constexpr (!SEQ) return 0;
  const bool starts = lane == 0 || seq_of<SEQ>(p, b, t0 + lane) != seq_of<SEQ>(p, b, t0 + lane - 1);
  const unsigned long long upto = __ballot(starts) & (~0ull >> (63 - lane));
  return 63 - __clzll(upto);
}

// Whether the state entering chunk c carries through it: the ids at the ends
// of chunks c - 1 and c agree (ids do not decrease, so none changes between).
template <bool SEQ>
__device__ __forceinline__ bool carries(const SsdParams& p, int64_t b, int64_t c) {
  if constexpr (!SEQ) return true;
  const int64_t end = (c + 1) * Q < p.seqlen ? (c + 1) * Q - 1 : p.seqlen - 1;
  return seq_of<SEQ>(p, b, end) == seq_of<SEQ>(p, b, c * Q - 1);
}

}  // namespace

// F1: steps and running decays of each head's chunk (saved for F3 and the
// backward), and the chunk-end state S(p, n) = sum_s exp(cs_L - cs_s) dt_s
// x_s(p) B_s(n). Grid (nchunks, nhb, batch); wave w computes state rows p in
// [16 w, 16 w + 16).
template <typename Tx, bool SEQ>
__global__ void __launch_bounds__(kThreads) ssd_chunk_state_kernel(const SsdParams p) {
  __shared__ __align__(16) float s_B[Q][NP];
  __shared__ __align__(16) float s_x[Q][XP];
  __shared__ float s_sc[Q];
  const int64_t c = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t h0 = static_cast<int64_t>(blockIdx.y) * p.hb;
  const int64_t g = h0 / (H / G);
  const int64_t t0 = c * Q;
  const int nvalid = chunk_steps(p, t0);
  stage<Tx, kVecN>(&s_B[0][0], NP, static_cast<const Tx*>(p.B) + ((b * L + t0) * G + g) * N, G * N, Q, nvalid,
            static_cast<int>(N));
  for (int i = 0; i < p.hb; ++i) {
    const int64_t h = h0 + i;
    if (wave == 0) {
      const float st = ssd_step(p, b, t0 + lane, h, nullptr);
      float cs, csl;
      wave_prefix_sum2(st * p.A[h], cs, csl);
      const int64_t row = chunk_row(p, b, h, c);
      p.cs[row + lane] = cs;
      p.cs_lo[row + lane] = csl;
      p.step[row + lane] = st;
      const float csL = __shfl(cs, Q - 1, 64), cslL = __shfl(csl, Q - 1, 64);
      // steps of another sequence than the chunk's last do not reach its end state
      const bool reach = seq_of<SEQ>(p, b, t0 + lane) == seq_of<SEQ>(p, b, t0 + nvalid - 1);
      s_sc[lane] = reach ? st * fast_exp((csL - cs) + (cslL - csl)) : 0.f;
    }
    __syncthreads();
    stage<Tx, kVecX>(&s_x[0][0], XP, static_cast<const Tx*>(p.x) + ((b * L + t0) * H + h) * P, H * P, Q, nvalid,
              static_cast<int>(P), s_sc);
    __syncthreads();
    if (16 * wave < P) {
      v4f acc[kSsdMaxN / 16];
      zero(acc);
      mma(acc, static_cast<int>(N / 16), &s_x[0][16 * wave], 1, XP, &s_B[0][0], NP, 1, Q);
      float* dst = p.states + state_block(p, b, c, h);
#pragma unroll
      for (int j = 0; j < kSsdMaxN / 16; ++j)
        if (j < N / 16)
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[(16 * wave + 4 * q + e) * N + 16 * j + r] = acc[j][e];
    }
    __syncthreads();
  }
}

// F2: walks the chunks in order, replacing each chunk-end state by the state
// entering the chunk, H_c = exp(cs_L(c-1)) H_{c-1} + S_{c-1} (H_0 = the
// initial state or 0), and writes the final state. One thread per state
// element; grid (nslices, nheads, batch). The next chunk's loads issue before
// this chunk's store.
template <bool SEQ>
__global__ void __launch_bounds__(kThreads) ssd_state_pass_kernel(const SsdParams p) {
  const int64_t PN = p.headdim * p.dstate, H = p.nheads;
  const int64_t e = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x;
  const int64_t h = blockIdx.y, b = blockIdx.z;
  if (e >= PN) return;
  float run = p.init ? p.init[(b * H + h) * PN + e] : 0.f;
  float* st = p.states + state_block(p, b, 0, h) + e;
  const int64_t cstride = H * PN;
  const float* csl = p.cs + chunk_row(p, b, h, 0) + (Q - 1);
  float s = st[0], d = csl[0];
  for (int64_t c = 0; c < p.nchunks; ++c) {
    const float sc = s, dc = carries<SEQ>(p, b, c) ? fast_exp(d) : 0.f;
    if (c + 1 < p.nchunks) {
      s = st[(c + 1) * cstride];
      d = csl[(c + 1) * Q];
    }
    st[c * cstride] = run;
    run = fmaf(dc, run, sc);
  }
  if (p.final_states) p.final_states[(b * H + h) * PN + e] = run;
}

// The steps and running decays of every chunk, for the in-order kernels:
// one wave per (b, h, chunk), lane t owning step t. Grid (ceil(nchunks / 4),
// nheads, batch).
__global__ void __launch_bounds__(kThreads) ssd_chunk_decay_kernel(const SsdParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t h = blockIdx.y, b = blockIdx.z;
  if (c >= p.nchunks) return;
  const float st = ssd_step(p, b, c * Q + lane, h, nullptr);
  float cs, csl;
  wave_prefix_sum2(st * p.A[h], cs, csl);
  const int64_t row = chunk_row(p, b, h, c);
  p.cs[row + lane] = cs;
  p.cs_lo[row + lane] = csl;
  p.step[row + lane] = st;
}

// Rows of the float4 entries a thread holds of a (64 x ncols) tile
// (tile_load's mapping), clamped to the tile.
template <int V>
__device__ __forceinline__ void tile_rows(int (&rows)[V], int ncols) {
  const float inv = 1.0f / static_cast<float>(ncols >> 2);
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const int r = tile_row(static_cast<int>(threadIdx.x) + k * kThreads, inv);
    rows[k] = r < Q ? r : Q - 1;
  }
}

// F1 and F2 in one launch: the workgroup of (b, h, column block) walks the
// chunks in order, holding state columns [64 x, 64 x + 64) of every row in
// matrix-core accumulators. Per chunk c it stores H_c (the state entering c)
// and forms H_{c+1} = exp(cs_L) H_c + sum_s exp(cs_L - cs_s) dt_s x_s B_s^T by
// starting the products from the scaled H_c, so chunk-end states never reach
// memory. The chunks' steps and running decays come from
// ssd_chunk_decay_kernel; each thread loads those of its own x rows with the
// next chunk's x and B while the current chunk's products run.
// Grid (column blocks, nheads, batch); wave w owns state rows [16 w, 16 w + 16).
// Three waves per SIMD, as the backward's.
template <typename Tx, bool SEQ>
__global__ void __launch_bounds__(kThreads, 3) ssd_state_scan_kernel(const SsdParams p) {
  constexpr int VX = vec_x();
  constexpr int VB = Q * kSsdPassCols / 4 / kThreads;
  constexpr int BP = kSsdPassCols + 4;
  __shared__ __align__(16) float s_x[Q][XP];    // dt_s exp(cs_L - cs_s) x_s
  __shared__ __align__(16) float s_B[Q][BP];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kSsdPassCols;
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int64_t g = h / (H / G);
  const int ncol = static_cast<int>(N - n0 < kSsdPassCols ? N - n0 : kSsdPassCols);
  const int nt = ncol >> 4;
  const bool act = 16 * wave < P;
  // Accumulator element (j, e) of this lane: state row 16 wave + 4 q + e,
  // column n0 + 16 j + r, at offset eo + e N + 16 j of a (headdim x dstate) block.
  const int64_t eo = (16 * wave + 4 * q) * N + n0 + r;
  v4f acc[kSsdPassCols / 16];
#pragma unroll
  for (int j = 0; j < kSsdPassCols / 16; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[j][e] = (act && j < nt && p.init) ? p.init[(b * H + h) * P * N + eo + e * N + 16 * j] : 0.f;

  const Tx* xh = static_cast<const Tx*>(p.x) + b * L * H * P + h * P;
  const Tx* Bg = static_cast<const Tx*>(p.B) + b * L * G * N + g * N + n0;
  raw4<Tx> nx[VX], nB[VB];
  int rows[VX];
  tile_rows(rows, static_cast<int>(P));
  float ncs[VX], nlo[VX], nst[VX], ncsL = 0.f, nloL = 0.f;
  // packed sequences: the chunk's last run starts at step nlast (its steps
  // reach the chunk's end state); H_c carries through the chunk
  int nlast = 0;
  bool ncarry = true;
  auto fetch = [&](int64_t c) {
    const int64_t t0 = c * Q;
    const int nv = chunk_steps(p, t0);
    tile_load<Tx, VX>(nx, xh + t0 * H * P, H * P, Q, nv, static_cast<int>(P));
    tile_load<Tx, VB>(nB, Bg + t0 * G * N, G * N, Q, nv, ncol);
    const int64_t row = chunk_row(p, b, h, c);
#pragma unroll
    for (int k = 0; k < VX; ++k) {
      ncs[k] = p.cs[row + rows[k]];
      nlo[k] = p.cs_lo[row + rows[k]];
      nst[k] = p.step[row + rows[k]];
    }
    ncsL = p.cs[row + Q - 1];
    nloL = p.cs_lo[row + Q - 1];
    if constexpr (SEQ) {  // the last run's first step, from a ballot over the chunk's steps
      nlast = __ffsll(static_cast<long long>(
                  __ballot(seq_of<SEQ>(p, b, t0 + lane) == seq_of<SEQ>(p, b, t0 + nv - 1)))) - 1;
      ncarry = carries<SEQ>(p, b, c);
    }
  };
  fetch(0);
  for (int64_t c = 0; c < p.nchunks; ++c) {
    const float decay = ncarry ? fast_exp(ncsL + nloL) : 0.f;
    float sc[VX];  // dt_s exp(cs_L - cs_s) of this thread's rows s
#pragma unroll
    for (int k = 0; k < VX; ++k) sc[k] = rows[k] >= nlast ? nst[k] * fast_exp((ncsL - ncs[k]) + (nloL - nlo[k])) : 0.f;
    __syncthreads();  // the previous chunk's products are done with s_x and s_B
    tile_store_scaled<Tx, VX>(&s_x[0][0], XP, nx, Q, static_cast<int>(P), sc);
    tile_store<Tx, VB>(&s_B[0][0], BP, nB, Q, ncol);
    if (c + 1 < p.nchunks) fetch(c + 1);
    __syncthreads();
    if (act) {
      float* dst = p.states + state_block(p, b, c, h) + eo;
#pragma unroll
      for (int j = 0; j < kSsdPassCols / 16; ++j)
        if (j < nt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            dst[e * N + 16 * j] = acc[j][e];
            acc[j][e] *= decay;
          }
      mma(acc, nt, &s_x[0][16 * wave], 1, XP, &s_B[0][0], BP, 1, Q);
    }
  }
  if (p.final_states && act) {
    float* dst = p.final_states + (b * H + h) * P * N + eo;
#pragma unroll
    for (int j = 0; j < kSsdPassCols / 16; ++j)
      if (j < nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e * N + 16 * j] = acc[j][e];
  }
}

// F3: the chunk's outputs, Y = (C B^T o M) (dt x) + diag(exp(cs)) C H^T + D x,
// out = Y silu(z) (and Y itself into ysave when the backward needs it).
// Grid (nchunks, nhb, batch), 8 waves: wave w computes rows t in
// [16 (w % 4), 16 (w % 4) + 16) and half w / 4 of the column tiles (C B^T:
// tiles 2h, 2h + 1; Y: the first or second half of the headdim tiles), so each
// SIMD runs two waves. C B^T is formed once for the block's heads.
template <typename Tx, bool HAS_Z, bool SEQ>
__global__ void __launch_bounds__(kThreads3, 2) ssd_chunk_scan_kernel(const SsdParams p) {
  constexpr int TPB = kThreads3;
  constexpr int VX = vec_x<TPB>(), VN = vec_n<TPB>();
  __shared__ __align__(16) float s_C[Q][NP];
  __shared__ __align__(16) float s_BH[Q][NP];     // B (Q x N), then each head's entering state H (P x N)
  __shared__ __align__(16) float s_G[Q][QP];      // (C B^T o M)[t][s] dt_s, then Y
  __shared__ __align__(16) float s_X[Q][XP];      // x
  __shared__ float s_cs[Q], s_csl[Q], s_dt[Q];
  __shared__ __align__(4) uint8_t s_first[Q];     // first step of each step's sequence run in the chunk
  const int64_t c = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ws = wave & 3, hf = wave >> 2;        // row strip, column half
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t h0 = static_cast<int64_t>(blockIdx.y) * p.hb;
  const int64_t g = h0 / (H / G);
  const int64_t t0 = c * Q;
  const int nvalid = chunk_steps(p, t0);
  const int np = static_cast<int>(P / 16);
  const int pa = (np + 1) / 2;
  const int p0 = hf ? pa : 0, npw = hf ? np - pa : pa;   // this wave's headdim tiles
  {
    const int64_t off = ((b * L + t0) * G + g) * N;
    stage<Tx, VN, TPB>(&s_C[0][0], NP, static_cast<const Tx*>(p.C) + off, G * N, Q, nvalid, static_cast<int>(N));
    stage<Tx, VN, TPB>(&s_BH[0][0], NP, static_cast<const Tx*>(p.B) + off, G * N, Q, nvalid, static_cast<int>(N));
  }
  if (SEQ && wave == 0) s_first[lane] = static_cast<uint8_t>(run_first<SEQ>(p, b, t0, lane));
  // the entering state reaches the chunk's first run
  const bool enter = seq_of<SEQ>(p, b, t0) == seq_of<SEQ>(p, b, t0 - 1);
  __syncthreads();
  // runs of this thread's rows t = 16 ws + 4 q + e: M[t][s] needs first_t <= s <= t
  const uint32_t firsts = SEQ ? *reinterpret_cast<const uint32_t*>(&s_first[16 * ws + 4 * q]) : 0u;
  v4f cb[2];
  zero(cb);
  mma(cb, 2, &s_C[16 * ws][0], NP, 1, &s_BH[32 * hf][0], 1, NP, static_cast<int>(N));
  // The next head's x tile, entering state and decays load into registers
  // while this head's products run.
  raw4<Tx> rx[VX], zc[VX];
  float4 rh[VN], rD[VX];
  float rcs = 0.f, rcsl = 0.f, rdt = 0.f;
  // The headdim column of this thread's output entries (fixed over heads).
  int ocol[VX];
  {
    const float inv = 1.0f / static_cast<float>(np * 4);
#pragma unroll
    for (int k = 0; k < VX; ++k) {
      const int v = tid + k * TPB;
      const int t = tile_row(v, inv);
      ocol[k] = v < Q * np * 4 ? (v - t * np * 4) << 2 : 0;
    }
  }
  auto fetch = [&](int64_t h) {
    const int64_t row = chunk_row(p, b, h, c);
    if (tid < Q) {
      rcs = p.cs[row + tid];
      rcsl = p.cs_lo[row + tid];
      rdt = p.step[row + tid];
    }
    tile_load<Tx, VX, TPB>(rx, static_cast<const Tx*>(p.x) + ((b * L + t0) * H + h) * P, H * P, Q, nvalid,
                           static_cast<int>(P));
    tile_load<float, VN, TPB>(rh, p.states + state_block(p, b, c, h), N, static_cast<int>(P), static_cast<int>(P),
                              static_cast<int>(N));
#pragma unroll
    for (int k = 0; k < VX; ++k)
      rD[k] = p.D ? *reinterpret_cast<const float4*>(p.D + h * P + ocol[k]) : make_float4(0.f, 0.f, 0.f, 0.f);
  };
  fetch(h0);
  for (int i = 0; i < p.hb; ++i) {
    const int64_t h = h0 + i;
    const int64_t xoff = ((b * L + t0) * H + h) * P;
    float4 dcol[VX];  // this head's D at the output columns (rD moves on to the next head below)
#pragma unroll
    for (int k = 0; k < VX; ++k) dcol[k] = rD[k];
    __syncthreads();  // every wave is done with s_BH, s_G, s_X and s_cs
    if (tid < Q) {
      s_cs[tid] = rcs;
      s_csl[tid] = rcsl;
      s_dt[tid] = rdt;
    }
    tile_store<Tx, VX, TPB>(&s_X[0][0], XP, rx, Q, static_cast<int>(P));
    tile_store<float, VN, TPB>(&s_BH[0][0], NP, rh, static_cast<int>(P), static_cast<int>(N));
    __syncthreads();
    if (HAS_Z)
      tile_load<Tx, VX, TPB>(zc, static_cast<const Tx*>(p.z) + xoff, H * P, Q, nvalid, static_cast<int>(P));
    if (i + 1 < p.hb) fetch(h + 1);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 16 * ws + 4 * q + e, s = 32 * hf + 16 * j + r;
        const int ft = (firsts >> (8 * e)) & 0xff;
        s_G[t][s] = (s <= t && s >= ft) ? cb[j][e] * seg_exp(s_cs, s_csl, t, s) * s_dt[s] : 0.f;
      }
    __syncthreads();
    v4f y1[2], y2[2];
    zero(y1);
    zero(y2);
    mma(y1, npw, &s_G[16 * ws][0], QP, 1, &s_X[0][16 * p0], XP, 1, Q);
    mma(y2, npw, &s_C[16 * ws][0], NP, 1, &s_BH[16 * p0][0], 1, NP, static_cast<int>(N));
    __syncthreads();  // every wave is done reading s_G
    // Y (float32) into s_G, then out = (Y + D x) silu(z) four elements at a time.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * ws + 4 * q + e;
      const bool from = enter && ((firsts >> (8 * e)) & 0xff) == 0;
      const float ecs = from ? fast_exp(s_cs[t] + s_csl[t]) : 0.f;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        if (j < npw) s_G[t][16 * (p0 + j) + r] = fmaf(ecs, y2[j][e], y1[j][e]);
    }
    __syncthreads();
    {
      const int nv = np * 4;
      const float inv = 1.0f / static_cast<float>(nv);
#pragma unroll
      for (int k = 0; k < VX; ++k) {
        const int v = tid + k * TPB;
        if (v >= Q * nv) continue;
        const int t = tile_row(v, inv);
        if (t >= nvalid) continue;
        const int pp = (v - t * nv) << 2;
        const int64_t at = xoff + t * H * P + pp;
        float y[4] = {s_G[t][pp], s_G[t][pp + 1], s_G[t][pp + 2], s_G[t][pp + 3]};
        if (p.D) {
          const float4 d = dcol[k];
          y[0] = fmaf(d.x, s_X[t][pp], y[0]);
          y[1] = fmaf(d.y, s_X[t][pp + 1], y[1]);
          y[2] = fmaf(d.z, s_X[t][pp + 2], y[2]);
          y[3] = fmaf(d.w, s_X[t][pp + 3], y[3]);
        }
        if (HAS_Z) {
          if (p.ysave) st4<Tx>(static_cast<Tx*>(p.ysave) + at, make_float4(y[0], y[1], y[2], y[3]));
          const float4 z4 = widen<Tx>(zc[k]);
          const float zx[4] = {z4.x, z4.y, z4.z, z4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) y[u] *= zx[u] * sigmoid(zx[u]);
        }
        st4<Tx>(static_cast<Tx*>(p.out) + at, make_float4(y[0], y[1], y[2], y[3]));
      }
    }
  }
}

// K1: the seed E_c[p][n] = sum_t exp(cs_t) dY[t][p] C[t][n] of dL/dH_c from
// the chunk's own outputs, for each head of the block, into dstates. Grid
// (nchunks, nhb, batch); wave w computes rows p in [16 w, 16 w + 16).
template <typename Tx, bool HAS_Z, bool SEQ>
__global__ void __launch_bounds__(kThreads) ssd_bwd_seed_kernel(const SsdParams p) {
  __shared__ __align__(16) float s_C[Q][NP];
  __shared__ __align__(16) float s_dY[Q][XP];     // exp(cs_t) dY[t][p]
  __shared__ float s_ecs[Q];
  const int64_t c = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t h0 = static_cast<int64_t>(blockIdx.y) * p.hb;
  const int64_t g = h0 / (H / G);
  const int64_t t0 = c * Q;
  const int nvalid = chunk_steps(p, t0);
  stage<Tx, kVecN>(&s_C[0][0], NP, static_cast<const Tx*>(p.C) + ((b * L + t0) * G + g) * N, G * N, Q, nvalid,
            static_cast<int>(N));
  // packed sequences: step tid reads the entering state only within its sequence
  const bool from = tid < Q && seq_of<SEQ>(p, b, t0 + tid) == seq_of<SEQ>(p, b, t0 - 1);
  for (int i = 0; i < p.hb; ++i) {
    const int64_t h = h0 + i;
    const int64_t row = chunk_row(p, b, h, c);
    __syncthreads();  // every wave is done with s_dY and s_ecs
    if (tid < Q) s_ecs[tid] = from ? fast_exp(p.cs[row + tid] + p.cs_lo[row + tid]) : 0.f;
    __syncthreads();
    {
      const int64_t off = ((b * L + t0) * H + h) * P;
      DyTiles<Tx, HAS_Z> dyt;
      dyt.load(p, off, H * P, nvalid, static_cast<int>(P), false);
      dyt.store(&s_dY[0][0], XP, p, off, H * P, nvalid, static_cast<int>(P), false, s_ecs);
    }
    __syncthreads();
    if (16 * wave < P) {
      v4f ev[kSsdMaxN / 16];
      zero(ev);
      mma(ev, static_cast<int>(N / 16), &s_dY[0][16 * wave], 1, XP, &s_C[0][0], NP, 1, Q);
      float* dst = p.dstates + state_block(p, b, c, h);
#pragma unroll
      for (int j = 0; j < kSsdMaxN / 16; ++j)
        if (j < N / 16)
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[(16 * wave + 4 * q + e) * N + 16 * j + r] = ev[j][e];
    }
  }
}

// K2: walks the chunks from the last: dH^out_c (gradient of the state leaving
// chunk c) replaces E_c in dstates, dH^in_c = exp(cs_L) dH^out_c + E_c
// carries on, and <dH^out_c, exp(cs_L) H_c> (this slice's share of dL/dcs_L)
// goes to dcsL. The gradient of the initial state is what is left after
// chunk 0. Grid (nslices, nheads, batch). The next chunk's loads issue before
// this chunk's store.
template <bool SEQ>
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
  float* dcsl = p.dcsL + (chunk_row(p, b, h, 0) / Q) * p.nslices + blockIdx.x;
  const int64_t last = p.nchunks - 1;
  float ec = ok ? p.dstates[base + last * cstride] : 0.f;
  float hin = ok ? p.states[base + last * cstride] : 0.f;
  float dl = csl[last * Q];
  for (int64_t c = last; c >= 0; --c) {
    const float ecc = ec, hc = hin, d = carries<SEQ>(p, b, c) ? fast_exp(dl) : 0.f;
    if (c > 0) {
      ec = ok ? p.dstates[base + (c - 1) * cstride] : 0.f;
      hin = ok ? p.states[base + (c - 1) * cstride] : 0.f;
      dl = csl[(c - 1) * Q];
    }
    if (ok) p.dstates[base + c * cstride] = run;
    const float part = wave_total(run * d * hc);
    if (lane == 0) s_part[wave] = part;
    __syncthreads();
    if (threadIdx.x == 0) dcsl[c * p.nslices] = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    __syncthreads();
    run = fmaf(d, run, ecc);
  }
  if (ok && p.dinit) p.dinit[(b * H + h) * PN + e] = run;
}

// K1 and K2 in one launch: the workgroup of (b, h, column block) walks the
// chunks from the last, holding columns [64 x, 64 x + 64) of dL/d(state
// leaving the chunk) in matrix-core accumulators. Per chunk c it stores
// dH^out_c, adds <dH^out_c, exp(cs_L) H_c> over its columns to dcsL (slice x),
// and forms dH^in_c = exp(cs_L) dH^out_c + (diag(exp(cs)) C)^T dY by starting
// the products from the scaled dH^out_c, so the seeds never reach memory.
// What is left after chunk 0 is the initial state's gradient. The next
// chunk's dout, z, C, running decays and H load while the current chunk's
// products run. Grid (column blocks, nheads, batch); wave w owns rows
// [16 w, 16 w + 16). Three waves per SIMD: 640 workgroups (the Mamba-2 2.7B
// layer at batch 4) run in one round.
template <typename Tx, bool HAS_Z, bool SEQ>
__global__ void __launch_bounds__(kThreads, 3) ssd_bwd_state_scan_kernel(const SsdParams p) {
  constexpr int VB = Q * kSsdPassCols / 4 / kThreads;
  constexpr int BP = kSsdPassCols + 4;
  using Dy = DyTiles<Tx, HAS_Z>;
  __shared__ __align__(16) float s_dY[Q][XP];   // exp(cs_t) dY[t][p]
  __shared__ __align__(16) float s_C[Q][BP];
  __shared__ float s_part[kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kSsdPassCols;
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int64_t g = h / (H / G);
  const int ncol = static_cast<int>(N - n0 < kSsdPassCols ? N - n0 : kSsdPassCols);
  const int nt = ncol >> 4;
  const bool act = 16 * wave < P;
  const int64_t eo = (16 * wave + 4 * q) * N + n0 + r;
  v4f acc[kSsdPassCols / 16];
#pragma unroll
  for (int j = 0; j < kSsdPassCols / 16; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      acc[j][e] = (act && j < nt && p.dfinal) ? p.dfinal[(b * H + h) * P * N + eo + e * N + 16 * j] : 0.f;

  const Tx* Cg = static_cast<const Tx*>(p.C) + b * L * G * N + g * N + n0;
  Dy dyt;
  raw4<Tx> nC[VB];
  float ncs = 0.f, nlo = 0.f, nH[kSsdPassCols / 16][4];
  bool nfrom = true, ncarry = true;  // packed sequences: step lane reads H_c; H_c carries through the chunk
  auto fetch = [&](int64_t c) {
    const int64_t t0 = c * Q;
    const int nv = chunk_steps(p, t0);
    dyt.load(p, ((b * L + t0) * H + h) * P, H * P, nv, static_cast<int>(P), false);
    tile_load<Tx, VB>(nC, Cg + t0 * G * N, G * N, Q, nv, ncol);
    const int64_t row = chunk_row(p, b, h, c);
    ncs = p.cs[row + lane];
    nlo = p.cs_lo[row + lane];
    nfrom = seq_of<SEQ>(p, b, t0 + lane) == seq_of<SEQ>(p, b, t0 - 1);
    ncarry = carries<SEQ>(p, b, c);
    const float* hs = p.states + state_block(p, b, c, h) + eo;
#pragma unroll
    for (int j = 0; j < kSsdPassCols / 16; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) nH[j][e] = (act && j < nt) ? hs[e * N + 16 * j] : 0.f;
  };
  float* dcsl = p.dcsL + (chunk_row(p, b, h, 0) / Q) * p.nslices + blockIdx.x;
  int64_t pend = -1;        // chunk whose dcsL share awaits the cross-wave sum
  float pend_decay = 0.f;
  fetch(p.nchunks - 1);
  for (int64_t c = p.nchunks - 1; c >= 0; --c) {
    const float ecs_all = fast_exp(ncs + nlo);
    const float decay = ncarry ? __shfl(ecs_all, Q - 1, 64) : 0.f;
    const float ecs = nfrom ? ecs_all : 0.f;
    // dH^out_c out, its share of dL/dcs_L, and the decayed carry, before the
    // next chunk's H_c loads into the same registers.
    float part = 0.f;
    if (act) {
      float* dst = p.dstates + state_block(p, b, c, h) + eo;
#pragma unroll
      for (int j = 0; j < kSsdPassCols / 16; ++j)
        if (j < nt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            dst[e * N + 16 * j] = acc[j][e];
            part = fmaf(acc[j][e], nH[j][e], part);
            acc[j][e] *= decay;
          }
    }
    part = wave_total(part);
    float sc[Dy::V];  // exp(cs_t) of this thread's dY rows t, from the lanes that own them
    {
      int rows[Dy::V];
      tile_rows(rows, static_cast<int>(P));
#pragma unroll
      for (int k = 0; k < Dy::V; ++k) sc[k] = __shfl(ecs, rows[k], 64);
    }
    __syncthreads();  // the previous chunk's products are done with s_dY and s_C; its parts are in
    if (pend >= 0 && tid == 0)
      dcsl[pend * p.nslices] = pend_decay * ((s_part[0] + s_part[1]) + (s_part[2] + s_part[3]));
    dyt.store_scaled(&s_dY[0][0], XP, static_cast<int>(P), sc);
    tile_store<Tx, VB>(&s_C[0][0], BP, nC, Q, ncol);
    if (c > 0) fetch(c - 1);
    __syncthreads();
    if (lane == 0) s_part[wave] = part;
    pend = c;
    pend_decay = decay;
    if (act) mma(acc, nt, &s_dY[0][16 * wave], 1, XP, &s_C[0][0], BP, 1, Q);
  }
  __syncthreads();
  if (pend >= 0 && tid == 0)
    dcsl[pend * p.nslices] = pend_decay * ((s_part[0] + s_part[1]) + (s_part[2] + s_part[3]));
  if (p.dinit && act) {
    float* dst = p.dinit + (b * H + h) * P * N + eo;
#pragma unroll
    for (int j = 0; j < kSsdPassCols / 16; ++j)
      if (j < nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e * N + 16 * j] = acc[j][e];
  }
}

// K3: every gradient of a chunk, for each head of the block. Grid (nchunks,
// nhb, batch), 8 waves: wave w owns rows [16 (w % 4), 16 (w % 4) + 16) of
// every Q-row product and half h = w / 4 of its column tiles (Q columns:
// tiles 2h, 2h + 1; headdim columns: the first or second half of the tiles;
// state columns: tiles 2h, 2h + 1 of each 64-state group). Two waves per SIMD
// hide each other's LDS and memory latency. Row sums over columns are
// combined across the two halves through LDS. dB and dC of the block's heads
// stay in accumulators and are written once, as the block's partial sums.
template <typename Tx, bool HAS_Z, bool SEQ>
__global__ void __launch_bounds__(kThreads3, 2) ssd_bwd_chunk_kernel(const SsdParams p) {
  constexpr int TPB = kThreads3;
  constexpr int VX = vec_x<TPB>(), VN = vec_n<TPB>();
  __shared__ __align__(16) float s_C[Q][NP];
  __shared__ __align__(16) float s_B[Q][NP];
  __shared__ __align__(16) float s_X[Q][XP];      // x
  __shared__ __align__(16) float s_dY[Q][XP];     // dY
  __shared__ __align__(16) float s_U[Q][QP];      // G = C B^T o M, then dH^out (P x 64-state group)
  __shared__ __align__(16) float s_V[Q][QP];      // dCB, then H (P x 64-state group), then dx
  __shared__ float s_colp[16][Q];                 // column sums of dG o G, per (row strip, lane quarter)
  __shared__ float s_dD[16][kSsdMaxP];
  __shared__ float s_half[2][4][Q];               // per column half: sum_s R, sum_n C.., sum_n B~.., sum_p ..
  __shared__ float s_cs[Q], s_csl[Q], s_dt[Q], s_w[Q], s_ecs[Q], s_dcs[Q];
  __shared__ float s_tot[8], s_wa[8], s_wb[8];
  __shared__ __align__(4) uint8_t s_first[Q];     // first step of each step's sequence run in the chunk
  const int64_t c = blockIdx.x, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ws = wave & 3, hf = wave >> 2;        // row strip, column half
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t h0 = static_cast<int64_t>(blockIdx.y) * p.hb;
  const int64_t g = h0 / (H / G);
  const int64_t t0 = c * Q;
  const int nvalid = chunk_steps(p, t0);
  const int np = static_cast<int>(P / 16), nn = static_cast<int>(N / 16);
  // headdim tiles of this wave: [p0, p0 + npw)
  const int pa = (np + 1) / 2;
  const int p0 = hf ? pa : 0, npw = hf ? np - pa : pa;
  // state tiles of this wave in the 64-state group starting at tile 4 grp
  auto ntw = [&](int grp) {
    const int nt = nn - 4 * grp < 4 ? nn - 4 * grp : 4;
    const int k = nt - 2 * hf;
    return k < 0 ? 0 : (k > 2 ? 2 : k);
  };
  {
    const int64_t off = ((b * L + t0) * G + g) * N;
    stage<Tx, VN, TPB>(&s_C[0][0], NP, static_cast<const Tx*>(p.C) + off, G * N, Q, nvalid, static_cast<int>(N));
    stage<Tx, VN, TPB>(&s_B[0][0], NP, static_cast<const Tx*>(p.B) + off, G * N, Q, nvalid, static_cast<int>(N));
  }
  // Packed sequences: step tid reaches the chunk's end state (w) and reads the
  // entering state (exp(cs)) only within one sequence.
  bool reach = true, from = true;
  if (wave == 0) {
    if (SEQ) s_first[lane] = static_cast<uint8_t>(run_first<SEQ>(p, b, t0, lane));
    const int32_t id = seq_of<SEQ>(p, b, t0 + lane);
    reach = id == seq_of<SEQ>(p, b, t0 + nvalid - 1);
    from = id == seq_of<SEQ>(p, b, t0 - 1);
  }
  __syncthreads();
  // runs of this thread's rows t = 16 ws + 4 q + e: M[t][s] needs first_t <= s <= t
  const uint32_t firsts = SEQ ? *reinterpret_cast<const uint32_t*>(&s_first[16 * ws + 4 * q]) : 0u;
  // C B^T, rows t of this strip, Q-column tiles 2 hf, 2 hf + 1
  v4f cb[2];
  zero(cb);
  mma(cb, 2, &s_C[16 * ws][0], NP, 1, &s_B[32 * hf][0], 1, NP, static_cast<int>(N));
  v4f dBa[2][2], dCa[2][2];   // [64-state group][tile of this wave]
#pragma unroll
  for (int grp = 0; grp < 2; ++grp) {
    zero(dBa[grp]);
    zero(dCa[grp]);
  }
  // The next head's x, dout, z and ysave tiles and decays load into
  // registers while this head's products run.
  raw4<Tx> rx[VX];
  DyTiles<Tx, HAS_Z, TPB> rdy;
  float rcs = 0.f, rcsl = 0.f, rdt = 0.f, rcsL = 0.f, rcslL = 0.f;
  auto fetch = [&](int64_t h) {
    const int64_t row = chunk_row(p, b, h, c);
    const int64_t xoff = ((b * L + t0) * H + h) * P;
    if (tid < Q) {
      rcs = p.cs[row + tid];
      rcsl = p.cs_lo[row + tid];
      rdt = p.step[row + tid];
      rcsL = p.cs[row + Q - 1];
      rcslL = p.cs_lo[row + Q - 1];
    }
    tile_load<Tx, VX, TPB>(rx, static_cast<const Tx*>(p.x) + xoff, H * P, Q, nvalid, static_cast<int>(P));
    rdy.load(p, xoff, H * P, nvalid, static_cast<int>(P), true);
  };
  fetch(h0);
  for (int i = 0; i < p.hb; ++i) {
    const int64_t h = h0 + i;
    const int64_t xoff = ((b * L + t0) * H + h) * P;
    const int64_t row = chunk_row(p, b, h, c);
    const int64_t sb = state_block(p, b, c, h);
    __syncthreads();  // every wave is done with the previous head's tiles
    if (tid < Q) {
      s_cs[tid] = rcs;
      s_csl[tid] = rcsl;
      s_dt[tid] = rdt;
      s_w[tid] = reach ? fast_exp((rcsL - rcs) + (rcslL - rcsl)) : 0.f;
      s_ecs[tid] = from ? fast_exp(rcs + rcsl) : 0.f;
    }
    tile_store<Tx, VX, TPB>(&s_X[0][0], XP, rx, Q, static_cast<int>(P));
    rdy.store(&s_dY[0][0], XP, p, xoff, H * P, nvalid, static_cast<int>(P), true);
    __syncthreads();
    if (i + 1 < p.hb) fetch(h + 1);
    // dGraw = dY x^T (rows t of this strip, this half's columns s); with M and
    // dt: G = CB o M, dCB = dt_s dGraw o M, R = dCB o CB (= dG o G). Row sums
    // of R per half and column sums per strip through LDS, in a fixed order.
    float rowsum[4] = {0.f, 0.f, 0.f, 0.f};
    {
      v4f dg[2];
      zero(dg);
      mma(dg, 2, &s_dY[16 * ws][0], XP, 1, &s_X[32 * hf][0], 1, XP, static_cast<int>(P));
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float colsum = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = 16 * ws + 4 * q + e, s = 32 * hf + 16 * j + r;
          const float m = (s <= t && s >= static_cast<int>((firsts >> (8 * e)) & 0xff)) ? seg_exp(s_cs, s_csl, t, s)
                                                                                     : 0.f;
          const float dcb = dg[j][e] * s_dt[s] * m;
          const float rv = dcb * cb[j][e];
          s_U[t][s] = cb[j][e] * m;
          s_V[t][s] = dcb;
          rowsum[e] += rv;
          colsum += rv;
        }
        s_colp[4 * ws + q][32 * hf + 16 * j + r] = colsum;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) rowsum[e] = row_allreduce16(rowsum[e]);
    if (r < 4) {
      float mine = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (r == e) mine = rowsum[e];
      s_half[hf][0][16 * ws + 4 * q + r] = mine;
    }
    __syncthreads();
    // dcs_intra[t] = sum_s R[t][s] - sum_s R[s][t] (half 0's quarter lanes r < 4 own row t).
    if (hf == 0 && r < 4) {
      const int t = 16 * ws + 4 * q + r;
      float col = 0.f;
      for (int k = 0; k < 16; ++k) col += s_colp[k][t];
      s_dcs[t] = (s_half[0][0][t] + s_half[1][0][t]) - col;
    }
    // d(dt x)[s][p] = sum_t G[t][s] dY[t][p] (rows s of this strip, this half's headdim tiles).
    v4f dxa[2];
    zero(dxa);
    mma(dxa, npw, &s_U[0][16 * ws], 1, QP, &s_dY[0][16 * p0], XP, 1, Q);
    // dH^out and H of a 64-state group into registers, parked in s_U / s_V
    // once the products reading them are done: group 0's load under the dC /
    // dB products, group 1's under group 0's state products.
    float4 su[VX], sv[VX];
    auto load_states = [&](int grp) {
      const int n0 = 64 * grp;
      const int nw = static_cast<int>(N - n0 < 64 ? N - n0 : 64);
      tile_load<float, VX, TPB>(su, p.dstates + sb + n0, N, static_cast<int>(P), static_cast<int>(P), nw);
      tile_load<float, VX, TPB>(sv, p.states + sb + n0, N, static_cast<int>(P), static_cast<int>(P), nw);
    };
    load_states(0);
    // dC[t][n] += sum_s dCB[t][s] B[s][n] ; dB[s][n] += sum_t dCB[t][s] C[t][n] (this wave's state tiles).
#pragma unroll
    for (int grp = 0; grp < 2; ++grp) {
      const int nt = ntw(grp);
      const int col = 64 * grp + 32 * hf;
      mma(dCa[grp], nt, &s_V[16 * ws][0], QP, 1, &s_B[0][col], NP, 1, Q);
      mma(dBa[grp], nt, &s_V[0][16 * ws], 1, QP, &s_C[0][col], NP, 1, Q);
    }
    // State terms, over 64-state groups of dH^out and H.
    float a_row[4] = {0.f, 0.f, 0.f, 0.f};  // sum_n C[t][n] exp(cs_t) (dY H)[t][n]
    float b_row[4] = {0.f, 0.f, 0.f, 0.f};  // sum_n w_s B[s][n] ((dt x) dH)[s][n]
    const float dt_row = s_dt[16 * ws + r], w_row = s_w[16 * ws + r];
#pragma unroll
    for (int grp = 0; grp < kSsdMaxN / 64; ++grp) {
      const int n0 = 64 * grp;
      if (n0 >= N) break;
      const int nw = static_cast<int>(N - n0 < 64 ? N - n0 : 64);
      const int nt = ntw(grp);
      __syncthreads();  // every wave is done reading s_U / s_V
      tile_store<float, VX, TPB>(&s_U[0][0], QP, su, static_cast<int>(P), nw);
      tile_store<float, VX, TPB>(&s_V[0][0], QP, sv, static_cast<int>(P), nw);
      __syncthreads();
      if (n0 + 64 < N) load_states(grp + 1);
      v4f tv[2], yh[2];
      zero(tv);
      zero(yh);
      // tv[s][n] = sum_p dt_s x[s][p] dH[p][n] ; yh[t][n] = sum_p dY[t][p] H[p][n]
      mma<2, true>(tv, nt, &s_X[16 * ws][0], XP, 1, &s_U[0][32 * hf], QP, 1, static_cast<int>(P), dt_row);
      mma(yh, nt, &s_dY[16 * ws][0], XP, 1, &s_V[0][32 * hf], QP, 1, static_cast<int>(P));
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j >= nt) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = 16 * ws + 4 * q + e;
          const int n = n0 + 32 * hf + 16 * j + r;
          const float wt = s_w[t] * tv[j][e];
          const float ys = s_ecs[t] * yh[j][e];
          dBa[grp][j][e] += wt;
          dCa[grp][j][e] += ys;
          b_row[e] = fmaf(s_B[t][n], wt, b_row[e]);
          a_row[e] = fmaf(s_C[t][n], ys, a_row[e]);
        }
      }
      // d(dt x)[s][p] += sum_n w_s B[s][n] dH[p][n] (all states of the group, this half's headdim tiles)
      mma<2, true>(dxa, npw, &s_B[16 * ws][n0], NP, 1, &s_U[16 * p0][0], 1, QP, nw, w_row);
    }
    // sum_p d(dt x) x (for dstep) and dD partial sums over this half's headdim tiles.
    float c_row[4] = {0.f, 0.f, 0.f, 0.f};
    float dD_col[2] = {0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int s = 16 * ws + 4 * q + e;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j >= npw) continue;
        const int pp = 16 * (p0 + j) + r;
        const float xv = s_X[s][pp];
        c_row[e] = fmaf(dxa[j][e], xv, c_row[e]);
        dD_col[j] = fmaf(s_dY[s][pp], xv, dD_col[j]);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a_row[e] = row_allreduce16(a_row[e]);
      b_row[e] = row_allreduce16(b_row[e]);
      c_row[e] = row_allreduce16(c_row[e]);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (j < npw) s_dD[4 * ws + q][16 * (p0 + j) + r] = dD_col[j];
    // the chunk's sum of b_row is the cs_L term of the states' dependence on w
    float bsum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) bsum += b_row[e];  // this quarter's 4 rows, alike in every lane of the row
    bsum = wave_total(r == 0 ? bsum : 0.f);
    if (lane == 0) s_tot[wave] = bsum;
    if (r < 4) {
      float av = 0.f, bv = 0.f, cv = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (r == e) {
          av = a_row[e];
          bv = b_row[e];
          cv = c_row[e];
        }
      const int t = 16 * ws + 4 * q + r;
      s_half[hf][1][t] = av;
      s_half[hf][2][t] = bv;
      s_half[hf][3][t] = cv;
    }
    __syncthreads();  // every wave is done reading s_U / s_V; halves' row sums are in
    // dx = dt d(dt x) + D dY into s_V, stored below four elements at a time
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int s = 16 * ws + 4 * q + e;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j >= npw) continue;
        const int pp = 16 * (p0 + j) + r;
        float dxv = dxa[j][e] * s_dt[s];
        if (p.D) dxv = fmaf(p.D[h * P + pp], s_dY[s][pp], dxv);
        s_V[s][pp] = dxv;
      }
    }
    if (wave == 0) {
      // dcs with the state terms, the cs_L terms, then da = suffix sums over the chunk
      float v = s_dcs[lane] + (s_half[0][1][lane] + s_half[1][1][lane]) -
                (s_half[0][2][lane] + s_half[1][2][lane]);
      if (lane == Q - 1) {
        float l = ((s_tot[0] + s_tot[1]) + (s_tot[2] + s_tot[3])) + ((s_tot[4] + s_tot[5]) + (s_tot[6] + s_tot[7]));
        const float* dl = p.dcsL + (row / Q) * p.nslices;
        for (int64_t k = 0; k < p.nslices; ++k) l += dl[k];
        v += l;
      }
      s_dcs[lane] = wave_suffix_sum(v);
    }
    __syncthreads();
    // dstep = sum_p d(dt x) x + da A, then through softplus / clamp / bias (half 0's quarter lanes).
    float ddt_raw = 0.f, dA_term = 0.f;
    if (hf == 0 && r < 4) {
      const int t = 16 * ws + 4 * q + r;
      if (t < nvalid) {
        float gfac;
        ssd_step(p, b, t0 + t, h, &gfac);
        const float da = s_dcs[t];
        const float c_all = s_half[0][3][t] + s_half[1][3][t];
        ddt_raw = fmaf(da, p.A[h], c_all) * gfac;
        dA_term = da * s_dt[t];
        p.ddt[(b * L + t0 + t) * H + h] = ddt_raw;
      }
    }
    {
      const int nv = np * 4;
      const float inv = 1.0f / static_cast<float>(nv);
#pragma unroll
      for (int k = 0; k < VX; ++k) {
        const int v = tid + k * TPB;
        if (v >= Q * nv) continue;
        const int s = tile_row(v, inv);
        if (s >= nvalid) continue;
        const int pp = (v - s * nv) << 2;
        st4<Tx>(static_cast<Tx*>(p.dx) + xoff + s * H * P + pp, *reinterpret_cast<const float4*>(&s_V[s][pp]));
      }
    }
    const float wa = wave_total(dA_term), wb = wave_total(ddt_raw);
    if (lane == 0) {
      s_wa[wave] = wa;
      s_wb[wave] = wb;
    }
    __syncthreads();
    const int64_t prt = (b * p.nchunks + c) * H + h;
    if (tid == 0) {
      p.dA_part[prt] = ((s_wa[0] + s_wa[1]) + (s_wa[2] + s_wa[3])) + ((s_wa[4] + s_wa[5]) + (s_wa[6] + s_wa[7]));
      p.dbias_part[prt] = ((s_wb[0] + s_wb[1]) + (s_wb[2] + s_wb[3])) + ((s_wb[4] + s_wb[5]) + (s_wb[6] + s_wb[7]));
    }
    if (tid < P) {
      float v = 0.f;
      for (int k = 0; k < 16; ++k) v += s_dD[k][tid];
      p.dD_part[prt * P + tid] = v;
    }
  }
  // the block's dB and dC partial sums (this wave's rows and state tiles)
  const int64_t hbk = blockIdx.y;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int t = 16 * ws + 4 * q + e;
    if (t >= nvalid) continue;
    const int64_t at = ((b * L + t0 + t) * p.nhb + hbk) * N;
#pragma unroll
    for (int grp = 0; grp < 2; ++grp) {
      const int nt = ntw(grp);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (j >= nt) continue;
        const int n = 64 * grp + 32 * hf + 16 * j + r;
        p.dC_part[at + n] = dCa[grp][j][e];
        p.dB_part[at + n] = dBa[grp][j][e];
      }
    }
  }
}

// Per-sequence final states of packed sequences in batch row 0 (mamba_ssm's
// varlen states): entry i is the state after step e = cu[i + 1] - 1. From the
// chunk c holding e, h_e = exp(cs_e) H_c (when step e is in the entering
// state's sequence) + sum_s exp(cs_e - cs_s) dt_s x_s B_s^T over the steps
// s <= e of e's sequence in the chunk: one product on the matrix cores,
// started from the decayed entering state. Empty sequences, and offsets
// outside [0, seqlen], give zeros. Grid (nseqs, nheads); wave w computes state
// rows [16 w, 16 w + 16).
template <typename Tx, bool SEQ>
__global__ void __launch_bounds__(kThreads) ssd_varlen_state_kernel(const SsdParams p, const int32_t* cu,
                                                                     float* out) {
  __shared__ __align__(16) float s_B[Q][NP];
  __shared__ __align__(16) float s_x[Q][XP];
  __shared__ float s_sc[Q];
  const int64_t i = blockIdx.x, h = blockIdx.y, b = 0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t L = p.seqlen, H = p.nheads, P = p.headdim, N = p.dstate, G = p.ngroups;
  const int64_t g = h / (H / G);
  const int nt = static_cast<int>(N / 16);
  const bool act = 16 * wave < P;
  const int64_t eo = (16 * wave + 4 * q) * N + r;   // accumulator (j, e) at eo + e N + 16 j of a block
  float* dst = out + (i * H + h) * P * N + eo;
  v4f acc[kSsdMaxN / 16];
  zero(acc);
  const int64_t start = cu[i], end = cu[i + 1];
  if (start < 0 || end > L || end <= start) {  // the same for the whole workgroup
    if (act)
#pragma unroll
      for (int j = 0; j < kSsdMaxN / 16; ++j)
        if (j < nt)
#pragma unroll
          for (int e = 0; e < 4; ++e) dst[e * N + 16 * j] = 0.f;
    return;
  }
  const int64_t last = end - 1, c = last / Q, t0 = c * Q;
  const int nv = static_cast<int>(last - t0 + 1);
  const int64_t row = chunk_row(p, b, h, c);
  const float cse = p.cs[row + nv - 1], loe = p.cs_lo[row + nv - 1];
  stage<Tx, kVecN>(&s_B[0][0], NP, static_cast<const Tx*>(p.B) + ((b * L + t0) * G + g) * N, G * N, Q, nv,
                   static_cast<int>(N));
  if (wave == 0) {
    const bool in = lane < nv && seq_of<SEQ>(p, b, t0 + lane) == seq_of<SEQ>(p, b, last);
    s_sc[lane] = in ? p.step[row + lane] * fast_exp((cse - p.cs[row + lane]) + (loe - p.cs_lo[row + lane])) : 0.f;
  }
  __syncthreads();
  stage<Tx, kVecX>(&s_x[0][0], XP, static_cast<const Tx*>(p.x) + ((b * L + t0) * H + h) * P, H * P, Q, nv,
                   static_cast<int>(P), s_sc);
  if (act && seq_of<SEQ>(p, b, last) == seq_of<SEQ>(p, b, t0 - 1)) {
    const float hd = fast_exp(cse + loe);
    const float* hs = p.states + state_block(p, b, c, h) + eo;
#pragma unroll
    for (int j = 0; j < kSsdMaxN / 16; ++j)
      if (j < nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[j][e] = hd * hs[e * N + 16 * j];
  }
  __syncthreads();
  if (act) {
    mma(acc, nt, &s_x[0][16 * wave], 1, XP, &s_B[0][0], NP, 1, Q);
#pragma unroll
    for (int j = 0; j < kSsdMaxN / 16; ++j)
      if (j < nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[e * N + 16 * j] = acc[j][e];
  }
}

namespace {

template <typename Tx, bool SEQ>
hipError_t fwd_t(const SsdParams& p, hipStream_t st) {
  const dim3 chunks(static_cast<unsigned>(p.nchunks), static_cast<unsigned>(p.nhb), static_cast<unsigned>(p.batch));
  const dim3 slices(static_cast<unsigned>(p.nslices), static_cast<unsigned>(p.nheads),
                    static_cast<unsigned>(p.batch));
  if (p.in_order) {
    const dim3 rows(static_cast<unsigned>((p.nchunks + kThreads / 64 - 1) / (kThreads / 64)),
                    static_cast<unsigned>(p.nheads), static_cast<unsigned>(p.batch));
    hipLaunchKernelGGL(ssd_chunk_decay_kernel, rows, dim3(kThreads), 0, st, p);
    if (hipError_t e = hipGetLastError()) return e;
    hipLaunchKernelGGL((ssd_state_scan_kernel<Tx, SEQ>), slices, dim3(kThreads), 0, st, p);
  } else {
    // F1 with one head per workgroup whatever the chunk kernels' head block:
    // each of its heads stages its own x and product, so more, smaller
    // workgroups fill the GPU better (28 against 39 us at batch 4, seqlen
    // 1024, 24 heads with blocks of 6); its outputs are per head.
    SsdParams q = p;
    q.hb = 1;
    q.nhb = static_cast<int>(p.nheads);
    const dim3 heads(static_cast<unsigned>(p.nchunks), static_cast<unsigned>(p.nheads), static_cast<unsigned>(p.batch));
    hipLaunchKernelGGL((ssd_chunk_state_kernel<Tx, SEQ>), heads, dim3(kThreads), 0, st, q);
    if (hipError_t e = hipGetLastError()) return e;
    hipLaunchKernelGGL(ssd_state_pass_kernel<SEQ>, slices, dim3(kThreads), 0, st, p);
  }
  if (hipError_t e = hipGetLastError()) return e;
  if (p.z) hipLaunchKernelGGL((ssd_chunk_scan_kernel<Tx, true, SEQ>), chunks, dim3(kThreads3), 0, st, p);
  else hipLaunchKernelGGL((ssd_chunk_scan_kernel<Tx, false, SEQ>), chunks, dim3(kThreads3), 0, st, p);
  return hipGetLastError();
}

template <typename Tx, bool SEQ>
hipError_t bwd_t(const SsdParams& p, hipStream_t st) {
  const dim3 chunks(static_cast<unsigned>(p.nchunks), static_cast<unsigned>(p.nhb), static_cast<unsigned>(p.batch));
  const dim3 slices(static_cast<unsigned>(p.nslices), static_cast<unsigned>(p.nheads),
                    static_cast<unsigned>(p.batch));
  if (p.in_order) {
    if (p.z) hipLaunchKernelGGL((ssd_bwd_state_scan_kernel<Tx, true, SEQ>), slices, dim3(kThreads), 0, st, p);
    else hipLaunchKernelGGL((ssd_bwd_state_scan_kernel<Tx, false, SEQ>), slices, dim3(kThreads), 0, st, p);
  } else {
    // K1 with one head per workgroup, as F1 in the forward
    SsdParams q = p;
    q.hb = 1;
    q.nhb = static_cast<int>(p.nheads);
    const dim3 heads(static_cast<unsigned>(p.nchunks), static_cast<unsigned>(p.nheads), static_cast<unsigned>(p.batch));
    if (p.z) hipLaunchKernelGGL((ssd_bwd_seed_kernel<Tx, true, SEQ>), heads, dim3(kThreads), 0, st, q);
    else hipLaunchKernelGGL((ssd_bwd_seed_kernel<Tx, false, SEQ>), heads, dim3(kThreads), 0, st, q);
    if (hipError_t e = hipGetLastError()) return e;
    hipLaunchKernelGGL(ssd_bwd_pass_kernel<SEQ>, slices, dim3(kThreads), 0, st, p);
  }
  if (hipError_t e = hipGetLastError()) return e;
  if (p.z) hipLaunchKernelGGL((ssd_bwd_chunk_kernel<Tx, true, SEQ>), chunks, dim3(kThreads3), 0, st, p);
  else hipLaunchKernelGGL((ssd_bwd_chunk_kernel<Tx, false, SEQ>), chunks, dim3(kThreads3), 0, st, p);
  return hipGetLastError();
}

}  // namespace

hipError_t ssd_fwd_launch(const SsdParams& p, int dtype, hipStream_t st) {
  const bool seq = p.seq_idx != nullptr;
  switch (dtype) {
    case MCPU_F32: return seq ? fwd_t<float, true>(p, st) : fwd_t<float, false>(p, st);
    case MCPU_BF16: return seq ? fwd_t<bf16, true>(p, st) : fwd_t<bf16, false>(p, st);
    default: return seq ? fwd_t<f16, true>(p, st) : fwd_t<f16, false>(p, st);
  }
}

hipError_t ssd_varlen_launch(const SsdParams& p, const int32_t* cu, int64_t nseqs, float* out, int dtype,
                             hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(nseqs), static_cast<unsigned>(p.nheads));
  const bool seq = p.seq_idx != nullptr;
  switch (dtype) {
    case MCPU_F32:
      if (seq) hipLaunchKernelGGL((ssd_varlen_state_kernel<float, true>), grid, dim3(kThreads), 0, st, p, cu, out);
      else hipLaunchKernelGGL((ssd_varlen_state_kernel<float, false>), grid, dim3(kThreads), 0, st, p, cu, out);
      break;
    case MCPU_BF16:
      if (seq) hipLaunchKernelGGL((ssd_varlen_state_kernel<bf16, true>), grid, dim3(kThreads), 0, st, p, cu, out);
      else hipLaunchKernelGGL((ssd_varlen_state_kernel<bf16, false>), grid, dim3(kThreads), 0, st, p, cu, out);
      break;
    default:
      if (seq) hipLaunchKernelGGL((ssd_varlen_state_kernel<f16, true>), grid, dim3(kThreads), 0, st, p, cu, out);
      else hipLaunchKernelGGL((ssd_varlen_state_kernel<f16, false>), grid, dim3(kThreads), 0, st, p, cu, out);
  }
  return hipGetLastError();
}

hipError_t ssd_bwd_launch(const SsdParams& p, int dtype, hipStream_t st) {
  const bool seq = p.seq_idx != nullptr;
  switch (dtype) {
    case MCPU_F32: return seq ? bwd_t<float, true>(p, st) : bwd_t<float, false>(p, st);
    case MCPU_BF16: return seq ? bwd_t<bf16, true>(p, st) : bwd_t<bf16, false>(p, st);
    default: return seq ? bwd_t<f16, true>(p, st) : bwd_t<f16, false>(p, st);
  }
}

}  // namespace mcpu
