// One decode step of a Mamba-1 block for a batch of single tokens (batch <=
// 8), in three launches:
//   1. block_in_kernel: RMSNorm of the hidden rows (every workgroup, into
//      LDS), the in_proj rows of this workgroup (RW rows per wave, the batch
//      rows at once), and for the x half the depthwise conv update of that
//      channel (conv state shifted in place) with silu. A workgroup of x rows
//      then multiplies its channels' conv outputs by the matching x_proj
//      columns: a partial x_proj sum over those channels, for every output
//      (dt, B, C) and batch row;
//   2. block_ssm_kernel: x_proj = those partial sums added in a fixed order,
//      then dt_proj, softplus, the selective state update (state in place),
//      the D skip and the silu(z) gate;
//   3. gemv_kernel: out_proj, plus the residual.
// Where adding the partial sums would cost block_ssm_kernel more than a
// separate product (wide blocks: many x workgroups times many x_proj
// outputs), x_proj runs as a gemv_kernel between 1 and 2 instead.
// The in_proj, x_proj and out_proj products are matrix-vector products over
// a handful of rows: they read each weight once, four elements per lane
// (coalesced rows), against the batch rows held in LDS, and reduce across
// the wave with DPP and permlane swaps. Intermediate vectors live in a small
// float32 workspace holding values already rounded to the storage type, as
// transformers' separate ops would have stored them.
// Each kernel requests all of its global loads before it waits on any, and
// keeps the values as stored (a float4, or two 32-bit words holding four
// 16-bit values) until then: a conversion next to a conditional load makes
// the compiler wait for that load on the spot, which turns a kernel's
// prologue into a chain of memory round trips.
#include <cstring>
#include <type_traits>

#include "abi_util.h"
#include "mcpu_common.h"

namespace mcpu {

namespace {

constexpr int kThreads = 256;
constexpr int kSsmThreads = 1024;                  // block_ssm_kernel: 64 channels x 16 lanes
constexpr int kSsmChannels = kSsmThreads / 16;
constexpr int kMaxBatch = 8;
constexpr int kMaxLdsFloats = 32768;
constexpr int kMaxConvState = 8;
constexpr int kMaxXdb = 2048;                      // dt_rank + 2 dstate
constexpr int kPartLoads = 16;                     // partial sums one block_ssm thread adds
constexpr int kDtLoads = 8;                        // dt_proj weights per lane requested at once

struct MixerParams {
  const void* hidden;
  const void* norm_w;
  const void* in_w;
  const void* in_b;
  const void* conv_w;
  const void* conv_b;
  void* conv_state;
  const void* x_w;
  const void* dt_w;
  const float* dt_b;
  const float* A;
  const float* D;
  void* ssm_state;
  const void* out_w;
  const void* out_b;
  void* out;
  float* xc;     // (batch, d_inner): silu(conv) of the x half
  float* zg;     // (batch, d_inner): the z half
  float* xdb;    // (batch, dt_rank + 2 dstate): x_proj, when it runs as its own product
  float* xpart;  // (batch, xpp, dt_rank + 2 dstate): partial x_proj sums, or null
  float* yv;     // (batch, d_inner): gated scan output
  int64_t batch, dm, di, R, N, W, S;
  // in_proj rows: nin of them; rows conv_lo .. conv_lo + nconv - 1 go through
  // the conv (into xc, (batch, nconv)), the others, in order, into zg
  // (batch, nin - nconv). Mamba-1: [x | z], conv on x. Mamba-2: [gate | xBC |
  // dt], conv on xBC.
  int64_t nin, conv_lo, nconv;
  int64_t zst;  // zg row stride: nin - nconv rounded up to a multiple of 4
  // Mamba-2 heads: nh heads of hd channels, ng groups of N states; the gated
  // norm's weight and epsilon.
  int64_t nh, hd, ng;
  const void* gn_w;
  float gn_eps;
  int nxwg;      // block_in workgroups holding x rows: partial sums 0 .. nxwg - 1
  int xq, xs;    // block_ssm_kernel adds xq groups of xs partial sums per output
  int xpp;       // = xq xs >= nxwg: partial sums per output, nxwg .. xpp - 1 zero
  float eps;
  int add_residual, hidden_dtype, state_dtype, out_dtype;
};

struct NormLinearParams {
  const void* x;     // (batch, K): float32 when HF, else T
  const void* nw;    // (K), T, or null
  const void* w;     // (nout, K), T
  const void* bias;  // (nout), T, or null
  void* out;         // (batch, nout): float32 when out_f32, else T
  int64_t batch, nout, ngroups;
  int K, out_f32;
  float eps;
};

// v rounded to the storage type T (exact in float32).
template <typename T> __device__ __forceinline__ float rnd(float v) { return to_f32(from_f32<T>(v)); }

// Four consecutive elements of a T tensor as stored: a float4 for float32,
// two 32-bit words for the 16-bit types.
template <typename T> struct Raw4 { using type = uint2; };
template <> struct Raw4<float> { using type = float4; };
template <typename T> using raw4 = typename Raw4<T>::type;

template <typename T> __device__ __forceinline__ raw4<T> ld_raw4(const void* base, int64_t i) {
  return *reinterpret_cast<const raw4<T>*>(static_cast<const T*>(base) + i);
}
template <typename T> __device__ __forceinline__ float4 cvt4(const raw4<T>& r);
template <> __device__ __forceinline__ float4 cvt4<float>(const float4& r) { return r; }
template <> __device__ __forceinline__ float4 cvt4<bf16>(const uint2& u) {
  return make_float4(__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xffff0000u),
                     __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xffff0000u));
}
template <> __device__ __forceinline__ float4 cvt4<f16>(const uint2& u) {
  auto h = [](uint32_t bits) { return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(bits))); };
  return make_float4(h(u.x & 0xffff), h(u.x >> 16), h(u.y & 0xffff), h(u.y >> 16));
}

// Element i of a T tensor as stored, in the low bits of a 32-bit word: each
// 16-bit element gets a register of its own (two 16-bit loads into halves of
// one register would make the second wait for the first).
template <typename T> __device__ __forceinline__ uint32_t ld_bits(const T* base, int64_t i) {
  if constexpr (std::is_same_v<T, float>) return __builtin_bit_cast(uint32_t, base[i]);
  else return *reinterpret_cast<const uint16_t*>(base + i);
}
template <typename T> __device__ __forceinline__ float bits_f32(uint32_t b) {
  if constexpr (std::is_same_v<T, float>) return __builtin_bit_cast(float, b);
  else if constexpr (std::is_same_v<T, bf16>) return __builtin_bit_cast(float, b << 16);
  else return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(b)));
}
template <typename T> __device__ __forceinline__ void st_bits(T* base, int64_t i, uint32_t b) {
  if constexpr (std::is_same_v<T, float>) base[i] = __builtin_bit_cast(float, b);
  else *reinterpret_cast<uint16_t*>(base + i) = static_cast<uint16_t>(b);
}

// Sum over the 64 lanes of a wave, in a fixed order, in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v = row_allreduce16(v);
  v = swap_sum<32>(v, v);
  return swap_sum<16>(v, v);
}

// float4 chunks (256 elements of a row per wave) each lane loads per pass.
constexpr int kChunks = 8;

// This wave's weight rows row0 .. row0 + RW - 1 of a matrix with rows
// 0 .. last, as stored, chunk u of pass k0 at k = k0 + 4 lane + 256 u
// (u < KC). The loads are unconditional, from addresses clamped into the
// matrix (row last, columns K - 4 ..): rows past last and columns past K
// hold copies whose products are never used.
template <typename T, int RW, int KC = kChunks>
struct RowTiles {
  static constexpr int kc = KC;
  raw4<T> w[RW][KC];

  __device__ __forceinline__ void load(const void* wt, int64_t row0, int64_t last, int K, int k0) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int rr = 0; rr < RW; ++rr)
#pragma unroll
      for (int u = 0; u < KC; ++u) {
        const int k = min(k0 + 4 * lane + 256 * u, K - 4);
        w[rr][u] = ld_raw4<T>(wt, (row0 + rr < last ? row0 + rr : last) * K + k);
      }
  }

  // acc[r][m] += sum over this pass's k of X[m][k] W[r][k]; X (MT, K) in LDS.
  template <int MT>
  __device__ __forceinline__ void fma(float (&acc)[RW][MT], const float* sx, int K, int k0) const {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < KC; ++u) {
      const int k = k0 + 4 * lane + 256 * u;
      if (k >= K) break;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float4 xv = *reinterpret_cast<const float4*>(sx + m * K + k);
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) {
          const float4 wv = cvt4<T>(w[rr][u]);
          float a = acc[rr][m];
          a = fmaf(wv.x, xv.x, a);
          a = fmaf(wv.y, xv.y, a);
          a = fmaf(wv.z, xv.z, a);
          a = fmaf(wv.w, xv.w, a);
          acc[rr][m] = a;
        }
      }
    }
  }
};

// acc[r][m] = sum_k X[m][k] W[row0 + r][k], summed over the wave: every lane
// ends with every row's sums. `tiles` holds the first pass's weights,
// requested before X was staged (so their latency overlapped the staging);
// further passes (K > 256 KC) load and multiply in turn.
template <typename T, int MT, int RW, int KC>
__device__ __forceinline__ void rows_dot(float (&acc)[RW][MT], RowTiles<T, RW, KC>& tiles, const float* sx,
                                         const void* w, int64_t row0, int64_t last, int K) {
#pragma unroll
  for (int rr = 0; rr < RW; ++rr)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[rr][m] = 0.f;
  tiles.template fma<MT>(acc, sx, K, 0);
  for (int k0 = 256 * KC; k0 < K; k0 += 256 * KC) {
    tiles.load(w, row0, last, K, k0);
    tiles.template fma<MT>(acc, sx, K, k0);
  }
#pragma unroll
  for (int rr = 0; rr < RW; ++rr)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[rr][m] = wave_sum(acc[rr][m]);
}

// Lane m's value of a wave-uniform array indexed by lane (m < MT).
template <int MT>
__device__ __forceinline__ float pick_lane(const float (&v)[MT], int lane) {
  float y = 0.f;
#pragma unroll
  for (int m = 0; m < MT; ++m)
    if (lane == m) y = v[m];
  return y;
}

// The batch rows of x (batch, K), float32 when HF else T, staged in LDS as
// s_u (MT, K) and RMS-normalised as transformers' MambaRMSNorm does, with
// the weight nw (T) when given:
//   s_u = round_T(nw * round_R(x * rsqrt(mean(x^2) + eps)))
// where x is the row as given, or rounded to T first (CAST: a Mamba block
// casts its input to the weights' dtype before its norm), and round_R
// rounds to the dtype the norm sees (T when CAST or the rows are T, nothing
// for float32 rows). Without a weight s_u = round_T(x). Rows from batch on
// are zero. Four steps, so that a kernel can request loads between them:
// issue() requests the rows and the weight (an absent weight reads alt, any
// T tensor of at least K elements); stage() waits for the rows, stores them
// and sums each row's squares; finish() stores the weight and reduces the
// sums over the workgroup, ending with a barrier; normalize() applies the
// norm, ending with a barrier.
template <typename T, int MT, bool HF, bool CAST>
struct RowStage {
  using TH = std::conditional_t<HF, float, T>;
  static constexpr int kStage = 8, kNorm = 4;
  const void* x;
  const void* nw;
  int K, nbk;
  raw4<TH> hv[kStage];
  raw4<T> nv[kNorm];
  float ss[MT];

  __device__ __forceinline__ RowStage(const void* x_, const void* nw_, int64_t batch, int K_)
      : x(x_), nw(nw_), K(K_), nbk(static_cast<int>(batch) * K_) {}

  __device__ __forceinline__ void issue(const void* alt) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int u = 0; u < kStage; ++u) hv[u] = ld_raw4<TH>(x, min(4 * (tid + kThreads * u), nbk - 4));
#pragma unroll
    for (int u = 0; u < kNorm; ++u) nv[u] = ld_raw4<T>(nw ? nw : alt, min(4 * (tid + kThreads * u), K - 4));
  }

  __device__ __forceinline__ void stage(float* s_u) {
    const int tid = threadIdx.x;
    const bool to_t = CAST || nw == nullptr;
#pragma unroll
    for (int m = 0; m < MT; ++m) ss[m] = 0.f;
    for (int base = 0; base < MT * K; base += 4 * kThreads * kStage) {
      if (base > 0) {
#pragma unroll
        for (int u = 0; u < kStage; ++u) hv[u] = ld_raw4<TH>(x, min(base + 4 * (tid + kThreads * u), nbk - 4));
      }
#pragma unroll
      for (int u = 0; u < kStage; ++u) {
        const int i = base + 4 * (tid + kThreads * u);
        if (i >= MT * K) break;
        const int m = i / K;
        float4 v = i < nbk ? cvt4<TH>(hv[u]) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (to_t) v = make_float4(rnd<T>(v.x), rnd<T>(v.y), rnd<T>(v.z), rnd<T>(v.w));
#pragma unroll
        for (int mm = 0; mm < MT; ++mm)
          if (mm == m) ss[mm] += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        *reinterpret_cast<float4*>(s_u + i) = v;
      }
    }
  }

  __device__ __forceinline__ void finish(float* s_nw, float (*s_red)[kThreads / 64]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (nw) {
#pragma unroll
      for (int u = 0; u < kNorm; ++u) {
        const int i = 4 * (tid + kThreads * u);
        if (i < K) *reinterpret_cast<float4*>(s_nw + i) = cvt4<T>(nv[u]);
      }
      for (int i = 4 * (tid + kThreads * kNorm); i < K; i += 4 * kThreads)
        *reinterpret_cast<float4*>(s_nw + i) = cvt4<T>(ld_raw4<T>(nw, i));
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float t = wave_sum(ss[m]);
        if (lane == 0) s_red[m][wave] = t;
      }
    }
    __syncthreads();
  }

  __device__ __forceinline__ void normalize(float* s_u, const float* s_nw, float (*s_red)[kThreads / 64],
                                            float eps) {
    if (!nw) return;
    for (int i = 4 * threadIdx.x; i < MT * K; i += 4 * kThreads) {
      const int m = i / K;
      float tot = 0.f;
#pragma unroll
      for (int mm = 0; mm < MT; ++mm)
        if (mm == m) tot = (s_red[mm][0] + s_red[mm][1]) + (s_red[mm][2] + s_red[mm][3]);
      const float rs = rsqrtf(tot / static_cast<float>(K) + eps);
      float4 v = *reinterpret_cast<const float4*>(s_u + i);
      const float4 w = *reinterpret_cast<const float4*>(s_nw + (i - m * K));
      if (CAST || !HF)
        v = make_float4(rnd<T>(w.x * rnd<T>(v.x * rs)), rnd<T>(w.y * rnd<T>(v.y * rs)),
                        rnd<T>(w.z * rnd<T>(v.z * rs)), rnd<T>(w.w * rnd<T>(v.w * rs)));
      else
        v = make_float4(rnd<T>(w.x * (v.x * rs)), rnd<T>(w.y * (v.y * rs)), rnd<T>(w.z * (v.z * rs)),
                        rnd<T>(w.w * (v.w * rs)));
      *reinterpret_cast<float4*>(s_u + i) = v;
    }
    __syncthreads();
  }
};

}  // namespace

// 1. RMSNorm (optional) + in_proj + conv update + partial x_proj. Grid:
// ceil(2 d_inner / (4 RW)) workgroups; wave w handles in_proj rows
// (4 blockIdx.x + w) RW + rr, so workgroups 0 .. nxwg - 1 hold the x rows
// (channels 4 RW blockIdx.x onwards). HF: the hidden rows are float32 (else T).
template <typename T, int MT, int RW, bool HF>
__global__ void __launch_bounds__(kThreads) block_in_kernel(const MixerParams p) {
  extern __shared__ __align__(16) float s_u[];   // (MT, d_model) rows, then the norm weight
  __shared__ float s_red[MT][kThreads / 64];
  __shared__ float s_xc[MT][4 * RW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = static_cast<int>(p.dm);
  float* s_nw = s_u + MT * K;
  const int64_t nout = p.nin, nplain = p.zst;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + wave) * RW;
  const int nrows = row0 >= nout ? 0 : static_cast<int>(nout - row0 < RW ? nout - row0 : RW);
  // Loads: first the hidden rows and the norm weight; once the rows are in,
  // what the epilogue needs (lane m < batch: the bias and, for x rows, batch
  // row m's conv window, weights and bias) and, in an x workgroup, the x_proj
  // columns of its channels (thread j: output j); after the first barrier
  // this wave's in_proj rows, which stream in while the norm runs. Requested
  // before the rows arrive, the in_proj rows of every workgroup delay them
  // (by about 1.4 us at Mamba-130M widths) more than issuing them later
  // costs. Every load is unconditional, from an index clamped into its
  // tensor (an absent optional tensor reads another one of its type); values
  // read for positions outside it are never used. The scheduling barriers
  // keep the groups in this order.
  RowStage<T, MT, HF, true> rows(p.hidden, p.norm_w, p.batch, K);
  rows.issue(p.in_w);
  __builtin_amdgcn_sched_barrier(0);
  rows.stage(s_u);
  __builtin_amdgcn_sched_barrier(0);
  const T* tb = static_cast<const T*>(p.in_b);
  const T* cb = static_cast<const T*>(p.conv_b ? p.conv_b : p.conv_w);
  const T* tbl = tb ? tb : static_cast<const T*>(p.in_w);
  const int64_t ml = lane < p.batch ? lane : p.batch - 1;
  uint32_t eb[RW], ecb[RW], est[RW][kMaxConvState], ecw[RW][kMaxConvState];
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int64_t n = row0 + rr < nout ? row0 + rr : nout - 1;
    const int64_t cn = n - p.conv_lo;  // conv channel of the row, clamped into the conv rows
    const int64_t nx = cn < 0 ? 0 : (cn < p.nconv ? cn : p.nconv - 1);
    eb[rr] = ld_bits(tbl, n);
    ecb[rr] = ld_bits(cb, nx);
    const T* stt = static_cast<const T*>(p.conv_state) + (ml * p.nconv + nx) * p.S;
    const T* cw = static_cast<const T*>(p.conv_w) + nx * p.W;
#pragma unroll
    for (int i = 0; i < kMaxConvState; ++i) {
      est[rr][i] = ld_bits(stt, min(i, static_cast<int>(p.S) - 1));
      ecw[rr][i] = ld_bits(cw, min(i, static_cast<int>(p.W) - 1));
    }
  }
  const int64_t J = p.R + 2 * p.N;
  const bool xpart = p.xpart != nullptr && static_cast<int>(blockIdx.x) < p.nxwg;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 4 * RW;
  const int cw = xpart ? static_cast<int>(p.di - c0 < 4 * RW ? p.di - c0 : 4 * RW) : 0;
  raw4<T> xw[RW];
  if (xpart) {
    const int64_t jl = tid < J ? tid : J - 1;
#pragma unroll
    for (int u = 0; u < RW; ++u) xw[u] = ld_raw4<T>(p.x_w, jl * p.di + c0 + min(4 * u, cw - 4));
  }
  __builtin_amdgcn_sched_barrier(0);
  rows.finish(s_nw, s_red);
  RowTiles<T, RW> tiles;
  tiles.load(p.in_w, row0, nout - 1, K, 0);
  __builtin_amdgcn_sched_barrier(0);
  rows.normalize(s_u, s_nw, s_red, p.eps);
  if (nrows > 0) {
    float acc[RW][MT];
    rows_dot<T, MT, RW>(acc, tiles, s_u, p.in_w, row0, nout - 1, K);
    // Lane m finishes batch row m of each of the wave's rows.
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
      const int64_t n = row0 + rr;
      float y = pick_lane<MT>(acc[rr], lane);
      if (rr >= nrows || lane >= p.batch) continue;
      const int64_t m = lane;
      y = rnd<T>(tb ? y + bits_f32<T>(eb[rr]) : y);
      const int64_t cn = n - p.conv_lo;
      if (cn < 0 || cn >= p.nconv) {
        p.zg[m * nplain + (cn < 0 ? n : n - p.nconv)] = y;
        continue;
      }
      // Depthwise conv update of channel cn: taps 0 .. W-2 read the newest W-1
      // state entries, tap W-1 reads y; the state shifts left by one and y
      // becomes its newest entry.
      float c = p.conv_b ? bits_f32<T>(ecb[rr]) : 0.f;
      for (int k = 0; k < p.W - 1; ++k) {
        uint32_t v = 0, wk = 0;
#pragma unroll
        for (int i = 0; i < kMaxConvState; ++i) {
          if (i == p.S - (p.W - 1) + k) v = est[rr][i];
          if (i == k) wk = ecw[rr][i];
        }
        c = fmaf(bits_f32<T>(wk), bits_f32<T>(v), c);
      }
      uint32_t wl = 0;
#pragma unroll
      for (int i = 0; i < kMaxConvState; ++i)
        if (i == p.W - 1) wl = ecw[rr][i];
      c = fmaf(bits_f32<T>(wl), y, c);
      c = c * sigmoid(c);
      T* stt = static_cast<T*>(p.conv_state) + (m * p.nconv + cn) * p.S;
#pragma unroll
      for (int i = 0; i < kMaxConvState - 1; ++i)
        if (i < p.S - 1) st_bits(stt, i, est[rr][i + 1]);
      stt[p.S - 1] = from_f32<T>(y);
      c = rnd<T>(c);
      p.xc[m * p.nconv + cn] = c;
      if (p.xpart) s_xc[m][wave * RW + rr] = c;
    }
  }
  if (!xpart) return;  // uniform across the workgroup
  // Partial x_proj over this workgroup's channels c0 .. c0 + cw - 1: thread j
  // sums output j for every batch row, into partial-sum row blockIdx.x (rows
  // of the outputs, so consecutive threads store consecutive words); the last
  // x workgroup also zeroes the padding rows.
  __syncthreads();
  for (int64_t j = tid; j < J; j += kThreads) {
    raw4<T> wr[RW];
#pragma unroll
    for (int u = 0; u < RW; ++u) {
      wr[u] = xw[u];
      if (j != tid) {
        wr[u] = raw4<T>{};
        if (4 * u < cw) wr[u] = ld_raw4<T>(p.x_w, j * p.di + c0 + 4 * u);
      }
    }
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.f;
#pragma unroll
    for (int u = 0; u < RW; ++u) {
      if (4 * u >= cw) break;
      const float4 w = cvt4<T>(wr[u]);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float a = acc[m];
        a = fmaf(s_xc[m][4 * u], w.x, a);
        a = fmaf(s_xc[m][4 * u + 1], w.y, a);
        a = fmaf(s_xc[m][4 * u + 2], w.z, a);
        a = fmaf(s_xc[m][4 * u + 3], w.w, a);
        acc[m] = a;
      }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m >= p.batch) break;
      float* dst = p.xpart + m * p.xpp * J + j;
      dst[blockIdx.x * J] = acc[m];
      if (static_cast<int>(blockIdx.x) == p.nxwg - 1)
        for (int q = p.nxwg; q < p.xpp; ++q) dst[q * J] = 0.f;
    }
  }
}

// 3 (and x_proj where it runs alone). Rows n of y[m][n] = round_T(sum_k
// x[m][k] W[n][k] + bias[n]) for x (batch, K) float32 from the workspace:
// into outf (batch, nout) float32 when given, else out (out_dtype) =
// residual + y when add_residual (residual: the hidden rows, float32 when HF,
// else T), else y.
template <typename T, int MT, int RW, bool HF>
__global__ void __launch_bounds__(kThreads) gemv_kernel(const MixerParams p, const float* x, const void* w,
                                                        const void* bias, int64_t nout, int K, float* outf) {
  using TH = std::conditional_t<HF, float, T>;
  extern __shared__ __align__(16) float s_x[];   // (MT, K)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + wave) * RW;
  const int nrows = row0 >= nout ? 0 : static_cast<int>(nout - row0 < RW ? nout - row0 : RW);
  const int nbk = static_cast<int>(p.batch) * K;
  // Loads: the x rows (staged into LDS first), this wave's weight rows, the
  // epilogue's bias and residual.
  // Unconditional, from indexes clamped into each tensor.
  // An absent bias reads the weights; the residual is read from the hidden
  // rows (batch, nout) of an out_proj, from x itself (float32, HF) for an
  // x_proj, whose result takes none.
  constexpr int kStage = 16;
  float4 xv[kStage];
#pragma unroll
  for (int u = 0; u < kStage; ++u)
    xv[u] = *reinterpret_cast<const float4*>(x + min(4 * (tid + kThreads * u), nbk - 4));
  __builtin_amdgcn_sched_barrier(0);
  RowTiles<T, RW> tiles;
  tiles.load(w, row0, nout - 1, K, 0);
  const int64_t ml = lane < p.batch ? lane : p.batch - 1;
  const T* bl = static_cast<const T*>(bias ? bias : w);
  const TH* hb = outf ? reinterpret_cast<const TH*>(x) : static_cast<const TH*>(p.hidden);
  const int64_t hmax = outf ? nbk - 1 : p.batch * nout - 1;
  uint32_t eb[RW], er[RW];
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int64_t n = row0 + rr < nout ? row0 + rr : nout - 1;
    eb[rr] = ld_bits(bl, n);
    er[rr] = ld_bits(hb, min(ml * nout + n, hmax));
  }
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int i = 4 * (tid + kThreads * u);
    if (i < MT * K) *reinterpret_cast<float4*>(s_x + i) = i < nbk ? xv[u] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int i = 4 * (tid + kThreads * kStage); i < MT * K; i += 4 * kThreads) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < nbk) v = *reinterpret_cast<const float4*>(x + i);
    *reinterpret_cast<float4*>(s_x + i) = v;
  }
  __syncthreads();
  if (nrows == 0) return;
  float acc[RW][MT];
  rows_dot<T, MT, RW>(acc, tiles, s_x, w, row0, nout - 1, K);
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int64_t n = row0 + rr;
    float y = pick_lane<MT>(acc[rr], lane);
    if (rr >= nrows || lane >= p.batch) continue;
    const int64_t m = lane;
    y = rnd<T>(bias ? y + bits_f32<T>(eb[rr]) : y);
    if (outf) {
      outf[m * nout + n] = y;
    } else {
      if (p.add_residual) y = bits_f32<TH>(er[rr]) + y;
      if (p.out_dtype == MCPU_F32) static_cast<float*>(p.out)[m * nout + n] = y;
      else st<T>(p.out, m * nout + n, y);
    }
  }
}

// 2. x_proj (the partial sums added, FUSED, or the finished row) + dt_proj +
// softplus + selective state update + D skip + silu(z) gate. 16 lanes per
// channel (state n = lane + 16 s), 64 channels per workgroup; grid
// (ceil(d_inner / 64), batch). The arithmetic of each channel is the
// selective state update kernel's.
template <typename T, typename Ts, int SPL, bool FUSED>
__global__ void __launch_bounds__(kSsmThreads) block_ssm_kernel(const MixerParams p) {
  __shared__ float s_red[kSsmThreads];
  __shared__ float s_xdb[kMaxXdb];
  const int tid = threadIdx.x, j = tid & 15;
  const int64_t d = blockIdx.x * static_cast<int64_t>(kSsmChannels) + (tid >> 4);
  const int64_t m = blockIdx.y;
  const int64_t R = p.R, N = p.N, J = R + 2 * N;
  const bool live = d < p.di;
  // Loads first. x_proj of batch row m: thread (q, oj) = (tid / J, tid % J)
  // reads partial sums q xs .. q xs + xs - 1 of output oj (a wave reads
  // consecutive words of a partial-sum row).
  // All loads are unconditional, from indexes clamped into each tensor;
  // values read for positions outside it are never used.
  const int pq = FUSED ? tid / static_cast<int>(J) : 0;
  const int pj = FUSED ? tid - pq * static_cast<int>(J) : 0;
  const bool pa = FUSED && pq < p.xq;
  float pv[FUSED ? kPartLoads : 1];
  constexpr int kXr = kMaxXdb / kSsmThreads;
  float xr[FUSED ? 1 : kXr];
  if constexpr (FUSED) {
    const float* src = p.xpart + (m * p.xpp + (pa ? pq : p.xq - 1) * p.xs) * J + pj;
#pragma unroll
    for (int u = 0; u < kPartLoads; ++u) pv[u] = src[min(u, p.xs - 1) * J];
  } else {
#pragma unroll
    for (int u = 0; u < kXr; ++u) xr[u] = p.xdb[m * J + min(static_cast<int64_t>(tid + kSsmThreads * u), J - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);
  // This channel: its dt_proj row (lane j: r = j + 16 i), state, A, x, z, D
  // and dt bias.
  const int64_t dl = live ? d : p.di - 1;
  const T* dtw = static_cast<const T*>(p.dt_w) + dl * R;
  Ts* state = static_cast<Ts*>(p.ssm_state) + (m * p.di + dl) * N;
  uint32_t dw[kDtLoads];
#pragma unroll
  for (int i = 0; i < kDtLoads; ++i) dw[i] = ld_bits(dtw, min(static_cast<int64_t>(j + 16 * i), R - 1));
  uint32_t sv0[SPL];
  float av[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int64_t n = min(static_cast<int64_t>(j + 16 * s), N - 1);
    sv0[s] = ld_bits(state, n);
    av[s] = p.A[dl * N + n];
  }
  const float x = p.xc[m * p.di + dl], zz = p.zg[m * p.di + dl];
  const float Dd = (p.D ? p.D : p.A)[dl], bias = (p.dt_b ? p.dt_b : p.A)[dl];
  __builtin_amdgcn_sched_barrier(0);
  // x_proj into LDS, rounded to T as the product's output.
  if constexpr (FUSED) {
    // Selects, not a loop bound: a load used only under a condition would
    // be moved next to its use.
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < kPartLoads; ++u) sum = u < p.xs ? sum + pv[u] : sum;
    if (pa) s_red[pq * J + pj] = sum;
    __syncthreads();
    for (int t = tid; t < J; t += kSsmThreads) {
      float a = 0.f;
      for (int q = 0; q < p.xq; ++q) a += s_red[q * J + t];
      s_xdb[t] = rnd<T>(a);
    }
  } else {
#pragma unroll
    for (int u = 0; u < kXr; ++u) {
      const int t = tid + kSsmThreads * u;
      if (t < J) s_xdb[t] = xr[u];
    }
  }
  __syncthreads();
  if (!live) return;  // whole 16-lane rows leave together, after the last barrier
  float part = 0.f;
#pragma unroll
  for (int i = 0; i < kDtLoads; ++i)
    if (j + 16 * i < R) part = fmaf(s_xdb[j + 16 * i], bits_f32<T>(dw[i]), part);
  for (int64_t r0 = 16 * kDtLoads; r0 < R; r0 += 16 * kDtLoads) {  // dt_rank > 128: one round trip per 128
#pragma unroll
    for (int i = 0; i < kDtLoads; ++i) dw[i] = ld_bits(dtw, min(r0 + j + 16 * i, R - 1));
#pragma unroll
    for (int i = 0; i < kDtLoads; ++i)
      if (r0 + j + 16 * i < R) part = fmaf(s_xdb[r0 + j + 16 * i], bits_f32<T>(dw[i]), part);
  }
  float dt = rnd<T>(row_allreduce16(part));
  if (p.dt_b) dt += bias;
  dt = softplus(dt);
  const float dtx = dt * x;
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int64_t n = j + 16 * s;
    if (n < N) {
      const float a = fast_exp(dt * av[s]);
      const float sv = fmaf(bits_f32<Ts>(sv0[s]), a, dtx * s_xdb[R + n]);
      state[n] = from_f32<Ts>(sv);
      acc = fmaf(sv, s_xdb[R + N + n], acc);
    }
  }
  float y = row_allreduce16(acc);
  if (j == 0) {
    if (p.D) y = fmaf(x, Dd, y);
    y *= zz * sigmoid(zz);
    p.yv[m * p.di + d] = rnd<T>(y);
  }
}

// Mamba-2 step, launch 2: the selective state update of every (head,
// channel) row, in the state update kernel's layout and arithmetic (16 lanes
// per row, states n = lane + 16 s, the same fixed-order sums):
//   dt = softplus(dt_raw[h] + dt_bias[h]),
//   state = state exp(dt A[h]) + dt x B_g,   y = <state, C_g> + D[h] x,
// y rounded to T. x, B and C are the conv outputs (xc: x | B | C of every
// group), dt_raw the in_proj rows after the gate (zg). Grid
// (ceil(nh hd / 16), batch).
template <typename T, typename Ts, int SPL>
__global__ void __launch_bounds__(256) m2_ssm_kernel(const MixerParams p) {
  const int j = threadIdx.x & 15;
  const int64_t hp = blockIdx.x * 16ll + (threadIdx.x >> 4);
  const int64_t m = blockIdx.y;
  if (hp >= p.nh * p.hd) return;  // whole 16-lane rows leave together
  const int64_t h = hp / p.hd, g = h / (p.nh / p.ng), N = p.N;
  const float* xr = p.xc + m * p.nconv;
  const float* Bg = xr + p.di + g * N;
  const float* Cg = xr + p.di + p.ng * N + g * N;
  Ts* state = static_cast<Ts*>(p.ssm_state) + (m * p.nh * p.hd + hp) * N;
  // Loads first, unconditional from indexes clamped into the row.
  uint32_t sv[SPL];
  float bv[SPL], cv[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int64_t n = min(static_cast<int64_t>(j + 16 * s), N - 1);
    sv[s] = ld_bits(state, n);
    bv[s] = Bg[n];
    cv[s] = Cg[n];
  }
  const float x = xr[hp];
  float dt = p.zg[m * p.zst + p.di + h];
  const float Ah = p.A[h];
  const float bias = (p.dt_b ? p.dt_b : p.A)[h], Dh = (p.D ? p.D : p.A)[h];
  if (p.dt_b) dt += bias;
  dt = softplus(dt);
  const float dtx = dt * x;
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int64_t n = j + 16 * s;
    if (n < N) {
      const float v = fmaf(bits_f32<Ts>(sv[s]), fast_exp(dt * Ah), dtx * bv[s]);
      state[n] = from_f32<Ts>(v);
      acc = fmaf(v, cv[s], acc);
    }
  }
  float y = row_allreduce16(acc);
  if (j == 0) {
    if (p.D) y = fmaf(x, Dh, y);
    p.yv[m * p.di + hp] = rnd<T>(y);
  }
}

// Mamba-2 step, launch 3: transformers' MambaRMSNormGated of the scan output
// and out_proj, plus the residual:
//   r = y silu(gate) (float32),  u = round_T(w round_T(r rsqrt(mean(r^2) + eps))),
//   out = round_T(out_w u + out_b) [+ residual]
// y (batch, d_inner) from yv, the gate from the first d_inner plain rows of
// zg. Every workgroup stages and normalises the rows; its waves then take
// their out_proj rows as gemv_kernel does. HF: the residual is float32.
template <typename T, int MT, int RW, bool HF>
__global__ void __launch_bounds__(kThreads) m2_out_kernel(const MixerParams p) {
  using TH = std::conditional_t<HF, float, T>;
  extern __shared__ __align__(16) float s_u[];   // (MT, d_inner) rows, then the norm weight
  __shared__ float s_red[MT][kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = static_cast<int>(p.di);
  const int64_t nout = p.dm;
  float* s_nw = s_u + MT * K;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + wave) * RW;
  const int nrows = row0 >= nout ? 0 : static_cast<int>(nout - row0 < RW ? nout - row0 : RW);
  const int nbk = static_cast<int>(p.batch) * K;
  // Loads: the rows and their gates, the norm weight; then the epilogue's
  // bias and residual; the out_proj rows after the first barrier. All
  // unconditional, from indexes clamped into their tensors.
  constexpr int kStage = 8, kNorm = 4;
  float4 yv4[kStage], gv4[kStage];
  auto load_rows = [&](int base) {
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int i = min(base + 4 * (tid + kThreads * u), nbk - 4);
      const int m = i / K;
      yv4[u] = *reinterpret_cast<const float4*>(p.yv + i);
      gv4[u] = *reinterpret_cast<const float4*>(p.zg + m * p.zst + (i - m * K));
    }
  };
  load_rows(0);
  raw4<T> nv[kNorm];
#pragma unroll
  for (int u = 0; u < kNorm; ++u) nv[u] = ld_raw4<T>(p.gn_w, min(4 * (tid + kThreads * u), K - 4));
  __builtin_amdgcn_sched_barrier(0);
  float ss[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) ss[m] = 0.f;
  for (int base = 0; base < MT * K; base += 4 * kThreads * kStage) {
    if (base > 0) load_rows(base);
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int i = base + 4 * (tid + kThreads * u);
      if (i >= MT * K) break;
      const int m = i / K;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < nbk) {
        const float4 y = yv4[u], gt = gv4[u];
        v = make_float4(y.x * (gt.x * sigmoid(gt.x)), y.y * (gt.y * sigmoid(gt.y)), y.z * (gt.z * sigmoid(gt.z)),
                        y.w * (gt.w * sigmoid(gt.w)));
      }
#pragma unroll
      for (int mm = 0; mm < MT; ++mm)
        if (mm == m) ss[mm] += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
      *reinterpret_cast<float4*>(s_u + i) = v;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const int64_t ml = lane < p.batch ? lane : p.batch - 1;
  const T* bl = static_cast<const T*>(p.out_b ? p.out_b : p.out_w);
  const TH* hb = static_cast<const TH*>(p.hidden);
  uint32_t eb[RW], er[RW];
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int64_t n = row0 + rr < nout ? row0 + rr : nout - 1;
    eb[rr] = ld_bits(bl, n);
    er[rr] = ld_bits(hb, ml * nout + n);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < kNorm; ++u) {
    const int i = 4 * (tid + kThreads * u);
    if (i < K) *reinterpret_cast<float4*>(s_nw + i) = cvt4<T>(nv[u]);
  }
  for (int i = 4 * (tid + kThreads * kNorm); i < K; i += 4 * kThreads)
    *reinterpret_cast<float4*>(s_nw + i) = cvt4<T>(ld_raw4<T>(p.gn_w, i));
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float t = wave_sum(ss[m]);
    if (lane == 0) s_red[m][wave] = t;
  }
  __syncthreads();
  RowTiles<T, RW> tiles;
  tiles.load(p.out_w, row0, nout - 1, K, 0);
  __builtin_amdgcn_sched_barrier(0);
  for (int i = 4 * tid; i < MT * K; i += 4 * kThreads) {
    const int m = i / K;
    float tot = 0.f;
#pragma unroll
    for (int mm = 0; mm < MT; ++mm)
      if (mm == m) tot = (s_red[mm][0] + s_red[mm][1]) + (s_red[mm][2] + s_red[mm][3]);
    const float rs = rsqrtf(tot / static_cast<float>(K) + p.gn_eps);
    float4 v = *reinterpret_cast<const float4*>(s_u + i);
    const float4 w = *reinterpret_cast<const float4*>(s_nw + (i - m * K));
    v = make_float4(rnd<T>(w.x * rnd<T>(v.x * rs)), rnd<T>(w.y * rnd<T>(v.y * rs)),
                    rnd<T>(w.z * rnd<T>(v.z * rs)), rnd<T>(w.w * rnd<T>(v.w * rs)));
    *reinterpret_cast<float4*>(s_u + i) = v;
  }
  __syncthreads();
  if (nrows == 0) return;
  float acc[RW][MT];
  rows_dot<T, MT, RW>(acc, tiles, s_u, p.out_w, row0, nout - 1, K);
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int64_t n = row0 + rr;
    float y = pick_lane<MT>(acc[rr], lane);
    if (rr >= nrows || lane >= p.batch) continue;
    y = rnd<T>(p.out_b ? y + bits_f32<T>(eb[rr]) : y);
    if (p.add_residual) y = bits_f32<TH>(er[rr]) + y;
    if (p.out_dtype == MCPU_F32) static_cast<float*>(p.out)[lane * nout + n] = y;
    else st<T>(p.out, lane * nout + n, y);
  }
}

// Final RMSNorm and a wide product for a handful of rows (a decode step's
// norm_f + lm_head): out[m][n] = round_T(sum_k u[m][k] W[n][k] + bias[n])
// with u the normalised rows (RowStage, rows as given). Persistent: each of
// gridDim.x workgroups stages and normalises the rows once, then walks the
// row groups g = blockIdx.x, blockIdx.x + gridDim.x, ... (RW rows per wave,
// 4 RW per group), requesting the next group's weights and bias before it
// multiplies the current one, so a workgroup keeps one group in flight
// while it computes. The request for a group past the end reads the last
// group again (unconditional: a conditional request would make the wait
// for the current group cover it too).
template <typename T, int MT, int RW, int KC, bool HF>
__global__ void __launch_bounds__(kThreads) norm_linear_kernel(const NormLinearParams p) {
  extern __shared__ __align__(16) float s_u[];   // (MT, K) rows, then the norm weight
  __shared__ float s_red[MT][kThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int K = p.K;
  const int64_t last = p.nout - 1;
  const T* bl = static_cast<const T*>(p.bias ? p.bias : p.w);
  auto row_of = [&](int64_t g) { return (g * (kThreads / 64) + wave) * RW; };
  RowStage<T, MT, HF, false> rows(p.x, p.nw, p.batch, K);
  rows.issue(p.w);
  __builtin_amdgcn_sched_barrier(0);
  rows.stage(s_u);
  __builtin_amdgcn_sched_barrier(0);
  rows.finish(s_u + MT * K, s_red);
  int64_t g = blockIdx.x;
  RowTiles<T, RW, KC> cur, nxt;
  uint32_t eb[RW], ebn[RW];
  cur.load(p.w, row_of(g), last, K, 0);
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) eb[rr] = ld_bits(bl, min(row_of(g) + rr, last));
  __builtin_amdgcn_sched_barrier(0);
  rows.normalize(s_u, s_u + MT * K, s_red, p.eps);
  for (; g < p.ngroups; g += gridDim.x) {
    const int64_t gn = min(g + static_cast<int64_t>(gridDim.x), p.ngroups - 1);
    nxt.load(p.w, row_of(gn), last, K, 0);
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) ebn[rr] = ld_bits(bl, min(row_of(gn) + rr, last));
    __builtin_amdgcn_sched_barrier(0);
    const int64_t row0 = row_of(g);
    float acc[RW][MT];
    rows_dot<T, MT, RW, KC>(acc, cur, s_u, p.w, row0, last, K);
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) {
      const int64_t n = row0 + rr;
      float y = pick_lane<MT>(acc[rr], lane);
      if (n > last || lane >= p.batch) continue;
      y = rnd<T>(p.bias ? y + bits_f32<T>(eb[rr]) : y);
      if (p.out_f32) static_cast<float*>(p.out)[lane * p.nout + n] = y;
      else st<T>(p.out, lane * p.nout + n, y);
    }
    cur = nxt;
#pragma unroll
    for (int rr = 0; rr < RW; ++rr) eb[rr] = ebn[rr];
  }
}

namespace {

// Rows per wave: as many as keep at least 256 workgroups.
int rows_per_wave(int64_t nout) {
  for (int rw = 4; rw > 1; rw /= 2)
    if ((nout + 4 * rw - 1) / (4 * rw) >= 256) return rw;
  return 1;
}

// How block_ssm_kernel adds the partial x_proj sums of nxwg workgroups for
// J outputs: xq groups of xs (at most kPartLoads) per output, xq J <=
// kSsmThreads. Returns false where that does not fit: then x_proj runs as
// its own product.
bool partial_plan(int64_t nxwg, int64_t J, int* xq, int* xs) {
  if (J > kSsmThreads) return false;
  int64_t q = kSsmThreads / J;
  if (q > nxwg) q = nxwg;
  const int64_t s = (nxwg + q - 1) / q;
  if (s > kPartLoads) return false;
  *xq = static_cast<int>(q);
  *xs = static_cast<int>(s);
  return true;
}

template <typename T, int MT, int RW>
hipError_t launch_in(const MixerParams& p, bool hf, hipStream_t st) {
  const int64_t nin = p.nin;
  const dim3 grid(static_cast<unsigned>((nin + 4 * RW - 1) / (4 * RW)));
  const size_t lds = sizeof(float) * (MT + 1) * p.dm;
  if (hf || std::is_same_v<T, float>)
    hipLaunchKernelGGL((block_in_kernel<T, MT, RW, true>), grid, dim3(kThreads), lds, st, p);
  else
    hipLaunchKernelGGL((block_in_kernel<T, MT, RW, false>), grid, dim3(kThreads), lds, st, p);
  return hipGetLastError();
}

template <typename T, int MT, int RW, bool HF>
void launch_gemv(const MixerParams& p, const float* x, const void* w, const void* bias, int64_t nout, int64_t K,
                 float* outf, hipStream_t st) {
  const size_t lds = sizeof(float) * MT * K;
  hipLaunchKernelGGL((gemv_kernel<T, MT, RW, HF>), dim3(static_cast<unsigned>((nout + 4 * RW - 1) / (4 * RW))),
                     dim3(kThreads), lds, st, p, x, w, bias, nout, static_cast<int>(K), outf);
}

template <typename T, int MT, bool HF>
hipError_t gemv(const MixerParams& p, const float* x, const void* w, const void* bias, int64_t nout, int64_t K,
                float* outf, hipStream_t st) {
  const int rw = rows_per_wave(nout);
  if (rw == 4) launch_gemv<T, MT, 4, HF>(p, x, w, bias, nout, K, outf, st);
  else if (rw == 2) launch_gemv<T, MT, 2, HF>(p, x, w, bias, nout, K, outf, st);
  else launch_gemv<T, MT, 1, HF>(p, x, w, bias, nout, K, outf, st);
  return hipGetLastError();
}

template <typename T, typename Ts, bool FUSED>
hipError_t launch_ssm(const MixerParams& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((p.di + kSsmChannels - 1) / kSsmChannels), static_cast<unsigned>(p.batch));
  if (p.N <= 16) hipLaunchKernelGGL((block_ssm_kernel<T, Ts, 1, FUSED>), grid, dim3(kSsmThreads), 0, st, p);
  else if (p.N <= 32) hipLaunchKernelGGL((block_ssm_kernel<T, Ts, 2, FUSED>), grid, dim3(kSsmThreads), 0, st, p);
  else if (p.N <= 64) hipLaunchKernelGGL((block_ssm_kernel<T, Ts, 4, FUSED>), grid, dim3(kSsmThreads), 0, st, p);
  else hipLaunchKernelGGL((block_ssm_kernel<T, Ts, 8, FUSED>), grid, dim3(kSsmThreads), 0, st, p);
  return hipGetLastError();
}

template <typename T, bool FUSED>
hipError_t launch_ssm_state(const MixerParams& p, hipStream_t st) {
  switch (p.state_dtype) {
    case MCPU_F32: return launch_ssm<T, float, FUSED>(p, st);
    case MCPU_BF16: return launch_ssm<T, bf16, FUSED>(p, st);
    default: return launch_ssm<T, f16, FUSED>(p, st);
  }
}

template <typename T, int MT>
hipError_t step_t(const MixerParams& p, hipStream_t st) {
  const int rw = rows_per_wave(p.nin);
  const bool hf = p.hidden_dtype == MCPU_F32;
  hipError_t e = rw == 4 ? launch_in<T, MT, 4>(p, hf, st) : rw == 2 ? launch_in<T, MT, 2>(p, hf, st)
                                                                    : launch_in<T, MT, 1>(p, hf, st);
  if (e != hipSuccess) return e;
  if (p.xpart) {
    e = launch_ssm_state<T, true>(p, st);
  } else {
    if ((e = gemv<T, MT, true>(p, p.xc, p.x_w, nullptr, p.R + 2 * p.N, p.di, p.xdb, st)) != hipSuccess) return e;
    e = launch_ssm_state<T, false>(p, st);
  }
  if (e != hipSuccess) return e;
  return hf || std::is_same_v<T, float> ? gemv<T, MT, true>(p, p.yv, p.out_w, p.out_b, p.dm, p.di, nullptr, st)
                                        : gemv<T, MT, false>(p, p.yv, p.out_w, p.out_b, p.dm, p.di, nullptr, st);
}

template <typename T>
hipError_t step_dtype(const MixerParams& p, hipStream_t st) {
  if (p.batch <= 1) return step_t<T, 1>(p, st);
  if (p.batch <= 2) return step_t<T, 2>(p, st);
  if (p.batch <= 4) return step_t<T, 4>(p, st);
  return step_t<T, 8>(p, st);
}

int pow2_batch(int64_t b) { return b <= 1 ? 1 : b <= 2 ? 2 : b <= 4 ? 4 : 8; }

struct StepLayout {
  size_t xc = 0, zg = 0, xdb = 0, xpart = 0, yv = 0, total = 0;
  int nxwg = 0, xq = 0, xs = 0;
  bool fused = false;
};
StepLayout step_layout(const mcpu_mixer_step_args* a) {
  StepLayout w;
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t at = off;
    off += align_up(sizeof(float) * n);
    return at;
  };
  const int64_t J = a->dt_rank + 2 * a->dstate;
  const int rw = rows_per_wave(2 * a->d_inner);
  w.nxwg = static_cast<int>((a->d_inner + 4 * rw - 1) / (4 * rw));
  w.fused = partial_plan(w.nxwg, J, &w.xq, &w.xs);
  w.xc = take(a->batch * a->d_inner);
  w.zg = take(a->batch * a->d_inner);
  if (w.fused) w.xpart = take(a->batch * J * w.xq * w.xs);
  else w.xdb = take(a->batch * J);
  w.yv = take(a->batch * a->d_inner);
  w.total = off;
  return w;
}

int check_step(const mcpu_mixer_step_args* a) {
  if (a == nullptr) return fail(MCPU_ERR_INVALID, "mixer_step: null argument block");
  if (a->hidden == nullptr || a->in_w == nullptr || a->conv_w == nullptr || a->conv_state == nullptr ||
      a->x_w == nullptr || a->dt_w == nullptr || a->A == nullptr || a->ssm_state == nullptr ||
      a->out_w == nullptr || a->out == nullptr)
    return fail(MCPU_ERR_INVALID, "mixer_step: hidden, in_w, conv_w, conv_state, x_w, dt_w, A, ssm_state, "
                                  "out_w and out are required");
  if (a->batch < 1 || a->d_model < 4 || a->d_inner < 4 || a->dt_rank < 1 || a->dstate < 1 || a->width < 1)
    return fail(MCPU_ERR_INVALID, "mixer_step: bad sizes");
  if (a->batch > kMaxBatch)
    return fail(MCPU_ERR_UNSUPPORTED, "mixer_step: batch %lld > %d", (long long)a->batch, kMaxBatch);
  if (a->d_model % 4 != 0 || a->d_inner % 4 != 0)
    return fail(MCPU_ERR_UNSUPPORTED, "mixer_step: d_model and d_inner must be multiples of 4");
  if (a->dstate > 128) return fail(MCPU_ERR_UNSUPPORTED, "mixer_step: dstate %lld > 128", (long long)a->dstate);
  if (a->dt_rank + 2 * a->dstate > kMaxXdb)
    return fail(MCPU_ERR_UNSUPPORTED, "mixer_step: dt_rank + 2 dstate = %lld > %d",
                (long long)(a->dt_rank + 2 * a->dstate), kMaxXdb);
  if (a->state_len < a->width - 1 || a->state_len < 1 || a->state_len > kMaxConvState)
    return fail(MCPU_ERR_UNSUPPORTED, "mixer_step: conv state length must be in [max(1, width - 1), %d]",
                kMaxConvState);
  if (a->width > kMaxConvState)
    return fail(MCPU_ERR_UNSUPPORTED, "mixer_step: conv width %lld > %d", (long long)a->width, kMaxConvState);
  const int64_t mt = pow2_batch(a->batch);
  if ((mt + 1) * a->d_model > kMaxLdsFloats || mt * a->d_inner > kMaxLdsFloats)
    return fail(MCPU_ERR_UNSUPPORTED, "mixer_step: batch x width too large for one workgroup's LDS");
  if (!valid_dtype(a->dtype) || !valid_dtype(a->state_dtype) ||
      (a->hidden_dtype != a->dtype && a->hidden_dtype != MCPU_F32) ||
      (a->out_dtype != a->dtype && a->out_dtype != MCPU_F32))
    return fail(MCPU_ERR_INVALID, "mixer_step: bad dtype");
  if (a->norm_eps < 0.f) return fail(MCPU_ERR_INVALID, "mixer_step: norm_eps < 0");
  for (const void* t : {a->hidden, a->in_w, a->x_w, a->out_w, a->norm_weight, static_cast<const void*>(a->out)})
    if (reinterpret_cast<uintptr_t>(t) % 16 != 0)
      return fail(MCPU_ERR_INVALID, "mixer_step: hidden, weights and out must be 16-byte aligned");
  return MCPU_OK;
}

}  // namespace
}  // namespace mcpu

using namespace mcpu;

extern "C" size_t mcpu_mixer_step_workspace_size(const mcpu_mixer_step_args* a) {
  if (check_step(a) != MCPU_OK) {
    clear_error();
    return 0;
  }
  return step_layout(a).total;
}

extern "C" int mcpu_mixer_step(const mcpu_mixer_step_args* a, void* workspace, size_t workspace_bytes,
                               void* stream) {
  clear_error();
  if (int rc = check_step(a)) return rc;
  const StepLayout w = step_layout(a);
  if (workspace == nullptr || workspace_bytes < w.total)
    return fail(MCPU_ERR_INVALID, "mixer_step: workspace of %zu bytes needed, got %zu", w.total, workspace_bytes);
  if (int rc = mcpu_check_device()) return rc;
  MixerParams p;
  std::memset(&p, 0, sizeof(p));
  p.hidden = a->hidden;
  p.norm_w = a->norm_weight;
  p.in_w = a->in_w;
  p.in_b = a->in_b;
  p.conv_w = a->conv_w;
  p.conv_b = a->conv_b;
  p.conv_state = a->conv_state;
  p.x_w = a->x_w;
  p.dt_w = a->dt_w;
  p.dt_b = a->dt_b;
  p.A = a->A;
  p.D = a->D;
  p.ssm_state = a->ssm_state;
  p.out_w = a->out_w;
  p.out_b = a->out_b;
  p.out = a->out;
  char* ws = static_cast<char*>(workspace);
  p.xc = reinterpret_cast<float*>(ws + w.xc);
  p.zg = reinterpret_cast<float*>(ws + w.zg);
  if (w.fused) {
    p.xpart = reinterpret_cast<float*>(ws + w.xpart);
    p.nxwg = w.nxwg;
    p.xq = w.xq;
    p.xs = w.xs;
    p.xpp = w.xq * w.xs;
  } else {
    p.xdb = reinterpret_cast<float*>(ws + w.xdb);
  }
  p.yv = reinterpret_cast<float*>(ws + w.yv);
  p.batch = a->batch;
  p.dm = a->d_model;
  p.di = a->d_inner;
  p.nin = 2 * a->d_inner;
  p.conv_lo = 0;
  p.nconv = a->d_inner;
  p.zst = a->d_inner;
  p.R = a->dt_rank;
  p.N = a->dstate;
  p.W = a->width;
  p.S = a->state_len;
  p.eps = a->norm_eps;
  p.add_residual = a->add_residual != 0;
  p.hidden_dtype = a->hidden_dtype;
  p.state_dtype = a->state_dtype;
  p.out_dtype = a->out_dtype;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (a->dtype) {
    case MCPU_F32: e = step_dtype<float>(p, st); break;
    case MCPU_BF16: e = step_dtype<bf16>(p, st); break;
    default: e = step_dtype<f16>(p, st); break;
  }
  return hip_status(e, "mixer_step launch");
}

namespace mcpu {
namespace {

constexpr int kNormLinearRW = 2;
constexpr int64_t kNormLinearGrid = 1024;   // 4 workgroups per CU on 256 CUs

template <typename T, int MT, int KC>
void launch_norm_linear(const NormLinearParams& p, bool hf, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>(p.ngroups < kNormLinearGrid ? p.ngroups : kNormLinearGrid));
  const size_t lds = sizeof(float) * (MT + 1) * p.K;
  if (hf || std::is_same_v<T, float>)
    hipLaunchKernelGGL((norm_linear_kernel<T, MT, kNormLinearRW, KC, true>), grid, dim3(kThreads), lds, st, p);
  else
    hipLaunchKernelGGL((norm_linear_kernel<T, MT, kNormLinearRW, KC, false>), grid, dim3(kThreads), lds, st, p);
}

template <typename T, int MT>
void norm_linear_mt(const NormLinearParams& p, bool hf, hipStream_t st) {
  if (p.K <= 256 * 4) launch_norm_linear<T, MT, 4>(p, hf, st);
  else launch_norm_linear<T, MT, kChunks>(p, hf, st);
}

template <typename T>
void norm_linear_t(const NormLinearParams& p, bool hf, hipStream_t st) {
  if (p.batch <= 1) norm_linear_mt<T, 1>(p, hf, st);
  else if (p.batch <= 2) norm_linear_mt<T, 2>(p, hf, st);
  else if (p.batch <= 4) norm_linear_mt<T, 4>(p, hf, st);
  else norm_linear_mt<T, 8>(p, hf, st);
}

int check_norm_linear(const mcpu_norm_linear_args* a) {
  if (a == nullptr) return fail(MCPU_ERR_INVALID, "norm_linear: null argument block");
  if (a->hidden == nullptr || a->weight == nullptr || a->out == nullptr)
    return fail(MCPU_ERR_INVALID, "norm_linear: hidden, weight and out are required");
  if (a->batch < 1 || a->d_in < 4 || a->d_out < 1) return fail(MCPU_ERR_INVALID, "norm_linear: bad sizes");
  if (a->batch > kMaxBatch)
    return fail(MCPU_ERR_UNSUPPORTED, "norm_linear: batch %lld > %d", (long long)a->batch, kMaxBatch);
  if (a->d_in % 4 != 0) return fail(MCPU_ERR_UNSUPPORTED, "norm_linear: d_in must be a multiple of 4");
  if ((pow2_batch(a->batch) + 1) * a->d_in > kMaxLdsFloats)
    return fail(MCPU_ERR_UNSUPPORTED, "norm_linear: batch x d_in too large for one workgroup's LDS");
  if (!valid_dtype(a->dtype) || (a->hidden_dtype != a->dtype && a->hidden_dtype != MCPU_F32) ||
      (a->out_dtype != a->dtype && a->out_dtype != MCPU_F32))
    return fail(MCPU_ERR_INVALID, "norm_linear: bad dtype");
  if (a->norm_eps < 0.f) return fail(MCPU_ERR_INVALID, "norm_linear: norm_eps < 0");
  for (const void* t : {a->hidden, a->weight, a->norm_weight})
    if (reinterpret_cast<uintptr_t>(t) % 16 != 0)
      return fail(MCPU_ERR_INVALID, "norm_linear: hidden, weight and norm_weight must be 16-byte aligned");
  return MCPU_OK;
}

}  // namespace
}  // namespace mcpu

extern "C" int mcpu_norm_linear(const mcpu_norm_linear_args* a, void* stream) {
  clear_error();
  if (int rc = check_norm_linear(a)) return rc;
  if (int rc = mcpu_check_device()) return rc;
  NormLinearParams p;
  std::memset(&p, 0, sizeof(p));
  p.x = a->hidden;
  p.nw = a->norm_weight;
  p.w = a->weight;
  p.bias = a->bias;
  p.out = a->out;
  p.batch = a->batch;
  p.nout = a->d_out;
  p.ngroups = (a->d_out + 4 * kNormLinearRW - 1) / (4 * kNormLinearRW);
  p.K = static_cast<int>(a->d_in);
  p.out_f32 = a->out_dtype == MCPU_F32;
  p.eps = a->norm_eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool hf = a->hidden_dtype == MCPU_F32;
  switch (a->dtype) {
    case MCPU_F32: norm_linear_t<float>(p, hf, st); break;
    case MCPU_BF16: norm_linear_t<bf16>(p, hf, st); break;
    default: norm_linear_t<f16>(p, hf, st); break;
  }
  return hip_status(hipGetLastError(), "norm_linear launch");
}

// ---- Mamba-2 block step --------------------------------------------------------

namespace mcpu {
namespace {

struct Step2Layout {
  size_t xc = 0, zg = 0, yv = 0, total = 0;
  int64_t conv_dim = 0, nin = 0, zst = 0;
};

Step2Layout step2_layout(const mcpu_mamba2_step_args* a) {
  Step2Layout w;
  w.conv_dim = a->d_inner + 2 * a->ngroups * a->dstate;
  w.nin = a->d_inner + w.conv_dim + a->nheads;
  w.zst = (a->d_inner + a->nheads + 3) / 4 * 4;
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t at = off;
    off += align_up(sizeof(float) * n);
    return at;
  };
  w.xc = take(a->batch * w.conv_dim);
  w.zg = take(a->batch * w.zst);
  w.yv = take(a->batch * a->d_inner);
  w.total = off;
  return w;
}

int check_step2(const mcpu_mamba2_step_args* a) {
  if (a == nullptr) return fail(MCPU_ERR_INVALID, "mamba2_step: null argument block");
  if (a->hidden == nullptr || a->in_w == nullptr || a->conv_w == nullptr || a->conv_state == nullptr ||
      a->A == nullptr || a->ssm_state == nullptr || a->gate_norm_weight == nullptr || a->out_w == nullptr ||
      a->out == nullptr)
    return fail(MCPU_ERR_INVALID, "mamba2_step: hidden, in_w, conv_w, conv_state, A, ssm_state, "
                                  "gate_norm_weight, out_w and out are required");
  if (a->batch < 1 || a->d_model < 4 || a->nheads < 1 || a->headdim < 1 || a->ngroups < 1 || a->dstate < 1 ||
      a->width < 1 || a->d_inner != a->nheads * a->headdim || a->nheads % a->ngroups != 0)
    return fail(MCPU_ERR_INVALID, "mamba2_step: bad sizes (d_inner must be nheads x headdim, nheads a "
                                  "multiple of ngroups)");
  if (a->batch > kMaxBatch)
    return fail(MCPU_ERR_UNSUPPORTED, "mamba2_step: batch %lld > %d", (long long)a->batch, kMaxBatch);
  if (a->d_model % 4 != 0 || a->d_inner % 4 != 0)
    return fail(MCPU_ERR_UNSUPPORTED, "mamba2_step: d_model and d_inner must be multiples of 4");
  if (a->dstate > 128) return fail(MCPU_ERR_UNSUPPORTED, "mamba2_step: dstate %lld > 128", (long long)a->dstate);
  if (a->state_len < a->width - 1 || a->state_len < 1 || a->state_len > kMaxConvState || a->width > kMaxConvState)
    return fail(MCPU_ERR_UNSUPPORTED, "mamba2_step: conv width and state length must be at most %d, "
                                      "state length at least max(1, width - 1)", kMaxConvState);
  const int64_t mt = pow2_batch(a->batch);
  if ((mt + 1) * a->d_model > kMaxLdsFloats || (mt + 1) * a->d_inner > kMaxLdsFloats)
    return fail(MCPU_ERR_UNSUPPORTED, "mamba2_step: batch x width too large for one workgroup's LDS");
  if (!valid_dtype(a->dtype) || !valid_dtype(a->state_dtype) ||
      (a->hidden_dtype != a->dtype && a->hidden_dtype != MCPU_F32) ||
      (a->out_dtype != a->dtype && a->out_dtype != MCPU_F32))
    return fail(MCPU_ERR_INVALID, "mamba2_step: bad dtype");
  if (a->norm_eps < 0.f || a->gate_norm_eps < 0.f) return fail(MCPU_ERR_INVALID, "mamba2_step: eps < 0");
  for (const void* t : {a->hidden, a->in_w, a->out_w, a->norm_weight, a->gate_norm_weight,
                        static_cast<const void*>(a->out)})
    if (reinterpret_cast<uintptr_t>(t) % 16 != 0)
      return fail(MCPU_ERR_INVALID, "mamba2_step: hidden, weights and out must be 16-byte aligned");
  return MCPU_OK;
}

template <typename T, typename Ts>
void launch_m2_ssm(const MixerParams& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((p.nh * p.hd + 15) / 16), static_cast<unsigned>(p.batch));
  if (p.N <= 16) hipLaunchKernelGGL((m2_ssm_kernel<T, Ts, 1>), grid, dim3(256), 0, st, p);
  else if (p.N <= 32) hipLaunchKernelGGL((m2_ssm_kernel<T, Ts, 2>), grid, dim3(256), 0, st, p);
  else if (p.N <= 64) hipLaunchKernelGGL((m2_ssm_kernel<T, Ts, 4>), grid, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((m2_ssm_kernel<T, Ts, 8>), grid, dim3(256), 0, st, p);
}

template <typename T, int MT, int RW>
void launch_m2_out(const MixerParams& p, bool hf, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((p.dm + 4 * RW - 1) / (4 * RW)));
  const size_t lds = sizeof(float) * (MT + 1) * p.di;
  if (hf || std::is_same_v<T, float>)
    hipLaunchKernelGGL((m2_out_kernel<T, MT, RW, true>), grid, dim3(kThreads), lds, st, p);
  else
    hipLaunchKernelGGL((m2_out_kernel<T, MT, RW, false>), grid, dim3(kThreads), lds, st, p);
}

template <typename T, int MT>
hipError_t step2_t(const MixerParams& p, hipStream_t st) {
  const bool hf = p.hidden_dtype == MCPU_F32;
  const int rw = rows_per_wave(p.nin);
  hipError_t e = rw == 4 ? launch_in<T, MT, 4>(p, hf, st) : rw == 2 ? launch_in<T, MT, 2>(p, hf, st)
                                                                    : launch_in<T, MT, 1>(p, hf, st);
  if (e != hipSuccess) return e;
  switch (p.state_dtype) {
    case MCPU_F32: launch_m2_ssm<T, float>(p, st); break;
    case MCPU_BF16: launch_m2_ssm<T, bf16>(p, st); break;
    default: launch_m2_ssm<T, f16>(p, st); break;
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int ro = rows_per_wave(p.dm);
  if (ro == 4) launch_m2_out<T, MT, 4>(p, hf, st);
  else if (ro == 2) launch_m2_out<T, MT, 2>(p, hf, st);
  else launch_m2_out<T, MT, 1>(p, hf, st);
  return hipGetLastError();
}

template <typename T>
hipError_t step2_dtype(const MixerParams& p, hipStream_t st) {
  if (p.batch <= 1) return step2_t<T, 1>(p, st);
  if (p.batch <= 2) return step2_t<T, 2>(p, st);
  if (p.batch <= 4) return step2_t<T, 4>(p, st);
  return step2_t<T, 8>(p, st);
}

}  // namespace
}  // namespace mcpu

extern "C" size_t mcpu_mamba2_step_workspace_size(const mcpu_mamba2_step_args* a) {
  if (check_step2(a) != MCPU_OK) {
    clear_error();
    return 0;
  }
  return step2_layout(a).total;
}

extern "C" int mcpu_mamba2_step(const mcpu_mamba2_step_args* a, void* workspace, size_t workspace_bytes,
                                void* stream) {
  clear_error();
  if (int rc = check_step2(a)) return rc;
  const Step2Layout w = step2_layout(a);
  if (workspace == nullptr || workspace_bytes < w.total)
    return fail(MCPU_ERR_INVALID, "mamba2_step: workspace of %zu bytes needed, got %zu", w.total, workspace_bytes);
  if (int rc = mcpu_check_device()) return rc;
  MixerParams p;
  std::memset(&p, 0, sizeof(p));
  p.hidden = a->hidden;
  p.norm_w = a->norm_weight;
  p.in_w = a->in_w;
  p.in_b = a->in_b;
  p.conv_w = a->conv_w;
  p.conv_b = a->conv_b;
  p.conv_state = a->conv_state;
  p.dt_b = a->dt_bias;
  p.A = a->A;
  p.D = a->D;
  p.ssm_state = a->ssm_state;
  p.gn_w = a->gate_norm_weight;
  p.gn_eps = a->gate_norm_eps;
  p.out_w = a->out_w;
  p.out_b = a->out_b;
  p.out = a->out;
  char* ws = static_cast<char*>(workspace);
  p.xc = reinterpret_cast<float*>(ws + w.xc);
  p.zg = reinterpret_cast<float*>(ws + w.zg);
  p.yv = reinterpret_cast<float*>(ws + w.yv);
  p.batch = a->batch;
  p.dm = a->d_model;
  p.di = a->d_inner;
  p.N = a->dstate;
  p.W = a->width;
  p.S = a->state_len;
  p.nin = w.nin;
  p.conv_lo = a->d_inner;
  p.nconv = w.conv_dim;
  p.zst = w.zst;
  p.nh = a->nheads;
  p.hd = a->headdim;
  p.ng = a->ngroups;
  p.eps = a->norm_eps;
  p.add_residual = a->add_residual != 0;
  p.hidden_dtype = a->hidden_dtype;
  p.state_dtype = a->state_dtype;
  p.out_dtype = a->out_dtype;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (a->dtype) {
    case MCPU_F32: e = step2_dtype<float>(p, st); break;
    case MCPU_BF16: e = step2_dtype<bf16>(p, st); break;
    default: e = step2_dtype<f16>(p, st); break;
  }
  return hip_status(e, "mamba2_step launch");
}
