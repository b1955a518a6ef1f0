// One decode step of a Mamba-1 block for a batch of single tokens (batch <=
// 8), in four launches:
//   1. block_in_kernel: RMSNorm of the hidden rows (every workgroup, into
//      LDS), the in_proj rows of this workgroup (one wave per row, the batch
//      rows at once), and for the x half the depthwise conv update of that
//      channel (conv state shifted in place) with silu;
//   2. gemv_kernel: x_proj over the conv outputs (dt, B, C);
//   3. block_ssm_kernel: dt_proj row, softplus, the selective state update
//      (state in place), D skip and the silu(z) gate;
//   4. gemv_kernel: out_proj, plus the residual.
// The in_proj, x_proj and out_proj products are matrix-vector products over
// a handful of rows: they read each weight once, four elements per lane
// (coalesced rows), against the batch rows held in LDS, and reduce across
// the wave with DPP and permlane swaps. Intermediate vectors live in a small
// float32 workspace holding values already rounded to the storage type, as
// transformers' separate ops would have stored them.
#include <cstring>

#include "abi_util.h"
#include "mcpu_common.h"

namespace mcpu {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxBatch = 8;
constexpr int kMaxLdsFloats = 32768;
constexpr int kMaxConvState = 8;

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
  float* xc;    // (batch, d_inner): silu(conv) of the x half
  float* zg;    // (batch, d_inner): the z half
  float* xdb;   // (batch, dt_rank + 2 dstate): x_proj
  float* yv;    // (batch, d_inner): gated scan output
  int64_t batch, dm, di, R, N, W, S;
  float eps;
  int add_residual, hidden_dtype, state_dtype, out_dtype;
};

// v rounded to the storage type T (exact in float32).
template <typename T> __device__ __forceinline__ float rnd(float v) { return to_f32(from_f32<T>(v)); }

template <typename T> __device__ __forceinline__ float4 ld4t(const void* base, int64_t i);
template <> __device__ __forceinline__ float4 ld4t<float>(const void* base, int64_t i) {
  return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
}
template <> __device__ __forceinline__ float4 ld4t<bf16>(const void* base, int64_t i) {
  const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + i);
  return make_float4(__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xffff0000u),
                     __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xffff0000u));
}
template <> __device__ __forceinline__ float4 ld4t<f16>(const void* base, int64_t i) {
  const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + i);
  auto h = [](uint32_t bits) { return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(bits))); };
  return make_float4(h(u.x & 0xffff), h(u.x >> 16), h(u.y & 0xffff), h(u.y >> 16));
}

// Element i of a tensor of storage type dt (float32, bf16 or f16) as float.
__device__ __forceinline__ float ld_any(const void* base, int64_t i, int dt) {
  if (dt == MCPU_F32) return static_cast<const float*>(base)[i];
  if (dt == MCPU_BF16) return ld<bf16>(base, i);
  return ld<f16>(base, i);
}
__device__ __forceinline__ void st_any(void* base, int64_t i, float v, int dt) {
  if (dt == MCPU_F32) static_cast<float*>(base)[i] = v;
  else if (dt == MCPU_BF16) st<bf16>(base, i, v);
  else st<f16>(base, i, v);
}

// Sum over the 64 lanes of a wave, in a fixed order, in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  v = row_allreduce16(v);
  v = swap_sum<32>(v, v);
  return swap_sum<16>(v, v);
}

// float4 chunks (256 elements of a row per wave) each lane loads per pass.
constexpr int kChunks = 8;

// This wave's weight rows row0 .. row0 + RW - 1 (rows from nrows on, and
// columns past K, read as 0), chunk u of pass k0 at k = k0 + 4 lane + 256 u.
template <typename T, int RW>
struct RowTiles {
  float4 w[RW][kChunks];

  __device__ __forceinline__ void load(const void* wt, int64_t row0, int nrows, int K, int k0) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int rr = 0; rr < RW; ++rr)
#pragma unroll
      for (int u = 0; u < kChunks; ++u) {
        const int k = k0 + 4 * lane + 256 * u;
        w[rr][u] = (rr < nrows && k < K) ? ld4t<T>(wt, (row0 + rr) * K + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
  }

  // acc[r][m] += sum over this pass's k of X[m][k] W[r][k]; X (MT, K) in LDS.
  template <int MT>
  __device__ __forceinline__ void fma(float (&acc)[RW][MT], const float* sx, int K, int k0) const {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < kChunks; ++u) {
      const int k = k0 + 4 * lane + 256 * u;
      if (k >= K) break;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float4 xv = *reinterpret_cast<const float4*>(sx + m * K + k);
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) {
          float a = acc[rr][m];
          a = fmaf(w[rr][u].x, xv.x, a);
          a = fmaf(w[rr][u].y, xv.y, a);
          a = fmaf(w[rr][u].z, xv.z, a);
          a = fmaf(w[rr][u].w, xv.w, a);
          acc[rr][m] = a;
        }
      }
    }
  }
};

// acc[r][m] = sum_k X[m][k] W[row0 + r][k], summed over the wave: every lane
// ends with every row's sums. `tiles` holds the first pass's weights,
// loaded before X was staged (so their latency overlapped the staging);
// further passes (K > 2048) load and multiply in turn.
template <typename T, int MT, int RW>
__device__ __forceinline__ void rows_dot(float (&acc)[RW][MT], RowTiles<T, RW>& tiles, const float* sx,
                                         const void* w, int64_t row0, int nrows, int K) {
#pragma unroll
  for (int rr = 0; rr < RW; ++rr)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[rr][m] = 0.f;
  tiles.template fma<MT>(acc, sx, K, 0);
  for (int k0 = 256 * kChunks; k0 < K; k0 += 256 * kChunks) {
    tiles.load(w, row0, nrows, K, k0);
    tiles.template fma<MT>(acc, sx, K, k0);
  }
#pragma unroll
  for (int rr = 0; rr < RW; ++rr)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[rr][m] = wave_sum(acc[rr][m]);
}

// LDS rows sx[m][k] (m < MT; rows past batch are 0) = float32 vectors of
// length K from a float32 workspace.
template <int MT>
__device__ __forceinline__ void load_rows(float* sx, const float* src, int64_t batch, int K) {
  for (int i = 4 * threadIdx.x; i < MT * K; i += 4 * kThreads) {
    const int m = i / K;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (m < batch) v = *reinterpret_cast<const float4*>(src + i);
    *reinterpret_cast<float4*>(sx + i) = v;
  }
}

}  // namespace

// 1. RMSNorm (optional) + in_proj + conv update. Grid: ceil(2 d_inner / (4 RW))
// workgroups; wave w handles in_proj rows (4 blockIdx.x + w) RW + rr.
template <typename T, int MT, int RW>
__global__ void __launch_bounds__(kThreads) block_in_kernel(const MixerParams p) {
  extern __shared__ __align__(16) float s_u[];   // (MT, d_model) rows, then the norm weight
  __shared__ float s_red[MT][kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = static_cast<int>(p.dm);
  float* s_nw = s_u + MT * K;
  const int64_t nout = 2 * p.di;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + wave) * RW;
  const int nrows = row0 >= nout ? 0 : static_cast<int>(nout - row0 < RW ? nout - row0 : RW);
  // Everything this wave reads from memory is requested up front: its
  // in_proj rows, then what its epilogue needs (lane m < batch: the bias and,
  // for x rows, batch row m's conv window, weights and bias).
  RowTiles<T, RW> tiles;
  tiles.load(p.in_w, row0, nrows, K, 0);
  const T* tb = static_cast<const T*>(p.in_b);
  float eb[RW], ecb[RW], est[RW][kMaxConvState], ecw[RW][kMaxConvState];
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int64_t n = row0 + rr;
    const bool mine = rr < nrows && lane < p.batch;
    const bool xrow = mine && n < p.di;
    eb[rr] = (mine && tb) ? to_f32(tb[n]) : 0.f;
    ecb[rr] = (xrow && p.conv_b) ? to_f32(static_cast<const T*>(p.conv_b)[n]) : 0.f;
    const T* stt = static_cast<const T*>(p.conv_state) + (lane * p.di + n) * p.S;
    const T* cw = static_cast<const T*>(p.conv_w) + n * p.W;
#pragma unroll
    for (int i = 0; i < kMaxConvState; ++i) {
      est[rr][i] = (xrow && i < p.S) ? to_f32(stt[i]) : 0.f;
      ecw[rr][i] = (xrow && i < p.W) ? to_f32(cw[i]) : 0.f;
    }
  }
  // The block's input rows, rounded to T as transformers casts them for the
  // norm, four elements per thread-step, loads first; the norm weight beside them.
  constexpr int kStage = 4;
  float ss[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) ss[m] = 0.f;
  for (int base = 4 * tid; base < MT * K; base += 4 * kThreads * kStage) {
    float4 hv[kStage];
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int i = base + 4 * kThreads * u;
      hv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < MT * K && i / K < p.batch)
        hv[u] = p.hidden_dtype == MCPU_F32 ? ld4t<float>(p.hidden, i) : ld4t<T>(p.hidden, i);
    }
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int i = base + 4 * kThreads * u;
      if (i >= MT * K) break;
      const int m = i / K;
      const float4 v = make_float4(rnd<T>(hv[u].x), rnd<T>(hv[u].y), rnd<T>(hv[u].z), rnd<T>(hv[u].w));
#pragma unroll
      for (int mm = 0; mm < MT; ++mm)
        if (mm == m) ss[mm] += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
      *reinterpret_cast<float4*>(s_u + i) = v;
    }
  }
  if (p.norm_w) {
    for (int i = 4 * tid; i < K; i += 4 * kThreads)
      *reinterpret_cast<float4*>(s_nw + i) = ld4t<T>(p.norm_w, i);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const float t = wave_sum(ss[m]);
      if (lane == 0) s_red[m][wave] = t;
    }
  }
  __syncthreads();
  if (p.norm_w) {
    // u = w * round_T(x * rsqrt(mean(x^2) + eps)), rounded to T.
    for (int i = 4 * tid; i < MT * K; i += 4 * kThreads) {
      const int m = i / K;
      float tot = 0.f;
#pragma unroll
      for (int mm = 0; mm < MT; ++mm)
        if (mm == m) tot = (s_red[mm][0] + s_red[mm][1]) + (s_red[mm][2] + s_red[mm][3]);
      const float rs = rsqrtf(tot / static_cast<float>(K) + p.eps);
      float4 v = *reinterpret_cast<const float4*>(s_u + i);
      const float4 w = *reinterpret_cast<const float4*>(s_nw + (i - m * K));
      v = make_float4(rnd<T>(w.x * rnd<T>(v.x * rs)), rnd<T>(w.y * rnd<T>(v.y * rs)),
                      rnd<T>(w.z * rnd<T>(v.z * rs)), rnd<T>(w.w * rnd<T>(v.w * rs)));
      *reinterpret_cast<float4*>(s_u + i) = v;
    }
    __syncthreads();
  }
  if (nrows == 0) return;
  float acc[RW][MT];
  rows_dot<T, MT, RW>(acc, tiles, s_u, p.in_w, row0, nrows, K);
  // Lane m finishes batch row m of each of the wave's rows.
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int64_t n = row0 + rr;
    if (rr >= nrows) continue;
    float y = 0.f;
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (lane == m) y = acc[rr][m];
    if (lane >= p.batch) continue;
    const int64_t m = lane;
    y = rnd<T>(y + eb[rr]);
    if (n >= p.di) {
      p.zg[m * p.di + (n - p.di)] = y;
      continue;
    }
    // Depthwise conv update of channel n: taps 0 .. W-2 read the newest W-1
    // state entries, tap W-1 reads y; the state shifts left by one and y
    // becomes its newest entry.
    float c = ecb[rr];
    for (int k = 0; k < p.W - 1; ++k) {
      float v = 0.f, wk = 0.f;
#pragma unroll
      for (int i = 0; i < kMaxConvState; ++i) {
        if (i == p.S - (p.W - 1) + k) v = est[rr][i];
        if (i == k) wk = ecw[rr][i];
      }
      c = fmaf(wk, v, c);
    }
    float wl = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxConvState; ++i)
      if (i == p.W - 1) wl = ecw[rr][i];
    c = fmaf(wl, y, c);
    c = c * sigmoid(c);
    T* stt = static_cast<T*>(p.conv_state) + (m * p.di + n) * p.S;
#pragma unroll
    for (int i = 0; i < kMaxConvState - 1; ++i)
      if (i < p.S - 1) stt[i] = from_f32<T>(est[rr][i + 1]);
    stt[p.S - 1] = from_f32<T>(y);
    p.xc[m * p.di + n] = rnd<T>(c);
  }
}

// 2 / 4. Rows n of y[m][n] = round_T(sum_k x[m][k] W[n][k] + bias[n]) for
// x (batch, K) float32 from the workspace: into outf (batch, nout) float32
// when given, else out (out_dtype) = residual + y when add_residual, else y.
template <typename T, int MT, int RW>
__global__ void __launch_bounds__(kThreads) gemv_kernel(const MixerParams p, const float* x, const void* w,
                                                        const void* bias, int64_t nout, int K, float* outf) {
  extern __shared__ __align__(16) float s_x[];   // (MT, K)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + wave) * RW;
  const int nrows = row0 >= nout ? 0 : static_cast<int>(nout - row0 < RW ? nout - row0 : RW);
  RowTiles<T, RW> tiles;
  tiles.load(w, row0, nrows, K, 0);
  // the epilogue's bias and residual, requested with the weights
  float eb[RW], er[RW];
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int64_t n = row0 + rr;
    const bool mine = rr < nrows && lane < p.batch;
    eb[rr] = (mine && bias) ? to_f32(static_cast<const T*>(bias)[n]) : 0.f;
    er[rr] = (mine && !outf && p.add_residual) ? ld_any(p.hidden, lane * nout + n, p.hidden_dtype) : 0.f;
  }
  load_rows<MT>(s_x, x, p.batch, K);
  __syncthreads();
  if (nrows == 0) return;
  float acc[RW][MT];
  rows_dot<T, MT, RW>(acc, tiles, s_x, w, row0, nrows, K);
#pragma unroll
  for (int rr = 0; rr < RW; ++rr) {
    const int64_t n = row0 + rr;
    if (rr >= nrows) continue;
    float y = 0.f;
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (lane == m) y = acc[rr][m];
    if (lane >= p.batch) continue;
    const int64_t m = lane;
    y = rnd<T>(y + eb[rr]);
    if (outf) {
      outf[m * nout + n] = y;
    } else {
      if (p.add_residual) y = er[rr] + y;
      st_any(p.out, m * nout + n, y, p.out_dtype);
    }
  }
}

// 3. dt_proj + softplus + selective state update + D skip + silu(z) gate.
// 16 lanes per channel (state n = lane + 16 s), 16 channels per workgroup;
// grid (ceil(d_inner / 16), batch). The arithmetic of each channel is the
// selective state update kernel's.
template <typename T, typename Ts, int SPL>
__global__ void __launch_bounds__(kThreads) block_ssm_kernel(const MixerParams p) {
  const int j = threadIdx.x & 15;
  const int64_t d = blockIdx.x * 16ll + (threadIdx.x >> 4);
  const int64_t m = blockIdx.y;
  if (d >= p.di) return;  // whole 16-lane rows leave together
  const int64_t R = p.R, N = p.N;
  const float* xdb = p.xdb + m * (R + 2 * N);
  const T* dtw = static_cast<const T*>(p.dt_w) + d * R;
  Ts* state = static_cast<Ts*>(p.ssm_state) + (m * p.di + d) * N;
  // Every load of the channel first: none of them waits on another.
  float sv0[SPL], av[SPL], bv[SPL], cv[SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s) {
    const int64_t n = j + 16 * s;
    const bool ok = n < N;
    sv0[s] = ok ? to_f32(state[n]) : 0.f;
    av[s] = ok ? p.A[d * N + n] : 0.f;
    bv[s] = ok ? xdb[R + n] : 0.f;
    cv[s] = ok ? xdb[R + N + n] : 0.f;
  }
  const float x = p.xc[m * p.di + d], zz = p.zg[m * p.di + d];
  const float Dd = p.D ? p.D[d] : 0.f, bias = p.dt_b ? p.dt_b[d] : 0.f;
  float part = 0.f;
  for (int64_t r = j; r < R; r += 16) part = fmaf(xdb[r], to_f32(dtw[r]), part);
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
      const float sv = fmaf(sv0[s], a, dtx * bv[s]);
      state[n] = from_f32<Ts>(sv);
      acc = fmaf(sv, cv[s], acc);
    }
  }
  float y = row_allreduce16(acc);
  if (j == 0) {
    if (p.D) y = fmaf(x, Dd, y);
    y *= zz * sigmoid(zz);
    p.yv[m * p.di + d] = rnd<T>(y);
  }
}

namespace {

// Rows per wave: as many as keep at least 256 workgroups.
int rows_per_wave(int64_t nout) {
  for (int rw = 4; rw > 1; rw /= 2)
    if ((nout + 4 * rw - 1) / (4 * rw) >= 256) return rw;
  return 1;
}

template <typename T, int MT, int RW>
hipError_t launch_rw(const MixerParams& p, hipStream_t st) {
  const int64_t nin = 2 * p.di;
  hipLaunchKernelGGL((block_in_kernel<T, MT, RW>), dim3(static_cast<unsigned>((nin + 4 * RW - 1) / (4 * RW))),
                     dim3(kThreads), sizeof(float) * (MT + 1) * p.dm, st, p);
  return hipGetLastError();
}

template <typename T, int MT>
hipError_t gemv(const MixerParams& p, const float* x, const void* w, const void* bias, int64_t nout, int64_t K,
                float* outf, hipStream_t st) {
  const int rw = rows_per_wave(nout);
  const size_t lds = sizeof(float) * MT * K;
  auto grid = [&](int r) { return dim3(static_cast<unsigned>((nout + 4 * r - 1) / (4 * r))); };
  if (rw == 4)
    hipLaunchKernelGGL((gemv_kernel<T, MT, 4>), grid(4), dim3(kThreads), lds, st, p, x, w, bias, nout,
                       static_cast<int>(K), outf);
  else if (rw == 2)
    hipLaunchKernelGGL((gemv_kernel<T, MT, 2>), grid(2), dim3(kThreads), lds, st, p, x, w, bias, nout,
                       static_cast<int>(K), outf);
  else
    hipLaunchKernelGGL((gemv_kernel<T, MT, 1>), grid(1), dim3(kThreads), lds, st, p, x, w, bias, nout,
                       static_cast<int>(K), outf);
  return hipGetLastError();
}

template <typename T, typename Ts>
hipError_t launch_ssm(const MixerParams& p, hipStream_t st) {
  const dim3 grid(static_cast<unsigned>((p.di + 15) / 16), static_cast<unsigned>(p.batch));
  if (p.N <= 16) hipLaunchKernelGGL((block_ssm_kernel<T, Ts, 1>), grid, dim3(kThreads), 0, st, p);
  else if (p.N <= 32) hipLaunchKernelGGL((block_ssm_kernel<T, Ts, 2>), grid, dim3(kThreads), 0, st, p);
  else if (p.N <= 64) hipLaunchKernelGGL((block_ssm_kernel<T, Ts, 4>), grid, dim3(kThreads), 0, st, p);
  else hipLaunchKernelGGL((block_ssm_kernel<T, Ts, 8>), grid, dim3(kThreads), 0, st, p);
  return hipGetLastError();
}

template <typename T, int MT>
hipError_t step_t(const MixerParams& p, hipStream_t st) {
  const int rw = rows_per_wave(2 * p.di);
  hipError_t e = rw == 4 ? launch_rw<T, MT, 4>(p, st) : rw == 2 ? launch_rw<T, MT, 2>(p, st)
                                                                : launch_rw<T, MT, 1>(p, st);
  if (e != hipSuccess) return e;
  if ((e = gemv<T, MT>(p, p.xc, p.x_w, nullptr, p.R + 2 * p.N, p.di, p.xdb, st)) != hipSuccess) return e;
  switch (p.state_dtype) {
    case MCPU_F32: e = launch_ssm<T, float>(p, st); break;
    case MCPU_BF16: e = launch_ssm<T, bf16>(p, st); break;
    default: e = launch_ssm<T, f16>(p, st); break;
  }
  if (e != hipSuccess) return e;
  return gemv<T, MT>(p, p.yv, p.out_w, p.out_b, p.dm, p.di, nullptr, st);
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
  size_t xc = 0, zg = 0, xdb = 0, yv = 0, total = 0;
};
StepLayout step_layout(const mcpu_mixer_step_args* a) {
  StepLayout w;
  size_t off = 0;
  auto take = [&](size_t n) {
    const size_t at = off;
    off += align_up(sizeof(float) * n);
    return at;
  };
  w.xc = take(a->batch * a->d_inner);
  w.zg = take(a->batch * a->d_inner);
  w.xdb = take(a->batch * (a->dt_rank + 2 * a->dstate));
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
  p.xdb = reinterpret_cast<float*>(ws + w.xdb);
  p.yv = reinterpret_cast<float*>(ws + w.yv);
  p.batch = a->batch;
  p.dm = a->d_model;
  p.di = a->d_inner;
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
