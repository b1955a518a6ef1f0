// Shared device helpers for the gfx950 Mamba-1 kernels: storage-type loads and
// stores, wave64 lane exchange (DPP, permlane swaps) and scalar math.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>
#include <utility>

#include "mamba_hip.h"

namespace mcpu {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- storage types -----------------------------------------------------------

struct bf16 { uint16_t bits; };
using f16 = _Float16;

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(x.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16 x) { return static_cast<float>(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float x) { return static_cast<f16>(x); }
// Round to nearest even; NaN stays a (quiet) NaN.
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return bf16{static_cast<uint16_t>((u >> 16) | 0x40)};
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16{static_cast<uint16_t>(u >> 16)};
}

template <typename T> __device__ __forceinline__ float ld(const void* base, int64_t idx) {
  return to_f32(static_cast<const T*>(base)[idx]);
}
template <typename T> __device__ __forceinline__ void st(void* base, int64_t idx, float v) {
  static_cast<T*>(base)[idx] = from_f32<T>(v);
}

// ---- buffer loads ---------------------------------------------------------------
// Loads through a raw buffer descriptor built from a wave-uniform base pointer
// (scalar registers) and a 32-bit per-lane byte offset: the address
// arithmetic stays in the scalar unit instead of a 64-bit add per lane. The
// descriptor spans 4 GiB (no range check is relied on); 0x00020000 is the
// gfx9 raw-buffer format word.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wave_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, -1, 0x00020000);
}
template <typename T> __device__ __forceinline__ float buf_ld(__amdgpu_buffer_rsrc_t r, uint32_t off);
template <> __device__ __forceinline__ float buf_ld<float>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
template <> __device__ __forceinline__ float buf_ld<bf16>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return to_f32(bf16{static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0))});
}
template <> __device__ __forceinline__ float buf_ld<f16>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return to_f32(__builtin_bit_cast(f16, static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0))));
}

template <typename T> __device__ __forceinline__ void buf_st(__amdgpu_buffer_rsrc_t r, uint32_t off, float v);
template <> __device__ __forceinline__ void buf_st<float>(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, 0);
}
template <> __device__ __forceinline__ void buf_st<bf16>(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b16(from_f32<bf16>(v).bits, r, off, 0, 0);
}
template <> __device__ __forceinline__ void buf_st<f16>(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<f16>(v)), r, off, 0, 0);
}

// ---- scalar math ----------------------------------------------------------------

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float sigmoid(float x) { return fast_rcp(1.0f + fast_exp(-x)); }

// softplus with threshold 20 (the torch default): x > 20 ? x : log1p(exp(x)),
// without branches. NaN propagates. log1p(e) uses the u = 1 + e correction
// log(u) * e / (u - 1), accurate to a few ulp also where e is tiny.
// Also returns sigmoid(x) = e / (1 + e) from the same exponential.
__device__ __forceinline__ float softplus_sigmoid(float x, float& sg) {
  const bool big = !(x <= 20.f);  // also true for NaN
  const float e = fast_exp(big ? 20.f : x);
  const float u = 1.0f + e;
  const float d = u - 1.0f;
  const float l = __builtin_amdgcn_logf(u) * kLn2;  // natural log of u
  const float sp = d == 0.0f ? e : l * e * fast_rcp(d);
  sg = big ? (x == x ? 1.0f : x) : e * fast_rcp(u);
  return big ? x : sp;
}
__device__ __forceinline__ float softplus(float x) {
  float sg;
  return softplus_sigmoid(x, sg);
}

// ---- wave64 lane exchange ---------------------------------------------------------
// Lanes are numbered l = 16 * row + j. DPP control codes (gfx9 encoding):
//   0x00-0xFF quad_perm, 0x120+n row_ror:n, 0x140 row_mirror (j -> 15 - j),
//   0x141 row_half_mirror (j -> 7 - j within each 8), 0x150+n row_newbcast:n
//   (every lane of a row reads lane n of that row).

template <int CTRL> __device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

constexpr int kRowMirror = 0x140;
constexpr int kRowHalfMirror = 0x141;
constexpr int kQuadXor3 = 0x1B;   // quad_perm [3,2,1,0]
constexpr int kQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]

// Value of x held by lane N of the caller's row.
template <int N> __device__ __forceinline__ float row_bcast(float x) { return dpp<0x150 + N>(x); }

// Sum over the 16 lanes of a row, result in every lane of the row.
__device__ __forceinline__ float row_allreduce16(float x) {
  x += dpp<kQuadXor1>(x);
  x += dpp<kQuadXor2>(x);
  x += dpp<kRowHalfMirror>(x);
  x += dpp<kRowMirror>(x);
  return x;
}

// Reduce-scatter over a row: lane j of every row returns sum_{lanes of row} p[j].
// Butterfly with partner masks 15 (row_mirror), 7 (row_half_mirror), 3 and 1
// (quad_perm); they span all four lane bits, and at each step the lane keeps
// the half selected by bits 3, 2, 1, 0 of j in turn.
__device__ __forceinline__ float row_reduce_scatter16(const float (&p)[16], int j) {
  const bool b3 = j & 8, b2 = j & 4, b1 = j & 2, b0 = j & 1;
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float keep = b3 ? p[i + 8] : p[i];
    const float send = b3 ? p[i] : p[i + 8];
    q[i] = keep + dpp<kRowMirror>(send);
  }
  float r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float keep = b2 ? q[i + 4] : q[i];
    const float send = b2 ? q[i] : q[i + 4];
    r[i] = keep + dpp<kRowHalfMirror>(send);
  }
  float s[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float keep = b1 ? r[i + 2] : r[i];
    const float send = b1 ? r[i] : r[i + 2];
    s[i] = keep + dpp<kQuadXor3>(send);
  }
  const float keep = b0 ? s[1] : s[0];
  const float send = b0 ? s[0] : s[1];
  return keep + dpp<kQuadXor1>(send);
}

// Sum of the two registers a permlane swap leaves behind: with W = 32,
// lanes 32-63 of a trade places with lanes 0-31 of b; with W = 16, the odd
// rows of a trade places with the even rows of b. The two results are
// copied into plain scalars before use: applying __builtin_bit_cast directly
// to an element of the returned vector makes this compiler read element 0
// twice.
template <int W>
__device__ __forceinline__ float swap_sum(float a, float b) {
  const uint32_t ua = __builtin_bit_cast(uint32_t, a), ub = __builtin_bit_cast(uint32_t, b);
  uint32_t r0, r1;
  if constexpr (W == 32) {
    const auto w = __builtin_amdgcn_permlane32_swap(ua, ub, false, false);
    r0 = w[0];
    r1 = w[1];
  } else {
    const auto w = __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
    r0 = w[0];
    r1 = w[1];
  }
  return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

// Reduce over the 4 rows of a wave, scattered over time: x[i] (i = 0..15) is a
// per-lane value for step i. On return, y[k] (k = 0..3) in lane (row, j) holds
// sum over the 4 rows of x[4 * row + k] of lane j. Uses the gfx950 permlane
// swaps: one swap exchanges half a register between two registers.
__device__ __forceinline__ void wave_rows_reduce_scatter(const float (&x)[16], float (&y)[4]) {
  float s[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // lanes 32-63 of x[i] <-> lanes 0-31 of x[i+8]
    s[i] = swap_sum<32>(x[i], x[i + 8]);
  }
  // rows 0,1 now hold steps 0..7 summed over rows {r, r+2}; rows 2,3 hold steps 8..15.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // odd rows of s[i] <-> even rows of s[i+4]
    y[i] = swap_sum<16>(s[i], s[i + 4]);
  }
}

// Compile-time loop: f(std::integral_constant<int, I>{}) for I = 0 .. N-1.
template <int... Is, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, Is...>, F&& f) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F> __device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

}  // namespace mcpu
