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
// Round to nearest even; NaN stays a (quiet) NaN. gfx950 converts in hardware
// (v_cvt_pk_bf16_f32, two values per instruction when neighbours convert together).
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) {
  return bf16{__builtin_bit_cast(uint16_t, static_cast<__bf16>(x))};
}
// Two values rounded to bf16 by one v_cvt_pk_bf16_f32; lo in bits 0-15.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
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

// The element's bits as a buffer load returns them (16-bit types in the low
// half, zero-extended), and their float32 value. Prefetch registers hold the
// bits and are widened where the value is consumed: widening next to the load
// would make the wave wait for the load there.
template <typename T> __device__ __forceinline__ uint32_t buf_ld_raw(__amdgpu_buffer_rsrc_t r, uint32_t off);
template <> __device__ __forceinline__ uint32_t buf_ld_raw<float>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
template <> __device__ __forceinline__ uint32_t buf_ld_raw<bf16>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
template <> __device__ __forceinline__ uint32_t buf_ld_raw<f16>(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
template <typename T> __device__ __forceinline__ float raw_f32(uint32_t bits);
template <> __device__ __forceinline__ float raw_f32<float>(uint32_t bits) { return __builtin_bit_cast(float, bits); }
template <> __device__ __forceinline__ float raw_f32<bf16>(uint32_t bits) {
  return __builtin_bit_cast(float, bits << 16);
}
template <> __device__ __forceinline__ float raw_f32<f16>(uint32_t bits) {
  return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(bits)));
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
//   (every lane of a row reads lane n of that row), 0x130 / 0x138 wave_shl:1 /
//   wave_shr:1 (across the whole wave).

template <int CTRL> __device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}

// Whole-wave shifts: lane l reads lane l + 1 (kWaveShl1) or l - 1 (kWaveShr1);
// lane 63 (resp. 0), whose source is outside the wave, reads 0.
constexpr int kWaveShl1 = 0x130;
constexpr int kWaveShr1 = 0x138;
constexpr int kRowMirror = 0x140;
constexpr int kRowHalfMirror = 0x141;
constexpr int kQuadXor3 = 0x1B;   // quad_perm [3,2,1,0]
constexpr int kQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]

// Value of x held by lane N of the caller's row.
template <int N> __device__ __forceinline__ float row_bcast(float x) { return dpp<0x150 + N>(x); }

// One VOP2 instruction whose first operand is x as held by lane N of the
// caller's row (row_newbcast), for the uses the compiler cannot fold a DPP
// move into (v_fmac, or a multiply far from the broadcast). Each statement
// starts with the two wait states a DPP instruction needs after a vector ALU
// write of any of its operands, so it is safe wherever it is scheduled; the
// wait stalls only the issuing wave. Nothing the compiler emits reads their
// results through DPP.

// acc + bcast_N(x) * m
template <int N> __device__ __forceinline__ float fmac_bcast(float acc, float x, float m) {
  asm("s_nop 1\n\tv_fmac_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
      : "+v"(acc)
      : "v"(x), "v"(m), "n"(N));
  return acc;
}
// bcast_N(x) * m
template <int N> __device__ __forceinline__ float mul_bcast(float x, float m) {
  float r;
  asm("s_nop 1\n\tv_mul_f32_dpp %0, %1, %2 row_newbcast:%3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
      : "=v"(r)
      : "v"(x), "v"(m), "n"(N));
  return r;
}

// Sum over the 16 lanes of a row, result in every lane of the row.
__device__ __forceinline__ float row_allreduce16(float x) {
  x += dpp<kQuadXor1>(x);
  x += dpp<kQuadXor2>(x);
  x += dpp<kRowHalfMirror>(x);
  x += dpp<kRowMirror>(x);
  return x;
}

// Reduce-scatter over a row: lane j of every row returns sum_{lanes of row} p[j].
// The first two halvings split the row by DPP bank masks (a bank is 4 lanes):
// one v_add_f32_dpp per half writes only the lanes that keep that half, so a
// halving costs one instruction per output and no selects. Partners are
// lane j ^ 8 (row_ror:8; banks 0-1 keep steps 0-7, banks 2-3 steps 8-15) and
// lane j ^ 7 (row_half_mirror; banks 0, 2 keep the lower four, banks 1, 3 the
// upper four), so lane j then holds steps i + 4 b2 + 8 b3 (i < 4) summed over
// lanes {j, j^8, j^7, j^15}. The last two halvings pair j with j ^ 3 and
// j ^ 1 within the quad (quad_perm) and select by bits 1 and 0. The 24 adds are
// one statement with the two wait states a DPP read needs after the vector ALU
// wrote its operand at its head; inside it no instruction reads a register
// written fewer than seven instructions earlier.
__device__ __forceinline__ float row_reduce_scatter16(const float (&p)[16], int j) {
  const bool b1 = j & 2, b0 = j & 1;
  float t0, t1, t2, t3, t4, t5, t6, t7;
  asm volatile(
      "s_nop 1\n\t"
      "v_add_f32_dpp %0, %8, %8 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %0, %16, %16 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %1, %9, %9 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %1, %17, %17 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %2, %10, %10 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %2, %18, %18 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %3, %11, %11 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %3, %19, %19 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %4, %12, %12 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %4, %20, %20 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %5, %13, %13 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %5, %21, %21 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %6, %14, %14 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %6, %22, %22 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %7, %15, %15 row_ror:8 row_mask:0xf bank_mask:0x3\n\t"
      "v_add_f32_dpp %7, %23, %23 row_ror:8 row_mask:0xf bank_mask:0xc\n\t"
      "v_add_f32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
      "v_add_f32_dpp %0, %4, %4 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %1, %1, %1 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
      "v_add_f32_dpp %1, %5, %5 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %2, %2, %2 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
      "v_add_f32_dpp %2, %6, %6 row_half_mirror row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %3, %3, %3 row_half_mirror row_mask:0xf bank_mask:0x5\n\t"
      "v_add_f32_dpp %3, %7, %7 row_half_mirror row_mask:0xf bank_mask:0xa"
      : "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3), "=&v"(t4), "=&v"(t5), "=&v"(t6), "=&v"(t7)
      : "v"(p[0]), "v"(p[1]), "v"(p[2]), "v"(p[3]), "v"(p[4]), "v"(p[5]), "v"(p[6]), "v"(p[7]),
        "v"(p[8]), "v"(p[9]), "v"(p[10]), "v"(p[11]), "v"(p[12]), "v"(p[13]), "v"(p[14]), "v"(p[15]));
  const float r[4] = {t0, t1, t2, t3};
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

// The same over 8 per-lane values x[i] (i = 0..7): y[k] (k = 0..1) in lane
// (row, j) holds the sum over the 4 rows of x[2 * row + k] of lane j.
__device__ __forceinline__ void wave_rows_reduce_scatter8(const float (&x)[8], float (&y)[2]) {
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = swap_sum<32>(x[i], x[i + 4]);
  // rows 0,1 now hold values 0..3 summed over rows {r, r+2}; rows 2,3 hold 4..7.
#pragma unroll
  for (int i = 0; i < 2; ++i) y[i] = swap_sum<16>(s[i], s[i + 2]);
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
