// Host-side helpers shared by the C-ABI entry points: per-thread error text,
// HIP status mapping, alignment, and a fill kernel (used instead of
// hipMemsetAsync so the entry points stay safe to record into HIP graphs).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "mamba_hip.h"

namespace mcpu {

// Records a formatted message for mcpu_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// MCPU_OK for hipSuccess, otherwise records "<what>: <hip error>" and returns MCPU_ERR_HIP.
int hip_status(hipError_t e, const char* what);

inline bool valid_dtype(int dt) { return dt == MCPU_F32 || dt == MCPU_BF16 || dt == MCPU_F16; }
inline int64_t dtype_size(int dt) { return dt == MCPU_F32 ? 4 : 2; }
inline size_t align_up(size_t bytes) { return (bytes + 255) & ~size_t(255); }

// Fills n floats with zero on `stream`.
int zero_f32(float* p, int64_t n, hipStream_t stream);

}  // namespace mcpu
