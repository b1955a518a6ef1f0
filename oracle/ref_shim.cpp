// Test infrastructure only: a plain C entry point over the reference's own CPU
// selective-scan kernels, so tests and the CPU-baseline leg of bench.py can call
// them through ctypes. The reference binds the same functions with nanobind
// (csrc/bindings.cpp:23-84), which is not installed here; this file plays that
// role and nothing else. It is compiled together with the reference sources
// where they lie (see oracle/Makefile) into oracle/_ref/libmcpu_ref.so.
//
// Argument order and meaning follow bindings.cpp:25-28 and 49-53: raw pointers
// (NULL = None), sizes, delta_softplus, num_threads.
#include <cstdint>

#include "selective_scan.h"

extern "C" {

// Replaces _C.selective_scan_fwd_f32 (csrc/bindings.cpp:23-45).
void mcpu_ref_selective_scan_fwd_f32(const float* u, const float* delta, const float* A,
                                     const float* B, const float* C, const float* D,
                                     const float* z, const float* delta_bias, float* out,
                                     float* last_state, int64_t batch, int64_t dim,
                                     int64_t seqlen, int64_t dstate, int64_t ngroups,
                                     int delta_softplus, int num_threads) {
  mamba_cpu::SelectiveScanParams p{u,          delta,      A,     B,      C,
                                   D,          z,          delta_bias,    out,
                                   last_state, batch,      dim,   seqlen, dstate,
                                   ngroups,    delta_softplus != 0};
  mamba_cpu::selective_scan_fwd_f32(p, num_threads);
}

// Replaces _C.selective_scan_bwd_f32 (csrc/bindings.cpp:47-84). dB and dC must
// be zeroed by the caller; dA/dD/ddelta_bias are per-batch partials
// (csrc/selective_scan.h:42-50).
void mcpu_ref_selective_scan_bwd_f32(const float* u, const float* delta, const float* A,
                                     const float* B, const float* C, const float* D,
                                     const float* z, const float* delta_bias, const float* dout,
                                     const float* dlast_state, float* du, float* ddelta,
                                     float* dA_part, float* dB, float* dC, float* dD_part,
                                     float* dz, float* ddelta_bias_part, int64_t batch,
                                     int64_t dim, int64_t seqlen, int64_t dstate,
                                     int64_t ngroups, int delta_softplus, int num_threads) {
  mamba_cpu::SelectiveScanBwdParams p{
      {u, delta, A, B, C, D, z, delta_bias, nullptr, nullptr, batch, dim, seqlen, dstate,
       ngroups, delta_softplus != 0},
      dout, dlast_state, du, ddelta, dA_part, dB, dC, dD_part, dz, ddelta_bias_part};
  mamba_cpu::selective_scan_bwd_f32(p, num_threads);
}

// Replaces _C.cpu_isa / _C.set_cpu_isa (csrc/bindings.cpp:20-21).
const char* mcpu_ref_cpu_isa() { return mamba_cpu::cpu_isa(); }
int mcpu_ref_set_cpu_isa(const char* name) { return mamba_cpu::set_cpu_isa(name) ? 1 : 0; }

}  // extern "C"
