// Error reporting, device check and small utilities behind the C ABI.
#include "abi_util.h"

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace mcpu {

namespace {
thread_local char g_err[512] = {0};

// Per-device result of the architecture check: 0 unknown, 1 gfx950, 2 other.
constexpr int kMaxDevices = 64;
std::atomic<int> g_dev_ok[kMaxDevices];

__global__ void fill_zero_kernel(float* p, int64_t n) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += 256ll * gridDim.x) p[i] = 0.f;
}
}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = 0; }

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MCPU_OK;
  return fail(MCPU_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int zero_f32(float* p, int64_t n, hipStream_t stream) {
  if (n <= 0) return MCPU_OK;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p, n);
  return hip_status(hipGetLastError(), "fill launch");
}

}  // namespace mcpu

extern "C" const char* mcpu_last_error(void) { return mcpu::g_err; }

extern "C" const char* mcpu_version(void) { return "mamba_hip 0.3.0 (gfx950)"; }

extern "C" size_t mcpu_args_size(const char* name) {
  if (name == nullptr) return 0;
  if (std::strcmp(name, "scan") == 0) return sizeof(mcpu_scan_args);
  if (std::strcmp(name, "conv") == 0) return sizeof(mcpu_conv_args);
  if (std::strcmp(name, "conv_update") == 0) return sizeof(mcpu_conv_update_args);
  if (std::strcmp(name, "state_update") == 0) return sizeof(mcpu_state_update_args);
  if (std::strcmp(name, "ssd") == 0) return sizeof(mcpu_ssd_args);
  if (std::strcmp(name, "mixer_step") == 0) return sizeof(mcpu_mixer_step_args);
  if (std::strcmp(name, "norm_linear") == 0) return sizeof(mcpu_norm_linear_args);
  if (std::strcmp(name, "mamba2_step") == 0) return sizeof(mcpu_mamba2_step_args);
  return 0;
}

extern "C" int mcpu_check_device(void) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return mcpu::hip_status(e, "hipGetDevice");
  if (dev >= 0 && dev < mcpu::kMaxDevices) {
    const int known = mcpu::g_dev_ok[dev].load(std::memory_order_relaxed);
    if (known == 1) return MCPU_OK;
    if (known == 2) return mcpu::fail(MCPU_ERR_DEVICE, "device %d is not gfx950", dev);
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return mcpu::hip_status(e, "hipGetDeviceProperties");
  const bool ok = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  if (dev >= 0 && dev < mcpu::kMaxDevices) mcpu::g_dev_ok[dev].store(ok ? 1 : 2, std::memory_order_relaxed);
  if (!ok)
    return mcpu::fail(MCPU_ERR_DEVICE, "device %d is %s, this library is built for gfx950 only", dev,
                      prop.gcnArchName);
  return MCPU_OK;
}
