// Error reporting, initialisation and host-only helpers of the C ABI.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "rg_common.hpp"

namespace rg {

static thread_local std::string t_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  t_last_error.assign(buf);
  return code;
}

int ok() {
  t_last_error.clear();
  return RG_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(RG_ERR_HIP, "%s kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return ok();
}

int device_cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
    n = 256;
  }
  return n;
}

}  // namespace rg

extern "C" const char* rg_last_error(void) { return rg::t_last_error.c_str(); }

extern "C" int rg_abi_version(void) { return RG_ABI_VERSION; }

// Kernel handles the library launches; defined next to each kernel.
namespace rg {
int probe_cache_kernels();
int probe_decode_kernels();
int probe_prefill_kernels();
int setup_no_alloc_scratch();
}  // namespace rg

extern "C" int rg_init(int device_ordinal) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) {
    return rg::fail(RG_ERR_HIP, "failed to initialise device %d: no HIP device (%s)",
                    device_ordinal, hipGetErrorString(e));
  }
  if (device_ordinal < 0 || device_ordinal >= count) {
    return rg::fail(RG_ERR_INVALID_ARGUMENT, "device ordinal %d out of range [0, %d)",
                    device_ordinal, count);
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device_ordinal);
  if (e != hipSuccess) {
    return rg::fail(RG_ERR_HIP, "failed to initialise device %d: %s", device_ordinal,
                    hipGetErrorString(e));
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    return rg::fail(RG_ERR_NOT_SUPPORTED,
                    "failed to initialise device %d: built for gfx950, device is %s",
                    device_ordinal, prop.gcnArchName);
  }
  int cur = 0;
  (void)hipGetDevice(&cur);
  (void)hipSetDevice(device_ordinal);
  int st = rg::probe_cache_kernels();
  if (st == RG_OK) st = rg::probe_decode_kernels();
  if (st == RG_OK) st = rg::probe_prefill_kernels();
  if (st == RG_OK) st = rg::setup_no_alloc_scratch();
  (void)hipSetDevice(cur);
  if (st != RG_OK) return st;
  return rg::ok();
}

extern "C" int rg_rope_cos_sin_table(float* table, int32_t max_position, int32_t head_dim,
                                     double theta) {
  if (table == nullptr) return rg::fail(RG_ERR_INVALID_ARGUMENT, "rope table: null table");
  if (max_position < 0 || head_dim <= 0 || head_dim % 2 != 0) {
    return rg::fail(RG_ERR_INVALID_ARGUMENT,
                    "rope table: need max_position >= 0 and an even head_dim > 0, got %d, %d",
                    (int)max_position, (int)head_dim);
  }
  if (!(theta > 0.0)) return rg::fail(RG_ERR_INVALID_ARGUMENT, "rope table: theta must be > 0");
  const int half = head_dim / 2;
  for (int32_t pos = 0; pos < max_position; ++pos) {
    float* row = table + (int64_t)pos * head_dim;
    for (int i = 0; i < half; ++i) {
      const double inv_freq = std::pow(theta, -2.0 * (double)i / (double)head_dim);
      const double ang = (double)pos * inv_freq;
      row[i] = (float)std::cos(ang);
      row[half + i] = (float)std::sin(ang);
    }
  }
  return rg::ok();
}
