// C-ABI bookkeeping for libmamba3_hip.so: version, thread-local error string, argument checks.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "m3_host.hpp"

namespace m3 {

static thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int check_tensor(const m3_tensor& t, const char* name, int dims, int64_t inner_extent,
                 bool required, int want_dtype) {
  if (t.ptr == nullptr) {
    return required ? fail(M3_EINVAL, "%s: required tensor is NULL", name) : M3_OK;
  }
  if (!valid_dtype(t.dtype)) return fail(M3_EINVAL, "%s: invalid dtype %d", name, t.dtype);
  if (want_dtype >= 0 && t.dtype != want_dtype) {
    return fail(M3_EUNSUPPORTED, "%s: dtype %d, expected %d", name, t.dtype, want_dtype);
  }
  if (reinterpret_cast<uintptr_t>(t.ptr) % elem_size(t.dtype) != 0) {
    return fail(M3_EINVAL, "%s: pointer not aligned to its element size", name);
  }
  if (dims > 0 && inner_extent > 1 && t.stride[dims - 1] != 1) {
    return fail(M3_EUNSUPPORTED, "%s: innermost stride must be 1 (got %lld)", name,
                static_cast<long long>(t.stride[dims - 1]));
  }
  for (int i = 0; i < dims; ++i) {
    if (t.stride[i] < 0) return fail(M3_EUNSUPPORTED, "%s: negative stride", name);
  }
  return M3_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(M3_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return M3_OK;
}

}  // namespace m3

extern "C" {

const char* m3_last_error(void) { return m3::g_error; }

int m3_abi_version(void) { return M3_ABI_VERSION; }

}  // extern "C"
