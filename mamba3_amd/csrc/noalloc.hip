// m3_scan_fwd_noalloc: the chunked scan with the library's own device scratch in place of a
// caller-allocated workspace, for callers that cannot allocate device memory.
//
// The scratch is one file-scope __device__ array of M3_SCRATCH_BYTES per GPU, alive until the
// process ends. Host code never passes the array's name to a kernel (on the host it names a
// stand-in, not device memory): the first call on each device looks up the array's device
// address with hipGetSymbolAddress, with that device current, and keeps it; every later call on
// that device passes the kept address as the scan's workspace.
//
// The scan's workspace needs no clearing between calls: prep writes every region the scan reads
// (the RMSNorm factors, the angle tiles, the scalar blocks), and a split call's segment buffers
// are written by its pass 1 and composition before pass 2 reads them. So nothing is zeroed here,
// and no call allocates, frees or synchronises.
#include <hip/hip_runtime.h>

#include <mutex>

#include "m3_host.hpp"

namespace m3 {
namespace {

__device__ __align__(256) unsigned char scratch[M3_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device (looked up once per device).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    return fail(M3_ELAUNCH, "m3_scan_fwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  }
  if (dev < 0 || dev >= kMaxDevices) {
    return fail(M3_EUNSUPPORTED, "m3_scan_fwd_noalloc: device %d >= %d", dev, kMaxDevices);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      return fail(M3_ELAUNCH, "m3_scan_fwd_noalloc: hipGetSymbolAddress: %s",
                  hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return M3_OK;
}

}  // namespace
}  // namespace m3

extern "C" int m3_scan_fwd_noalloc(const m3_scan_args* args, hipStream_t stream) {
  using namespace m3;
  clear_error();
  if (args == nullptr) return fail(M3_EINVAL, "m3_scan_fwd_noalloc: args is NULL");
  size_t need = 0;
  int rc = m3_scan_workspace_size(args, &need);
  if (rc != M3_OK) return rc;
  if (need > M3_SCRATCH_BYTES) {
    return fail(M3_EWORKSPACE,
                "m3_scan_fwd_noalloc: the call needs %zu bytes of scratch, above the %u-byte "
                "maximum (use m3_scan_fwd with a workspace)",
                need, static_cast<unsigned>(M3_SCRATCH_BYTES));
  }
  void* ptr = nullptr;
  if ((rc = scratch_address(&ptr)) != M3_OK) return rc;
  m3_scan_args a = *args;
  a.workspace = ptr;
  a.workspace_bytes = M3_SCRATCH_BYTES;
  return m3_scan_fwd(&a, stream);
}
