// rkv_scratch.hip -- the decode's static device scratch: split-K partials
// for rkv_decode_q8_noalloc, a variant of rkv_decode_q8 that allocates
// nothing and takes no workspace (for callers that cannot call hipMalloc).
//
// The array is a file-scope __device__ variable, so every device the library
// runs on holds its own copy from module load until the process ends.  Host
// code never passes `scratch` itself to a kernel or a copy: in host code the
// name is a stand-in, not a device address.  scratch_address() resolves the
// device address once per device (hipGetSymbolAddress with that device
// current) and every later use goes through the resolved pointer.
#include <mutex>

#include "rkv_launch.h"

namespace rkv {

namespace {
static __device__ __align__(256) uint8_t scratch[kDecodeScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};
}  // namespace

hipError_t scratch_address(int device, void **ptr) {
  *ptr = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] == nullptr) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device) return hipErrorInvalidDevice;  // the caller makes `device` current
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = p;
  }
  *ptr = g_scratch_ptr[device];
  return hipSuccess;
}

}  // namespace rkv
