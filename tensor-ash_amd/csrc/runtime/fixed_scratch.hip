// Fixed device scratch of the allocation-free split-K entry point
// (ta_matmul_split_k2_noalloc).  This file is compiled by hipcc into
// libtensor_ash.so itself, not into a code object, so the array below is
// registered with the HIP runtime and each device that the library runs on
// holds its own copy until the process ends.
//
// On the host, `scratch` names a host-side stand-in, not device memory:
// only the address hipGetSymbolAddress returns for the current device may
// reach a kernel argument.  That address is looked up once per device and
// kept in `g_addr`.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "../kernels/kernel_args.h"

static __device__ __align__(256) unsigned char scratch[TA_FIXED_SCRATCH_BYTES];
static_assert(sizeof(scratch) == TA_FIXED_SCRATCH_BYTES, "fixed scratch size");

namespace tensor_ash {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_addr[kMaxDevices] = {};
std::mutex g_run_mu[kMaxDevices];
} // namespace

// Device address of `scratch` on `device`, which must be the current
// device.  The first call on a device resolves it; later calls return the
// kept address.  Returns hipSuccess or the lookup's error.
hipError_t fixed_scratch_address(int device, void **out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices)
    return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_addr[device]) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess)
      return e;
    if (cur != device)
      return hipErrorInvalidDevice;
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
      return e;
    if (!p)
      return hipErrorInvalidSymbol;
    g_addr[device] = p;
  }
  *out = g_addr[device];
  return hipSuccess;
}

// Serialises the users of one device's array within this process (the
// caller holds it from the first launch until the stream has drained).
std::mutex &fixed_scratch_mutex(int device) { return g_run_mu[device]; }

} // namespace tensor_ash
