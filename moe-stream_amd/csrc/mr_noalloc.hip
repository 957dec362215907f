// mr_noalloc.hip -- the static scratch of mr_moe_forward_batched_noalloc.
//
// One file-scope device array, `scratch`, of kStaticScratchBytes: every GPU the library
// runs on holds its own copy at its own address until the process ends. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in for the symbol):
// static_scratch_init resolves this device's address with hipGetSymbolAddress, once per
// device with that device current, and every later use goes through that address.
#include <mutex>

#include "mr_internal.h"

namespace mr {

static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_addr[kMaxDevices];  // device address of `scratch` on each device (nullptr: not resolved)
}  // namespace

hipError_t static_scratch_init(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_addr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_addr[device] = p;
  }
  *out = g_addr[device];
  return hipSuccess;
}

}  // namespace mr
