// Device scratch of the allocation-free entry point (fe_engine_diffusion_denoise_noalloc).
//
// A file-scope device array holds that entry point's whole workspace (FiLM rows, staged input,
// activations, split-K partials), so the call itself needs no device allocation.  Each GPU the
// library runs on holds its own copy of the array for the life of the process.  The host-side
// name `scratch` is only a stand-in for the symbol: its device address, different on every GPU,
// comes from hipGetSymbolAddress with that GPU current, once per device, and only that address is
// ever handed to kernels or copies.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <mutex>

#include "kernels.h"

namespace {

static __device__ __align__(256) unsigned char scratch[fe::hip::kScratchBytes];

constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mutex;

}  // namespace

namespace fe::hip {

hipError_t scratch_setup(int device, void** ptr) {
  *ptr = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[device] == nullptr) {
    int current = -1;
    hipError_t st = hipGetDevice(&current);
    if (st != hipSuccess) return st;
    if (current != device) return hipErrorInvalidDevice;
    void* p = nullptr;
    st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (st != hipSuccess) return st;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch[device] = p;
  }
  *ptr = g_scratch[device];
  return hipSuccess;
}

}  // namespace fe::hip
