// Fixed device scratch for the entry points that allocate nothing
// (nsr_attention_splitkv_f16_noalloc). The array lives in this library's own
// registered code object, one copy per GPU, for the life of the process.
// Host code never passes the array's name to a kernel (in host code it is a
// stand-in, not a device address): nsr_scratch_device_ptr resolves each
// device's copy once with hipGetSymbolAddress, with that device current, and
// callers use only the pointer it returns.
#include <hip/hip_runtime.h>

#include <mutex>

#include "nsr_scratch.h"

static __device__ __align__(256) float scratch[NSR_NOALLOC_SCRATCH_FLOATS];

namespace {

constexpr int kMaxDevices = 64;

struct ScratchSlot {
  std::once_flag once;
  hipError_t err = hipErrorNotInitialized;
  void* ptr = nullptr;
};

ScratchSlot g_scratch[kMaxDevices];

}  // namespace

__attribute__((visibility("hidden"))) hipError_t nsr_scratch_device_ptr(int device, float** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  ScratchSlot& s = g_scratch[device];
  std::call_once(s.once, [&] {
    s.err = hipGetSymbolAddress(&s.ptr, HIP_SYMBOL(scratch));
    if (s.err != hipSuccess) {
      (void)hipGetLastError();  // reported through the return value, not left sticky
      s.ptr = nullptr;
    }
  });
  *out = static_cast<float*>(s.ptr);
  return s.err;
}
