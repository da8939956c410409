// Scratch memory of the no-allocation entry point (cq_matmul_noalloc): a
// fixed device array, present on every device the library runs on from the
// moment the HIP runtime loads this file's code object there until the
// process ends.  Host code never passes the array's name to a kernel (in
// host code it is only a stand-in for the device symbol): its device address
// is looked up once per device with hipGetSymbolAddress, with that device
// current, and that address is what the prefill launches receive.
//
// Compiled by hipcc into an object that the host library links (the HIP
// runtime registers its code object at load); the library's kernels live in
// the separately loaded code objects and take the address as an argument.
#include <hip/hip_runtime.h>

#include <mutex>

#define CQ_SCRATCH_BYTES (32u << 20)

static __device__ __attribute__((aligned(256))) unsigned char scratch[CQ_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::once_flag g_once[kMaxDevices];
void* g_ptr[kMaxDevices];
hipError_t g_status[kMaxDevices];
}  // namespace

// Device address and size of the scratch array on the current device.
extern "C" __attribute__((visibility("hidden"))) hipError_t cq_scratch_device_ptr(void** out, size_t* bytes) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::call_once(g_once[dev], [dev]() {
    void* p = nullptr;
    g_status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_ptr[dev] = p;
  });
  if (g_status[dev] != hipSuccess) return g_status[dev];
  *out = g_ptr[dev];
  *bytes = CQ_SCRATCH_BYTES;
  return hipSuccess;
}
