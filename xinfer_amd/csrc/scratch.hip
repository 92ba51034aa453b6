// Static device scratch for the allocation-free batched attention entry point
// (xinfer_batched_flash_attention_noalloc in capi.cpp).
//
// `scratch` is a file-scope device array in this library's code object: the
// HIP runtime gives every GPU that loads the library its own copy, at its own
// address, for the life of the process.  In host code the name `scratch` is
// only a host-side stand-in for the symbol, not a device address, so host code
// never passes it to a kernel or a copy.  scratch_pointer() asks the runtime
// for the current device's address of the array once per device
// (hipGetSymbolAddress) and keeps it; the attention kernels then receive that
// pointer as their split-record workspace, exactly as they receive a
// caller-supplied workspace.
//
// The first call on a device may come while the caller's stream is being
// captured into a HIP graph (the callers this entry point is for).  The
// lookup enqueues no work, but the runtime may load the code object behind
// it, which a capture in global or thread-local mode forbids; so this thread
// switches to relaxed capture mode for the lookup alone and restores its mode
// afterwards.
//
// Nothing in the array needs clearing between calls: every work item that
// splits a query group writes each of its records (running max, sum and
// unnormalised output) before the merge reads them, splits that see no key
// included (their records carry max = -inf).  Calls that overlap in time on
// one GPU share the array and race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "launch.h"

namespace xattn {

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

hipError_t scratch_pointer(void **pointer) {
  constexpr int kMaxDevices = 64;
  static std::mutex mutex;
  static void *device_pointers[kMaxDevices] = {};
  int device = -1;
  hipError_t status = hipGetDevice(&device);
  if (status != hipSuccess) return status;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mutex);
  if (device_pointers[device] == nullptr) {
    void *address = nullptr;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    status = hipThreadExchangeStreamCaptureMode(&mode);
    if (status != hipSuccess) return status;
    status = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    const hipError_t restored = hipThreadExchangeStreamCaptureMode(&mode);
    if (status != hipSuccess) return status;
    if (restored != hipSuccess) return restored;
    if (address == nullptr) return hipErrorInvalidSymbol;
    device_pointers[device] = address;
  }
  *pointer = device_pointers[device];
  return hipSuccess;
}

}  // namespace xattn
