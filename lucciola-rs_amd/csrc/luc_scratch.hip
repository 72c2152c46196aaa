// luc_scratch.hip -- the library's fixed split-K scratch, for the entry point
// that allocates nothing (luc_decode_step_noalloc in include/luc_attn.h).
//
// The array below is device memory that the library owns for the life of the
// process, one copy per GPU.  Its host-side name is only a stand-in for the
// symbol: host code never passes `scratch` itself to a kernel or a copy.  At
// set-up (every luc_init, with its device current) hipGetSymbolAddress gives
// that device's address of its copy; the context keeps it, and every later
// use goes through that address.
//
// Compiled by hipcc for gfx950 and linked into liblucattn.so.
#include <hip/hip_runtime.h>

#include <mutex>

#include "luc_attn.h"

namespace {

// The split-K workspace of luc_decode_step_noalloc: the same layout as a
// caller's workspace (arrival counters first, then the partials).
static __device__ __align__(256) unsigned char scratch[LUC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// Zero fill by a plain kernel (no memset node), 16 bytes per thread.
__global__ void luc_scratch_clear(uint4* p, size_t n16) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n16) p[i] = make_uint4(0, 0, 0, 0);
}

}  // namespace

namespace luc_internal {

int fail(int code, const char* fmt, ...);

// Address of this device's scratch (the caller has made `device` current),
// resolved on every call: the first call for `device`, and any call that
// finds the address changed since (the device was reset and its code
// reloaded), zero-fills it.  Otherwise the contents are kept: every decode
// launch leaves the arrival counters at zero again.
int scratch_setup(int device, void** out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices)
    return fail(LUC_E_INVALID, "scratch: device %d outside [0, %d)", device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr)
    return fail(LUC_E_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  if (g_ptr[device] != ptr) {
    // the arrival counters must start at zero
    const size_t n16 = LUC_SCRATCH_BYTES / 16;
    hipLaunchKernelGGL(luc_scratch_clear, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0,
                       nullptr, static_cast<uint4*>(ptr), n16);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) return fail(LUC_E_HIP, "scratch clear: %s", hipGetErrorString(e));
    g_ptr[device] = ptr;
  }
  *out = g_ptr[device];
  return LUC_OK;
}

}  // namespace luc_internal
