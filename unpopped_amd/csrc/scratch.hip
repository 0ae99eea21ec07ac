// The no-allocation launch: unp_hip_exec_launch with every workspace (the scan's tile status and
// ticket counter, the full reduction's partials and counter, the column reduction's partials and
// strip counters, the dequant GEMM's repacked activations and column sums) taken from one static
// device array instead of the executor's own allocations.  For callers that cannot call hipMalloc:
// code under HIP graph capture, tight serving loops, harnesses that forbid allocation.
//
// The array lives in this library's own code object, one copy per GPU, zero-filled at load and
// held until the process ends.  Its device address is looked up once per device, with that device
// current, through hipGetSymbolAddress; host code only ever uses that address, never the array's
// name (which in host code is a stand-in, not a device pointer).  Every launch clears the part it
// uses on its stream before its kernels run, so no call depends on what an earlier one left; the
// clear is a kernel (scratch_zero), not hipMemsetAsync, so a captured call records kernel nodes
// only.  Calls that overlap on one GPU share the array and race: a caller serialises them (one
// stream, or events).
#include <hip/hip_runtime.h>

#include <mutex>

#include "unp_internal.hpp"

static __device__ __align__(256) unsigned char scratch[UNP_STATIC_SCRATCH_BYTES];

// Zero n 16-byte words at p (grid-strided).
__global__ void __launch_bounds__(256) scratch_zero(uint4* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = uint4{0, 0, 0, 0};
}

namespace unp {

int32_t scratch_clear(void* base, size_t bytes, void* stream, unp_error* err) {
  if (bytes % 16 != 0) {
    set_error(err, UNP_INVALID_ARGUMENT, "a scratch clear covers whole 16-byte words");
    return UNP_INVALID_ARGUMENT;
  }
  const size_t n = bytes / 16;
  if (n == 0) return UNP_OK;
  const size_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(scratch_zero, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0,
                     static_cast<hipStream_t>(stream),
                     static_cast<uint4*>(base), n);
  const hipError_t h = hipGetLastError();
  if (h != hipSuccess) {
    set_error(err, UNP_HIP_ERROR, std::string("scratch_zero launch: ") + hipGetErrorString(h));
    return UNP_HIP_ERROR;
  }
  return UNP_OK;
}

}  // namespace unp

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices];  // the array's device address, per device (null until looked up)
std::mutex g_scratch_mu;

}  // namespace

extern "C" int32_t unp_hip_exec_launch_static(unp_exec* e, const unp_arg* args, size_t nargs, void* stream,
                                              unp_error* err) {
  int dev = -1;
  hipError_t h = hipGetDevice(&dev);
  if (h != hipSuccess) {
    unp::set_error(err, UNP_HIP_ERROR, std::string("hipGetDevice: ") + hipGetErrorString(h));
    return UNP_HIP_ERROR;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    unp::set_error(err, UNP_INVALID_ARGUMENT, "device ordinal out of range for the static scratch");
    return UNP_INVALID_ARGUMENT;
  }
  void* ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
      void* p = nullptr;
      h = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (h != hipSuccess || !p) {
        unp::set_error(err, UNP_HIP_ERROR,
                       std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(h));
        return UNP_HIP_ERROR;
      }
      g_scratch[dev] = p;
    }
    ptr = g_scratch[dev];
  }
  return unp::exec_launch_in(e, args, nargs, stream, ptr, UNP_STATIC_SCRATCH_BYTES, err);
}
