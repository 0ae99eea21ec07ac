// Storage images for the forms whose kernels read and write dense storage (the dequants, RowReduce,
// and the reductions and scans with a pre-map body): a view that is not dense row-major is staged.
// Before the launch each such input view is packed, element by element in row-major order of its
// shape, into a dense buffer the executor owns; the form's dense kernels run on the packed copies;
// after them each staged output is unpacked into its view's elements.  Elements outside a view are
// never read or written.  A buffer's view (shape, signed strides in elements, base) follows the
// reference's storage image (crates/unpopped-cpu-c/src/base.rs:65-103, oracle/buffers.rs:16-42).
//
// Sub-byte (4-bit) elements are nibbles, element i of a buffer in the low nibble of byte i / 2 when i
// is even and the high nibble when it is odd (kernel_subbyte_load.rs); the packer writes one output
// byte per lane, so two lanes never share a byte.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "unp_internal.hpp"

namespace {

struct view_desc {
  long long rank, base, count;
  long long shape[UNP_MAX_RANK], stride[UNP_MAX_RANK];
};

// The storage offset (in elements) of row-major element i of the view.
__device__ __forceinline__ long long view_offset(const view_desc& v, long long i) {
  long long off = v.base;
  for (long long d = v.rank - 1; d >= 0; --d) {
    const long long c = i % v.shape[d];
    i /= v.shape[d];
    off += c * v.stride[d];
  }
  return off;
}

template <class E>
__global__ void __launch_bounds__(256) view_pack(const E* __restrict__ src, view_desc v, E* __restrict__ dst) {
  const long long step = (long long)gridDim.x * 256;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < v.count; i += step) dst[i] = src[view_offset(v, i)];
}

template <class E>
__global__ void __launch_bounds__(256) view_unpack(const E* __restrict__ src, view_desc v, E* __restrict__ dst) {
  const long long step = (long long)gridDim.x * 256;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < v.count; i += step) dst[view_offset(v, i)] = src[i];
}

// 4-bit elements: lane j writes packed byte j, nibbles 2j and 2j + 1 of the view (the high nibble
// zero past an odd count).
__global__ void __launch_bounds__(256) view_pack4(const uint8_t* __restrict__ src, view_desc v, uint8_t* __restrict__ dst) {
  const long long bytes = (v.count + 1) / 2, step = (long long)gridDim.x * 256;
  for (long long j = (long long)blockIdx.x * 256 + threadIdx.x; j < bytes; j += step) {
    unsigned b = 0;
    for (int h = 0; h < 2; ++h) {
      const long long i = 2 * j + h;
      if (i >= v.count) break;
      const long long o = view_offset(v, i);
      const unsigned q = (src[o >> 1] >> ((o & 1) * 4)) & 15u;
      b |= q << (4 * h);
    }
    dst[j] = (uint8_t)b;
  }
}

view_desc desc_of(const unp_view& v) {
  view_desc d{};
  d.rank = v.rank;
  d.base = v.base;
  d.count = 1;
  for (int i = 0; i < v.rank; ++i) {
    d.shape[i] = v.shape[i];
    d.stride[i] = v.stride[i];
    d.count *= v.shape[i];
  }
  return d;
}

unsigned grid_for(long long items) {
  const long long b = (items + 255) / 256;
  return (unsigned)(b < 1 ? 1 : (b > 2048 ? 2048 : b));
}

int32_t launched(unp_error* err, const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return UNP_OK;
  unp::set_error(err, UNP_HIP_ERROR, std::string(what) + ": " + hipGetErrorString(e));
  return UNP_HIP_ERROR;
}

}  // namespace

namespace unp {

size_t view_stage_bytes(const unp_view& v, int bits) {
  const view_desc d = desc_of(v);
  return bits == 4 ? (size_t)((d.count + 1) / 2) : (size_t)d.count * (size_t)(bits / 8);
}

int32_t view_stage_in(const unp_view& v, int bits, void* dst, void* stream, unp_error* err) {
  const view_desc d = desc_of(v);
  if (d.count == 0) return UNP_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const void* src = reinterpret_cast<const void*>(v.data);
  switch (bits) {
    case 4:
      hipLaunchKernelGGL(view_pack4, dim3(grid_for((d.count + 1) / 2)), dim3(256), 0, s,
                         static_cast<const uint8_t*>(src), d, static_cast<uint8_t*>(dst));
      break;
    case 8:
      hipLaunchKernelGGL(view_pack<uint8_t>, dim3(grid_for(d.count)), dim3(256), 0, s,
                         static_cast<const uint8_t*>(src), d, static_cast<uint8_t*>(dst));
      break;
    case 16:
      hipLaunchKernelGGL(view_pack<uint16_t>, dim3(grid_for(d.count)), dim3(256), 0, s,
                         static_cast<const uint16_t*>(src), d, static_cast<uint16_t*>(dst));
      break;
    case 32:
      hipLaunchKernelGGL(view_pack<uint32_t>, dim3(grid_for(d.count)), dim3(256), 0, s,
                         static_cast<const uint32_t*>(src), d, static_cast<uint32_t*>(dst));
      break;
    case 64:
      hipLaunchKernelGGL(view_pack<unsigned long long>, dim3(grid_for(d.count)), dim3(256), 0, s,
                         static_cast<const unsigned long long*>(src), d, static_cast<unsigned long long*>(dst));
      break;
    default:
      set_error(err, UNP_INVALID_ARGUMENT, "a staged view of an element width other than 4, 8, 16, 32 or 64 bits");
      return UNP_INVALID_ARGUMENT;
  }
  return launched(err, "view_pack");
}

int32_t view_stage_out(const void* src, const unp_view& v, int bits, void* stream, unp_error* err) {
  const view_desc d = desc_of(v);
  if (d.count == 0) return UNP_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* dst = reinterpret_cast<void*>(v.data);
  switch (bits) {
    case 8:
      hipLaunchKernelGGL(view_unpack<uint8_t>, dim3(grid_for(d.count)), dim3(256), 0, s,
                         static_cast<const uint8_t*>(src), d, static_cast<uint8_t*>(dst));
      break;
    case 16:
      hipLaunchKernelGGL(view_unpack<uint16_t>, dim3(grid_for(d.count)), dim3(256), 0, s,
                         static_cast<const uint16_t*>(src), d, static_cast<uint16_t*>(dst));
      break;
    case 32:
      hipLaunchKernelGGL(view_unpack<uint32_t>, dim3(grid_for(d.count)), dim3(256), 0, s,
                         static_cast<const uint32_t*>(src), d, static_cast<uint32_t*>(dst));
      break;
    case 64:
      hipLaunchKernelGGL(view_unpack<unsigned long long>, dim3(grid_for(d.count)), dim3(256), 0, s,
                         static_cast<const unsigned long long*>(src), d, static_cast<unsigned long long*>(dst));
      break;
    default:
      set_error(err, UNP_INVALID_ARGUMENT, "a staged output view of an element width other than 8, 16, 32 or 64 bits");
      return UNP_INVALID_ARGUMENT;
  }
  return launched(err, "view_unpack");
}

}  // namespace unp
