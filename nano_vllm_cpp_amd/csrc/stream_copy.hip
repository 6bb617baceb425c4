// Plain streaming copy: the bandwidth and traffic-counter reference for the
// op kernels.  It uses the same instruction forms as they do (16-byte
// non-temporal loads and stores, one vector per lane), so the bytes a copy of
// known size moves calibrate rocprofv3's FETCH_SIZE / WRITE_SIZE for them, and
// its GB/s is the attainable HBM rate the op kernels are compared with.
#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                          int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) st16_nt(dst + i, ld16_nt(src + i));
}

// The same with the gather's 1:2 read:write mix: each 8 bytes read become one
// 16-byte non-temporal store (the 8 bytes twice), one store per lane -- the
// attainable rate for a kernel that writes twice what it reads.
__global__ __launch_bounds__(256) void stream_expand_kernel(const uint2* __restrict__ src, u32x4* __restrict__ dst,
                                                            int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const uint2 v = src[i];
    st16_nt(dst + i, u32x4{v.x, v.y, v.x, v.y});
  }
}

}  // namespace nvf

extern "C" int nvf_stream_expand(void* dst, const void* src, int64_t src_bytes, void* stream) {
  using namespace nvf;
  if (src_bytes < 0 || src_bytes % 8 != 0)
    return fail(NVF_ERR_INVALID, "nvf_stream_expand: %lld bytes is not a multiple of 8", (long long)src_bytes);
  if (src_bytes == 0) return NVF_OK;
  if (!dst || !src || !aligned16(dst) || (reinterpret_cast<uintptr_t>(src) & 7u))
    return fail(NVF_ERR_INVALID, "nvf_stream_expand: NULL or unaligned pointer");
  const int64_t n = src_bytes / 8;
  if ((n + 255) / 256 > INT32_MAX) return fail(NVF_ERR_INVALID, "nvf_stream_expand: too large for one launch");
  stream_expand_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, as_stream(stream)>>>(
      static_cast<const uint2*>(src), static_cast<u32x4*>(dst), n);
  return launch_status("stream_expand");
}

extern "C" int nvf_stream_copy(void* dst, const void* src, int64_t bytes, void* stream) {
  using namespace nvf;
  if (bytes < 0 || bytes % 16 != 0)
    return fail(NVF_ERR_INVALID, "nvf_stream_copy: %lld bytes is not a multiple of 16", (long long)bytes);
  if (bytes == 0) return NVF_OK;
  if (!dst || !src || !aligned16(dst) || !aligned16(src))
    return fail(NVF_ERR_INVALID, "nvf_stream_copy: NULL or unaligned pointer");
  const int64_t n = bytes / 16;
  if ((n + 255) / 256 > INT32_MAX) return fail(NVF_ERR_INVALID, "nvf_stream_copy: too large for one launch");
  stream_copy_kernel<<<dim3((unsigned)((n + 255) / 256)), 256, 0, as_stream(stream)>>>(
      static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n);
  return launch_status("stream_copy");
}
