// Row gather ahead of the LM head: out[r, :] = rows[indices[r], :].
//
// Reference: gather_rows_kernel (src/hip_ops.hip:611-619) and hip_gather_rows
// (:788-795), called by Qwen3Model::forward_logits to keep each sequence's last
// token row before the LM-head projection (src/model.cpp:839).  A plain copy,
// bit-exact in every dtype.
//
// Design: one wave per output row (the index is read once, wave-uniform); lanes
// move 16-byte vectors, so each instruction copies 1 KiB of contiguous row.  Odd
// widths or unaligned rows take a one-element-per-thread kernel.
#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

constexpr int kGatherThreads = 256;
constexpr int kGatherWaves = kGatherThreads / kWave;

__device__ __forceinline__ bool gather_bad(int64_t i, int64_t rows_count) {
  return rows_count > 0 && (i < 0 || i >= rows_count);
}

template <typename T>
__global__ __launch_bounds__(kGatherThreads) void gather_rows_vec_kernel(const T* __restrict__ rows,
                                                                         const int32_t* __restrict__ indices,
                                                                         T* __restrict__ out, int64_t out_rows,
                                                                         int64_t cols, int64_t rows_count) {
  constexpr int N = Pack<T>::N;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t r = (int64_t)blockIdx.x * kGatherWaves + __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  if (r >= out_rows) return;  // wave-uniform
  const int64_t src = indices[r];
  const int64_t nvec = cols / N;
  T* dst = out + r * cols;
  if (gather_bad(src, rows_count)) {  // out-of-range index: a NaN row instead of a read
    float nan[N];
#pragma unroll
    for (int i = 0; i < N; ++i) nan[i] = __builtin_nanf("");
    for (int64_t c = lane; c < nvec; c += kWave) st16(dst + c * N, Pack<T>::pack(nan));
    return;
  }
  const T* s = rows + src * cols;
  for (int64_t c = lane; c < nvec; c += kWave) st16(dst + c * N, ld16(s + c * N));
}

template <typename T>
__global__ __launch_bounds__(kGatherThreads) void gather_rows_generic_kernel(const T* __restrict__ rows,
                                                                             const int32_t* __restrict__ indices,
                                                                             T* __restrict__ out, int64_t total,
                                                                             int64_t cols, int64_t rows_count) {
  const int64_t i = (int64_t)blockIdx.x * kGatherThreads + threadIdx.x;
  if (i >= total) return;
  const int64_t r = i / cols, c = i - r * cols;
  const int64_t src = indices[r];
  out[i] = gather_bad(src, rows_count) ? from_f32<T>(__builtin_nanf("")) : rows[src * cols + c];
}

template <typename T>
int launch_gather_rows(const void* rows, const int32_t* indices, int64_t cols, int64_t out_rows, int64_t rows_count,
                       void* out, hipStream_t st) {
  constexpr int N = Pack<T>::N;
  const T* rp = static_cast<const T*>(rows);
  T* op = static_cast<T*>(out);
  if (cols % N == 0 && aligned16(rows) && aligned16(out)) {
    const dim3 grid((unsigned)((out_rows + kGatherWaves - 1) / kGatherWaves));
    gather_rows_vec_kernel<T><<<grid, kGatherThreads, 0, st>>>(rp, indices, op, out_rows, cols, rows_count);
  } else {
    const int64_t total = out_rows * cols;
    gather_rows_generic_kernel<T><<<dim3((unsigned)((total + kGatherThreads - 1) / kGatherThreads)), kGatherThreads,
                                    0, st>>>(rp, indices, op, total, cols, rows_count);
  }
  return launch_status("gather_rows");
}

}  // namespace nvf

using namespace nvf;

extern "C" int nvf_gather_rows(const void* rows, const int32_t* indices, int64_t rows_count, int64_t cols,
                               int64_t out_rows, void* out, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "nvf_gather_rows: bad dtype %d", dtype);
  if (cols < 0 || out_rows < 0) return fail(NVF_ERR_INVALID, "nvf_gather_rows: negative size");
  if (cols == 0 || out_rows == 0) return NVF_OK;
  if (!rows || !indices || !out) return fail(NVF_ERR_INVALID, "nvf_gather_rows: NULL pointer");
  if ((out_rows * cols + kGatherThreads - 1) / kGatherThreads > INT32_MAX ||
      (out_rows + kGatherWaves - 1) / kGatherWaves > INT32_MAX)
    return fail(NVF_ERR_INVALID, "nvf_gather_rows: too many elements for one launch");
  int rc = NVF_OK;
  NVF_DISPATCH_DTYPE(dtype, T, rc = launch_gather_rows<T>(rows, indices, cols, out_rows, rows_count, out,
                                                          as_stream(stream)));
  return rc;
}

// Drop-in: include/nanovllm/hip_ops.hpp:34 / src/hip_ops.hip:788-795 (fp32, null
// stream).  The reference ignores rows_count and reads wherever an index points; here
// a positive rows_count bounds the indices (an index outside gives a NaN row), which
// changes nothing for valid indices.
extern "C" void hip_gather_rows(const float* rows, const int32_t* indices, int rows_count, int cols, int out_rows,
                                float* out) {
  if (out_rows <= 0 || cols <= 0) return;
  dropin_check(nvf_gather_rows(rows, indices, rows_count, cols, out_rows, out, NVF_F32, nullptr), "hip_gather_rows");
}
