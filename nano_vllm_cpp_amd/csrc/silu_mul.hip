// SiLU(gate) * up (SwiGLU) for gfx950.
//
// Reference semantics: src/hip_ops.hip:419-429 (silu_and_mul_kernel):
//   out[r, c] = g / (1 + expf(-g)) * u,  g = gate_up[r, c], u = gate_up[r, I + c].
//
// Design: a flat grid with one 16-byte output vector per lane (one gate and
// one up load in flight), the row/column split by a launch-constant mul-hi
// divide.  Pure streaming: 3 x T x I x e bytes, read once and written once,
// all with non-temporal hints (nothing here is reused from L2/MALL).  Measured
// at Qwen2.5-7B prefill shape this beat 2 or 4 vectors per lane and a 2-D
// (row, chunk) grid: more vectors per lane lowered the achieved bandwidth.
//
// fp32 keeps the reference's exact expression (IEEE divide, precise expf).
// fp16/bf16 use v_exp_f32 + v_rcp_f32 (relative error a few fp32 ulp, far below
// one 16-bit ulp) because the precise path is VALU-bound at 16-bit widths.
#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

constexpr int kSiluThreads = 256;
constexpr int kSiluUnroll = 1;

template <typename T>
__device__ __forceinline__ float silu_mul(float g, float u) {
  if constexpr (sizeof(T) == 4) {
    return g / (1.0f + expf(-g)) * u;
  } else {
    const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
  }
}

template <typename T>
__global__ __launch_bounds__(kSiluThreads) void silu_mul_vec_kernel(const T* __restrict__ gu, T* __restrict__ out,
                                                                    uint32_t total_vec, FastDiv vpr, int64_t inter) {
  constexpr int N = Pack<T>::N;
  const uint32_t base = blockIdx.x * (kSiluThreads * kSiluUnroll) + threadIdx.x;
  u32x4 ga[kSiluUnroll], ua[kSiluUnroll];
  int64_t oo[kSiluUnroll];
#pragma unroll
  for (int k = 0; k < kSiluUnroll; ++k) {
    const uint32_t g = base + k * kSiluThreads;
    if (g < total_vec) {
      const uint32_t r = vpr.div(g);
      const int64_t c = (int64_t)(g - r * vpr.d) * N;
      const int64_t gi = (int64_t)r * 2 * inter + c;
      ga[k] = ld16_nt(gu + gi);
      ua[k] = ld16_nt(gu + gi + inter);
      oo[k] = (int64_t)r * inter + c;
    }
  }
#pragma unroll
  for (int k = 0; k < kSiluUnroll; ++k) {
    const uint32_t g = base + k * kSiluThreads;
    if (g < total_vec) {
      float a[N], b[N];
      Pack<T>::unpack(ga[k], a);
      Pack<T>::unpack(ua[k], b);
#pragma unroll
      for (int j = 0; j < N; ++j) a[j] = silu_mul<T>(a[j], b[j]);
      st16_nt(out + oo[k], Pack<T>::pack(a));
    }
  }
}

// Any shape / alignment: one element per thread.
template <typename T>
__global__ __launch_bounds__(kSiluThreads) void silu_mul_generic_kernel(const T* __restrict__ gu, T* __restrict__ out,
                                                                        int64_t total, int64_t inter) {
  const int64_t i = (int64_t)blockIdx.x * kSiluThreads + threadIdx.x;
  if (i >= total) return;
  const int64_t r = i / inter, c = i - r * inter;
  const float g = to_f32(gu[r * 2 * inter + c]);
  const float u = to_f32(gu[r * 2 * inter + inter + c]);
  out[i] = from_f32<T>(silu_mul<T>(g, u));
}

template <typename T>
static int launch_silu(const void* gate_up, void* out, int64_t rows, int64_t inter, hipStream_t st) {
  constexpr int N = Pack<T>::N;
  const T* gp = static_cast<const T*>(gate_up);
  T* op = static_cast<T*>(out);
  const int64_t total_vec = rows * inter / N;
  if (inter % N == 0 && aligned16(gate_up) && aligned16(out) && total_vec < (1ll << 32) - kSiluThreads * kSiluUnroll) {
    const int64_t per_block = kSiluThreads * kSiluUnroll;
    const dim3 grid((unsigned)((total_vec + per_block - 1) / per_block));
    silu_mul_vec_kernel<T><<<grid, kSiluThreads, 0, st>>>(gp, op, (uint32_t)total_vec, FastDiv((uint32_t)(inter / N)),
                                                          inter);
    return launch_status("silu_and_mul");
  }
  const int64_t total = rows * inter;
  const dim3 grid((unsigned)((total + kSiluThreads - 1) / kSiluThreads));
  silu_mul_generic_kernel<T><<<grid, kSiluThreads, 0, st>>>(gp, op, total, inter);
  return launch_status("silu_and_mul(generic)");
}

}  // namespace nvf

extern "C" int nvf_silu_and_mul(const void* gate_up, void* out, int64_t rows, int64_t inter, int dtype,
                                void* stream) {
  using namespace nvf;
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "nvf_silu_and_mul: bad dtype %d", dtype);
  if (rows < 0 || inter < 0 || (rows > 0 && inter > (INT64_MAX / 4) / rows))
    return fail(NVF_ERR_INVALID, "nvf_silu_and_mul: bad shape rows=%lld inter=%lld", (long long)rows,
                (long long)inter);
  if (rows == 0 || inter == 0) return NVF_OK;
  if (!gate_up || !out) return fail(NVF_ERR_INVALID, "nvf_silu_and_mul: NULL pointer");
  if ((rows * inter + kSiluThreads - 1) / kSiluThreads > INT32_MAX)
    return fail(NVF_ERR_INVALID, "nvf_silu_and_mul: %lld elements exceed one launch", (long long)(rows * inter));
  int s = NVF_OK;
  NVF_DISPATCH_DTYPE(dtype, T, s = launch_silu<T>(gate_up, out, rows, inter, as_stream(stream)));
  return s;
}

// Drop-in: include/nanovllm/hip_ops.hpp:17 / src/hip_ops.hip:707-713.
extern "C" void hip_silu_and_mul(const float* gate_up, float* out, int rows, int intermediate) {
  if (rows <= 0 || intermediate <= 0) return;
  nvf::dropin_check(nvf_silu_and_mul(gate_up, out, rows, intermediate, NVF_F32, nullptr), "hip_silu_and_mul");
}
