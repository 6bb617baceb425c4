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

// ---------------------------------------------------------------------------
// SwiGLU that also quantizes its output for the Q8_0 down projection: the
// stored SwiGLU row (rounded to T, exactly what silu_mul_vec_kernel stores) is
// reduced to scale = 127/max|v| and written as int8 rows
// (int8)min(127, max(-127, v * scale)) -- the reference's q8_row_scale_kernel
// and quantizer (src/hip_ops.hip:205-217, :244-245) applied to the output of
// silu_and_mul_kernel (:419-429), without the fp round trip through HBM.  One
// 512-thread workgroup per row holds the row in VGPRs (kSiluQ8Vpl vectors per
// lane at most); the fp output is optional.
constexpr int kSiluQ8Threads = 512;
constexpr int kSiluQ8MaxVpl = 8;

template <typename T, int VPL>
__global__ __launch_bounds__(kSiluQ8Threads) void silu_mul_q8_kernel(const T* __restrict__ gu, T* __restrict__ out,
                                                                     float* __restrict__ scale,
                                                                     int8_t* __restrict__ q, int64_t inter) {
  constexpr int N = Pack<T>::N;
  __shared__ float part[kSiluQ8Threads / 64];
  const int64_t r = blockIdx.x;
  const int64_t nvec = inter / N;
  const T* g_row = gu + r * 2 * inter;
  float v[VPL][N];
  u32x4 ga[VPL], ua[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int64_t c = threadIdx.x + (int64_t)i * kSiluQ8Threads;
    if (c < nvec) {
      ga[i] = ld16_nt(g_row + c * N);
      ua[i] = ld16_nt(g_row + inter + c * N);
    }
  }
  float mx = 0.0f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int64_t c = threadIdx.x + (int64_t)i * kSiluQ8Threads;
    if (c < nvec) {
      float a[N], b[N];
      Pack<T>::unpack(ga[i], a);
      Pack<T>::unpack(ua[i], b);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        v[i][j] = to_f32(from_f32<T>(silu_mul<T>(a[j], b[j])));  // the stored value
        mx = fmaxf(mx, fabsf(v[i][j]));
      }
      if (out) st16_nt(out + r * inter + c * N, Pack<T>::pack(v[i]));
    }
  }
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = part[0];
#pragma unroll
  for (int w = 1; w < kSiluQ8Threads / 64; ++w) mx = fmaxf(mx, part[w]);
  const float sc = q8_row_scale(mx);
  if (threadIdx.x == 0) scale[r] = sc;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int64_t c = threadIdx.x + (int64_t)i * kSiluQ8Threads;
    if (c < nvec) {
      uint32_t w[N / 4];
#pragma unroll
      for (int d = 0; d < N / 4; ++d) {
        w[d] = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[d] |= (uint32_t)(q8_quantize(v[i][4 * d + e], sc) & 0xff) << (8 * e);
      }
      if constexpr (N == 8) {
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        __builtin_nontemporal_store(u32x2{w[0], w[1]}, reinterpret_cast<u32x2*>(q + r * inter + c * N));
      } else {
        __builtin_nontemporal_store(w[0], reinterpret_cast<uint32_t*>(q + r * inter + c * N));
      }
    }
  }
}

// Any shape / alignment: one workgroup per row, the SwiGLU computed twice
// (once for the maximum, once to quantize).
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_q8_generic_kernel(const T* __restrict__ gu, T* __restrict__ out,
                                                                  float* __restrict__ scale, int8_t* __restrict__ q,
                                                                  int64_t inter) {
  __shared__ float part[4];
  const int64_t r = blockIdx.x;
  const T* g_row = gu + r * 2 * inter;
  float mx = 0.0f;
  for (int64_t c = threadIdx.x; c < inter; c += 256) {
    const float v = to_f32(from_f32<T>(silu_mul<T>(to_f32(g_row[c]), to_f32(g_row[inter + c]))));
    mx = fmaxf(mx, fabsf(v));
    if (out) out[r * inter + c] = from_f32<T>(v);
  }
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
  const float sc = q8_row_scale(mx);
  if (threadIdx.x == 0) scale[r] = sc;
  for (int64_t c = threadIdx.x; c < inter; c += 256) {
    const float v = to_f32(from_f32<T>(silu_mul<T>(to_f32(g_row[c]), to_f32(g_row[inter + c]))));
    q[r * inter + c] = (int8_t)q8_quantize(v, sc);
  }
}

template <typename T, int VPL>
static void launch_silu_q8_vec(const T* gp, T* op, float* sc, int8_t* q, int64_t rows, int64_t inter,
                               hipStream_t st) {
  silu_mul_q8_kernel<T, VPL><<<dim3((unsigned)rows), kSiluQ8Threads, 0, st>>>(gp, op, sc, q, inter);
}

template <typename T>
static int launch_silu_q8(const void* gate_up, void* out, float* scale, int8_t* q, int64_t rows, int64_t inter,
                          hipStream_t st) {
  constexpr int N = Pack<T>::N;
  const T* gp = static_cast<const T*>(gate_up);
  T* op = static_cast<T*>(out);
  const int64_t nvec = inter / N;
  const int vpl = (int)((nvec + kSiluQ8Threads - 1) / kSiluQ8Threads);
  // q rows start N-byte aligned (N int8 per lane store) when inter % N == 0 and q is
  const bool vec = inter % N == 0 && aligned16(gate_up) && (out == nullptr || aligned16(out)) &&
                   (reinterpret_cast<uintptr_t>(q) & (N - 1)) == 0 && vpl <= kSiluQ8MaxVpl;
  if (vec) {
    switch (vpl) {
      case 1: launch_silu_q8_vec<T, 1>(gp, op, scale, q, rows, inter, st); break;
      case 2: launch_silu_q8_vec<T, 2>(gp, op, scale, q, rows, inter, st); break;
      case 3: launch_silu_q8_vec<T, 3>(gp, op, scale, q, rows, inter, st); break;
      case 4: launch_silu_q8_vec<T, 4>(gp, op, scale, q, rows, inter, st); break;
      case 5: launch_silu_q8_vec<T, 5>(gp, op, scale, q, rows, inter, st); break;
      case 6: launch_silu_q8_vec<T, 6>(gp, op, scale, q, rows, inter, st); break;
      case 7: launch_silu_q8_vec<T, 7>(gp, op, scale, q, rows, inter, st); break;
      default: launch_silu_q8_vec<T, 8>(gp, op, scale, q, rows, inter, st); break;
    }
    return launch_status("silu_and_mul_q8");
  }
  silu_mul_q8_generic_kernel<T><<<dim3((unsigned)rows), 256, 0, st>>>(gp, op, scale, q, inter);
  return launch_status("silu_and_mul_q8(generic)");
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

extern "C" int nvf_silu_and_mul_q8(const void* gate_up, void* out, float* row_scale, int8_t* q_out, int64_t rows,
                                   int64_t inter, int dtype, void* stream) {
  using namespace nvf;
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "nvf_silu_and_mul_q8: bad dtype %d", dtype);
  if (rows < 0 || inter < 0 || (rows > 0 && inter > (INT64_MAX / 4) / rows))
    return fail(NVF_ERR_INVALID, "nvf_silu_and_mul_q8: bad shape rows=%lld inter=%lld", (long long)rows,
                (long long)inter);
  if (rows > INT32_MAX) return fail(NVF_ERR_INVALID, "nvf_silu_and_mul_q8: rows=%lld exceeds the grid", (long long)rows);
  if (rows == 0 || inter == 0) return NVF_OK;
  if (!gate_up || !row_scale || !q_out) return fail(NVF_ERR_INVALID, "nvf_silu_and_mul_q8: NULL pointer");
  int s = NVF_OK;
  NVF_DISPATCH_DTYPE(dtype, T, s = launch_silu_q8<T>(gate_up, out, row_scale, q_out, rows, inter, as_stream(stream)));
  return s;
}

// Drop-in: include/nanovllm/hip_ops.hpp:17 / src/hip_ops.hip:707-713.
extern "C" void hip_silu_and_mul(const float* gate_up, float* out, int rows, int intermediate) {
  if (rows <= 0 || intermediate <= 0) return;
  nvf::dropin_check(nvf_silu_and_mul(gate_up, out, rows, intermediate, NVF_F32, nullptr), "hip_silu_and_mul");
}
