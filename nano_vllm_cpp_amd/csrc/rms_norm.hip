// Fused residual-add + RMSNorm and plain RMSNorm for gfx950.
//
// Reference semantics: src/hip_ops.hip:373-417 (rms_norm_kernel,
// rms_norm_add_kernel) -- residual <- x + residual is written back, then
// out = residual * rsqrt(sum(residual^2)/hidden + eps) * weight.
//
// Design: a row is split over WPR = 1, 2 or 4 wave64s of a 256-thread
// workgroup (4 / WPR rows per workgroup).  Each lane reads VPL 16-byte vectors
// of x and residual with non-temporal loads and keeps them in VGPRs, so x and
// residual cross HBM once and residual/out are written once (4 row passes
// instead of the reference's 5).  The sum of squares is reduced inside each
// wave with DPP row ops + one ds_swizzle (wave_sum), and the WPR partial sums
// of a row are combined through LDS in a fixed order, so every wave of the row
// computes the bit-identical 1/rms.  Vector i of lane l in wave w is
// (i * WPR + w) * 64 + l: each load/store instruction of a wave covers 1 KiB of
// contiguous row.  At Qwen2.5-7B prefill shape 4 waves per row measured ~77%
// of the 8 TB/s HBM peak against ~63% for one wave per row.
//
// nvf_rms_norm_q8 also emits what the reference's INT8 GEMM path computes in a
// separate pass over the normalised row (q8_row_scale_kernel,
// src/hip_ops.hip:205-217): the per-row scale 127 / max|out| from a DPP + LDS
// max reduction of the row already in registers, and optionally the int8 row
// its GEMM forms on the fly (:244-245).
#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

constexpr int kNormThreads = 256;
constexpr int kNormWaves = kNormThreads / kWave;
constexpr int kNormMaxVpl = kRmsMaxVpl;  // 16 x 4 waves x 64 lanes x 16 B = a 64 KiB row in registers

template <typename T, int VPL, int WPR, bool ADD, bool Q8>
__global__ __launch_bounds__(kNormThreads) void rms_norm_vec_kernel(const T* x, T* residual, const T* __restrict__ w,
                                                                    T* out, int64_t rows, int hidden, float eps,
                                                                    float* row_scale, int8_t* q_out) {
  constexpr int N = Pack<T>::N;
  constexpr int RPB = kNormWaves / WPR;  // rows per workgroup
  __shared__ float partial[kNormWaves];
  __shared__ float partial_max[kNormWaves];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int sub = wave % WPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + wave / WPR;
  const bool active = row < rows;  // no early return: the row's waves meet at a barrier
  const int nvec = hidden / N;
  const int64_t off = (active ? row : 0) * (int64_t)hidden;
  const T* xr = x + off;
  T* rr = residual + off;
  T* orow = out + off;

  u32x4 xa[VPL], ra[VPL], wa[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = (i * WPR + sub) * kWave + lane;
    if (active && c < nvec) {
      xa[i] = ld16_nt(xr + c * N);
      if constexpr (ADD) ra[i] = ld16_nt(rr + c * N);
      wa[i] = ld16(w + c * N);
    }
  }

  float v[VPL][N];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = (i * WPR + sub) * kWave + lane;
    if (active && c < nvec) {
      Pack<T>::unpack(xa[i], v[i]);
      if constexpr (ADD) {
        float r[N];
        Pack<T>::unpack(ra[i], r);
#pragma unroll
        for (int j = 0; j < N; ++j) v[i][j] += r[j];
        const u32x4 stored = Pack<T>::pack(v[i]);
        st16_nt(rr + c * N, stored);
        Pack<T>::unpack(stored, v[i]);  // the norm sees the stored (rounded) row
      }
#pragma unroll
      for (int j = 0; j < N; ++j) ss = fmaf(v[i][j], v[i][j], ss);
    }
  }
  ss = wave_sum(ss);
  if constexpr (WPR > 1) {
    if (lane == 0) partial[wave] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int k = 0; k < WPR; ++k) ss += partial[(wave / WPR) * WPR + k];
  }
  const float inv = rsqrtf(ss / (float)hidden + eps);

  float mx = 0.f;  // max |out| as stored, for the Q8 row scale
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = (i * WPR + sub) * kWave + lane;
    if (active && c < nvec) {
      float g[N], o[N];
      Pack<T>::unpack(wa[i], g);
#pragma unroll
      for (int j = 0; j < N; ++j) o[j] = v[i][j] * inv * g[j];
      const u32x4 stored = Pack<T>::pack(o);
      if (out) st16_nt(orow + c * N, stored);
      if constexpr (Q8) {
        Pack<T>::unpack(stored, v[i]);  // keep the stored values for the quantizer
#pragma unroll
        for (int j = 0; j < N; ++j) mx = fmaxf(mx, fabsf(v[i][j]));
      }
    }
  }
  if constexpr (Q8) {
    mx = wave_max(mx);
    if constexpr (WPR > 1) {
      if (lane == 0) partial_max[wave] = mx;
      __syncthreads();
      mx = 0.f;
#pragma unroll
      for (int k = 0; k < WPR; ++k) mx = fmaxf(mx, partial_max[(wave / WPR) * WPR + k]);
    }
    const float scale = q8_row_scale(mx);
    if (active && sub == 0 && lane == 0) row_scale[row] = scale;
    if (q_out) {
      int8_t* qrow = q_out + off;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = (i * WPR + sub) * kWave + lane;
        if (active && c < nvec) {
          uint32_t pk[N / 4];
#pragma unroll
          for (int w4 = 0; w4 < N / 4; ++w4) {
            uint32_t b = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) b |= ((uint32_t)q8_quantize(v[i][4 * w4 + k], scale) & 0xffu) << (8 * k);
            pk[w4] = b;
          }
          if constexpr (N == 8) {
            *reinterpret_cast<uint2*>(qrow + c * N) = make_uint2(pk[0], pk[1]);
          } else {
            *reinterpret_cast<uint32_t*>(qrow + c * N) = pk[0];
          }
        }
      }
    }
  }
}

// Any hidden / alignment: one wave per row, scalar two-pass (the second pass
// re-reads the row this lane wrote, an L2 hit); Q8 adds a third pass over the
// stored output for the int8 row.
template <typename T, bool ADD, bool Q8>
__global__ __launch_bounds__(kNormThreads) void rms_norm_generic_kernel(const T* x, T* residual, const T* w, T* out,
                                                                        int64_t rows, int hidden, float eps,
                                                                        float* row_scale, int8_t* q_out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * kNormWaves + (threadIdx.x / kWave);
  if (row >= rows) return;
  const int64_t off = row * (int64_t)hidden;
  float ss = 0.f;
  for (int c = lane; c < hidden; c += kWave) {
    float v = to_f32(x[off + c]);
    if constexpr (ADD) {
      const T s = from_f32<T>(v + to_f32(residual[off + c]));
      residual[off + c] = s;
      v = to_f32(s);
    }
    ss += v * v;
  }
  ss = wave_sum(ss);
  const float inv = rsqrtf(ss / (float)hidden + eps);
  float mx = 0.f;
  for (int c = lane; c < hidden; c += kWave) {
    const float v = ADD ? to_f32(residual[off + c]) : to_f32(x[off + c]);
    const T o = from_f32<T>(v * inv * to_f32(w[c]));
    if (out) out[off + c] = o;
    mx = fmaxf(mx, fabsf(to_f32(o)));
  }
  if constexpr (Q8) {
    const float scale = q8_row_scale(wave_max(mx));
    if (lane == 0) row_scale[row] = scale;
    if (q_out) {
      for (int c = lane; c < hidden; c += kWave) {  // recompute: out may be absent
        const float v = ADD ? to_f32(residual[off + c]) : to_f32(x[off + c]);
        const T o = from_f32<T>(v * inv * to_f32(w[c]));
        q_out[off + c] = (int8_t)q8_quantize(to_f32(o), scale);
      }
    }
  }
}

template <typename T, bool ADD, bool Q8>
static int launch_rms(const void* x, void* residual, const void* w, void* out, int64_t rows, int64_t hidden,
                      float eps, float* row_scale, int8_t* q_out, hipStream_t st) {
  constexpr int N = Pack<T>::N;
  const int64_t nvec = hidden / N;
  // waves per row: 4 once a row has >= 256 vectors, else fewer, so lanes stay busy
  const int wpr = rms_waves_per_row(nvec);
  const int vpl = (int)((nvec + (int64_t)wpr * kWave - 1) / ((int64_t)wpr * kWave));
  const bool vec_ok = hidden % N == 0 && vpl >= 1 && vpl <= (wpr == 4 ? kNormMaxVpl : 2) && aligned16(x) &&
                      aligned16(w) && (!out || aligned16(out)) && (!ADD || aligned16(residual)) &&
                      (!q_out || (reinterpret_cast<uintptr_t>(q_out) & (N - 1)) == 0);
  const dim3 block(kNormThreads);
  const T* xp = static_cast<const T*>(x);
  T* rp = static_cast<T*>(residual);
  const T* wp = static_cast<const T*>(w);
  T* op = static_cast<T*>(out);
  const int h = (int)hidden;
  if (!vec_ok) {
    const dim3 grid((unsigned)((rows + kNormWaves - 1) / kNormWaves));
    rms_norm_generic_kernel<T, ADD, Q8><<<grid, block, 0, st>>>(xp, rp, wp, op, rows, h, eps, row_scale, q_out);
    return launch_status("rms_norm(generic)");
  }
  const int rpb = kNormWaves / wpr;
  const dim3 grid((unsigned)((rows + rpb - 1) / rpb));
#define NVF_RMS_LAUNCH(V, W) \
  rms_norm_vec_kernel<T, V, W, ADD, Q8><<<grid, block, 0, st>>>(xp, rp, wp, op, rows, h, eps, row_scale, q_out)
  if (wpr == 1) {
    if (vpl == 1) NVF_RMS_LAUNCH(1, 1); else NVF_RMS_LAUNCH(2, 1);
  } else if (wpr == 2) {
    if (vpl == 1) NVF_RMS_LAUNCH(1, 2); else NVF_RMS_LAUNCH(2, 2);
  } else {
    switch (vpl) {
#define NVF_RMS_CASE(V) case V: NVF_RMS_LAUNCH(V, 4); break;
      NVF_RMS_CASE(1) NVF_RMS_CASE(2) NVF_RMS_CASE(3) NVF_RMS_CASE(4) NVF_RMS_CASE(5) NVF_RMS_CASE(6)
      NVF_RMS_CASE(7) NVF_RMS_CASE(8) NVF_RMS_CASE(9) NVF_RMS_CASE(10) NVF_RMS_CASE(11) NVF_RMS_CASE(12)
      NVF_RMS_CASE(13) NVF_RMS_CASE(14) NVF_RMS_CASE(15) NVF_RMS_CASE(16)
#undef NVF_RMS_CASE
    }
  }
#undef NVF_RMS_LAUNCH
  return launch_status("rms_norm");
}

static int rms_entry(const void* x, void* residual, const void* w, void* out, int64_t rows, int64_t hidden,
                     float eps, int dtype, void* stream, bool add, float* row_scale = nullptr,
                     int8_t* q_out = nullptr) {
  const bool q8 = row_scale != nullptr;
  const char* name = q8 ? "nvf_rms_norm_q8" : (add ? "nvf_rms_norm_add" : "nvf_rms_norm");
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "%s: bad dtype %d", name, dtype);
  if (rows < 0 || hidden < 0 || hidden > INT32_MAX)
    return fail(NVF_ERR_INVALID, "%s: bad shape rows=%lld hidden=%lld", name, (long long)rows, (long long)hidden);
  if (rows == 0 || hidden == 0) return NVF_OK;
  if (!x || !w || (!out && !q8) || (add && !residual)) return fail(NVF_ERR_INVALID, "%s: NULL pointer", name);
  if (q8 && !out && !q_out) return fail(NVF_ERR_INVALID, "%s: neither out nor q_out given", name);
  if ((int64_t)((rows + kNormWaves - 1) / kNormWaves) > INT32_MAX)
    return fail(NVF_ERR_INVALID, "%s: %lld rows exceed one launch", name, (long long)rows);
  int st = NVF_OK;
  const hipStream_t s = as_stream(stream);
#define NVF_RMS_GO(A, Q) NVF_DISPATCH_DTYPE(dtype, T, st = (launch_rms<T, A, Q>(x, residual, w, out, rows, hidden, eps, row_scale, q_out, s)))
  if (add && q8) NVF_RMS_GO(true, true);
  else if (add) NVF_RMS_GO(true, false);
  else if (q8) NVF_RMS_GO(false, true);
  else NVF_RMS_GO(false, false);
#undef NVF_RMS_GO
  return st;
}

}  // namespace nvf

extern "C" int nvf_rms_norm_add(const void* x, void* residual, const void* weight, void* out, int64_t rows,
                                int64_t hidden, float eps, int dtype, void* stream) {
  return nvf::rms_entry(x, residual, weight, out, rows, hidden, eps, dtype, stream, true);
}

extern "C" int nvf_rms_norm(const void* x, const void* weight, void* out, int64_t rows, int64_t hidden, float eps,
                            int dtype, void* stream) {
  return nvf::rms_entry(x, nullptr, weight, out, rows, hidden, eps, dtype, stream, false);
}

extern "C" int nvf_rms_norm_q8(const void* x, void* residual, const void* weight, void* out, float* row_scale,
                               int8_t* q_out, int64_t rows, int64_t hidden, float eps, int dtype, void* stream) {
  if (!row_scale) return nvf::fail(NVF_ERR_INVALID, "nvf_rms_norm_q8: NULL row_scale");
  return nvf::rms_entry(x, residual, weight, out, rows, hidden, eps, dtype, stream, residual != nullptr, row_scale,
                        q_out);
}

// Drop-in: include/nanovllm/hip_ops.hpp:14 / src/hip_ops.hip:694-698.
extern "C" void hip_rms_norm(const float* x, const float* weight, float* out, int rows, int hidden, float eps) {
  if (rows <= 0 || hidden <= 0) return;
  nvf::dropin_check(nvf::rms_entry(x, nullptr, weight, out, rows, hidden, eps, NVF_F32, nullptr, false),
                    "hip_rms_norm");
}

// Drop-in: include/nanovllm/hip_ops.hpp:15 / src/hip_ops.hip:700-705.
extern "C" void hip_rms_norm_add(const float* x, float* residual, const float* weight, float* out, int rows,
                                 int hidden, float eps) {
  if (rows <= 0 || hidden <= 0) return;
  nvf::dropin_check(nvf::rms_entry(x, residual, weight, out, rows, hidden, eps, NVF_F32, nullptr, true),
                    "hip_rms_norm_add");
}
