// Qwen3 per-head QK-norm fused with NeoX RoPE, on q and k in one launch.
//
// Reference semantics:
//   qkv bias: src/model.cpp:768-772 -> add_bias_kernel (src/hip_ops.hip:366-371):
//            x[t, c] += bias[c] on q, k and v after the qkv projection (Qwen2.5);
//   QK-norm: src/model.cpp:774-775 -> hip_rms_norm with rows = T*heads,
//            hidden = head_dim (src/hip_ops.hip:373-393), before RoPE;
//   RoPE:    src/model.cpp:777-778 -> rope_kernel (src/hip_ops.hip:431-450):
//            a = float(pos[t]) * inv_freq[d]; (x1, x2) -> (x1 c - x2 s, x2 c + x1 s)
//            for the pair (d, d + head_dim/2).
//
// Design: one 256-thread workgroup per token, walking the token's q and k heads
// in passes of 256 / LPH heads with the next pass's loads issued before the
// current pass's math (a 256-thread two-pass workgroup measured faster than
// one sized for all 40 heads of Qwen3-8B).  The head_dim/2 (cos, sin) pairs
// of the token are computed once (precise cosf/sinf, the reference's own
// functions) into LDS and reused by every q and k head -- the reference
// recomputes them per head.  The data loads of the first pass are issued before
// that table is built, and q/k are streamed with non-temporal loads/stores.  A head is LPH = (head_dim/2)/N lanes; lane l
// holds the 16-byte vectors at d0 = l*N and d0 + head_dim/2, so every rotation
// pair is lane-local.  QK-norm reduces the head's sum of squares over those LPH
// lanes with DPP (group_sum) and keeps the normalised values in registers, so q
// and k are read once and written once: 2 passes instead of the reference's 8
// (norm q, norm k, rope q, rope k, each read + write).
#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

constexpr int kRopeThreads = 256;     // generic kernel
constexpr int kRopeVecThreads = 256;   // vector kernel: a token's heads in passes of 256 / LPH

// KV store fused in (STORE; nvf_qk_norm_rope_store_kv): the rotated k heads also go
// to k_cache row slots[t], and the token's v row to v_cache row slots[t] (cache rows
// [kv_heads * HD]; slot < 0 skips the token), exactly what nvf_store_kv does after
// the RoPE launch.  The v row is loaded with the heads and stored at the end.
struct KvStoreArgs {
  const void* v;
  int64_t v_stride;
  void* kc;
  void* vc;
  const int32_t* slots;
};

// BIAS: the fp32 qkv bias [q_heads*HD | kv_heads*HD | kv_heads*HD] is added to each
// head in fp32 as it is loaded (head h of the q-then-k walk at bias + h*HD, the v row
// at bias + (q_heads + kv_heads)*HD), so the biased values are never rounded to the
// storage type before the norm and rotation.  In fp32 storage this is the reference's
// add-bias pass followed by the rest, bit for bit.
template <typename T, int HD, bool NORM, bool STORE, bool BIAS>
__global__ __launch_bounds__(kRopeVecThreads) void qk_norm_rope_kernel(T* q, T* k, const int64_t* __restrict__ positions,
                                                                    const T* __restrict__ qw, const T* __restrict__ kw,
                                                                    const float* __restrict__ inv_freq, int q_heads,
                                                                    int kv_heads, int64_t q_stride, int64_t k_stride,
                                                                    float eps, KvStoreArgs kv,
                                                                    const float* __restrict__ bias) {
  constexpr int N = Pack<T>::N;
  constexpr int HALF = HD / 2;
  constexpr int LPH = HALF / N;                   // lanes per head
  static_assert(LPH >= 1 && LPH <= 32 && (LPH & (LPH - 1)) == 0, "lanes per head");

  __shared__ float cs_lds[HALF];
  __shared__ float sn_lds[HALF];
  const int64_t t = blockIdx.x;
  const int sub = threadIdx.x % LPH;
  const int d0 = sub * N;
  const int total_heads = q_heads + kv_heads;
  constexpr int hpp = kRopeVecThreads / LPH;  // heads per pass
  auto head_base = [&](int h) -> T* {
    return h < q_heads ? q + t * q_stride + (int64_t)h * HD : k + t * k_stride + (int64_t)(h - q_heads) * HD;
  };

  // The first pass's loads go out before the (cos, sin) table is built, so
  // the HBM latency overlaps the sincos work and the barrier.
  // the fused store: slot of this token; the v row's 16-byte chunks, kVPer per thread
  constexpr int kVPer = 2;  // up to 2 * 256 chunks: kv_heads * HD <= 4096 elements (host-checked)
  int32_t slot = -1;
  u32x4 vrow[kVPer];
  const int64_t row = (int64_t)kv_heads * HD;
  if constexpr (STORE) {
    slot = kv.slots[t];
    const T* vsrc = static_cast<const T*>(kv.v) + t * kv.v_stride;
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      const int64_t c = threadIdx.x + (int64_t)i * kRopeVecThreads;
      if (slot >= 0 && c * N < row) vrow[i] = ld16_nt(vsrc + c * N);
    }
  }

  int h = threadIdx.x / LPH;
  u32x4 a, b;
  float ba[N], bb[N];  // the head's bias at d0 and HALF + d0 (BIAS)
  auto load_bias = [&](int hh, float* x1b, float* x2b) {
    const float* bh = bias + (int64_t)hh * HD;
#pragma unroll
    for (int j = 0; j < N; j += 4) {
      const u32x4 u = ld16(bh + d0 + j), w = ld16(bh + HALF + d0 + j);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t ui = u[i], wi = w[i];
        x1b[j + i] = __builtin_bit_cast(float, ui);
        x2b[j + i] = __builtin_bit_cast(float, wi);
      }
    }
  };
  if (h < total_heads) {
    T* base = head_base(h);
    a = ld16_nt(base + d0);
    b = ld16_nt(base + HALF + d0);
    if constexpr (BIAS) load_bias(h, ba, bb);
  }
  if (threadIdx.x < HALF) {
    const float ang = (float)positions[t] * inv_freq[threadIdx.x];
    cs_lds[threadIdx.x] = cosf(ang);
    sn_lds[threadIdx.x] = sinf(ang);
  }
  float qg1[N], qg2[N], kg1[N], kg2[N];
  if constexpr (NORM) {
    Pack<T>::unpack(ld16(qw + d0), qg1);
    Pack<T>::unpack(ld16(qw + HALF + d0), qg2);
    Pack<T>::unpack(ld16(kw + d0), kg1);
    Pack<T>::unpack(ld16(kw + HALF + d0), kg2);
  }
  __syncthreads();
  float c[N], s[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    c[j] = cs_lds[d0 + j];
    s[j] = sn_lds[d0 + j];
  }

  for (; h < total_heads; h += hpp) {
    T* base = head_base(h);
    const bool is_q = h < q_heads;
    // software pipeline: the next pass's loads go out before this pass's math
    const int hn = h + hpp;
    u32x4 an, bn;
    float ban[N], bbn[N];
    if (hn < total_heads) {
      T* nb = head_base(hn);
      an = ld16_nt(nb + d0);
      bn = ld16_nt(nb + HALF + d0);
      if constexpr (BIAS) load_bias(hn, ban, bbn);
    }
    float x1[N], x2[N];
    Pack<T>::unpack(a, x1);
    Pack<T>::unpack(b, x2);
    if constexpr (BIAS) {
#pragma unroll
      for (int j = 0; j < N; ++j) {
        x1[j] += ba[j];
        x2[j] += bb[j];
      }
    }
    if constexpr (NORM) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < N; ++j) ss += x1[j] * x1[j] + x2[j] * x2[j];
      ss = group_sum<LPH>(ss);
      const float inv = rsqrtf(ss / (float)HD + eps);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        x1[j] = x1[j] * inv * (is_q ? qg1[j] : kg1[j]);
        x2[j] = x2[j] * inv * (is_q ? qg2[j] : kg2[j]);
      }
    }
    float y1[N], y2[N];
#pragma unroll
    for (int j = 0; j < N; ++j) {
      y1[j] = x1[j] * c[j] - x2[j] * s[j];
      y2[j] = x2[j] * c[j] + x1[j] * s[j];
    }
    const u32x4 p1 = Pack<T>::pack(y1), p2 = Pack<T>::pack(y2);
    st16_nt(base + d0, p1);
    st16_nt(base + HALF + d0, p2);
    if constexpr (STORE) {
      if (!is_q && slot >= 0) {
        T* dst = static_cast<T*>(kv.kc) + (int64_t)slot * row + (int64_t)(h - q_heads) * HD;
        st16(dst + d0, p1);
        st16(dst + HALF + d0, p2);
      }
    }
    a = an;
    b = bn;
    if constexpr (BIAS) {
#pragma unroll
      for (int j = 0; j < N; ++j) {
        ba[j] = ban[j];
        bb[j] = bbn[j];
      }
    }
  }
  if constexpr (STORE) {
    T* vdst = static_cast<T*>(kv.vc) + (int64_t)slot * row;
    const float* vb = bias + (int64_t)total_heads * HD;
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      const int64_t c = threadIdx.x + (int64_t)i * kRopeVecThreads;
      if (slot >= 0 && c * N < row) {
        u32x4 out = vrow[i];
        if constexpr (BIAS) {
          float x[N];
          Pack<T>::unpack(vrow[i], x);
#pragma unroll
          for (int j = 0; j < N; j += 4) {
            const u32x4 u = ld16(vb + c * N + j);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t ue = u[e];
              x[j + e] += __builtin_bit_cast(float, ue);
            }
          }
          out = Pack<T>::pack(x);
        }
        st16(vdst + c * N, out);
      }
    }
  }
}

// Any head_dim / stride / alignment: one wave per (token, head); lanes walk the
// rotation pairs.  Norm uses a wave-wide sum.
template <typename T, bool NORM>
__global__ __launch_bounds__(kRopeThreads) void qk_norm_rope_generic_kernel(
    T* q, T* k, const int64_t* __restrict__ positions, const T* __restrict__ qw, const T* __restrict__ kw,
    const float* __restrict__ inv_freq, int64_t tokens, int q_heads, int kv_heads, int head_dim, int64_t q_stride,
    int64_t k_stride, float eps, const float* __restrict__ bias) {
  const int total_heads = q_heads + kv_heads;
  const int64_t item = (int64_t)blockIdx.x * (kRopeThreads / kWave) + threadIdx.x / kWave;
  if (item >= tokens * total_heads) return;  // wave-uniform
  const int lane = threadIdx.x % kWave;
  const int64_t t = item / total_heads;
  const int h = (int)(item - t * total_heads);
  const bool is_q = h < q_heads;
  T* base = is_q ? q + t * q_stride + (int64_t)h * head_dim : k + t * k_stride + (int64_t)(h - q_heads) * head_dim;
  const T* gw = is_q ? qw : kw;
  const int half = head_dim / 2;
  // the optional fp32 qkv bias of this head (q heads then k heads, h * head_dim apart)
  const float* bh = bias ? bias + (int64_t)h * head_dim : nullptr;
  auto at = [&](int d) { return bh ? to_f32(base[d]) + bh[d] : to_f32(base[d]); };
  float inv = 1.f;
  if constexpr (NORM) {
    float ss = 0.f;
    for (int d = lane; d < head_dim; d += kWave) {
      const float v = at(d);
      ss += v * v;
    }
    ss = wave_sum(ss);
    inv = rsqrtf(ss / (float)head_dim + eps);
  }
  const float pos = (float)positions[t];
  for (int d = lane; d < half; d += kWave) {
    float x1 = at(d), x2 = at(d + half);
    if constexpr (NORM) {
      x1 = x1 * inv * to_f32(gw[d]);
      x2 = x2 * inv * to_f32(gw[d + half]);
    }
    const float a = pos * inv_freq[d];
    const float c = cosf(a), s = sinf(a);
    base[d] = from_f32<T>(x1 * c - x2 * s);
    base[d + half] = from_f32<T>(x2 * c + x1 * s);
  }
}

// x[r, c] += bias[c] (fp32 bias, one rounding to the storage type), rows with a
// stride: the reference's add_bias_kernel (src/hip_ops.hip:366-371), one thread per
// element.  The separate-op path of the fused entry and the typed nvf_add_bias.
template <typename T>
__global__ __launch_bounds__(kRopeThreads) void add_bias_kernel(T* x, const float* __restrict__ bias, int64_t rows,
                                                                int64_t cols, int64_t stride) {
  const int64_t i = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x;
  if (i >= rows * cols) return;
  const int64_t r = i / cols, c = i - r * cols;
  T* p = x + r * stride + c;
  *p = from_f32<T>(to_f32(*p) + bias[c]);
}

// KV store with the v bias added on the way (the fused entry's separate-op path):
// k_cache[slot] = k[t], v_cache[slot] = v[t] + v_bias; slot < 0 skips the token.
template <typename T>
__global__ __launch_bounds__(kRopeThreads) void store_kv_bias_kernel(const T* k, const T* v,
                                                                     const float* __restrict__ v_bias, T* kc, T* vc,
                                                                     const int32_t* __restrict__ slots, int64_t tokens,
                                                                     int64_t row, int64_t k_stride, int64_t v_stride) {
  const int64_t i = (int64_t)blockIdx.x * kRopeThreads + threadIdx.x;
  if (i >= tokens * row) return;
  const int64_t t = i / row, c = i - t * row;
  const int32_t slot = slots[t];
  if (slot < 0) return;
  kc[(int64_t)slot * row + c] = k[t * k_stride + c];
  vc[(int64_t)slot * row + c] = from_f32<T>(to_f32(v[t * v_stride + c]) + v_bias[c]);
}

template <typename T>
static int launch_add_bias(void* x, const float* bias, int64_t rows, int64_t cols, int64_t stride, hipStream_t st) {
  const int64_t n = rows * cols;
  add_bias_kernel<T><<<dim3((unsigned)((n + kRopeThreads - 1) / kRopeThreads)), kRopeThreads, 0, st>>>(
      static_cast<T*>(x), bias, rows, cols, stride);
  return launch_status("add_bias");
}

// kv != nullptr: launch the fused RoPE + KV store kernel (adding the qkv bias first when
// bias != nullptr) when the vector kernel takes the shape (returns 1 without launching
// otherwise: the caller then runs the separate ops)
template <typename T, bool NORM>
static int launch_rope(void* q, void* k, const int64_t* pos, const void* qw, const void* kw, const float* inv_freq,
                       int64_t tokens, int q_heads, int kv_heads, int head_dim, int64_t q_stride, int64_t k_stride,
                       float eps, hipStream_t st, const KvStoreArgs* kv = nullptr, const float* bias = nullptr) {
  constexpr int N = Pack<T>::N;
  T* qp = static_cast<T*>(q);
  T* kp = static_cast<T*>(k);
  const T* qwp = static_cast<const T*>(qw);
  const T* kwp = static_cast<const T*>(kw);
  bool vec_ok = (q_heads == 0 || (aligned16(q) && q_stride % N == 0)) &&
                (kv_heads == 0 || (aligned16(k) && k_stride % N == 0)) &&
                (!NORM || (aligned16(qw) && aligned16(kw)));
  if (kv) {
    const int64_t row = (int64_t)kv_heads * head_dim;
    vec_ok = vec_ok && kv_heads > 0 && aligned16(kv->v) && kv->v_stride % N == 0 && aligned16(kv->kc) &&
             aligned16(kv->vc) && row <= 2 * kRopeVecThreads * N && (!bias || aligned16(bias));
  }
  if (bias && !kv) vec_ok = false;  // the vector kernel adds the bias only with the store fused in
  if (vec_ok && (head_dim == 64 || head_dim == 128 || head_dim == 256)) {
    const dim3 grid((unsigned)tokens);
    const unsigned block = kRopeVecThreads;
    const KvStoreArgs none{};
#define NVF_ROPE_LAUNCH(HDV)                                                                                          \
  if (kv && bias)                                                                                                     \
    qk_norm_rope_kernel<T, HDV, NORM, true, true><<<grid, block, 0, st>>>(qp, kp, pos, qwp, kwp, inv_freq, q_heads,   \
                                                                           kv_heads, q_stride, k_stride, eps, *kv,  \
                                                                           bias);                                   \
  else if (kv)                                                                                                        \
    qk_norm_rope_kernel<T, HDV, NORM, true, false><<<grid, block, 0, st>>>(qp, kp, pos, qwp, kwp, inv_freq, q_heads,  \
                                                                            kv_heads, q_stride, k_stride, eps, *kv, \
                                                                            nullptr);                               \
  else                                                                                                                \
    qk_norm_rope_kernel<T, HDV, NORM, false, false><<<grid, block, 0, st>>>(qp, kp, pos, qwp, kwp, inv_freq,         \
                                                                             q_heads, kv_heads, q_stride, k_stride, \
                                                                             eps, none, nullptr)
    if (head_dim == 64) {
      NVF_ROPE_LAUNCH(64);
      return launch_status("qk_norm_rope");
    }
    if (head_dim == 128) {
      NVF_ROPE_LAUNCH(128);
      return launch_status("qk_norm_rope");
    }
    if (head_dim == 256) {
      NVF_ROPE_LAUNCH(256);
      return launch_status("qk_norm_rope");
    }
#undef NVF_ROPE_LAUNCH
  }
  if (kv) return 1;  // not launched: the caller runs RoPE and the store separately
  const int64_t items = tokens * (q_heads + kv_heads);
  const int per_block = kRopeThreads / kWave;
  const dim3 grid((unsigned)((items + per_block - 1) / per_block));
  qk_norm_rope_generic_kernel<T, NORM><<<grid, kRopeThreads, 0, st>>>(qp, kp, pos, qwp, kwp, inv_freq, tokens, q_heads,
                                                                      kv_heads, head_dim, q_stride, k_stride, eps,
                                                                      bias);
  return launch_status("qk_norm_rope(generic)");
}

}  // namespace nvf

namespace nvf {
// nvf_qk_norm_rope's checks and dispatch; with kv, the fused kernel (1: shape not
// taken by it, nothing launched)
static int rope_entry(const char* name, void* q, void* k, const int64_t* positions, const void* q_w, const void* k_w,
                      const float* inv_freq, int64_t tokens, int q_heads, int kv_heads, int head_dim,
                      int64_t q_stride, int64_t k_stride, float eps, int dtype, void* stream, const KvStoreArgs* kv,
                      const float* bias = nullptr) {
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "%s: bad dtype %d", name, dtype);
  if (tokens < 0 || q_heads < 0 || kv_heads < 0 || head_dim < 2 || tokens > INT32_MAX)
    return fail(NVF_ERR_INVALID, "%s: bad shape tokens=%lld q_heads=%d kv_heads=%d head_dim=%d", name,
                (long long)tokens, q_heads, kv_heads, head_dim);
  if (tokens == 0 || q_heads + kv_heads == 0) return NVF_OK;
  if ((q_heads > 0 && (!q || q_stride < (int64_t)q_heads * head_dim)) ||
      (kv_heads > 0 && (!k || k_stride < (int64_t)kv_heads * head_dim)))
    return fail(NVF_ERR_INVALID, "%s: NULL tensor or stride smaller than heads*head_dim", name);
  if (!positions || !inv_freq) return fail(NVF_ERR_INVALID, "%s: NULL positions or inv_freq", name);
  const bool norm = q_w || k_w;
  if (norm && ((q_heads > 0 && !q_w) || (kv_heads > 0 && !k_w)))
    return fail(NVF_ERR_INVALID, "%s: q_w and k_w must both be given (or both NULL)", name);
  int s = NVF_OK;
  hipStream_t st = as_stream(stream);
  if (norm)
    NVF_DISPATCH_DTYPE(dtype, T, s = (launch_rope<T, true>(q, k, positions, q_w, k_w, inv_freq, tokens, q_heads,
                                                           kv_heads, head_dim, q_stride, k_stride, eps, st, kv, bias)));
  else
    NVF_DISPATCH_DTYPE(dtype, T, s = (launch_rope<T, false>(q, k, positions, nullptr, nullptr, inv_freq, tokens,
                                                            q_heads, kv_heads, head_dim, q_stride, k_stride, eps, st,
                                                            kv, bias)));
  return s;
}
}  // namespace nvf

extern "C" int nvf_add_bias(void* x, const float* bias, int64_t rows, int64_t cols, int64_t stride, int dtype,
                            void* stream) {
  using namespace nvf;
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "nvf_add_bias: bad dtype %d", dtype);
  if (rows < 0 || cols < 0 || stride < cols) return fail(NVF_ERR_INVALID, "nvf_add_bias: bad shape");
  if (rows == 0 || cols == 0) return NVF_OK;
  if (!x || !bias) return fail(NVF_ERR_INVALID, "nvf_add_bias: NULL pointer");
  if ((rows * cols + kRopeThreads - 1) / kRopeThreads > INT32_MAX)
    return fail(NVF_ERR_INVALID, "nvf_add_bias: too many elements");
  int s = NVF_OK;
  NVF_DISPATCH_DTYPE(dtype, T, s = launch_add_bias<T>(x, bias, rows, cols, stride, as_stream(stream)));
  return s;
}

extern "C" int nvf_qk_norm_rope(void* q, void* k, const int64_t* positions, const void* q_w, const void* k_w,
                                const float* inv_freq, int64_t tokens, int q_heads, int kv_heads, int head_dim,
                                int64_t q_stride, int64_t k_stride, float eps, int dtype, void* stream) {
  return nvf::rope_entry("nvf_qk_norm_rope", q, k, positions, q_w, k_w, inv_freq, tokens, q_heads, kv_heads, head_dim,
                         q_stride, k_stride, eps, dtype, stream, nullptr);
}

extern "C" int nvf_qkv_bias_qk_norm_rope_store_kv(void* q, void* k, const void* v, const float* qkv_bias,
                                                  const int64_t* positions, const void* q_w, const void* k_w,
                                                  const float* inv_freq, int64_t tokens, int q_heads, int kv_heads,
                                                  int head_dim, int64_t q_stride, int64_t k_stride, int64_t v_stride,
                                                  float eps, void* k_cache, void* v_cache,
                                                  const int32_t* slot_mapping, int dtype, void* stream) {
  using namespace nvf;
  const char* name = qkv_bias ? "nvf_qkv_bias_qk_norm_rope_store_kv" : "nvf_qk_norm_rope_store_kv";
  if (kv_heads <= 0 || head_dim <= 0) return fail(NVF_ERR_INVALID, "%s: kv_heads=%d head_dim=%d", name, kv_heads, head_dim);
  if (v_stride < (int64_t)kv_heads * head_dim)
    return fail(NVF_ERR_INVALID, "%s: v_stride must be >= kv_heads * head_dim", name);
  if (tokens > 0 && (!v || !k_cache || !v_cache || !slot_mapping)) return fail(NVF_ERR_INVALID, "%s: NULL pointer", name);
  const KvStoreArgs kv{v, v_stride, k_cache, v_cache, slot_mapping};
  const int s = rope_entry(name, q, k, positions, q_w, k_w, inv_freq, tokens, q_heads, kv_heads, head_dim, q_stride,
                           k_stride, eps, dtype, stream, &kv, qkv_bias);
  if (s != 1) return s;
  // a shape the fused kernel does not take: the generic (bias +) QK-norm + RoPE kernel, then
  // the store (with the v bias added on the way into the cache)
  const int64_t qn = (int64_t)q_heads * head_dim, kn = (int64_t)kv_heads * head_dim;
  const int r = rope_entry(name, q, k, positions, q_w, k_w, inv_freq, tokens, q_heads, kv_heads, head_dim, q_stride,
                           k_stride, eps, dtype, stream, nullptr, qkv_bias);
  if (r != NVF_OK) return r;
  if (!qkv_bias)
    return nvf_store_kv(k, v, k_cache, v_cache, slot_mapping, tokens, kv_heads, head_dim, k_stride, v_stride, dtype,
                        stream);
  if ((tokens * kn + kRopeThreads - 1) / kRopeThreads > INT32_MAX)
    return fail(NVF_ERR_INVALID, "%s: too many elements", name);
  const dim3 grid((unsigned)((tokens * kn + kRopeThreads - 1) / kRopeThreads));
  NVF_DISPATCH_DTYPE(dtype, T,
                     (store_kv_bias_kernel<T><<<grid, kRopeThreads, 0, as_stream(stream)>>>(
                         static_cast<const T*>(k), static_cast<const T*>(v), qkv_bias + qn + kn,
                         static_cast<T*>(k_cache), static_cast<T*>(v_cache), slot_mapping, tokens, kn, k_stride,
                         v_stride)));
  return launch_status("store_kv(bias)");
}

extern "C" int nvf_qk_norm_rope_store_kv(void* q, void* k, const void* v, const int64_t* positions, const void* q_w,
                                         const void* k_w, const float* inv_freq, int64_t tokens, int q_heads,
                                         int kv_heads, int head_dim, int64_t q_stride, int64_t k_stride,
                                         int64_t v_stride, float eps, void* k_cache, void* v_cache,
                                         const int32_t* slot_mapping, int dtype, void* stream) {
  return nvf_qkv_bias_qk_norm_rope_store_kv(q, k, v, nullptr, positions, q_w, k_w, inv_freq, tokens, q_heads,
                                            kv_heads, head_dim, q_stride, k_stride, v_stride, eps, k_cache, v_cache,
                                            slot_mapping, dtype, stream);
}

extern "C" void hip_add_bias_inplace(float* x, const float* bias, int rows, int cols) {
  if (rows <= 0 || cols <= 0) return;
  nvf::dropin_check(nvf_add_bias(x, bias, rows, cols, cols, NVF_F32, nullptr), "hip_add_bias_inplace");
}

extern "C" void hip_rope_inplace(float* data, const int64_t* positions, int tokens, int heads, int head_dim,
                                 int64_t stride, const float* inv_freq) {
  if (tokens <= 0 || heads <= 0 || head_dim / 2 <= 0) return;
  nvf::dropin_check(nvf_qk_norm_rope(data, nullptr, positions, nullptr, nullptr, inv_freq, tokens, heads, 0, head_dim,
                                     stride, 0, 0.f, NVF_F32, nullptr),
                    "hip_rope_inplace");
}
