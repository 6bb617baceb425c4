// KV-cache store and paged attention.
//
// Reference: store_kv_kernel (src/hip_ops.hip:452-466) and paged_attention_kernel
// (:468-550), called per layer from src/model.cpp:780-784.  The cache is
// [num_blocks * block_size, kv_heads, head_dim]; query token t of sequence
// query_seq[t] attends its first query_key_len[t] keys (causal prefill: its
// position + 1; decode: the whole context), key j at cache row
// block_tables[seq * max_blocks + j / block_size] * block_size + j % block_size;
// query head h reads kv head h / (q_heads / kv_heads).
//
// Kernels:
// * store_kv: one 16-byte chunk per lane, slot < 0 skipped.
// * attn_wave_kernel: one wave per (token, head), any head_dim <= 256 and any
//   dtype: scores 64 keys at a time (a lane per key, 16-byte K loads when
//   aligned), an online softmax over the chunks, P . V with the lane owning
//   head dimensions.  fp32 math; it serves the fp32 drop-in and the shapes the
//   tiled kernel does not take.
#include <hip/hip_runtime.h>

#include <math.h>

#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

constexpr int kAttnWaves = 4;

// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void store_kv_vec_kernel(const T* __restrict__ key, const T* __restrict__ value,
                                                           T* __restrict__ kc, T* __restrict__ vc,
                                                           const int32_t* __restrict__ slots, int64_t tokens,
                                                           int64_t chunks_per_row, int64_t key_stride,
                                                           int64_t value_stride) {
  constexpr int N = Pack<T>::N;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= tokens * chunks_per_row) return;
  const int64_t t = i / chunks_per_row, c = i - t * chunks_per_row;
  const int32_t slot = slots[t];
  if (slot < 0) return;
  const int64_t row = chunks_per_row * N;
  st16(kc + (int64_t)slot * row + c * N, ld16_nt(key + t * key_stride + c * N));
  st16(vc + (int64_t)slot * row + c * N, ld16_nt(value + t * value_stride + c * N));
}

template <typename T>
__global__ __launch_bounds__(256) void store_kv_generic_kernel(const T* __restrict__ key, const T* __restrict__ value,
                                                               T* __restrict__ kc, T* __restrict__ vc,
                                                               const int32_t* __restrict__ slots, int64_t tokens,
                                                               int64_t row, int64_t key_stride, int64_t value_stride) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= tokens * row) return;
  const int64_t t = i / row, c = i - t * row;
  const int32_t slot = slots[t];
  if (slot < 0) return;
  kc[(int64_t)slot * row + c] = key[t * key_stride + c];
  vc[(int64_t)slot * row + c] = value[t * value_stride + c];
}

// ---------------------------------------------------------------------------
// One wave per (token, head).  DPL = head dimensions per lane (head_dim <= 64 DPL).
template <typename T, int DPL, bool VEC>
__global__ __launch_bounds__(kAttnWaves * 64) void attn_wave_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kc, const T* __restrict__ vc,
    const int32_t* __restrict__ qseq, const int32_t* __restrict__ qlen, const int32_t* __restrict__ tables,
    int64_t tokens, int q_heads, int kv_heads, int hd, int bs, int max_blocks, float scale, int64_t q_stride) {
  constexpr int N = Pack<T>::N;
  __shared__ float q_sh[kAttnWaves][64 * DPL];
  __shared__ float p_sh[kAttnWaves][64];
  __shared__ int64_t row_sh[kAttnWaves][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t gw = (int64_t)blockIdx.x * kAttnWaves + w;
  if (gw >= tokens * q_heads) return;  // whole waves only; no workgroup barrier below
  const int64_t t = gw / q_heads;
  const int h = (int)(gw - t * q_heads);
  const int kvh = h / (q_heads / kv_heads);
  const int L = qlen[t];
  T* o = out + (t * q_heads + h) * hd;
  if (L <= 0) {  // the reference writes zeros (:488-491)
    for (int d = lane; d < hd; d += 64) o[d] = from_f32<T>(0.0f);
    return;
  }
  const int64_t seq = qseq[t];
  const T* qp = q + t * q_stride + (int64_t)h * hd;
  for (int d = lane; d < 64 * DPL; d += 64) q_sh[w][d] = d < hd ? to_f32(qp[d]) : 0.0f;
  __builtin_amdgcn_wave_barrier();  // wave-private LDS: other lanes read what this wave wrote
  const int64_t kv_stride = (int64_t)kv_heads * hd;
  const int32_t* tab = tables + seq * max_blocks;

  float m = -1e30f, s = 0.0f, acc[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) acc[i] = 0.0f;
  for (int k0 = 0; k0 < L; k0 += 64) {
    const int n = L - k0 < 64 ? L - k0 : 64;
    float sc = -1e30f;
    if (lane < n) {
      const int key = k0 + lane;
      const int64_t row = (int64_t)tab[key / bs] * bs + key % bs;
      row_sh[w][lane] = row;
      const T* kp = kc + row * kv_stride + (int64_t)kvh * hd;
      float dot = 0.0f;
      if constexpr (VEC) {
        for (int d0 = 0; d0 < hd; d0 += N) {
          float kv[N];
          Pack<T>::unpack(ld16(kp + d0), kv);
#pragma unroll
          for (int e = 0; e < N; ++e) dot = fmaf(q_sh[w][d0 + e], kv[e], dot);
        }
      } else {
        for (int d = 0; d < hd; ++d) dot = fmaf(q_sh[w][d], to_f32(kp[d]), dot);
      }
      sc = dot * scale;
    }
    const float cmax = wave_max(sc);
    const float new_m = fmaxf(m, cmax);
    const float p = lane < n ? expf(sc - new_m) : 0.0f;
    const float alpha = expf(m - new_m);
    s = s * alpha + wave_sum(p);
    p_sh[w][lane] = p;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] *= alpha;
    for (int j = 0; j < n; ++j) {
      const float pj = p_sh[w][j];
      const T* vp = vc + row_sh[w][j] * kv_stride + (int64_t)kvh * hd;
#pragma unroll
      for (int i = 0; i < DPL; ++i) {
        const int d = lane + 64 * i;
        if (d < hd) acc[i] = fmaf(pj, to_f32(vp[d]), acc[i]);
      }
    }
    m = new_m;
    __builtin_amdgcn_wave_barrier();  // the chunk's p_sh / row_sh reads finish before the next writes
  }
  const float inv = s > 0.0f ? 1.0f / s : 0.0f;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const int d = lane + 64 * i;
    if (d < hd) o[d] = from_f32<T>(acc[i] * inv);
  }
}

template <typename T, int DPL>
void launch_attn_wave(const void* q, void* out, const void* kc, const void* vc, const int32_t* qseq,
                      const int32_t* qlen, const int32_t* tables, int64_t tokens, int q_heads, int kv_heads, int hd,
                      int bs, int max_blocks, float scale, int64_t q_stride, bool vec, hipStream_t st) {
  const int64_t waves = tokens * q_heads;
  const dim3 grid((unsigned)((waves + kAttnWaves - 1) / kAttnWaves)), block(kAttnWaves * 64);
  const T* qt = static_cast<const T*>(q);
  T* ot = static_cast<T*>(out);
  const T* kt = static_cast<const T*>(kc);
  const T* vt = static_cast<const T*>(vc);
  if (vec) {
    attn_wave_kernel<T, DPL, true><<<grid, block, 0, st>>>(qt, ot, kt, vt, qseq, qlen, tables, tokens, q_heads,
                                                           kv_heads, hd, bs, max_blocks, scale, q_stride);
  } else {
    attn_wave_kernel<T, DPL, false><<<grid, block, 0, st>>>(qt, ot, kt, vt, qseq, qlen, tables, tokens, q_heads,
                                                            kv_heads, hd, bs, max_blocks, scale, q_stride);
  }
}

template <typename T>
int attention_generic(const void* q, void* out, const void* kc, const void* vc, const int32_t* qseq,
                      const int32_t* qlen, const int32_t* tables, int64_t tokens, int q_heads, int kv_heads, int hd,
                      int bs, int max_blocks, float scale, int64_t q_stride, hipStream_t st) {
  constexpr int N = Pack<T>::N;
  const bool vec = hd % N == 0 && aligned16(kc) && ((int64_t)kv_heads * hd) % N == 0;
  const int dpl = (hd + 63) / 64;
  switch (dpl) {
    case 1: launch_attn_wave<T, 1>(q, out, kc, vc, qseq, qlen, tables, tokens, q_heads, kv_heads, hd, bs, max_blocks,
                                   scale, q_stride, vec, st); break;
    case 2: launch_attn_wave<T, 2>(q, out, kc, vc, qseq, qlen, tables, tokens, q_heads, kv_heads, hd, bs, max_blocks,
                                   scale, q_stride, vec, st); break;
    case 3: launch_attn_wave<T, 3>(q, out, kc, vc, qseq, qlen, tables, tokens, q_heads, kv_heads, hd, bs, max_blocks,
                                   scale, q_stride, vec, st); break;
    default: launch_attn_wave<T, 4>(q, out, kc, vc, qseq, qlen, tables, tokens, q_heads, kv_heads, hd, bs,
                                    max_blocks, scale, q_stride, vec, st); break;
  }
  return launch_status("paged_attention");
}

template <typename T>
int store_kv_typed(const void* key, const void* value, void* kc, void* vc, const int32_t* slots, int64_t tokens,
                   int64_t row, int64_t key_stride, int64_t value_stride, hipStream_t st) {
  constexpr int N = Pack<T>::N;
  const T* k = static_cast<const T*>(key);
  const T* v = static_cast<const T*>(value);
  T* kt = static_cast<T*>(kc);
  T* vt = static_cast<T*>(vc);
  const bool vec = row % N == 0 && key_stride % N == 0 && value_stride % N == 0 && aligned16(key) &&
                   aligned16(value) && aligned16(kc) && aligned16(vc);
  if (vec) {
    const int64_t total = tokens * (row / N);
    store_kv_vec_kernel<T><<<dim3((unsigned)((total + 255) / 256)), 256, 0, st>>>(k, v, kt, vt, slots, tokens,
                                                                                 row / N, key_stride, value_stride);
  } else {
    const int64_t total = tokens * row;
    store_kv_generic_kernel<T><<<dim3((unsigned)((total + 255) / 256)), 256, 0, st>>>(k, v, kt, vt, slots, tokens,
                                                                                     row, key_stride, value_stride);
  }
  return launch_status("store_kv");
}

}  // namespace nvf

using namespace nvf;

extern "C" {

int nvf_store_kv(const void* key, const void* value, void* k_cache, void* v_cache, const int32_t* slot_mapping,
                 int64_t tokens, int kv_heads, int head_dim, int64_t key_stride, int64_t value_stride, int dtype,
                 void* stream) {
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "nvf_store_kv: bad dtype %d", dtype);
  if (tokens < 0 || kv_heads <= 0 || head_dim <= 0)
    return fail(NVF_ERR_INVALID, "nvf_store_kv: bad shape tokens=%lld kv_heads=%d head_dim=%d", (long long)tokens,
                kv_heads, head_dim);
  const int64_t row = (int64_t)kv_heads * head_dim;
  if (key_stride < row || value_stride < row)
    return fail(NVF_ERR_INVALID, "nvf_store_kv: strides must be >= kv_heads * head_dim");
  if (tokens == 0) return NVF_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) return fail(NVF_ERR_INVALID, "nvf_store_kv: NULL pointer");
  if ((tokens * row + 255) / 256 > INT32_MAX) return fail(NVF_ERR_INVALID, "nvf_store_kv: too many elements");
  int rc = NVF_OK;
  NVF_DISPATCH_DTYPE(dtype, T, rc = store_kv_typed<T>(key, value, k_cache, v_cache, slot_mapping, tokens, row,
                                                      key_stride, value_stride, as_stream(stream)));
  return rc;
}

int nvf_paged_attention(const void* q, void* out, const void* k_cache, const void* v_cache, const int32_t* query_seq,
                        const int32_t* query_key_len, const int32_t* block_tables, int64_t tokens, int q_heads,
                        int kv_heads, int head_dim, int block_size, int max_blocks, float scale, int64_t q_stride,
                        int dtype, void* stream) {
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "nvf_paged_attention: bad dtype %d", dtype);
  if (tokens < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || max_blocks <= 0)
    return fail(NVF_ERR_INVALID, "nvf_paged_attention: bad shape");
  if (q_heads % kv_heads != 0)
    return fail(NVF_ERR_INVALID, "nvf_paged_attention: q_heads=%d is not a multiple of kv_heads=%d", q_heads, kv_heads);
  if (head_dim > 256) return fail(NVF_ERR_INVALID, "nvf_paged_attention: head_dim=%d exceeds 256", head_dim);
  if (q_stride < (int64_t)q_heads * head_dim)
    return fail(NVF_ERR_INVALID, "nvf_paged_attention: q_stride must be >= q_heads * head_dim");
  if (tokens == 0) return NVF_OK;
  if (!q || !out || !k_cache || !v_cache || !query_seq || !query_key_len || !block_tables)
    return fail(NVF_ERR_INVALID, "nvf_paged_attention: NULL pointer");
  if ((tokens * q_heads + kAttnWaves - 1) / kAttnWaves > INT32_MAX)
    return fail(NVF_ERR_INVALID, "nvf_paged_attention: too many (token, head) pairs");
  int rc = NVF_OK;
  NVF_DISPATCH_DTYPE(dtype, T, rc = attention_generic<T>(q, out, k_cache, v_cache, query_seq, query_key_len,
                                                         block_tables, tokens, q_heads, kv_heads, head_dim, block_size,
                                                         max_blocks, scale, q_stride, as_stream(stream)));
  return rc;
}

// Drop-ins: include/nanovllm/hip_ops.hpp:22-28 / src/hip_ops.hip:724-744 (fp32 cache, null stream).
void hip_store_kv(const float* key, const float* value, float* k_cache, float* v_cache, const int32_t* slot_mapping,
                  int tokens, int kv_heads, int head_dim) {
  if (tokens <= 0 || kv_heads <= 0 || head_dim <= 0) return;
  const int64_t row = (int64_t)kv_heads * head_dim;
  dropin_check(nvf_store_kv(key, value, k_cache, v_cache, slot_mapping, tokens, kv_heads, head_dim, row, row, NVF_F32,
                            nullptr),
               "hip_store_kv");
}

void hip_paged_attention(const float* q, float* out, const float* k_cache, const float* v_cache,
                         const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                         int tokens, int q_heads, int kv_heads, int head_dim, int block_size, int max_blocks,
                         float scale) {
  if (tokens <= 0 || q_heads <= 0 || kv_heads <= 0) return;
  dropin_check(nvf_paged_attention(q, out, k_cache, v_cache, query_seq, query_key_len, block_tables, tokens, q_heads,
                                   kv_heads, head_dim, block_size, max_blocks, scale, (int64_t)q_heads * head_dim,
                                   NVF_F32, nullptr),
               "hip_paged_attention");
}

}  // extern "C"
