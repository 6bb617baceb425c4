// GEMM on fp32 / fp16 / bf16 and K-quant (Q4_K, Q5_K, Q6_K) weights on the fp32
// matrix cores: out[r][c] = sum_i x[r][i] * w(c, i), the weights decoded exactly to
// fp32 as they are staged.
//
// Reference: hip_matmul (matmul_kernel<float>, src/hip_ops.hip:43-64), hip_matmul_u16
// (matmul_kernel<uint16_t>: fp16/bf16 weights widened exactly) and hip_matmul_qk
// (matmul_qk_kernel :577-598 over qk_w :184-193, launcher :770-777).  matmul_dispatch
// (src/model.cpp:665-686) calls them for every weight that is not Q8_0, and for the
// LM head (:839-846).  The reference takes 16x16 fp32 tiles, one output per thread,
// fp32 sums in k order; weights w(c, i) = element c*k + i of the flat weight array
// (row-major [n][k]; K-quant superblocks cover 256 consecutive elements).
//
// Design for gfx950: the fp32 matrix-core tile kernel of gemm_tile.hpp for m > 16
// (m <= 32 takes 32-row tiles, so a small m does not multiply the matrix-core work),
// and the weight-streaming decode products below for m <= 16.  The sums are fp32
// in a different order from the reference's, so results agree within the
// recursive-summation bound the tests state.

#include "nvf_device.hpp"
#include "nvf_host.hpp"
#include "gemm_tile.hpp"

namespace nvf {

// ---------------------------------------------------------------------------
// 32-element group sources for the decode products: one lane decodes a whole
// 32-element group of a K-quant superblock per load (e0 % 32 == 0), so the
// superblock header and the group's scale / min are read and decoded once per 32
// values instead of once per 8.  Values are bit-identical to Q4K / Q5K / Q6K
// (weight_formats.hpp): the same formulas on the same bytes.

// a & 0x0f0f0f0f kept as one instruction: the byte-wise conversions that follow
// (v_cvt_f32_ubyte0..3) then take the masked bytes directly, where the compiler
// would otherwise fold a variable shift and the mask into a bit-field extract per
// nibble
__device__ __forceinline__ uint32_t low_nibbles(uint32_t a) {
  uint32_t r;
  asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(a));
  return r;
}

template <int LAYOUT>
struct Q4KGroup {  // GGML: group j = bytes 32 (j / 2) .. +32, nibble j % 2; HIP_LEGACY: bytes 16 j .. +16, both nibbles
  const uint8_t* wq;
  static constexpr int kQ = LAYOUT == NVF_QK_LAYOUT_GGML ? 8 : 4;
  struct Raw {
    u32x4 hdr;
    uint32_t q[kQ];
    int j;
  };
  __device__ __forceinline__ Raw load(int64_t e0) const {
    const uint8_t* blk = wq + (e0 >> 8) * 144;
    Raw r;
    r.j = (int)((e0 & 255) >> 5);
    r.hdr = ld16(blk);
    if constexpr (LAYOUT == NVF_QK_LAYOUT_GGML) {
      const u32x4 a = ld16(blk + 16 + 32 * (r.j >> 1)), b = ld16(blk + 32 + 32 * (r.j >> 1));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r.q[i] = a[i];
        r.q[4 + i] = b[i];
      }
    } else {
      const u32x4 a = ld16(blk + 16 + 16 * r.j);
#pragma unroll
      for (int i = 0; i < 4; ++i) r.q[i] = a[i];
    }
    return r;
  }
  __device__ __forceinline__ void decode(const Raw& r, float* v) const {
    uint32_t sc, mn;
    q4k_sm(r.hdr[1], r.hdr[2], r.hdr[3], r.j, sc, mn);
    const float s = half_bits_to_f32(r.hdr[0] & 0xffffu) * (float)sc;
    const float m = half_bits_to_f32(r.hdr[0] >> 16) * (float)mn;
    if constexpr (LAYOUT == NVF_QK_LAYOUT_GGML) {
      const int sh = (r.j & 1) * 4;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t w = low_nibbles(r.q[i] >> sh);
#pragma unroll
        for (int k = 0; k < 4; ++k) v[4 * i + k] = s * (float)byte_of(w, k) - m;
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w = (r.q[i] >> (4 * h)) & 0x0f0f0f0fu;
#pragma unroll
          for (int k = 0; k < 4; ++k) v[16 * h + 4 * i + k] = s * (float)byte_of(w, k) - m;
        }
    }
  }
};

struct Q5KGroup {  // group j = 2 g + s: low bits nibble s of ql[32 g .. +32], bit 4 = bit j of qh[0 .. 32]
  const uint8_t* wq;
  struct Raw {
    u32x4 hdr;
    uint32_t ql[8], qh[8];
    int j;
  };
  __device__ __forceinline__ Raw load(int64_t e0) const {
    const uint8_t* blk = wq + (e0 >> 8) * 176;
    Raw r;
    r.j = (int)((e0 & 255) >> 5);
    r.hdr = ld16(blk);
    const u32x4 a = ld16(blk + 48 + 32 * (r.j >> 1)), b = ld16(blk + 64 + 32 * (r.j >> 1));
    const u32x4 c = ld16(blk + 16), d = ld16(blk + 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.ql[i] = a[i];
      r.ql[4 + i] = b[i];
      r.qh[i] = c[i];
      r.qh[4 + i] = d[i];
    }
    return r;
  }
  __device__ __forceinline__ void decode(const Raw& r, float* v) const {
    uint32_t sc, mn;
    q4k_sm(r.hdr[1], r.hdr[2], r.hdr[3], r.j, sc, mn);
    const float s = half_bits_to_f32(r.hdr[0] & 0xffffu) * (float)sc;
    const float m = half_bits_to_f32(r.hdr[0] >> 16) * (float)mn;
    const int sh = (r.j & 1) * 4;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w = low_nibbles(r.ql[i] >> sh) | (((r.qh[i] >> r.j) & 0x01010101u) << 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * i + k] = s * (float)byte_of(w, k) - m;
    }
  }
};

struct Q6KGroup {  // elements 128 h + 32 s + l: ql[64 h + 32 (s & 1) + l] nibble s / 2, qh[32 h + l] bits 2 s;
                   // scales sc[8 h + 2 s + l / 16]; 2-byte aligned superblocks
  const uint8_t* wq;
  struct Raw {
    uint32_t ql[8], qh[8];
    uint32_t sd;  // two int8 scales | fp16 d << 16
    int slot;
  };
  __device__ __forceinline__ Raw load(int64_t e0) const {
    const uint8_t* blk = wq + (e0 >> 8) * 210;
    Raw r;
    const int i = (int)(e0 & 255), h = i >> 7;
    r.slot = (i & 127) >> 5;
    load_a2<32>(blk + 64 * h + 32 * (r.slot & 1), r.ql);
    load_a2<32>(blk + 128 + 32 * h, r.qh);
    r.sd = (uint32_t)*reinterpret_cast<const uint16_t*>(blk + 192 + 8 * h + 2 * r.slot) |
           ((uint32_t)*reinterpret_cast<const uint16_t*>(blk + 208) << 16);
    return r;
  }
  __device__ __forceinline__ void decode(const Raw& r, float* v) const {
    const int lsh = (r.slot >> 1) * 4, hsh = 2 * r.slot;
    const float d = half_bits_to_f32(r.sd >> 16);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const float ds = d * (float)(int8_t)((r.sd >> (8 * half)) & 0xffu);  // (d * sc) first, as the reference
#pragma unroll
      for (int i = 4 * half; i < 4 * half + 4; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int q = (int)(((byte_of(r.ql[i], k) >> lsh) & 0xfu) | (((byte_of(r.qh[i], k) >> hsh) & 3u) << 4));
          v[4 * i + k] = ds * (float)(q - 32);
        }
    }
  }
};

template <int L>
struct RunOf<Q4KGroup<L>> {
  static constexpr int value = 32;
};
template <>
struct RunOf<Q5KGroup> {
  static constexpr int value = 32;
};
template <>
struct RunOf<Q6KGroup> {
  static constexpr int value = 32;
};
template <>
struct GemvPrefetch<Q6KGroup> {
  static constexpr bool value = false;
};

// ---------------------------------------------------------------------------
// Decode-shaped products (m <= 16 rows, k a multiple of the run below): bound by streaming the
// weights once from HBM.  Every fp32 matrix-core shape consumes at most 64 weight
// elements per 32 cycles per SIMD (8 per clock per CU), below what HBM delivers
// for K-quant weights (~23 elements per clock per CU for Q4_K), so the smallest
// batches use plain FMAs.  The 4 waves of a workgroup split K (contiguous ranges
// of steps) and meet in LDS, summed in wave order.  The activations are read from
// global memory (L2-resident: every workgroup reads the same m rows).  A lane
// takes runs of R = 8 consecutive weights (dense rows) or R = 32 (one K-quant
// group: header and scale decoded once per run).
//
// m <= 2: gemv_fma_kernel (gemm_tile.hpp, plain FMAs) with the plain problem policy.
//
// 2 < m <= 16: gemv_mfma_kernel (gemm_tile.hpp, v_mfma_f32_16x16x4_f32) with the
// plain problem policy.
constexpr int kGemvRows = 16;

// Column sets / groups per wave: 4 (dense) or 2 (K-quants, larger runs) when that
// leaves >= ~1000 workgroups, fewer for narrow outputs.
template <typename TX, typename Src, int MR, typename TO>
int launch_gemv_fma(const TX* x, const Src& src, TO* out, int64_t m, int64_t n, int64_t k, hipStream_t st) {
  constexpr int CPS = RunOf<Src>::value == 8 ? 4 : 8;
  constexpr int CMAX = RunOf<Src>::value == 8 ? 4 : 2;
  const dim3 blk(kGvWaves * 64);
  auto grid = [&](int cols) { return dim3((unsigned)((n + cols - 1) / cols)); };
  // wide outputs: each wave walks the whole K of its own columns (S = 1); narrow
  // ones split K over the 4 waves to fill the GPU
  const PlainGemvProb<TO> prob{out, m, n, k};
  if (RunOf<Src>::value == 8 && n >= (int64_t)CPS * CMAX * kGvWaves * 1024)  // dense rows, 1 KB per load
    gemv_fma_kernel<TX, Src, MR, 2, 1, PlainGemvProb<TO>, 64><<<grid(2 * kGvWaves), blk, 0, st>>>(x, src, prob, k);
  else if (n >= (int64_t)CPS * CMAX * kGvWaves * 1024)
    gemv_fma_kernel<TX, Src, MR, CMAX, 1><<<grid(CPS * CMAX * kGvWaves), blk, 0, st>>>(x, src, prob, k);
  else if (RunOf<Src>::value == 8 && n >= (int64_t)CPS * CMAX * 1024)
    gemv_fma_kernel<TX, Src, MR, 2, 4, PlainGemvProb<TO>, 64><<<grid(2), blk, 0, st>>>(x, src, prob, k);
  else if (n >= (int64_t)CPS * CMAX * 1024)
    gemv_fma_kernel<TX, Src, MR, CMAX, 4><<<grid(CPS * CMAX), blk, 0, st>>>(x, src, prob, k);
  else
    gemv_fma_kernel<TX, Src, MR, 1, 4><<<grid(CPS), blk, 0, st>>>(x, src, prob, k);
  return launch_status("dense_gemv_fma");
}

template <typename TX, typename Src, typename TO>
int launch_gemv_mfma(const TX* x, const Src& src, TO* out, int64_t m, int64_t n, int64_t k, hipStream_t st) {
  const dim3 blk(kGvWaves * 64);
  const PlainGemvProb<TO> prob{out, m, n, k};
  if (n >= 64 * 1024)
    gemv_mfma_kernel<TX, Src, 4><<<dim3((unsigned)((n + 63) / 64)), blk, 0, st>>>(x, src, prob, k);
  else if (n >= 32 * 1024)
    gemv_mfma_kernel<TX, Src, 2><<<dim3((unsigned)((n + 31) / 32)), blk, 0, st>>>(x, src, prob, k);
  else
    gemv_mfma_kernel<TX, Src, 1><<<dim3((unsigned)((n + 15) / 16)), blk, 0, st>>>(x, src, prob, k);
  return launch_status("dense_gemv_mfma");
}

// The decode product for a weight format: dense rows by 8-element runs, K-quants
// by 32-element groups.
template <typename TX, typename G, typename TO>
int launch_gemv(const TX* x, const G& src, TO* out, int64_t m, int64_t n, int64_t k, hipStream_t st) {
  if (m == 1) return launch_gemv_fma<TX, G, 1, TO>(x, src, out, m, n, k, st);
  if (m == 2) return launch_gemv_fma<TX, G, 2, TO>(x, src, out, m, n, k, st);
  return launch_gemv_mfma<TX, G, TO>(x, src, out, m, n, k, st);
}
template <typename S>
struct GemvSource {  // dense rows: the gather source itself
  using type = S;
  static type make(const S& s) { return s; }
};
template <int L>
struct GemvSource<Q4K<8, L>> {
  using type = Q4KGroup<L>;
  static type make(const Q4K<8, L>& s) { return type{s.wq}; }
};
template <>
struct GemvSource<Q5K<8>> {
  using type = Q5KGroup;
  static type make(const Q5K<8>& s) { return type{s.wq}; }
};
template <>
struct GemvSource<Q6K<8>> {
  using type = Q6KGroup;
  static type make(const Q6K<8>& s) { return type{s.wq}; }
};

template <typename TX, typename Src, typename TO>
int launch_dense(const void* x, const Src& src, void* out, int64_t m, int64_t n, int64_t k, bool vec,
                 hipStream_t st) {
  const int tiles_n = (int)((n + kDgBN - 1) / kDgBN);
  const TX* xp = static_cast<const TX*>(x);
  TO* op = static_cast<TO*>(out);
  // decode product: whole runs per row (8 elements for dense rows, a 32-element group for K-quants)
  if (vec && m <= kGemvRows && k % RunOf<typename GemvSource<Src>::type>::value == 0)
    return launch_gemv<TX>(xp, GemvSource<Src>::make(src), op, m, n, k, st);
  const bool ragged = !vec || k % kDgKC != 0;
  if (m <= 32) {
    const dim3 g((unsigned)tiles_n);
    const PlainProb<32, TO> prob{op, m, n, k};
    if (ragged)
      gemm_tile_kernel<TX, Src, 32, true><<<g, kDgThreads, 0, st>>>(xp, src, prob, k, tiles_n);
    else
      gemm_tile_kernel<TX, Src, 32, false><<<g, kDgThreads, 0, st>>>(xp, src, prob, k, tiles_n);
  } else {
    const dim3 g((unsigned)(((m + 127) / 128) * tiles_n));
    const PlainProb<128, TO> prob{op, m, n, k};
    if constexpr (SplitTile<Src>::value) {  // fp16 / bf16 weights: the split product on the bf16 matrix cores
      if (!ragged) {
        gemm_tile_split_kernel<TX><<<g, kDgThreads, 0, st>>>(xp, src, prob, k, tiles_n);
        return launch_status("dense_gemm (split)");
      }
    }
    if (ragged)
      gemm_tile_kernel<TX, Src, 128, true><<<g, kDgThreads, 0, st>>>(xp, src, prob, k, tiles_n);
    else
      gemm_tile_kernel<TX, Src, 128, false><<<g, kDgThreads, 0, st>>>(xp, src, prob, k, tiles_n);
  }
  return launch_status("dense_gemm");
}

template <typename TX, typename TO>
int dispatch_weights(const void* x, const void* w, int w_format, int layout, void* out, int64_t m, int64_t n,
                     int64_t k, bool vec, hipStream_t st) {
  const uint8_t* wb = static_cast<const uint8_t*>(w);
  switch (w_format) {
    case NVF_W_F32:
      return launch_dense<TX, Table<8, float>, TO>(x, Table<8, float>{static_cast<const float*>(w)}, out, m, n, k, vec, st);
    case NVF_W_F16:
      return launch_dense<TX, Table<8, _Float16>, TO>(x, Table<8, _Float16>{static_cast<const _Float16*>(w)}, out, m,
                                                      n, k, vec, st);
    case NVF_W_BF16:
      return launch_dense<TX, Table<8, __bf16>, TO>(x, Table<8, __bf16>{static_cast<const __bf16*>(w)}, out, m, n, k,
                                                    vec, st);
    case NVF_W_Q4_K:
      if (layout == NVF_QK_LAYOUT_HIP_LEGACY)
        return launch_dense<TX, Q4K<8, NVF_QK_LAYOUT_HIP_LEGACY>, TO>(x, Q4K<8, NVF_QK_LAYOUT_HIP_LEGACY>{wb}, out, m,
                                                                      n, k, vec, st);
      return launch_dense<TX, Q4K<8, NVF_QK_LAYOUT_GGML>, TO>(x, Q4K<8, NVF_QK_LAYOUT_GGML>{wb}, out, m, n, k, vec, st);
    case NVF_W_Q5_K:
      return launch_dense<TX, Q5K<8>, TO>(x, Q5K<8>{wb}, out, m, n, k, vec, st);
    default:
      return launch_dense<TX, Q6K<8>, TO>(x, Q6K<8>{wb}, out, m, n, k, vec, st);
  }
}

}  // namespace nvf

using namespace nvf;

extern "C" int nvf_matmul(const void* x, int x_dtype, const void* w, int w_format, int qk_layout, int64_t m,
                          int64_t n, int64_t k, void* out, int out_dtype, void* stream) {
  static const char* who = "nvf_matmul";
  if (!dtype_ok(x_dtype) || !dtype_ok(out_dtype)) return fail(NVF_ERR_INVALID, "%s: bad dtype", who);
  const bool kq = w_format == NVF_W_Q4_K || w_format == NVF_W_Q5_K || w_format == NVF_W_Q6_K;
  if (!(w_format == NVF_W_F32 || w_format == NVF_W_F16 || w_format == NVF_W_BF16 || kq))
    return fail(NVF_ERR_INVALID, "%s: bad weight format %d", who, w_format);
  if (qk_layout != NVF_QK_LAYOUT_GGML && qk_layout != NVF_QK_LAYOUT_HIP_LEGACY)
    return fail(NVF_ERR_INVALID, "%s: bad Q4_K layout %d", who, qk_layout);
  if (m < 0 || n < 0 || k < 0) return fail(NVF_ERR_INVALID, "%s: negative size", who);
  if (m == 0 || n == 0 || k == 0) return NVF_OK;
  if (kq && (n * k) % 256 != 0)
    return fail(NVF_ERR_INVALID, "%s: n*k=%lld is not whole 256-element superblocks", who, (long long)(n * k));
  if (!x || !w || !out) return fail(NVF_ERR_INVALID, "%s: NULL pointer", who);
  // vector loads need 16-byte aligned x and dense weights; without them every value
  // is read on its own (K-quant superblocks always need their base alignment)
  const bool vec = aligned16(x) && (kq || aligned16(w));
  if (kq && (reinterpret_cast<uintptr_t>(w) & (w_format == NVF_W_Q6_K ? 1u : 15u)) != 0)
    return fail(NVF_ERR_INVALID, "%s: K-quant weights must be 16-byte aligned (Q6_K: 2)", who);
  const int64_t tiles = (m <= 32 ? 1 : (m + 127) / 128) * ((n + kDgBN - 1) / kDgBN);
  if (tiles > INT32_MAX) return fail(NVF_ERR_INVALID, "%s: too many output tiles", who);
  int rc = NVF_OK;
  hipStream_t st = as_stream(stream);
  NVF_DISPATCH_DTYPE(x_dtype, TX, NVF_DISPATCH_DTYPE(out_dtype, TO, rc = (dispatch_weights<TX, TO>(
                                                                          x, w, w_format, qk_layout, out, m, n, k,
                                                                          vec, st))));
  return rc;
}

// Drop-ins: include/nanovllm/hip_ops.hpp:8-11 / src/hip_ops.hip:746-777 (fp32
// activations and output, null stream, early return for a size <= 0).
extern "C" void hip_matmul(const float* x, const float* w, int m, int n, int k, float* out) {
  if (m <= 0 || n <= 0 || k <= 0) return;
  dropin_check(nvf_matmul(x, NVF_F32, w, NVF_W_F32, NVF_QK_LAYOUT_GGML, m, n, k, out, NVF_F32, nullptr), "hip_matmul");
}

extern "C" void hip_matmul_u16(const float* x, const uint16_t* w, int m, int n, int k, float* out, bool w_bf16) {
  if (m <= 0 || n <= 0 || k <= 0) return;
  dropin_check(nvf_matmul(x, NVF_F32, w, w_bf16 ? NVF_W_BF16 : NVF_W_F16, NVF_QK_LAYOUT_GGML, m, n, k, out, NVF_F32,
                          nullptr),
               "hip_matmul_u16");
}

// Q4_K nibble order: the process-wide drop-in setting (nvf_set_dropin_q4k_layout),
// as hip_embedding_qk.
extern "C" void hip_matmul_qk(const float* x, const uint8_t* wq, int m, int n, int k, float* out, int kind) {
  if (m <= 0 || n <= 0 || k <= 0) return;
  dropin_check(nvf_matmul(x, NVF_F32, wq, kind, dropin_q4k_layout(), m, n, k, out, NVF_F32, nullptr),
               "hip_matmul_qk");
}
