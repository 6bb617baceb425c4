// Embedding gathers with in-kernel dequant for gfx950.
//
// Reference semantics (all bit-exact: every product is exact in fp32):
//   Q8_0 split planes  src/hip_ops.hip:565-574 over src/model.cpp:394-404
//                      out[t,c] = fp16(ws[e>>5]) * int8(w8[e]),  e = id*H + c
//   Q8_0 34 B blocks   the same values read from the GGUF block bytes
//                      (src/gguf.cpp:353-362, decode tools/ref_top5.cpp:121-136)
//   K-quants           src/hip_ops.hip:600-609 + :96-193 (qk_w); Q4_K nibble
//                      order GGML (src/gguf.cpp:477-496) or HIP_LEGACY (:130-140)
//   F16/BF16/F32       src/hip_ops.hip:553-563
//
// Design: flat grids of independent threads, each owning a 16- or 32-element
// run of one output row, so table bytes are read with 16-byte (or aligned
// dword) loads and every output element is written once with 16-byte stores.
// The fp16 scale is decoded by v_cvt_f32_f16 (exact, subnormals included).
// Q4_K: eight lanes share a 144 B superblock; each lane loads the 16 B header
// (d, dmin, 12 B of 6-bit scales/mins -- one cache line serves the eight lanes)
// plus its own 16 B of nibbles, unpacks its two (scale, min) pairs in VGPRs and
// writes 32 outputs.
#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

constexpr int kEmbThreads = 256;

__device__ __forceinline__ float half_bits_to_f32(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

__device__ __forceinline__ bool bad_id(int64_t id, int64_t vocab) { return vocab > 0 && (id < 0 || id >= vocab); }

// Stores `n` (multiple of 8, or 4 for fp32) floats as TO with 16-byte stores.
template <typename TO, int NV>
__device__ __forceinline__ void store_run(TO* dst, const float* v) {
  constexpr int N = Pack<TO>::N;
  static_assert(NV % N == 0, "run length");
#pragma unroll
  for (int i = 0; i < NV / N; ++i) st16(dst + i * N, Pack<TO>::pack(v + i * N));
}

template <typename TO, int NV>
__device__ __forceinline__ void store_nan_run(TO* dst) {
  float v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = __builtin_nanf("");
  store_run<TO, NV>(dst, v);
}

__device__ __forceinline__ float sbyte(uint32_t w, int k) { return (float)(int8_t)((w >> (8 * k)) & 0xffu); }

// ---------------------------------------------------------------------------
// Q8_0, split planes: one thread per 16 outputs (one 16 B load of w8).
// ---------------------------------------------------------------------------
template <typename TO>
__global__ __launch_bounds__(kEmbThreads) void embed_q8_split_kernel(const int64_t* __restrict__ ids,
                                                                     const uint8_t* __restrict__ w8,
                                                                     const uint16_t* __restrict__ ws,
                                                                     TO* __restrict__ out, uint32_t total,
                                                                     FastDiv chunks_per_row, int64_t hidden,
                                                                     int64_t vocab) {
  const uint32_t g = blockIdx.x * kEmbThreads + threadIdx.x;
  if (g >= total) return;
  const uint32_t t = chunks_per_row.div(g);
  const int64_t c0 = (int64_t)(g - t * chunks_per_row.d) * 16;
  const int64_t id = ids[t];
  TO* dst = out + (int64_t)t * hidden + c0;
  if (bad_id(id, vocab)) {
    store_nan_run<TO, 16>(dst);
    return;
  }
  const int64_t e0 = id * hidden + c0;
  const u32x4 q = ld16(w8 + e0);
  const float s = half_bits_to_f32(ws[e0 >> 5]);
  float v[16];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) v[4 * i + k] = s * sbyte(q[i], k);
  store_run<TO, 16>(dst, v);
}

// ---------------------------------------------------------------------------
// Q8_0, interleaved 34 B blocks: one thread per block (32 outputs).  Block
// starts are 2 B aligned; the thread reads the aligned dwords covering its 34
// bytes (never a byte outside the block's dwords) and realigns with
// v_alignbyte.
// ---------------------------------------------------------------------------
template <typename TO>
__global__ __launch_bounds__(kEmbThreads) void embed_q8_blocks_kernel(const int64_t* __restrict__ ids,
                                                                      const uint8_t* __restrict__ blocks,
                                                                      TO* __restrict__ out, uint32_t total,
                                                                      FastDiv blocks_per_row, int64_t hidden,
                                                                      int64_t vocab) {
  const uint32_t g = blockIdx.x * kEmbThreads + threadIdx.x;
  if (g >= total) return;
  const uint32_t t = blocks_per_row.div(g);
  const uint32_t b = g - t * blocks_per_row.d;
  const int64_t id = ids[t];
  TO* dst = out + (int64_t)t * hidden + (int64_t)b * 32;
  if (bad_id(id, vocab)) {
    store_nan_run<TO, 32>(dst);
    return;
  }
  const uint8_t* blk = blocks + (id * blocks_per_row.d + b) * 34;
  const bool odd = (reinterpret_cast<uintptr_t>(blk) & 2u) != 0;  // block starts 2 B into a dword
  const uint32_t* w = reinterpret_cast<const uint32_t*>(reinterpret_cast<uintptr_t>(blk) & ~uintptr_t(3));
  uint32_t wd[9];
#pragma unroll
  for (int i = 0; i < 8; ++i) wd[i] = w[i];
  // dword 8: the whole dword when the block starts mid-dword (bytes 30..33),
  // else only the block's last two bytes (32, 33).
  if (odd)
    wd[8] = w[8];
  else
    wd[8] = reinterpret_cast<const uint16_t*>(w + 8)[0];
  const float s = half_bits_to_f32(odd ? (wd[0] >> 16) : (wd[0] & 0xffffu));
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t qd = odd ? wd[i + 1] : __builtin_amdgcn_alignbyte(wd[i + 1], wd[i], 2);
#pragma unroll
    for (int k = 0; k < 4; ++k) v[4 * i + k] = s * sbyte(qd, k);
  }
  store_run<TO, 32>(dst, v);
}

// ---------------------------------------------------------------------------
// Q4_K: one thread per 16 B of nibbles (32 outputs); needs hidden % 256 == 0.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int k) { return (w >> (8 * k)) & 0xffu; }

// (scale, min) of group j from the header dwords h1 = bytes 4..7, h2 = 8..11,
// h3 = 12..15 of the superblock (src/gguf.cpp:482-489).
__device__ __forceinline__ void q4k_sm(uint32_t h1, uint32_t h2, uint32_t h3, int j, uint32_t& sc, uint32_t& mn) {
  if (j < 4) {
    sc = byte_of(h1, j) & 63u;
    mn = byte_of(h2, j) & 63u;
  } else {
    const int jj = j - 4;
    sc = (byte_of(h3, jj) & 0xfu) | ((byte_of(h1, jj) >> 6) << 4);
    mn = (byte_of(h3, jj) >> 4) | ((byte_of(h2, jj) >> 6) << 4);
  }
}

template <typename TO, int LAYOUT>
__global__ __launch_bounds__(kEmbThreads) void embed_q4k_kernel(const int64_t* __restrict__ ids,
                                                                const uint8_t* __restrict__ wq, TO* __restrict__ out,
                                                                uint32_t total, FastDiv chunks_per_row, int64_t hidden,
                                                                int64_t vocab) {
  const uint32_t g = blockIdx.x * kEmbThreads + threadIdx.x;
  if (g >= total) return;
  const uint32_t t = chunks_per_row.div(g);
  const uint32_t rem = g - t * chunks_per_row.d;
  const uint32_t sb = rem >> 3, ch = rem & 7u;
  const int64_t id = ids[t];
  TO* row = out + (int64_t)t * hidden + (int64_t)sb * 256;
  int lo_off, j_lo, j_hi;
  if (LAYOUT == NVF_QK_LAYOUT_GGML) {
    // byte qs[32p + 16hh + k]: low nibble -> element 64p + 16hh + k (group 2p),
    // high nibble -> element 64p + 32 + 16hh + k (group 2p + 1)
    j_lo = 2 * (int)(ch >> 1);
    j_hi = j_lo + 1;
    lo_off = 64 * (int)(ch >> 1) + 16 * (int)(ch & 1u);
  } else {
    // byte qs[16j + k]: low nibble -> element 32j + k, high -> 32j + 16 + k
    j_lo = j_hi = (int)ch;
    lo_off = 32 * (int)ch;
  }
  const int hi_off = LAYOUT == NVF_QK_LAYOUT_GGML ? lo_off + 32 : lo_off + 16;
  if (bad_id(id, vocab)) {
    store_nan_run<TO, 16>(row + lo_off);
    store_nan_run<TO, 16>(row + hi_off);
    return;
  }
  const uint8_t* blk = wq + (id * (hidden >> 8) + sb) * 144;
  const u32x4 hdr = ld16(blk);
  const u32x4 qs = ld16(blk + 16 + ch * 16);
  const float d = half_bits_to_f32(hdr[0] & 0xffffu);
  const float dmin = half_bits_to_f32(hdr[0] >> 16);
  uint32_t sc, mn;
  q4k_sm(hdr[1], hdr[2], hdr[3], j_lo, sc, mn);
  const float s_lo = d * (float)sc, m_lo = dmin * (float)mn;
  q4k_sm(hdr[1], hdr[2], hdr[3], j_hi, sc, mn);
  const float s_hi = d * (float)sc, m_hi = dmin * (float)mn;
  float lo[16], hi[16];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t by = byte_of(qs[i], k);
      lo[4 * i + k] = s_lo * (float)(by & 0xfu) - m_lo;
      hi[4 * i + k] = s_hi * (float)(by >> 4) - m_hi;
    }
  store_run<TO, 16>(row + lo_off, lo);
  store_run<TO, 16>(row + hi_off, hi);
}

// ---------------------------------------------------------------------------
// Generic K-quant element decode (any hidden; Q5_K and Q6_K always).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fp16_at(const uint8_t* p) {
  return half_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}

__device__ __forceinline__ void q4k_sm_bytes(const uint8_t* s12, int j, uint32_t& sc, uint32_t& mn) {
  if (j < 4) {
    sc = s12[j] & 63u;
    mn = s12[j + 4] & 63u;
  } else {
    sc = (s12[j + 4] & 0xfu) | ((s12[j - 4] >> 6) << 4);
    mn = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4);
  }
}

__device__ __forceinline__ float qk_elem(const uint8_t* blk, int i, int kind, int layout) {
  if (kind == NVF_Q4_K) {
    const int j = i >> 5, e = i & 31;
    uint32_t sc, mn;
    q4k_sm_bytes(blk + 4, j, sc, mn);
    const float s = fp16_at(blk) * (float)sc, m = fp16_at(blk + 2) * (float)mn;
    int q;
    if (layout == NVF_QK_LAYOUT_GGML) {
      q = (blk[16 + (j >> 1) * 32 + e] >> ((j & 1) * 4)) & 0xf;
    } else {
      const uint8_t qb = blk[16 + j * 16 + (e & 15)];
      q = e < 16 ? (qb & 0xf) : (qb >> 4);
    }
    return s * (float)q - m;
  }
  if (kind == NVF_Q5_K) {  // src/hip_ops.hip:142-155
    const int group = i >> 6, slot = (i & 63) >> 5, l = i & 31;
    uint32_t sc, mn;
    q4k_sm_bytes(blk + 4, group * 2 + slot, sc, mn);
    const float s = fp16_at(blk) * (float)sc, m = fp16_at(blk + 2) * (float)mn;
    const uint8_t qlb = blk[48 + group * 32 + l];
    int q = slot == 0 ? (qlb & 0xf) : (qlb >> 4);
    if (blk[16 + l] & ((slot == 0 ? 1u : 2u) << (group * 2))) q += 16;
    return s * (float)q - m;
  }
  // Q6_K, src/hip_ops.hip:157-182: (d * sc) * (q - 32)
  const int half = i >> 7, tt = i & 127, l = tt & 31, slot = tt >> 5, is = l >> 4;
  const uint8_t* ql = blk + half * 64;
  const uint8_t qh = blk[128 + half * 32 + l];
  const int8_t* scs = reinterpret_cast<const int8_t*>(blk + 192 + half * 8);
  int q;
  if (slot == 0)
    q = (ql[l] & 0xf) | (((qh >> 0) & 3) << 4);
  else if (slot == 1)
    q = (ql[l + 32] & 0xf) | (((qh >> 2) & 3) << 4);
  else if (slot == 2)
    q = (ql[l] >> 4) | (((qh >> 4) & 3) << 4);
  else
    q = (ql[l + 32] >> 4) | (((qh >> 6) & 3) << 4);
  const float d = fp16_at(blk + 208);
  return d * (float)scs[is + 2 * slot] * (float)(q - 32);
}

template <typename TO>
__global__ __launch_bounds__(kEmbThreads) void embed_qk_generic_kernel(const int64_t* __restrict__ ids,
                                                                       const uint8_t* __restrict__ wq,
                                                                       TO* __restrict__ out, int64_t total,
                                                                       int64_t hidden, int64_t vocab, int kind,
                                                                       int layout, int block_bytes) {
  const int64_t g = (int64_t)blockIdx.x * kEmbThreads + threadIdx.x;
  if (g >= total) return;
  const int64_t t = g / hidden, c = g - t * hidden;
  const int64_t id = ids[t];
  if (bad_id(id, vocab)) {
    out[g] = from_f32<TO>(__builtin_nanf(""));
    return;
  }
  const int64_t e = id * hidden + c;
  out[g] = from_f32<TO>(qk_elem(wq + (e >> 8) * block_bytes, (int)(e & 255), kind, layout));
}

// Q8_0 at any hidden / alignment, one element per thread.
template <typename TO>
__global__ __launch_bounds__(kEmbThreads) void embed_q8_generic_kernel(const int64_t* __restrict__ ids,
                                                                       const uint8_t* __restrict__ w8,
                                                                       const uint16_t* __restrict__ ws,
                                                                       const uint8_t* __restrict__ blocks,
                                                                       TO* __restrict__ out, int64_t total,
                                                                       int64_t hidden, int64_t vocab) {
  const int64_t g = (int64_t)blockIdx.x * kEmbThreads + threadIdx.x;
  if (g >= total) return;
  const int64_t t = g / hidden, c = g - t * hidden;
  const int64_t id = ids[t];
  if (bad_id(id, vocab)) {
    out[g] = from_f32<TO>(__builtin_nanf(""));
    return;
  }
  const int64_t e = id * hidden + c;
  float v;
  if (blocks) {
    const uint8_t* b = blocks + (e >> 5) * 34;
    v = fp16_at(b) * (float)(int8_t)b[2 + (e & 31)];
  } else {
    v = half_bits_to_f32(ws[e >> 5]) * (float)(int8_t)w8[e];
  }
  out[g] = from_f32<TO>(v);
}

// ---------------------------------------------------------------------------
// Plain table gather: one thread per 8 elements.
// ---------------------------------------------------------------------------
template <typename TI, typename TO>
__global__ __launch_bounds__(kEmbThreads) void embed_table_kernel(const int64_t* __restrict__ ids,
                                                                  const TI* __restrict__ table, TO* __restrict__ out,
                                                                  uint32_t total, FastDiv chunks_per_row,
                                                                  int64_t hidden, int64_t vocab) {
  const uint32_t g = blockIdx.x * kEmbThreads + threadIdx.x;
  if (g >= total) return;
  const uint32_t t = chunks_per_row.div(g);
  const int64_t c0 = (int64_t)(g - t * chunks_per_row.d) * 8;
  const int64_t id = ids[t];
  TO* dst = out + (int64_t)t * hidden + c0;
  if (bad_id(id, vocab)) {
    store_nan_run<TO, 8>(dst);
    return;
  }
  const TI* src = table + id * hidden + c0;
  float v[8];
  constexpr int NI = Pack<TI>::N;
#pragma unroll
  for (int i = 0; i < 8 / NI; ++i) Pack<TI>::unpack(ld16(src + i * NI), v + i * NI);
  store_run<TO, 8>(dst, v);
}

template <typename TI, typename TO>
__global__ __launch_bounds__(kEmbThreads) void embed_table_generic_kernel(const int64_t* __restrict__ ids,
                                                                          const TI* __restrict__ table,
                                                                          TO* __restrict__ out, int64_t total,
                                                                          int64_t hidden, int64_t vocab) {
  const int64_t g = (int64_t)blockIdx.x * kEmbThreads + threadIdx.x;
  if (g >= total) return;
  const int64_t t = g / hidden, c = g - t * hidden;
  const int64_t id = ids[t];
  out[g] = from_f32<TO>(bad_id(id, vocab) ? __builtin_nanf("") : to_f32(table[id * hidden + c]));
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static inline dim3 grid_for(int64_t threads) { return dim3((unsigned)((threads + kEmbThreads - 1) / kEmbThreads)); }

static int check_common(const char* name, const int64_t* ids, const void* table, const void* out, int64_t tokens,
                        int64_t hidden, int out_dtype) {
  if (!dtype_ok(out_dtype)) return fail(NVF_ERR_INVALID, "%s: bad out dtype %d", name, out_dtype);
  if (tokens < 0 || hidden < 0) return fail(NVF_ERR_INVALID, "%s: bad shape", name);
  if (tokens == 0 || hidden == 0) return 1;  // nothing to do
  if (!ids || !table || !out) return fail(NVF_ERR_INVALID, "%s: NULL pointer", name);
  if (tokens * hidden > (int64_t)INT32_MAX * kEmbThreads)
    return fail(NVF_ERR_INVALID, "%s: %lld outputs exceed one launch", name, (long long)(tokens * hidden));
  return 0;
}

template <typename TO>
static int launch_q8(const int64_t* ids, const uint8_t* w8, const uint16_t* ws, const uint8_t* blocks, int64_t tokens,
                     int64_t hidden, int64_t vocab, void* out, hipStream_t st) {
  TO* o = static_cast<TO*>(out);
  if (blocks) {
    const int64_t total = tokens * (hidden / 32);
    if (hidden % 32 == 0 && aligned16(out) && (reinterpret_cast<uintptr_t>(blocks) & 3u) == 0 && total < UINT32_MAX) {
      embed_q8_blocks_kernel<TO><<<grid_for(total), kEmbThreads, 0, st>>>(ids, blocks, o, (uint32_t)total,
                                                                          FastDiv((uint32_t)(hidden / 32)), hidden, vocab);
      return launch_status("embedding_q8_0_blocks");
    }
  } else {
    const int64_t total = tokens * (hidden / 16);
    if (hidden % 32 == 0 && aligned16(out) && aligned16(w8) && (reinterpret_cast<uintptr_t>(ws) & 1u) == 0 &&
        total < UINT32_MAX) {
      embed_q8_split_kernel<TO><<<grid_for(total), kEmbThreads, 0, st>>>(ids, w8, ws, o, (uint32_t)total,
                                                                         FastDiv((uint32_t)(hidden / 16)), hidden, vocab);
      return launch_status("embedding_q8_0");
    }
  }
  const int64_t total = tokens * hidden;
  embed_q8_generic_kernel<TO><<<grid_for(total), kEmbThreads, 0, st>>>(ids, w8, ws, blocks, o, total, hidden, vocab);
  return launch_status("embedding_q8_0(generic)");
}

template <typename TO>
static int launch_qk(const int64_t* ids, const uint8_t* wq, int64_t tokens, int64_t hidden, int64_t vocab, int kind,
                     int layout, void* out, hipStream_t st) {
  TO* o = static_cast<TO*>(out);
  const int64_t chunks = tokens * (hidden / 256) * 8;
  if (kind == NVF_Q4_K && hidden % 256 == 0 && aligned16(wq) && aligned16(out) && chunks < UINT32_MAX) {
    const FastDiv cpr((uint32_t)(hidden / 256 * 8));
    if (layout == NVF_QK_LAYOUT_GGML)
      embed_q4k_kernel<TO, NVF_QK_LAYOUT_GGML>
          <<<grid_for(chunks), kEmbThreads, 0, st>>>(ids, wq, o, (uint32_t)chunks, cpr, hidden, vocab);
    else
      embed_q4k_kernel<TO, NVF_QK_LAYOUT_HIP_LEGACY>
          <<<grid_for(chunks), kEmbThreads, 0, st>>>(ids, wq, o, (uint32_t)chunks, cpr, hidden, vocab);
    return launch_status("embedding_q4_k");
  }
  const int bb = kind == NVF_Q4_K ? 144 : (kind == NVF_Q5_K ? 176 : 210);
  const int64_t total = tokens * hidden;
  embed_qk_generic_kernel<TO>
      <<<grid_for(total), kEmbThreads, 0, st>>>(ids, wq, o, total, hidden, vocab, kind, layout, bb);
  return launch_status("embedding_qk(generic)");
}

template <typename TI, typename TO>
static int launch_table(const int64_t* ids, const void* table, int64_t tokens, int64_t hidden, int64_t vocab, void* out,
                        hipStream_t st) {
  const TI* tb = static_cast<const TI*>(table);
  TO* o = static_cast<TO*>(out);
  const int64_t total = tokens * (hidden / 8);
  if (hidden % 8 == 0 && aligned16(table) && aligned16(out) && total < UINT32_MAX) {
    embed_table_kernel<TI, TO><<<grid_for(total), kEmbThreads, 0, st>>>(ids, tb, o, (uint32_t)total,
                                                                        FastDiv((uint32_t)(hidden / 8)), hidden, vocab);
    return launch_status("embedding");
  }
  embed_table_generic_kernel<TI, TO>
      <<<grid_for(tokens * hidden), kEmbThreads, 0, st>>>(ids, tb, o, tokens * hidden, hidden, vocab);
  return launch_status("embedding(generic)");
}

}  // namespace nvf

using namespace nvf;

extern "C" int nvf_embedding_q8_0(const int64_t* ids, const uint8_t* w8, const uint16_t* ws, int64_t tokens,
                                  int64_t hidden, int64_t vocab, void* out, int out_dtype, void* stream) {
  const int c = check_common("nvf_embedding_q8_0", ids, w8, out, tokens, hidden, out_dtype);
  if (c) return c < 0 ? c : NVF_OK;
  if (!ws) return fail(NVF_ERR_INVALID, "nvf_embedding_q8_0: NULL scale plane");
  int s = NVF_OK;
  NVF_DISPATCH_DTYPE(out_dtype, TO,
                     s = launch_q8<TO>(ids, w8, ws, nullptr, tokens, hidden, vocab, out, as_stream(stream)));
  return s;
}

extern "C" int nvf_embedding_q8_0_blocks(const int64_t* ids, const uint8_t* blocks, int64_t tokens, int64_t hidden,
                                         int64_t vocab, void* out, int out_dtype, void* stream) {
  const int c = check_common("nvf_embedding_q8_0_blocks", ids, blocks, out, tokens, hidden, out_dtype);
  if (c) return c < 0 ? c : NVF_OK;
  if (hidden % 32 != 0)
    return fail(NVF_ERR_INVALID, "nvf_embedding_q8_0_blocks: hidden %lld is not a multiple of 32", (long long)hidden);
  int s = NVF_OK;
  NVF_DISPATCH_DTYPE(out_dtype, TO,
                     s = launch_q8<TO>(ids, nullptr, nullptr, blocks, tokens, hidden, vocab, out, as_stream(stream)));
  return s;
}

extern "C" int nvf_embedding_qk(const int64_t* ids, const uint8_t* wq, int64_t tokens, int64_t hidden, int64_t vocab,
                                int kind, int layout, void* out, int out_dtype, void* stream) {
  const int c = check_common("nvf_embedding_qk", ids, wq, out, tokens, hidden, out_dtype);
  if (c) return c < 0 ? c : NVF_OK;
  if (kind != NVF_Q4_K && kind != NVF_Q5_K && kind != NVF_Q6_K)
    return fail(NVF_ERR_INVALID, "nvf_embedding_qk: unsupported kind %d (12, 13 or 14)", kind);
  if (layout != NVF_QK_LAYOUT_GGML && layout != NVF_QK_LAYOUT_HIP_LEGACY)
    return fail(NVF_ERR_INVALID, "nvf_embedding_qk: bad layout %d", layout);
  int s = NVF_OK;
  NVF_DISPATCH_DTYPE(out_dtype, TO,
                     s = launch_qk<TO>(ids, wq, tokens, hidden, vocab, kind, layout, out, as_stream(stream)));
  return s;
}

extern "C" int nvf_embedding(const int64_t* ids, const void* table, int64_t tokens, int64_t hidden, int64_t vocab,
                             int table_dtype, void* out, int out_dtype, void* stream) {
  const int c = check_common("nvf_embedding", ids, table, out, tokens, hidden, out_dtype);
  if (c) return c < 0 ? c : NVF_OK;
  if (!dtype_ok(table_dtype)) return fail(NVF_ERR_INVALID, "nvf_embedding: bad table dtype %d", table_dtype);
  int s = NVF_OK;
  hipStream_t st = as_stream(stream);
  NVF_DISPATCH_DTYPE(table_dtype, TI,
                     NVF_DISPATCH_DTYPE(out_dtype, TO,
                                        s = (launch_table<TI, TO>(ids, table, tokens, hidden, vocab, out, st))));
  return s;
}

// Drop-ins: include/nanovllm/hip_ops.hpp:30-33 / src/hip_ops.hip:746-786.
extern "C" void hip_embedding(const int64_t* ids, const float* table, int tokens, int hidden, float* out) {
  if (tokens <= 0 || hidden <= 0) return;
  dropin_check(nvf_embedding(ids, table, tokens, hidden, 0, NVF_F32, out, NVF_F32, nullptr), "hip_embedding");
}

extern "C" void hip_embedding_u16(const int64_t* ids, const uint16_t* table, int tokens, int hidden, float* out,
                                  bool table_bf16) {
  if (tokens <= 0 || hidden <= 0) return;
  dropin_check(nvf_embedding(ids, table, tokens, hidden, 0, table_bf16 ? NVF_BF16 : NVF_F16, out, NVF_F32, nullptr),
               "hip_embedding_u16");
}

extern "C" void hip_embedding_q8(const int64_t* ids, const uint8_t* w8, const uint16_t* ws, int tokens, int hidden,
                                 float* out) {
  if (tokens <= 0 || hidden <= 0) return;
  dropin_check(nvf_embedding_q8_0(ids, w8, ws, tokens, hidden, 0, out, NVF_F32, nullptr), "hip_embedding_q8");
}

extern "C" void hip_embedding_qk(const int64_t* ids, const uint8_t* wq, int tokens, int hidden, float* out, int kind) {
  if (tokens <= 0 || hidden <= 0) return;
  dropin_check(nvf_embedding_qk(ids, wq, tokens, hidden, 0, kind, NVF_QK_LAYOUT_GGML, out, NVF_F32, nullptr),
               "hip_embedding_qk");
}
