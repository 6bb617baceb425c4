// Weight / table element sources shared by the embedding gathers and the dense
// GEMM's weight loader: each turns a flat element index into N exact fp32 values.
//   Raw  load(e0)               -- issue the loads for elements e0 .. e0+N-1
//   void decode(Raw, float* v)  -- produce the N fp32 values (exact)
// e0 is N-aligned, and N consecutive elements never cross a 32-element group.
// Reference decoders: Q8_0 src/hip_ops.hip:565-574 (split planes, src/model.cpp:394-404);
// K-quants src/hip_ops.hip:96-193 (Q4_K in GGML order src/gguf.cpp:477-496 or the
// reference's device order :130-140); F16/BF16/F32 rows :553-563.
#pragma once

#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

__device__ __forceinline__ float half_bits_to_f32(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

__device__ __forceinline__ float sbyte(uint32_t w, int k) { return (float)(int8_t)((w >> (8 * k)) & 0xffu); }

__device__ __forceinline__ bool bad_id(int64_t id, int64_t vocab) { return vocab > 0 && (id < 0 || id >= vocab); }

template <int N>
struct Q8Split {  // int8 plane + fp16 scale plane (src/model.cpp:394-404)
  const uint8_t* w8;
  const uint16_t* ws;
  struct Raw {
    uint32_t q[N / 4];
    uint32_t s;
  };
  __device__ __forceinline__ Raw load(int64_t e0) const {
    Raw r;
    if constexpr (N == 8) {
      const uint2 v = *reinterpret_cast<const uint2*>(w8 + e0);
      r.q[0] = v.x;
      r.q[1] = v.y;
    } else {
      r.q[0] = *reinterpret_cast<const uint32_t*>(w8 + e0);
    }
    r.s = ws[e0 >> 5];
    return r;
  }
  __device__ __forceinline__ void decode(const Raw& r, float* v) const {
    const float s = half_bits_to_f32(r.s);
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * i + k] = s * sbyte(r.q[i], k);
  }
};

// Reads NB (4 or 8) bytes at a 2-byte-aligned address: only the dwords that
// hold those bytes are loaded (plus a 16-bit tail load when the run starts 2
// bytes into a dword), realigned with v_alignbyte.  Nothing outside the run's
// dwords is touched, so a run at the very end of a table stays in bounds.
template <int NB>
__device__ __forceinline__ void load_a2(const uint8_t* p, uint32_t* out) {
  const bool mid = (reinterpret_cast<uintptr_t>(p) & 2u) != 0;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(reinterpret_cast<uintptr_t>(p) & ~uintptr_t(3));
  uint32_t d[NB / 4 + 1];
#pragma unroll
  for (int i = 0; i < NB / 4; ++i) d[i] = w[i];
  d[NB / 4] = mid ? (uint32_t)reinterpret_cast<const uint16_t*>(w + NB / 4)[0] : 0u;
#pragma unroll
  for (int i = 0; i < NB / 4; ++i) out[i] = mid ? __builtin_amdgcn_alignbyte(d[i + 1], d[i], 2) : d[i];
}

template <int N>
struct Q8Blocks {  // interleaved 34-byte blocks [fp16 d][32 x int8]
  const uint8_t* blocks;
  struct Raw {
    uint32_t q[N / 4];
    uint32_t s;
  };
  __device__ __forceinline__ Raw load(int64_t e0) const {
    const uint8_t* blk = blocks + (e0 >> 5) * 34;
    Raw r;
    load_a2<N>(blk + 2 + (e0 & 31), r.q);  // the quants start 2 bytes into a dword for even blocks
    r.s = *reinterpret_cast<const uint16_t*>(blk);
    return r;
  }
  __device__ __forceinline__ void decode(const Raw& r, float* v) const {
    const float s = half_bits_to_f32(r.s);
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * i + k] = s * sbyte(r.q[i], k);
  }
};

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int k) { return (w >> (8 * k)) & 0xffu; }

// (scale, min) of group j from the header dwords h1 = bytes 4..7, h2 = 8..11,
// h3 = 12..15 of a K-quant superblock (src/gguf.cpp:482-489).
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

template <int N, int LAYOUT>
struct Q4K {  // 144-byte superblocks; N consecutive outputs share one group j = i >> 5
  const uint8_t* wq;
  struct Raw {
    u32x4 hdr;
    uint32_t q[N / 4];
    int i;  // element index inside the superblock
  };
  __device__ __forceinline__ Raw load(int64_t e0) const {
    const uint8_t* blk = wq + (e0 >> 8) * 144;
    Raw r;
    r.i = (int)(e0 & 255);
    // GGML: element 64p + 32h + k is byte 32p + k, nibble h; HIP_LEGACY:
    // element 32j + 16h + k is byte 16j + k, nibble h.  N-aligned runs of
    // elements map to N consecutive bytes with one nibble.
    const int off = LAYOUT == NVF_QK_LAYOUT_GGML ? 32 * (r.i >> 6) + (r.i & 31) : 16 * (r.i >> 5) + (r.i & 15);
    r.hdr = ld16(blk);  // d, dmin, 12 B of scales: shared by the row's lanes (cache hits)
    if constexpr (N == 8) {
      const uint2 v = *reinterpret_cast<const uint2*>(blk + 16 + off);
      r.q[0] = v.x;
      r.q[1] = v.y;
    } else {
      r.q[0] = *reinterpret_cast<const uint32_t*>(blk + 16 + off);
    }
    return r;
  }
  __device__ __forceinline__ void decode(const Raw& r, float* v) const {
    const int j = r.i >> 5;
    const int sh = LAYOUT == NVF_QK_LAYOUT_GGML ? ((r.i >> 5) & 1) * 4 : ((r.i >> 4) & 1) * 4;
    uint32_t sc, mn;
    q4k_sm(r.hdr[1], r.hdr[2], r.hdr[3], j, sc, mn);
    const float s = half_bits_to_f32(r.hdr[0] & 0xffffu) * (float)sc;
    const float m = half_bits_to_f32(r.hdr[0] >> 16) * (float)mn;
#pragma unroll
    for (int i = 0; i < N / 4; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * i + k] = s * (float)((byte_of(r.q[i], k) >> sh) & 0xfu) - m;
  }
};

template <int N>
__device__ __forceinline__ void load_n(const uint8_t* p, uint32_t* out) {  // N-byte aligned run
  if constexpr (N == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    out[0] = v.x;
    out[1] = v.y;
  } else {
    out[0] = *reinterpret_cast<const uint32_t*>(p);
  }
}

template <int N>
struct Q5K {  // 176-byte superblocks [d][dmin][12 B scales][32 B qh][128 B ql] (src/hip_ops.hip:142-155)
  const uint8_t* wq;
  struct Raw {
    u32x4 hdr;
    uint32_t ql[N / 4];
    uint32_t qh[N / 4];
    int i;
  };
  // element 64g + 32s + l: low bits = nibble s of ql[32g + l], bit 4 = bit (2g + s) of qh[l]
  __device__ __forceinline__ Raw load(int64_t e0) const {
    const uint8_t* blk = wq + (e0 >> 8) * 176;
    Raw r;
    r.i = (int)(e0 & 255);
    r.hdr = ld16(blk);
    load_n<N>(blk + 48 + 32 * (r.i >> 6) + (r.i & 31), r.ql);
    load_n<N>(blk + 16 + (r.i & 31), r.qh);
    return r;
  }
  __device__ __forceinline__ void decode(const Raw& r, float* v) const {
    const int j = r.i >> 5, sh = (j & 1) * 4, hb = j;  // j = 2g + s
    uint32_t sc, mn;
    q4k_sm(r.hdr[1], r.hdr[2], r.hdr[3], j, sc, mn);
    const float s = half_bits_to_f32(r.hdr[0] & 0xffffu) * (float)sc;
    const float m = half_bits_to_f32(r.hdr[0] >> 16) * (float)mn;
#pragma unroll
    for (int w = 0; w < N / 4; ++w)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t q = ((byte_of(r.ql[w], k) >> sh) & 0xfu) | (((byte_of(r.qh[w], k) >> hb) & 1u) << 4);
        v[4 * w + k] = s * (float)q - m;
      }
  }
};

template <int N>
struct Q6K {  // 210-byte superblocks [128 B ql][64 B qh][16 x int8 scales][fp16 d] (src/gguf.cpp:500-518)
  const uint8_t* wq;
  struct Raw {
    uint32_t ql[N / 4];
    uint32_t qh[N / 4];
    uint32_t sd;  // int8 scale (low byte) | fp16 d << 16
    int i;
  };
  // element 128h + 32s + l: low 4 bits = nibble (s >> 1) of ql[64h + 32(s & 1) + l],
  // high 2 bits = bits 2s..2s+1 of qh[32h + l], scale sc[8h + l/16 + 2s]
  __device__ __forceinline__ Raw load(int64_t e0) const {
    const uint8_t* blk = wq + (e0 >> 8) * 210;  // 2-byte aligned
    Raw r;
    r.i = (int)(e0 & 255);
    const int h = r.i >> 7, t = r.i & 127, l0 = t & 31, slot = t >> 5;
    load_a2<N>(blk + 64 * h + 32 * (slot & 1) + l0, r.ql);
    load_a2<N>(blk + 128 + 32 * h + l0, r.qh);
    const uint32_t sc = blk[192 + 8 * h + (l0 >> 4) + 2 * slot];
    r.sd = sc | ((uint32_t)*reinterpret_cast<const uint16_t*>(blk + 208) << 16);
    return r;
  }
  __device__ __forceinline__ void decode(const Raw& r, float* v) const {
    const int slot = (r.i & 127) >> 5;
    const int lsh = (slot >> 1) * 4, hsh = 2 * slot;
    const float ds = half_bits_to_f32(r.sd >> 16) * (float)(int8_t)(r.sd & 0xffu);  // (d * sc) first, as the reference
#pragma unroll
    for (int w = 0; w < N / 4; ++w)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int q = (int)(((byte_of(r.ql[w], k) >> lsh) & 0xfu) | (((byte_of(r.qh[w], k) >> hsh) & 3u) << 4));
        v[4 * w + k] = ds * (float)(q - 32);
      }
  }
};

template <int N, typename TI>
struct Table {  // plain fp32 / fp16 / bf16 rows
  const TI* table;
  static constexpr int kWords = N * (int)sizeof(TI) / 4;
  struct Raw {
    uint32_t w[kWords];
  };
  __device__ __forceinline__ Raw load(int64_t e0) const {
    Raw r;
    const TI* p = table + e0;
    if constexpr (kWords == 8) {
      const u32x4 a = ld16(p), b = ld16(p + 16 / sizeof(TI));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r.w[i] = a[i];
        r.w[4 + i] = b[i];
      }
    } else if constexpr (kWords == 4) {
      const u32x4 a = ld16(p);
#pragma unroll
      for (int i = 0; i < 4; ++i) r.w[i] = a[i];
    } else {
      const uint2 a = *reinterpret_cast<const uint2*>(p);
      r.w[0] = a.x;
      r.w[1] = a.y;
    }
    return r;
  }
  __device__ __forceinline__ void decode(const Raw& r, float* v) const {
    if constexpr (sizeof(TI) == 4) {
#pragma unroll
      for (int i = 0; i < N; ++i) v[i] = __builtin_bit_cast(float, r.w[i]);
    } else {
#pragma unroll
      for (int i = 0; i < N / 2; ++i) {
        const uint32_t w = r.w[i];
        if constexpr (sizeof(TI) == 2 && __is_same(TI, __bf16)) {
          v[2 * i] = __builtin_bit_cast(float, w << 16);
          v[2 * i + 1] = __builtin_bit_cast(float, w & 0xffff0000u);
        } else {
          v[2 * i] = half_bits_to_f32(w & 0xffffu);
          v[2 * i + 1] = half_bits_to_f32(w >> 16);
        }
      }
    }
  }
};

}  // namespace nvf
