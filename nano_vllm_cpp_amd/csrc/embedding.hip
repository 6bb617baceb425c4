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
// Design: wave64s own token rows (the id is read once per wave).  Lane l owns
// the 16-byte output chunks l, l + 64, ... of its wave, so every store
// instruction writes 1 KiB of contiguous output -- the output is the larger
// side of every gather (2 bytes out per 1.06 (Q8_0) or 0.56 (Q4_K) bytes in)
// -- and the output streams out with non-temporal stores.  The fp16 scales are
// decoded by v_cvt_f32_f16 (exact, subnormals included).
//   * Q8_0 split planes and plain tables: each lane issues the loads of all its
//     chunks (up to 8) straight from HBM before decoding any.
//   * Block formats (Q8_0 34 B blocks, Q4_K, Q5_K, Q6_K): the wave stages its
//     row's blocks in LDS with coalesced 16-byte loads, then each lane decodes
//     its chunks from LDS.  The 8 outputs of a chunk share one scale (and for
//     the K-quants one 6-bit (scale, min) pair, unpacked in VGPRs from the
//     staged 12-byte table).  Rows longer than the 16 KiB stage fall back to
//     direct per-chunk loads (Q4_K/Q5_K/Q6_K split a row over 4 waves there).
//   * A hidden that is not a multiple of the block takes a per-element kernel
//     (correct, not tuned).
#include <atomic>
#include <algorithm>
#include <type_traits>

#include "nvf_device.hpp"
#include "nvf_host.hpp"
#include "weight_formats.hpp"

namespace nvf {

constexpr int kEmbThreads = 256;

constexpr int kEmbWaves = kEmbThreads / kWave;
constexpr int64_t kEmbCapMinGroups = 4096;  // two rounds of 256 CUs x 8 resident workgroups
constexpr size_t kEmbCapLds = 40 * 1024;    // 160 KiB LDS per CU / 40 KiB = 4 workgroups per CU

// ---------------------------------------------------------------------------
// Row-gather kernel.  One wave per token row; lane l owns the 16-byte output
// chunks l, l + 64, ... (N = 8 outputs for fp16/bf16, 4 for fp32), so each
// store instruction writes 1 KiB of contiguous row.  Up to U chunks per lane
// have their loads in flight before any decode.  The table row is located
// once per wave (the id is wave-uniform).  The Source (weight_formats.hpp)
// loads and decodes each chunk's N outputs.
// ---------------------------------------------------------------------------
// WPR waves per row: wave w of a row covers its chunk groups w, w + WPR, ...
// Measured at Qwen2.5-7B prefill shapes: Q8_0 and tables gather best with one
// wave per row and exactly ceil(chunks / 64) chunks per lane in flight; Q4_K
// (smaller loads per output) with four waves per row.  Packing two rows into
// one wave was slower in this form.
template <typename TO, typename Src, int U, int WPR>
__global__ __launch_bounds__(kEmbThreads) void embed_rows_kernel(const int64_t* __restrict__ ids, Src src,
                                                                 TO* __restrict__ out, int64_t tokens, int hidden,
                                                                 int64_t vocab) {
  constexpr int N = Pack<TO>::N;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int64_t t = (int64_t)blockIdx.x * (kEmbWaves / WPR) + wave / WPR;
  const int part = wave % WPR;
  if (t >= tokens) return;  // wave-uniform
  const int nch = hidden / N;
  const int64_t id = ids[t];  // wave-uniform
  TO* dst = out + t * hidden;
  if (bad_id(id, vocab)) {  // out-of-range id: a NaN row instead of a read
    float nan[N];
#pragma unroll
    for (int i = 0; i < N; ++i) nan[i] = __builtin_nanf("");
    for (int c = part * kWave + lane; c < nch; c += WPR * kWave) st16(dst + c * N, Pack<TO>::pack(nan));
    return;
  }
  const int64_t row0 = id * hidden;
  for (int base = 0; base < nch; base += U * WPR * kWave) {
    typename Src::Raw raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = base + (u * WPR + part) * kWave + lane;
      if (c < nch) raw[u] = src.load(row0 + (int64_t)c * N);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = base + (u * WPR + part) * kWave + lane;
      if (c < nch) {
        float v[N];
        src.decode(raw[u], v);
        st16_nt(dst + (int64_t)c * N, Pack<TO>::pack(v));
      }
    }
  }
}

template <typename TO, typename Src, int WPR>
static int launch_rows(const int64_t* ids, const Src& src, TO* out, int64_t tokens, int64_t hidden, int64_t vocab,
                       hipStream_t st, const char* what, size_t occ_lds = 0) {
  constexpr int N = Pack<TO>::N;
  const int64_t per_lane = (hidden / N + WPR * kWave - 1) / (WPR * kWave);  // chunks per lane
  const int64_t rows_per_block = kEmbWaves / WPR;
  const dim3 grid((unsigned)((tokens + rows_per_block - 1) / rows_per_block));
  const int h = (int)hidden;
  switch (per_lane < 8 ? per_lane : 8) {  // exact up to 8 chunks per lane, then the row loops
#define NVF_EMB_CASE(UU)                                                                                          \
  case UU:                                                                                                        \
    embed_rows_kernel<TO, Src, UU, WPR><<<grid, kEmbThreads, occ_lds, st>>>(ids, src, out, tokens, h, vocab); \
    break;
    NVF_EMB_CASE(1) NVF_EMB_CASE(2) NVF_EMB_CASE(3) NVF_EMB_CASE(4)
    NVF_EMB_CASE(5) NVF_EMB_CASE(6) NVF_EMB_CASE(7) NVF_EMB_CASE(8)
#undef NVF_EMB_CASE
  }
  return launch_status(what);
}

// ---------------------------------------------------------------------------
// LDS-staged row gather for block formats.  A wave copies its row's blocks
// into LDS by buffer loads straight to LDS, 16 bytes per lane (from the
// 16-byte-aligned address at or below the row's first block), then every lane
// decodes its own chunks of N outputs out of LDS and stores them as before.
// This turns the many small per-chunk loads of the K-quant formats (header,
// nibbles, high bits, scales) into a few full-width loads per lane (measured at
// Qwen2.5-7B shape: Q5_K 57% -> 69%, Q6_K 50% -> 60%, Q8_0 blocks 65% -> 68%,
// Q4_K 74% -> 75% of the 8 TB/s peak, staged through registers; the direct LDS
// loads then took Q5_K 70-74% -> 77%).  The stage starts at the 16-byte-aligned
// address at or below the row and ends with the 16-byte granule holding the
// row's last byte; the buffer resource ends there too, so lanes past it read
// zeros (into their own slice of the stage) and no fault is possible.
// A format supplies
//   kBlockBytes, kBlockElems, decode(const uint8_t* blk, int i, float* v)
// reading the block from LDS (elements i .. i+N-1 of the block), and may supply
// kSpareBytes, the bytes its decode may read past the staged row.
// ---------------------------------------------------------------------------
// Q6_K superblocks are 210 bytes, so flat staging leaves every other one 2 bytes
// off dword alignment.  As for the 34-byte Q8_0 blocks, the quants are read as the
// aligned dwords that hold them (one more than their count) and realigned with
// v_alignbyte: a 2-byte-aligned dword LDS read would take the hardware's
// unaligned path.  The row is staged by aligned 16-byte global loads.  Every read
// stays inside its block (the quants end at byte 192 of 210).
template <int N>
struct StagedQ6K {
  static constexpr int kBlockBytes = 210, kBlockElems = 256;
  __device__ __forceinline__ static void decode(const uint8_t* blk, int i, float* v) {
    const int h = i >> 7, t = i & 127, l0 = t & 31, slot = t >> 5;
    const int lsh = (slot >> 1) * 4, hsh = 2 * slot;
    const float ds = half_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk + 208)) *
                     (float)(int8_t)blk[192 + 8 * h + (l0 >> 4) + 2 * slot];
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3);  // 0 or 2 (l0 % 4 == 0)
    const uint32_t* ql = reinterpret_cast<const uint32_t*>(blk - sh + 64 * h + 32 * (slot & 1) + l0);
    const uint32_t* qh = reinterpret_cast<const uint32_t*>(blk - sh + 128 + 32 * h + l0);
    uint32_t da[N / 4 + 1], db[N / 4 + 1];
#pragma unroll
    for (int w = 0; w <= N / 4; ++w) {
      da[w] = ql[w];
      db[w] = qh[w];
    }
    // four 6-bit values per dword at once (low nibbles | high 2 bits << 4), then per
    // byte an exact byte-to-float, an exact - 32 and the product, as the reference
    // (an fma with -32 ds folded in would give +0 where the reference gives -0)
#pragma unroll
    for (int w = 0; w < N / 4; ++w) {
      const uint32_t a = __builtin_amdgcn_alignbyte(da[w + 1], da[w], sh);
      const uint32_t b = __builtin_amdgcn_alignbyte(db[w + 1], db[w], sh);
      const uint32_t q4 = ((a >> lsh) & 0x0f0f0f0fu) | (((b >> hsh) & 0x03030303u) << 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * w + k] = ((float)byte_of(q4, k) - 32.0f) * ds;
    }
  }
};

// The four slots s of elements 128 h + 32 s + l0 .. + N - 1 share their quant bytes:
// s = 0 and 2 the low and high nibbles of ql[64 h + l0 ..], s = 1 and 3 those of
// ql[64 h + 32 + l0 ..], and all four the 2-bit fields 2 s of qh[32 h + l0 ..].  A
// lane decodes the four together: a third of the LDS reads and realignments
// (measured at Qwen2.5-7B's prefill shape: 31.7-32.0 -> 31.0-31.4 us).
template <int N>
struct StagedQ6KQuad : StagedQ6K<N> {
  static constexpr bool kQuad = true;
  __device__ __forceinline__ static void decode4(const uint8_t* blk, int h, int l0, float (&v)[4][N]) {
    const float d = half_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk + 208));
    float ds[4];
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) ds[sl] = d * (float)(int8_t)blk[192 + 8 * h + (l0 >> 4) + 2 * sl];
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3);  // 0 or 2 (l0 % 4 == 0)
    const uint32_t* q0 = reinterpret_cast<const uint32_t*>(blk - sh + 64 * h + l0);
    const uint32_t* q1 = reinterpret_cast<const uint32_t*>(blk - sh + 64 * h + 32 + l0);
    const uint32_t* qh = reinterpret_cast<const uint32_t*>(blk - sh + 128 + 32 * h + l0);
    uint32_t a0[N / 4 + 1], a1[N / 4 + 1], b[N / 4 + 1];
#pragma unroll
    for (int w = 0; w <= N / 4; ++w) {
      a0[w] = q0[w];
      a1[w] = q1[w];
      b[w] = qh[w];
    }
#pragma unroll
    for (int w = 0; w < N / 4; ++w) {
      const uint32_t x0 = __builtin_amdgcn_alignbyte(a0[w + 1], a0[w], sh);
      const uint32_t x1 = __builtin_amdgcn_alignbyte(a1[w + 1], a1[w], sh);
      const uint32_t hb = __builtin_amdgcn_alignbyte(b[w + 1], b[w], sh);
      const uint32_t q[4] = {(x0 & 0x0f0f0f0fu) | ((hb & 0x03030303u) << 4),
                             (x1 & 0x0f0f0f0fu) | (((hb >> 2) & 0x03030303u) << 4),
                             ((x0 >> 4) & 0x0f0f0f0fu) | (((hb >> 4) & 0x03030303u) << 4),
                             ((x1 >> 4) & 0x0f0f0f0fu) | (((hb >> 6) & 0x03030303u) << 4)};
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int k = 0; k < 4; ++k) v[sl][4 * w + k] = ((float)byte_of(q[sl], k) - 32.0f) * ds[sl];
    }
  }
};

template <int N>
struct StagedQ5K {
  static constexpr int kBlockBytes = 176, kBlockElems = 256;
  __device__ __forceinline__ static void decode(const uint8_t* blk, int i, float* v) {
    const int j = i >> 5, sh = (j & 1) * 4, l0 = i & 31;
    const uint32_t* hd = reinterpret_cast<const uint32_t*>(blk);  // 176 B blocks stay 16-byte aligned
    uint32_t sc, mn;
    q4k_sm(hd[1], hd[2], hd[3], j, sc, mn);
    const float s = half_bits_to_f32(hd[0] & 0xffffu) * (float)sc;
    const float m = half_bits_to_f32(hd[0] >> 16) * (float)mn;
    const uint32_t* ql = reinterpret_cast<const uint32_t*>(blk + 48 + 32 * (i >> 6) + l0);
    const uint32_t* qh = reinterpret_cast<const uint32_t*>(blk + 16 + l0);
    // four 5-bit values per dword at once; s * q is exact (22 bits), so fma(q, s, -m)
    // rounds the same exact difference once, as s * q - m does
#pragma unroll
    for (int w = 0; w < N / 4; ++w) {
      const uint32_t a = ql[w], b = qh[w];
      const uint32_t q4 = ((a >> sh) & 0x0f0f0f0fu) | (((b >> j) & 0x01010101u) << 4);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * w + k] = fmaf((float)byte_of(q4, k), s, -m);
    }
  }
};

template <int N, int LAYOUT>
struct StagedQ4K {
  static constexpr int kBlockBytes = 144, kBlockElems = 256;
  __device__ __forceinline__ static void decode(const uint8_t* blk, int i, float* v) {
    const int j = i >> 5;
    const int off = LAYOUT == NVF_QK_LAYOUT_GGML ? 32 * (i >> 6) + (i & 31) : 16 * (i >> 5) + (i & 15);
    const int sh = LAYOUT == NVF_QK_LAYOUT_GGML ? ((i >> 5) & 1) * 4 : ((i >> 4) & 1) * 4;
    const uint32_t* hd = reinterpret_cast<const uint32_t*>(blk);
    uint32_t sc, mn;
    q4k_sm(hd[1], hd[2], hd[3], j, sc, mn);
    const float s = half_bits_to_f32(hd[0] & 0xffffu) * (float)sc;
    const float m = half_bits_to_f32(hd[0] >> 16) * (float)mn;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(blk + 16 + off);
#pragma unroll
    for (int w = 0; w < N / 4; ++w) {
      const uint32_t a = q[w];
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * w + k] = s * (float)((byte_of(a, k) >> sh) & 0xfu) - m;
    }
  }
};

// Staged flat: every other 34-byte block sits 2 bytes off dword alignment.  Its
// quants are read as the aligned dwords that hold them (one more than their
// count) and realigned with v_alignbyte: a 2-byte-aligned 8-byte LDS read takes
// the hardware's unaligned path instead (17x the LDS issue stalls of Q5_K).  48-byte
// aligned slots, at three 16-byte loads per block, measured slower (38.5 against
// ~33 us at Qwen2.5-7B prefill shape): for 34-byte blocks the extra loads cost more.
// The last dword read may reach 2 bytes past the row: the stage holds 16 spare bytes.
// Four chunks per lane are decoded before their stores (measured at Qwen2.5-7B's
// prefill shape: 32.2 -> 31.4 us; the same for Q6_K and Q5_K was no faster).
template <int N>
struct StagedQ8Blocks {
  static constexpr int kBlockBytes = 34, kBlockElems = 32, kSpareBytes = 16, kDecodeUnroll = 4;
  __device__ __forceinline__ static void decode(const uint8_t* blk, int i, float* v) {
    const float s = half_bits_to_f32(*reinterpret_cast<const uint16_t*>(blk));
    const uint8_t* q8 = blk + 2 + i;
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(q8) & 3);  // 0 or 2
    const uint32_t* d = reinterpret_cast<const uint32_t*>(q8 - sh);       // (pointer arithmetic: stays in LDS)
    uint32_t dw[N / 4 + 1];
#pragma unroll
    for (int w = 0; w <= N / 4; ++w) dw[w] = d[w];
#pragma unroll
    for (int w = 0; w < N / 4; ++w) {
      const uint32_t q = __builtin_amdgcn_alignbyte(dw[w + 1], dw[w], sh);
#pragma unroll
      for (int k = 0; k < 4; ++k) v[4 * w + k] = s * sbyte(q, k);
    }
  }
};

// kSpareBytes of a format: LDS bytes its decode may read past the staged row
template <typename F, typename = void>
struct SpareBytes {
  static constexpr int value = 0;
};
template <typename F>
struct SpareBytes<F, decltype((void)F::kSpareBytes)> {
  static constexpr int value = F::kSpareBytes;
};

// kQuad of a format: true when it supplies decode4 (four slots of a 256-element block per lane)
template <typename F, typename = void>
struct QuadDecode {
  static constexpr bool value = false;
};
template <typename F>
struct QuadDecode<F, decltype((void)F::kQuad)> {
  static constexpr bool value = F::kQuad;
};

// kDecodeUnroll of a format: chunks a lane decodes before it stores them (default 1)
template <typename F, typename = void>
struct DecodeUnroll {
  static constexpr int value = 1;
};
template <typename F>
struct DecodeUnroll<F, decltype((void)F::kDecodeUnroll)> {
  static constexpr int value = F::kDecodeUnroll;
};

constexpr int kStageMaxBytesPerWave = 16384;  // LDS per wave: rows up to 16 KiB of blocks

// PARTS waves per row: wave p of a row stages and decodes blocks [nblk p / PARTS,
// nblk (p + 1) / PARTS) of it, so a row's blocks are spread over more waves.
template <typename TO, typename Fmt, int L16, int PARTS>  // L16: 16-byte loads per lane to stage a part
__global__ __launch_bounds__(kEmbThreads) void embed_rows_staged_kernel(const int64_t* __restrict__ ids,
                                                                        const uint8_t* __restrict__ table,
                                                                        TO* __restrict__ out, int64_t tokens,
                                                                        int hidden, int64_t vocab, int stage_bytes) {
  constexpr int N = Pack<TO>::N;
  extern __shared__ __attribute__((aligned(16))) uint8_t stage[];  // kEmbWaves slices of stage_bytes
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int64_t gw = (int64_t)blockIdx.x * kEmbWaves + wave;
  const int64_t t = gw / PARTS;
  const int part = (int)(gw % PARTS);
  if (t >= tokens) return;  // wave-uniform; the wave's LDS slice is its own (no workgroup barrier)
  const int64_t id = ids[t];
  const int nblk = hidden / Fmt::kBlockElems;
  const int b0 = nblk * part / PARTS, b1 = nblk * (part + 1) / PARTS;
  const int nch = (b1 - b0) * Fmt::kBlockElems / N;
  TO* dst = out + t * hidden + (int64_t)b0 * Fmt::kBlockElems;
  if (bad_id(id, vocab)) {
    float nan[N];
#pragma unroll
    for (int i = 0; i < N; ++i) nan[i] = __builtin_nanf("");
    for (int c = lane; c < nch; c += kWave) st16(dst + c * N, Pack<TO>::pack(nan));
    return;
  }
  const uint8_t* row = table + (id * (int64_t)nblk + b0) * Fmt::kBlockBytes;
  const uintptr_t a16 = reinterpret_cast<uintptr_t>(row) & ~uintptr_t(15);
  const int delta = (int)(reinterpret_cast<uintptr_t>(row) - a16);
  const int n16 = (delta + (b1 - b0) * Fmt::kBlockBytes + 15) >> 4;
  uint8_t* my = stage + wave * stage_bytes;
  {  // LDS DMA over the stage's 16-byte chunks (lanes past them read zeros, inside the slice)
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(row - delta), (short)0, n16 * 16, 0x00020000);
#pragma unroll
    for (int u = 0; u < L16; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(my + u * kWave * 16), 16,
                                               (uint32_t)(16 * lane), (uint32_t)(u * kWave * 16), 0, 0);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint8_t* rowl = my + delta;
  if constexpr (QuadDecode<Fmt>::value) {
    // quad qi: block qi / (64 / N), half h and first element l0 of its four slots
    constexpr int kPerBlock = 64 / N, kPerHalf = 32 / N;
    for (int qi = lane; qi < nch / 4; qi += kWave) {
      const int sb = qi / kPerBlock, r = qi % kPerBlock, h = r / kPerHalf, l0 = (r % kPerHalf) * N;
      float v[4][N];
      Fmt::decode4(rowl + sb * Fmt::kBlockBytes, h, l0, v);
#pragma unroll
      for (int sl = 0; sl < 4; ++sl) st16_nt(dst + (int64_t)sb * 256 + 128 * h + 32 * sl + l0, Pack<TO>::pack(v[sl]));
    }
    return;
  }
  constexpr int U = DecodeUnroll<Fmt>::value;
  for (int c0 = 0; c0 < nch; c0 += U * kWave) {  // wave-uniform trip count: U chunks per lane, decoded, then stored
    u32x4 o[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * kWave + lane;
      if (c < nch) {
        const int e = c * N;
        float v[N];
        Fmt::decode(rowl + (e / Fmt::kBlockElems) * Fmt::kBlockBytes, e % Fmt::kBlockElems, v);
        o[u] = Pack<TO>::pack(v);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * kWave + lane;
      if (c < nch) st16_nt(dst + (int64_t)c * N, o[u]);
    }
  }
}

template <typename TO, typename Fmt>
static bool launch_staged(const int64_t* ids, const uint8_t* table, TO* out, int64_t tokens, int64_t hidden,
                          int64_t vocab, hipStream_t st) {
  const int64_t row_bytes = hidden / Fmt::kBlockElems * Fmt::kBlockBytes;
  // the stage starts at the 16-byte boundary at or below the row: one chunk more
  const int64_t n16 = (15 + row_bytes + 15) / 16;
  if (hidden % Fmt::kBlockElems != 0 || n16 * 16 > kStageMaxBytesPerWave || hidden > INT32_MAX) return false;
  // two waves per row when the row has at least 8 blocks (measured at Qwen2.5-7B's
  // shape: Q5_K 70.7 -> 74.3%, Q4_K 75.4 -> 76.7%, Q6_K 63.1 -> 64.3%, Q8_0 blocks
  // 67.0 -> 67.8% of 8 TB/s; four waves per row was slower for every format)
  const int parts = hidden / Fmt::kBlockElems >= 8 ? 2 : 1;
  // 16-byte chunks of the larger part: ceil(nblk / 2) blocks plus the alignment lead
  const int64_t half_blocks = (hidden / Fmt::kBlockElems + parts - 1) / parts;
  const int64_t part_n16 = parts == 1 ? n16 : (15 + half_blocks * Fmt::kBlockBytes + 15) / 16;
  const int l16 = (int)((part_n16 + kWave - 1) / kWave);
  int stage_bytes = (int)(part_n16 * 16) + SpareBytes<Fmt>::value;
  stage_bytes = std::max(stage_bytes, l16 * kWave * 16);  // every DMA lane writes its 16 bytes
  const size_t lds = (size_t)stage_bytes * kEmbWaves;
  const int64_t waves = tokens * parts;
  const dim3 grid((unsigned)((waves + kEmbWaves - 1) / kEmbWaves));
  const int h = (int)hidden;
  switch (l16 * 2 + (parts - 1)) {
#define NVF_STAGE_CASE(L)                                                                                     \
  case 2 * L:                                                                                                 \
    embed_rows_staged_kernel<TO, Fmt, L, 1><<<grid, kEmbThreads, lds, st>>>(ids, table, out, tokens, h, vocab, \
                                                                             stage_bytes);                      \
    break;                                                                                                    \
  case 2 * L + 1:                                                                                             \
    embed_rows_staged_kernel<TO, Fmt, L, 2><<<grid, kEmbThreads, lds, st>>>(ids, table, out, tokens, h, vocab, \
                                                                             stage_bytes);                      \
    break;
    NVF_STAGE_CASE(1) NVF_STAGE_CASE(2) NVF_STAGE_CASE(3) NVF_STAGE_CASE(4)
    NVF_STAGE_CASE(5) NVF_STAGE_CASE(6) NVF_STAGE_CASE(7) NVF_STAGE_CASE(8)
    NVF_STAGE_CASE(9) NVF_STAGE_CASE(10) NVF_STAGE_CASE(11) NVF_STAGE_CASE(12)
    NVF_STAGE_CASE(13) NVF_STAGE_CASE(14) NVF_STAGE_CASE(15) NVF_STAGE_CASE(16)
#undef NVF_STAGE_CASE
    default:
      return false;
  }
  return true;
}

// ---------------------------------------------------------------------------
// Layer-0 embedding + residual-add + RMSNorm in one pass (src/model.cpp:756
// then :762: the residual buffer is zero-filled, so residual = emb + 0 and
// out = RMSNorm(residual) * w).  The embedding row never exists in HBM: the
// wave gathers it into VGPRs, stores the residual, reduces the sum of squares
// with DPP and stores the normalised row -- table rows + 2 row writes instead
// of table rows + 5 row passes.  U chunks of N per lane; long rows are split
// over 4 waves.
// ---------------------------------------------------------------------------
template <typename T, typename Src, int U, int WPR>
__global__ __launch_bounds__(kEmbThreads) void embed_rms_kernel(const int64_t* __restrict__ ids, Src src,
                                                                const T* __restrict__ w, T* __restrict__ residual,
                                                                T* __restrict__ out, int64_t tokens, int hidden,
                                                                int64_t vocab, float eps) {
  constexpr int N = Pack<T>::N;
  __shared__ float partial[kEmbWaves];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int part = wave % WPR;
  const int64_t t = (int64_t)blockIdx.x * (kEmbWaves / WPR) + wave / WPR;
  const bool live = t < tokens;  // no early return: the row's waves meet at a barrier
  const int nch = hidden / N;
  const int64_t id = live ? ids[t] : 0;
  const bool bad = bad_id(id, vocab);
  const int64_t row0 = (bad ? 0 : id) * hidden;  // a bad id reads row 0, stores NaN
  typename Src::Raw raw[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = (u * WPR + part) * kWave + lane;
    if (live && c < nch) raw[u] = src.load(row0 + (int64_t)c * N);
  }
  u32x4 wa[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = (u * WPR + part) * kWave + lane;
    if (live && c < nch) wa[u] = ld16(w + (int64_t)c * N);
  }
  float v[U][N];
  float ss = 0.f;
  T* rrow = residual + (live ? t : 0) * hidden;
  T* orow = out + (live ? t : 0) * hidden;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = (u * WPR + part) * kWave + lane;
    if (live && c < nch) {
      src.decode(raw[u], v[u]);
#pragma unroll
      for (int j = 0; j < N; ++j) v[u][j] = (bad ? __builtin_nanf("") : v[u][j]) + 0.0f;  // x + the zero residual
      const u32x4 stored = Pack<T>::pack(v[u]);
      st16_nt(rrow + (int64_t)c * N, stored);
      Pack<T>::unpack(stored, v[u]);  // the norm sees the stored residual
#pragma unroll
      for (int j = 0; j < N; ++j) ss += v[u][j] * v[u][j];
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
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = (u * WPR + part) * kWave + lane;
    if (live && c < nch) {
      float g[N], o[N];
      Pack<T>::unpack(wa[u], g);
#pragma unroll
      for (int j = 0; j < N; ++j) o[j] = v[u][j] * inv * g[j];
      st16_nt(orow + (int64_t)c * N, Pack<T>::pack(o));
    }
  }
}

// Rows of >= 256 chunks are split over 4 waves (LDS combine of the partial
// sums), as in the RMSNorm kernel; shorter rows keep one wave.
template <typename T, typename Src>
static bool launch_embed_rms(const int64_t* ids, const Src& src, const T* w, T* residual, T* out, int64_t tokens,
                             int64_t hidden, int64_t vocab, float eps, hipStream_t st) {
  constexpr int N = Pack<T>::N;
  const int64_t nch = hidden / N;
  // Long rows over 4 waves; 8-bit tables over 2 when there are at least 16384 rows
  // (measured, fp16 / bf16 out: 16384 x 3584 Q8_0 52.5 against 54.5 us at 4 waves;
  // 8192 x 4096 Q8_0 31.1 against 29.8 us, and 32768 x 3584 Q4_K 81-83 against
  // 79-81 us, so those keep 4; a 4-workgroup residency cap was slower everywhere)
  constexpr bool k8 = std::is_same<Src, Q8Split<N>>::value || std::is_same<Src, Q8Blocks<N>>::value;
  const int wpr = nch < 4 * kWave ? 1
                  : k8 && tokens >= 16384 && nch <= 2 * 16 * kWave ? 2
                                                                   : 4;
  const int64_t per_lane = (nch + wpr * kWave - 1) / (wpr * kWave);
  if (per_lane < 1 || per_lane > 16) return false;
  const dim3 grid((unsigned)((tokens + kEmbWaves / wpr - 1) / (kEmbWaves / wpr)));
  const int h = (int)hidden;
#define NVF_ER_LAUNCH(UU, W) \
  embed_rms_kernel<T, Src, UU, W><<<grid, kEmbThreads, 0, st>>>(ids, src, w, residual, out, tokens, h, vocab, eps)
  if (wpr == 1) {
    switch (per_lane) {
#define NVF_ER_CASE(UU) case UU: NVF_ER_LAUNCH(UU, 1); break;
      NVF_ER_CASE(1) NVF_ER_CASE(2) NVF_ER_CASE(3) NVF_ER_CASE(4)
#undef NVF_ER_CASE
      default: return false;
    }
  } else if (wpr == 2) {
    switch (per_lane) {
#define NVF_ER_CASE(UU) case UU: NVF_ER_LAUNCH(UU, 2); break;
      NVF_ER_CASE(1) NVF_ER_CASE(2) NVF_ER_CASE(3) NVF_ER_CASE(4) NVF_ER_CASE(5) NVF_ER_CASE(6) NVF_ER_CASE(7)
      NVF_ER_CASE(8) NVF_ER_CASE(9) NVF_ER_CASE(10) NVF_ER_CASE(11) NVF_ER_CASE(12) NVF_ER_CASE(13) NVF_ER_CASE(14)
      NVF_ER_CASE(15) NVF_ER_CASE(16)
#undef NVF_ER_CASE
    }
  } else {
    switch (per_lane) {
#define NVF_ER_CASE(UU) case UU: NVF_ER_LAUNCH(UU, 4); break;
      NVF_ER_CASE(1) NVF_ER_CASE(2) NVF_ER_CASE(3) NVF_ER_CASE(4) NVF_ER_CASE(5) NVF_ER_CASE(6) NVF_ER_CASE(7)
      NVF_ER_CASE(8) NVF_ER_CASE(9) NVF_ER_CASE(10) NVF_ER_CASE(11) NVF_ER_CASE(12) NVF_ER_CASE(13) NVF_ER_CASE(14)
      NVF_ER_CASE(15) NVF_ER_CASE(16)
#undef NVF_ER_CASE
      default: return false;
    }
  }
#undef NVF_ER_LAUNCH
  return true;
}

// ---------------------------------------------------------------------------
// Generic K-quant element decode (hidden not a multiple of 256).
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
  constexpr int N = Pack<TO>::N;
  TO* o = static_cast<TO*>(out);
  const bool row_ok = hidden % 32 == 0 && hidden <= INT32_MAX && aligned16(out);
  if (blocks) {
    if (row_ok && launch_staged<TO, StagedQ8Blocks<N>>(ids, blocks, o, tokens, hidden, vocab, st))
      return launch_status("embedding_q8_0_blocks(staged)");
    if (row_ok && (reinterpret_cast<uintptr_t>(blocks) & 3u) == 0)
      return launch_rows<TO, Q8Blocks<N>, 1>(ids, Q8Blocks<N>{blocks}, o, tokens, hidden, vocab, st,
                                                 "embedding_q8_0_blocks");
  } else if (row_ok && (reinterpret_cast<uintptr_t>(w8) & 7u) == 0 && (reinterpret_cast<uintptr_t>(ws) & 1u) == 0) {
    // Residency cap for long gathers: the table rows are cold random HBM reads, and with every wave
    // slot filled (8 workgroups per CU) the reads of 8192 rows are in flight at once.  Measured on
    // MI355X at 16384 x 3584 with the rows not in the Infinity Cache: 4 workgroups per CU (forced
    // by 40 KiB of unused dynamic LDS out of 160 KiB) take 31.5 us against 32.5 us; 3 or fewer
    // take 40 us.  A grid that fits in about one round at full residency (8192 x 4096: 2048
    // workgroups) gains nothing and keeps every slot.
    const int64_t groups = (tokens + kEmbWaves - 1) / kEmbWaves;
    const size_t occ_lds = groups >= kEmbCapMinGroups ? kEmbCapLds : 0;
    return launch_rows<TO, Q8Split<N>, 1>(ids, Q8Split<N>{w8, ws}, o, tokens, hidden, vocab, st, "embedding_q8_0",
                                          occ_lds);
  }
  const int64_t total = tokens * hidden;
  embed_q8_generic_kernel<TO><<<grid_for(total), kEmbThreads, 0, st>>>(ids, w8, ws, blocks, o, total, hidden, vocab);
  return launch_status("embedding_q8_0(generic)");
}

template <typename TO>
static int launch_qk(const int64_t* ids, const uint8_t* wq, int64_t tokens, int64_t hidden, int64_t vocab, int kind,
                     int layout, void* out, hipStream_t st) {
  constexpr int N = Pack<TO>::N;
  TO* o = static_cast<TO*>(out);
  if (hidden % 256 == 0 && hidden <= INT32_MAX && aligned16(wq) && aligned16(out)) {
    // rows up to the 16 KiB stage: LDS-staged (measured faster for every
    // K-quant); longer rows: the direct per-chunk loads below
    bool staged = false;
    if (kind == NVF_Q5_K)
      staged = launch_staged<TO, StagedQ5K<N>>(ids, wq, o, tokens, hidden, vocab, st);
    else if (kind == NVF_Q6_K)
      staged = launch_staged<TO, StagedQ6KQuad<N>>(ids, wq, o, tokens, hidden, vocab, st);
    else if (layout == NVF_QK_LAYOUT_GGML)
      staged = launch_staged<TO, StagedQ4K<N, NVF_QK_LAYOUT_GGML>>(ids, wq, o, tokens, hidden, vocab, st);
    else
      staged = launch_staged<TO, StagedQ4K<N, NVF_QK_LAYOUT_HIP_LEGACY>>(ids, wq, o, tokens, hidden, vocab, st);
    if (staged) return launch_status("embedding_qk(staged)");
    if (kind == NVF_Q5_K)
      return launch_rows<TO, Q5K<N>, 4>(ids, {wq}, o, tokens, hidden, vocab, st, "embedding_q5_k");
    if (kind == NVF_Q6_K)
      return launch_rows<TO, Q6K<N>, 4>(ids, {wq}, o, tokens, hidden, vocab, st, "embedding_q6_k");
    if (layout == NVF_QK_LAYOUT_GGML)
      return launch_rows<TO, Q4K<N, NVF_QK_LAYOUT_GGML>, 4>(ids, {wq}, o, tokens, hidden, vocab, st, "embedding_q4_k");
    return launch_rows<TO, Q4K<N, NVF_QK_LAYOUT_HIP_LEGACY>, 4>(ids, {wq}, o, tokens, hidden, vocab, st,
                                                                "embedding_q4_k");
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
  constexpr int N = Pack<TO>::N;
  const TI* tb = static_cast<const TI*>(table);
  TO* o = static_cast<TO*>(out);
  if (hidden % 8 == 0 && hidden <= INT32_MAX && aligned16(table) && aligned16(out)) {
    // the Q8_0 gather's residency cap: at 16384 x 3584 fp16, 43.2 -> 42.6 us (68.0 -> 69.1% of
    // 8 TB/s); two waves per row were slower (46.8 us)
    const int64_t groups = (tokens + kEmbWaves - 1) / kEmbWaves;
    const size_t occ_lds = groups >= kEmbCapMinGroups ? kEmbCapLds : 0;
    return launch_rows<TO, Table<N, TI>, 1>(ids, Table<N, TI>{tb}, o, tokens, hidden, vocab, st, "embedding",
                                            occ_lds);
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

extern "C" int nvf_embedding_rms_norm(const int64_t* ids, int format, const void* table, const void* scales,
                                      int64_t tokens, int64_t hidden, int64_t vocab, const void* weight,
                                      void* residual, void* out, float eps, int dtype, void* stream) {
  const int c = check_common("nvf_embedding_rms_norm", ids, table, out, tokens, hidden, dtype);
  if (c) return c < 0 ? c : NVF_OK;
  if (!weight || !residual) return fail(NVF_ERR_INVALID, "nvf_embedding_rms_norm: NULL weight or residual");
  if (format == NVF_EMB_Q8_0 && !scales) return fail(NVF_ERR_INVALID, "nvf_embedding_rms_norm: NULL scale plane");
  const int64_t blk = format == NVF_EMB_Q8_0 || format == NVF_EMB_Q8_0_BLOCKS ? 32 : 256;
  if ((format != NVF_EMB_Q8_0 && format != NVF_EMB_Q8_0_BLOCKS && format != NVF_EMB_Q4_K &&
       format != NVF_EMB_Q5_K && format != NVF_EMB_Q6_K) ||
      hidden % blk != 0 || hidden > INT32_MAX)
    return fail(NVF_ERR_INVALID, "nvf_embedding_rms_norm: format %d needs hidden %% %lld == 0 (got %lld)", format,
                (long long)blk, (long long)hidden);
  const uint8_t* tb = static_cast<const uint8_t*>(table);
  const bool aligned = aligned16(weight) && aligned16(residual) && aligned16(out) &&
                       (format == NVF_EMB_Q8_0 ? ((reinterpret_cast<uintptr_t>(tb) & 7u) == 0 &&
                                                 (reinterpret_cast<uintptr_t>(scales) & 1u) == 0)
                        : format == NVF_EMB_Q8_0_BLOCKS || format == NVF_EMB_Q6_K
                            ? (reinterpret_cast<uintptr_t>(tb) & 3u) == 0
                            : aligned16(tb));
  if (!aligned) return fail(NVF_ERR_INVALID, "nvf_embedding_rms_norm: misaligned pointer");
  bool ok = false;
  hipStream_t st = as_stream(stream);
  NVF_DISPATCH_DTYPE(dtype, T, {
    constexpr int N = Pack<T>::N;
    const T* wp = static_cast<const T*>(weight);
    T* rp = static_cast<T*>(residual);
    T* op = static_cast<T*>(out);
    if (format == NVF_EMB_Q8_0)
      ok = launch_embed_rms(ids, Q8Split<N>{tb, static_cast<const uint16_t*>(scales)}, wp, rp, op, tokens, hidden,
                            vocab, eps, st);
    else if (format == NVF_EMB_Q8_0_BLOCKS)
      ok = launch_embed_rms(ids, Q8Blocks<N>{tb}, wp, rp, op, tokens, hidden, vocab, eps, st);
    else if (format == NVF_EMB_Q4_K)
      ok = launch_embed_rms(ids, Q4K<N, NVF_QK_LAYOUT_GGML>{tb}, wp, rp, op, tokens, hidden, vocab, eps, st);
    else if (format == NVF_EMB_Q5_K)
      ok = launch_embed_rms(ids, Q5K<N>{tb}, wp, rp, op, tokens, hidden, vocab, eps, st);
    else
      ok = launch_embed_rms(ids, Q6K<N>{tb}, wp, rp, op, tokens, hidden, vocab, eps, st);
  });
  if (!ok)
    return fail(NVF_ERR_INVALID, "nvf_embedding_rms_norm: hidden %lld exceeds the fused row (4 x 16 x 64 chunks)",
                (long long)hidden);
  return launch_status("embedding_rms_norm");
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

// The nibble order the drop-in hip_embedding_qk reads Q4_K in: GGML (GGUF files) by
// default, or HIP_LEGACY to reproduce the reference's own device decoder
// (src/hip_ops.hip:130-140) bit for bit.  Process-wide.
static std::atomic<int> g_dropin_q4k_layout{NVF_QK_LAYOUT_GGML};
int nvf::dropin_q4k_layout() { return g_dropin_q4k_layout.load(); }

extern "C" int nvf_set_dropin_q4k_layout(int layout) {
  if (layout != NVF_QK_LAYOUT_GGML && layout != NVF_QK_LAYOUT_HIP_LEGACY)
    return fail(NVF_ERR_INVALID, "nvf_set_dropin_q4k_layout: bad layout %d", layout);
  g_dropin_q4k_layout.store(layout);
  return NVF_OK;
}

extern "C" void hip_embedding_qk(const int64_t* ids, const uint8_t* wq, int tokens, int hidden, float* out, int kind) {
  if (tokens <= 0 || hidden <= 0) return;
  dropin_check(nvf_embedding_qk(ids, wq, tokens, hidden, 0, kind, g_dropin_q4k_layout.load(), out, NVF_F32, nullptr),
               "hip_embedding_qk");
}
