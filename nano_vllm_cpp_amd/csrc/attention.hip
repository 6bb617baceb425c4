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
//   head dimensions.  fp32 math; it serves the fp32 drop-in, decode batches and
//   the shapes and tiles the tiled kernel does not take.
// * fa_prefill_kernel: 128-query tiles of one sequence on the matrix cores;
//   fa_decode_kernel: the remaining (decode-shaped) tokens, one workgroup per
//   (token, kv head) on the matrix cores, its 4 waves splitting the keys.
#include <hip/hip_runtime.h>

#include <math.h>

#include <algorithm>
#include <mutex>
#include <vector>

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
// Prefill tiles on the matrix cores: 16-bit q and cache, head_dim 128, block
// sizes a multiple of 64 (the reference's are multiples of 256,
// include/nanovllm/config.hpp:254).  A workgroup owns kFaBq = 128 consecutive
// query tokens of one sequence and one query head (32 per wave) and walks the
// keys in 64-key chunks staged in LDS by DMA: K double-buffered (the next chunk's
// K in flight during the softmax and PV), V single-buffered (the next chunk's V
// in flight during S and the softmax; a second barrier per chunk guards it).  48
// KiB of LDS and at most 168 VGPRs per wave: three workgroups per CU.
//
// Per wave and chunk, with 32x32x16 MFMAs:
//   S^T = K . Q^T   (keys x queries: A = K rows from LDS, B = the wave's q rows,
//                    held in registers for the whole tile)
//   online softmax per query -- a query is a lane column of S^T, so its max,
//                    sum and the O rescale are lane-local plus one swap with the
//                    other lane half
//   O^T += V^T . P^T (dims x queries: A = V^T by transpose reads of V's LDS rows; B = P^T,
//                    which is S^T's own register layout: the 8 values a lane
//                    holds for keys 16u + 4h + {0..3, 8..11} are its B operand
//                    for key step u once both operands index keys that way)
// P is rounded to the cache dtype for the MFMA; the row sums use the fp32 P.
// Tiles whose tokens span sequences (or are partial at a sequence switch) are
// left to attn_wave_kernel, which applies the same predicate.
constexpr int kFaHd = 128;
constexpr int kFaBq = 128;                       // query tokens per workgroup
constexpr int kFaBk = 64;                        // keys per chunk
constexpr float kFaLazy = 8.0f;                  // exp2 units the running max may lag behind (16-bit tiles)
// K row in LDS, written by DMA: unpadded, its 16-byte units swizzled by row
// (conflict-free 16 B reads)
constexpr int kFaKRow = kFaHd * 2;
constexpr int kFaKBytes = kFaBk * kFaKRow;
// V rows in LDS, written by DMA as K's: unpadded, 16-byte unit u of key row r at
// position u ^ 4 (r % 4), read transposed (ds_read_b64_tr_b16) into the MFMA operand
// [K chunk buffer 0][K chunk buffer 1][V chunk]: 48 KiB, three workgroups per CU
constexpr int kFaLds = 3 * kFaKBytes;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma16;
template <>
struct Mfma16<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma16<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 mma(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// True iff every token of the kFaBq-token tile `tile` (those < tokens) belongs to
// one sequence.  Evaluated per wave; every wave of a workgroup gets the same answer.
__device__ __forceinline__ bool fa_tile_uniform(const int32_t* __restrict__ qseq, int64_t tokens, int64_t tile) {
  const int lane = threadIdx.x & 63;
  const int64_t t0 = tile * kFaBq;
  const int32_t s0 = qseq[t0];
  bool same = true;
#pragma unroll
  for (int i = 0; i < kFaBq / 64; ++i) {
    const int64_t t = t0 + lane + 64 * i;
    if (t < tokens) same = same && qseq[t] == s0;
  }
  return __all(same);
}

template <typename T, bool SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void fa_prefill_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kc, const T* __restrict__ vc,
    const int32_t* __restrict__ qseq, const int32_t* __restrict__ qlen, const int32_t* __restrict__ tables,
    int64_t tokens, int q_heads, int kv_heads, int bs, int max_blocks, float scale_log2, int64_t q_stride,
    int64_t tiles, int split_keys, float* __restrict__ part) {
  using M = Mfma16<T>;
  using v8 = typename M::v8;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int half = lane >> 5;
  const int64_t bid = blockIdx.x;
  const int64_t tile = tiles - 1 - bid / q_heads;  // the longest tiles (latest positions) first
  const int h = (int)(bid % q_heads);
  const int64_t t0 = tile * kFaBq;
  if (!fa_tile_uniform(qseq, tokens, tile)) return;  // the whole workgroup: left to attn_wave_kernel
  const int64_t seq = qseq[t0];
  const int kvh = h / (q_heads / kv_heads);
  const int64_t kv_stride = (int64_t)kv_heads * kFaHd;
  const int32_t* tab = tables + seq * max_blocks;

  // the tile's longest key range (every wave computes the same value)
  float lmax = 0.0f;
#pragma unroll
  for (int i = 0; i < kFaBq / 64; ++i) {
    const int64_t t = t0 + lane + 64 * i;
    if (t < tokens) lmax = fmaxf(lmax, (float)qlen[t]);
  }
  const int Lmax = (int)wave_max(lmax);
  const int nchunks = (Lmax + kFaBk - 1) / kFaBk;

  // this lane's query (a column of S^T and O^T)
  const int64_t tq = t0 + 32 * wave + (lane & 31);
  const bool q_ok = tq < tokens;
  const int L = q_ok ? qlen[tq] : 0;
  // the smallest key count among the wave's queries (chunks below it need no mask)
  // (a wave with no query in range takes the masked path; its outputs are not stored)
  const float lmin = -wave_max(q_ok ? -(float)L : -INFINITY);
  const int Lmin = lmin < 2.0e9f ? (int)lmin : 0;
  v8 qf[kFaHd / 16];
#pragma unroll
  for (int s = 0; s < kFaHd / 16; ++s) {
    const u32x4 v = q_ok ? ld16(q + tq * q_stride + (int64_t)h * kFaHd + 16 * s + 8 * half) : u32x4{0, 0, 0, 0};
    qf[s] = __builtin_bit_cast(v8, v);
  }

  // K and V by LDS DMA: transfer i of wave w takes key rows 16 w + 4 i + lane / 16
  // whole, lane l fetching the 16-byte unit that belongs at position l % 16: for K
  // unit (l % 16) ^ (row % 16), for V unit (l % 16) ^ 4 (row % 4).  (Through
  // registers and padded LDS rows, K ran 614 against 594 us at config 2.)  Keys
  // past the tile's range may hold anything: V's resource ends at the range, so
  // those rows arrive as zeros (their p is 0, and 0 * NaN would not be); K's are
  // masked in the scores.
  uint32_t k_off[4], v_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * wave + 4 * i + (lane >> 4);
    const uint32_t rb = (uint32_t)((int64_t)row * kv_stride * sizeof(T));
    k_off[i] = rb + 16u * (uint32_t)((lane & 15) ^ (row & 15));
    v_off[i] = rb + 16u * (uint32_t)((lane & 15) ^ (4 * (row & 3)));
  }
  auto chunk_head = [&](int c) {
    const int k0 = c * kFaBk;
    const int64_t row0 = (int64_t)tab[k0 / bs] * bs + k0 % bs;
    return row0 * kv_stride + (int64_t)kvh * kFaHd;
  };
  auto load_k = [&](int c, uint8_t* dst) {
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(kc + chunk_head(c)), (short)0, (int)(kFaBk * kv_stride * sizeof(T)), 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rk, (__attribute__((address_space(3))) void*)(dst + (16 * wave + 4 * i) * kFaKRow), 16, k_off[i], 0, 0, 0);
  };
  auto load_v = [&](int c, uint8_t* dst) {
    const int k0 = c * kFaBk;
    const int vrows = Lmax - k0 < kFaBk ? Lmax - k0 : kFaBk;
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(vc + chunk_head(c)), (short)0, (int)(vrows * kv_stride * sizeof(T)), 0x00020000);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rv, (__attribute__((address_space(3))) void*)(dst + (16 * wave + 4 * i) * kFaKRow), 16, v_off[i], 0, 0, 0);
  };

  // The PV operand by transpose reads.  ds_read_b64_tr_b16 over a 16-lane group:
  // lane i receives, as its element e, 16-bit element i % 4 of the 8 bytes that
  // lane 4 e + i / 4 addresses.  So when lane s of the group addresses key row
  // key0 + s / 4, dims dim0 + 4 (s % 4) .. + 3, lane i receives dim dim0 + i of
  // keys key0 .. key0 + 3: the A operand (row = dim, k = key) of the 32x32x16 MFMA.
  // Lane l: dims 32 d + 16 ((l >> 4) & 1) + 4 (s % 4), keys 4 half + s / 4 (+ 8 for
  // the operand's second half) past the key step's first, s = l % 16.  Its 16-byte
  // unit 4 d + 2 ((l >> 4) & 1) + (s % 4) / 2 sits at that ^ 4 (key % 4) = ^ 4 (s / 4):
  // a lane base per d; the key step and the half are row offsets.  Each 32-lane half
  // of a read covers 4 keys x 4 units, at 16 distinct positions of one 256-byte row
  // span: no bank conflicts.
  uint32_t v_lane[kFaHd / 32];
  {
    const int s16 = lane & 15, g16 = (lane >> 4) & 1;
#pragma unroll
    for (int d = 0; d < kFaHd / 32; ++d)
      v_lane[d] = (uint32_t)((4 * half + s16 / 4) * kFaKRow + 16 * ((4 * d + 2 * g16 + (s16 & 3) / 2) ^ (4 * (s16 / 4))) +
                             8 * (s16 & 1));
  }

  f32x16 o[kFaHd / 32];
#pragma unroll
  for (int d = 0; d < kFaHd / 32; ++d) o[d] = f32x16{};
  float m = -INFINITY, l = 0.0f;

  // this workgroup's chunks: all of the tile's, or split blockIdx.z's split_keys keys
  int c0 = 0, c1 = nchunks;
  if constexpr (SPLIT) {
    c0 = (int)blockIdx.z * (split_keys / kFaBk);
    c1 = min(c1, c0 + split_keys / kFaBk);
  }
  uint8_t* const vbuf = lds + 2 * kFaKBytes;
  if (c0 < c1) {
    load_k(c0, lds);
    load_v(c0, vbuf);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the K transfers are in LDS
  __syncthreads();
  for (int c = c0; c < c1; ++c) {
    const uint8_t* buf = lds + ((c - c0) & 1) * kFaKBytes;
    // S^T = K . Q^T for keys [32 kt, 32 kt + 32)
    // (the two key tiles' MFMA chains interleaved: neither waits on its own accumulator)
    f32x16 st[2] = {f32x16{}, f32x16{}};
    // Wave priority over the MFMA blocks (S 2 here, PV 1 below), 0 over the softmax: a
    // SIMD's three waves then hand its issue slots to the one with matrix work first, and
    // the others' softmax fills the MFMAs' shadow (config 2: 545 -> 536 us with 1 for
    // both, 555 -> 545 with S above PV on another box; raising the softmax instead: 539).
    __builtin_amdgcn_s_setprio(2);
#pragma unroll
    for (int s = 0; s < kFaHd / 16; ++s)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int kr = 32 * kt + (lane & 31), ku = 2 * s + half;  // K row, 16-byte unit
        const v8 a = __builtin_bit_cast(v8, ld16(buf + kr * kFaKRow + 16 * (ku ^ (kr & 15))));
        st[kt] = M::mma(a, qf[s], st[kt]);
      }
    __builtin_amdgcn_s_setprio(0);
    if (c + 1 < c1) load_k(c + 1, lds + ((c + 1 - c0) & 1) * kFaKBytes);  // in flight during the softmax and PV
    // online softmax for this lane's query; element j of tile kt is key
    // c*64 + 32 kt + 8 (j/4) + 4 half + j%4.  The running max m is kept in
    // exp2 units (score * scale_log2); since scale_log2 > 0 and rounding is
    // monotonic, the max of the raw scores times scale_log2 is exactly the max
    // of the scaled ones, and each p takes one fma into exp2.
    // (four independent max and sum chains, not one chain of 32 dependent ops)
    float mx4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    if ((c + 1) * kFaBk <= Lmin) {  // every key of the chunk is visible to every query of the wave
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int j = 0; j < 16; ++j) mx4[j & 3] = fmaxf(mx4[j & 3], st[kt][j]);
    } else {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = c * kFaBk + 32 * kt + 8 * (j >> 2) + 4 * half + (j & 3);
          const float x = key < L ? st[kt][j] : -INFINITY;
          st[kt][j] = x;
          mx4[j & 3] = fmaxf(mx4[j & 3], x);
        }
    }
    float mx = fmaxf(fmaxf(mx4[0], mx4[1]), fmaxf(mx4[2], mx4[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // Lazy running max: m moves (and O and l are rescaled) only when some query of the
    // wave would see a weight above 2^kFaLazy under the current m.  Otherwise the chunk's
    // weights are taken against the stale m, at most 2^kFaLazy.  O and l always share one
    // m, so out = O / l is unchanged; only the point where the 16-bit P rounds moves,
    // with the same relative precision.  With m = -inf (every key so far masked) any
    // finite candidate moves it.
    const float m_cand = fmaxf(m, mx * scale_log2);
    if (__any(m_cand > m + kFaLazy)) {
      const float alpha = __builtin_amdgcn_exp2f(m - (m_cand == -INFINITY ? 0.0f : m_cand));
      l *= alpha;
#pragma unroll
      for (int d = 0; d < kFaHd / 32; ++d) o[d] *= alpha;
      m = m_cand;
    }
    const float m_use = m == -INFINITY ? 0.0f : m;
    float ls4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    v8 pb[2][2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = __builtin_amdgcn_exp2f(fmaf(st[kt][j], scale_log2, -m_use));
        ls4[j & 3] += p;
        pb[kt][j >> 3][j & 7] = (T)p;
      }
    float ls = (ls4[0] + ls4[1]) + (ls4[2] + ls4[3]);
    ls += __shfl_xor(ls, 32);
    l += ls;
    // O^T += V^T . P^T, key step u of tile kt: keys 32 kt + 16 u + 4 half + {0..3, 8..11},
    // P^T's keys, and V^T's by two transpose reads (+0 and +8 key rows)
    // V(c): issued after the previous chunk's second barrier, before K(c + 1).  (Bare
    // barriers: a workgroup fence would add a vmcnt(0) and drain K(c + 1); the
    // wavefront fences keep the compiler's LDS accesses on their side.)
    if (c > c0) {
      if (c + 1 < c1)
        __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4): all but K(c + 1)
      else
        __builtin_amdgcn_s_waitcnt(0x0F70);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    const uint8_t* vt = vbuf;
    __builtin_amdgcn_s_setprio(1);
    // (the four dim tiles' MFMA chains interleaved)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int d = 0; d < kFaHd / 32; ++d) {
          typedef short s16x4 __attribute__((ext_vector_type(4)));
          const uint8_t* r = vt + v_lane[d] + (32 * kt + 16 * u) * kFaKRow;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(r));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(r + 8 * kFaKRow));
          o[d] = M::mma(__builtin_bit_cast(v8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)), pb[kt][u],
                        o[d]);
        }
    if (c + 1 < c1) {
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): K(c + 1) is in LDS
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_s_barrier();  // and every wave is done with V(c)
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      load_v(c + 1, vbuf);
    }
  }

  // O^T layout: lane column = query, dims 32 d + 8 (j/4) + 4 half + j%4
  if constexpr (SPLIT) {  // unnormalised partial O, running max (exp2 units) and sum
    if (q_ok) {
      const int64_t pi = (tq * q_heads + h) * gridDim.z + blockIdx.z;
      float* po = part + pi * kFaHd;
#pragma unroll
      for (int d = 0; d < kFaHd / 32; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          st16(po + 32 * d + 8 * g + 4 * half,
               __builtin_bit_cast(u32x4, f32x4{o[d][4 * g], o[d][4 * g + 1], o[d][4 * g + 2], o[d][4 * g + 3]}));
      if (half == 0) {
        float* pml = part + tokens * q_heads * gridDim.z * kFaHd + 2 * pi;
        pml[0] = m;
        pml[1] = l;
      }
    }
  } else if (q_ok) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    T* orow = out + (tq * q_heads + h) * kFaHd;
#pragma unroll
    for (int d = 0; d < kFaHd / 32; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (T)(o[d][4 * g + e] * inv);
        *reinterpret_cast<t4*>(orow + 32 * d + 8 * g + 4 * half) = v;
      }
  }
}

// ---------------------------------------------------------------------------
// fp32 caches (the reference's own KV dtype) on the fp32 matrix cores,
// v_mfma_f32_32x32x2_f32 (exact fp32 products, fp32 sums).  The tiles are
// fa_prefill_kernel's (128 queries of one head, 4 waves of 32 queries, the same
// uniform-tile rule), over 32-key chunks:
//   S^T = K . Q^T   64 MFMAs over the 128 dims.  MFMA s contracts dim
//                   64 (lane / 32) + s, so a lane's A and B operands of 4
//                   consecutive MFMAs are 16 consecutive bytes of its K row / q.
//   O^T += V^T . P^T  MFMA s contracts key 8 (s / 4) + 4 (lane / 32) + s % 4,
//                   the key S^T's register s of this lane holds, so P^T is
//                   those registers as they are.  Row r of O^T tile d is dim
//                   4 r + d: the 4 tiles' A operands for one key are 16
//                   consecutive bytes of V's own row, read without a transpose.
constexpr int kF32Bk = 32;                       // keys per chunk
constexpr int kF32KRow = kFaHd * 4 + 16;         // K row in LDS: 528 B, the 8 lanes of a 16 B read phase on distinct banks
constexpr int kF32VRow = kFaHd * 4;              // V row in LDS: 512 B (read along the row)
constexpr int kF32KBytes = kF32Bk * kF32KRow;
constexpr int kF32Stage = kF32KBytes + kF32Bk * kF32VRow;
constexpr int kF32Lds = 2 * kF32Stage;           // 66560 B: two workgroups per CU

template <bool SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void fa_prefill_f32_kernel(
    const float* __restrict__ q, float* __restrict__ out, const float* __restrict__ kc, const float* __restrict__ vc,
    const int32_t* __restrict__ qseq, const int32_t* __restrict__ qlen, const int32_t* __restrict__ tables,
    int64_t tokens, int q_heads, int kv_heads, int bs, int max_blocks, float scale_log2, int64_t q_stride,
    int64_t tiles, int split_keys, float* __restrict__ part) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int half = lane >> 5;
  const int64_t bid = blockIdx.x;
  const int64_t tile = tiles - 1 - bid / q_heads;  // the longest tiles (latest positions) first
  const int h = (int)(bid % q_heads);
  const int64_t t0 = tile * kFaBq;
  if (!fa_tile_uniform(qseq, tokens, tile)) return;  // the whole workgroup: left to attn_wave_kernel
  const int64_t seq = qseq[t0];
  const int kvh = h / (q_heads / kv_heads);
  const int64_t kv_stride = (int64_t)kv_heads * kFaHd;
  const int32_t* tab = tables + seq * max_blocks;

  float lmax = 0.0f;
#pragma unroll
  for (int i = 0; i < kFaBq / 64; ++i) {
    const int64_t t = t0 + lane + 64 * i;
    if (t < tokens) lmax = fmaxf(lmax, (float)qlen[t]);
  }
  const int Lmax = (int)wave_max(lmax);
  const int nchunks = (Lmax + kF32Bk - 1) / kF32Bk;

  const int64_t tq = t0 + 32 * wave + (lane & 31);
  const bool q_ok = tq < tokens;
  const int L = q_ok ? qlen[tq] : 0;
  const float lmin = -wave_max(q_ok ? -(float)L : -INFINITY);
  const int Lmin = lmin < 2.0e9f ? (int)lmin : 0;
  // B operand of S^T: this lane's query, dims 64 half + 4 i + e
  f32x4 qf[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    qf[i] = q_ok ? __builtin_bit_cast(f32x4, ld16(q + tq * q_stride + (int64_t)h * kFaHd + 64 * half + 4 * i))
                 : f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // chunk loads: rows ld_r + 8 i (i < 4) of K and V, 16 B column ld_c of each
  const int tid = threadIdx.x;
  const int ld_c = tid & 31, ld_r = tid >> 5;
  u32x4 kreg[4], vreg[4];
  auto load_chunk = [&](int c) {
    const int k0 = c * kF32Bk;
    const int64_t row0 = (int64_t)tab[k0 / bs] * bs + k0 % bs;
    const float* kb = kc + row0 * kv_stride + (int64_t)kvh * kFaHd + ld_c * 4;
    const float* vb = vc + row0 * kv_stride + (int64_t)kvh * kFaHd + ld_c * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = ld_r + 8 * i;
      kreg[i] = ld16(kb + (int64_t)key * kv_stride);
      // keys past the tile's range may hold anything: zero their V (their p is 0).
      // The row itself lies inside the chunk's block, so the load is unconditional
      // and only the value is selected (no branch around the load).
      const u32x4 v = ld16(vb + (int64_t)key * kv_stride);
      vreg[i] = k0 + key < Lmax ? v : u32x4{0, 0, 0, 0};
    }
  };
  auto store_chunk = [&](uint8_t* st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      st16(st + (ld_r + 8 * i) * kF32KRow + ld_c * 16, kreg[i]);
      st16(st + kF32KBytes + (ld_r + 8 * i) * kF32VRow + ld_c * 16, vreg[i]);
    }
  };

  f32x16 o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) o[d] = f32x16{};
  float m = -INFINITY, l = 0.0f;

  // this workgroup's chunks: all of the tile's, or split blockIdx.z's split_keys keys
  int c0 = 0, c1 = nchunks;
  if constexpr (SPLIT) {
    c0 = (int)blockIdx.z * (split_keys / kF32Bk);
    c1 = min(c1, c0 + split_keys / kF32Bk);
  }
  if (c0 < c1) {
    load_chunk(c0);
    store_chunk(lds);
  }
  __syncthreads();
  for (int c = c0; c < c1; ++c) {
    const uint8_t* buf = lds + ((c - c0) & 1) * kF32Stage;
    if (c + 1 < c1) load_chunk(c + 1);  // in flight during this chunk
    // S^T: lane row (key) lane & 31 of the chunk, dims 64 half + ...
    f32x16 st = f32x16{};
    // wave priority as in fa_prefill_kernel: S 2, PV 1, the softmax 0 (3957-3968 ->
    // 3900-3908 us at config 2)
    __builtin_amdgcn_s_setprio(2);
    const uint8_t* krow = buf + (lane & 31) * kF32KRow + 256 * half;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const f32x4 a = __builtin_bit_cast(f32x4, ld16(krow + 16 * i));
#pragma unroll
      for (int e = 0; e < 4; ++e) st = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qf[i][e], st, 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    // online softmax for this lane's query over its keys c*32 + 8 (j/4) + 4 half + j%4
    // (the running max in exp2 units, as in fa_prefill_kernel)
    float mx = -INFINITY;
    if ((c + 1) * kF32Bk <= Lmin) {
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, st[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = c * kF32Bk + 8 * (j >> 2) + 4 * half + (j & 3);
        const float x = key < L ? st[j] : -INFINITY;
        st[j] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // lazy running max, as in fa_prefill_kernel (P stays fp32 here: no rounding moves)
    const float m_cand = fmaxf(m, mx * scale_log2);
    if (__any(m_cand > m + kFaLazy)) {
      const float alpha = __builtin_amdgcn_exp2f(m - (m_cand == -INFINITY ? 0.0f : m_cand));
      l *= alpha;
#pragma unroll
      for (int d = 0; d < 4; ++d) o[d] *= alpha;
      m = m_cand;
    }
    const float m_use = m == -INFINITY ? 0.0f : m;
    float ls = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      st[j] = __builtin_amdgcn_exp2f(fmaf(st[j], scale_log2, -m_use));
      ls += st[j];
    }
    ls += __shfl_xor(ls, 32);
    l += ls;
    // O^T += V^T . P^T: MFMA s takes key 8 (s/4) + 4 half + s%4 (P^T = st[s]); lane
    // row r = lane & 31 of tile d is dim 4 r + d
    const uint8_t* vrow = buf + kF32KBytes + 16 * (lane & 31);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int key = 8 * (s >> 2) + 4 * half + (s & 3);
      const f32x4 a = __builtin_bit_cast(f32x4, ld16(vrow + key * kF32VRow));
#pragma unroll
      for (int d = 0; d < 4; ++d) o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[d], st[s], o[d], 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    if (c + 1 < c1) store_chunk(lds + ((c + 1 - c0) & 1) * kF32Stage);
    __syncthreads();
  }

  // O^T: lane column = query; register j of tile d is dim 4 (8 (j/4) + 4 half + j%4) + d
  if constexpr (SPLIT) {  // unnormalised partial O, running max (exp2 units) and sum
    if (q_ok) {
      const int64_t pi = (tq * q_heads + h) * gridDim.z + blockIdx.z;
      float* po = part + pi * kFaHd;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int r = 8 * (j >> 2) + 4 * half + (j & 3);
        st16(po + 4 * r, __builtin_bit_cast(u32x4, f32x4{o[0][j], o[1][j], o[2][j], o[3][j]}));
      }
      if (half == 0) {
        float* pml = part + tokens * q_heads * gridDim.z * kFaHd + 2 * pi;
        pml[0] = m;
        pml[1] = l;
      }
    }
  } else if (q_ok) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float* orow = out + (tq * q_heads + h) * kFaHd;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = 8 * (j >> 2) + 4 * half + (j & 3);
      st16(orow + 4 * r, __builtin_bit_cast(u32x4, f32x4{o[0][j] * inv, o[1][j] * inv, o[2][j] * inv, o[3][j] * inv}));
    }
  }
}

// ---------------------------------------------------------------------------
// The decode kernels' end: a workgroup is one (token, kv head) whose 4 waves each
// hold a softmax state over their share of the keys.  Each wave has written its
// unnormalised O^T as [128 dims][16 heads] floats at pw(w), then m[16] (exp2
// units, -inf for a wave without keys) and l[16].  After the barrier, thread
// (head hc = tid % 16, dims d0 = 8 (tid / 16) .. + 7) merges the 4 states and
// stores either the normalised output or the merged partial of split blockIdx.z.
template <typename TO, bool SPLIT, typename PW>
__device__ __forceinline__ void decode_merge_store(PW pw, TO* __restrict__ out, float* __restrict__ part, int64_t t,
                                                   int64_t tokens, int q_heads, int kvh, int G) {
  __syncthreads();
  const int hc = threadIdx.x & 15, d0 = 8 * (threadIdx.x >> 4);
  float mw[4], mall = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mw[w] = pw(w)[kFaHd * 16 + hc];
    mall = fmaxf(mall, mw[w]);
  }
  float lsum = 0.0f, ov[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float sc = mw[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - mall);
    const float* pv = pw(w);
    lsum += sc * pv[kFaHd * 16 + 16 + hc];
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] += sc * pv[(d0 + e) * 16 + hc];
  }
  if (hc >= G) return;  // (callers that loop re-converge at their own barrier)
  const int hq = kvh * G + hc;
  if constexpr (SPLIT) {  // unnormalised partial O, running max (exp2 units) and sum
    const int64_t pi = (t * q_heads + hq) * gridDim.z + blockIdx.z;
    float* po = part + pi * kFaHd + d0;
    st16(po, __builtin_bit_cast(u32x4, f32x4{ov[0], ov[1], ov[2], ov[3]}));
    st16(po + 4, __builtin_bit_cast(u32x4, f32x4{ov[4], ov[5], ov[6], ov[7]}));
    if (d0 == 0) {
      float* pml = part + tokens * q_heads * gridDim.z * kFaHd + 2 * pi;
      pml[0] = mall;
      pml[1] = lsum;
    }
  } else {
    const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = ov[e] * inv;
    TO* orow = out + (t * q_heads + hq) * kFaHd + d0;
    if constexpr (sizeof(TO) == 4) {
      st16(orow, __builtin_bit_cast(u32x4, f32x4{v[0], v[1], v[2], v[3]}));
      st16(orow + 4, __builtin_bit_cast(u32x4, f32x4{v[4], v[5], v[6], v[7]}));
    } else {
      typedef TO t8 __attribute__((ext_vector_type(8)));
      t8 r;
#pragma unroll
      for (int e = 0; e < 8; ++e) r[e] = (TO)v[e];
      *reinterpret_cast<t8*>(orow) = r;
    }
  }
}
constexpr int kDecMergeFloats = kFaHd * 16 + 32;  // one wave's state in the merge

// ---------------------------------------------------------------------------
// Decode-shaped attention on the matrix cores (16-bit cache, head_dim 128,
// block sizes a multiple of 64, at most 16 query heads per kv head): a wave
// streams its share of one (token, kv head)'s keys in 64-key chunks.  The query
// heads of the group are the 16 columns of v_mfma_f32_16x16x32 tiles:
//   S^T = K . Q^T    (A = 16 keys x 32 dims, K rows loaded whole and passed
//                     through the wave's LDS buffer to that layout, B = q)
//   O^T += V^T . P^T (A = V^T from a wave-private LDS transpose of the chunk,
//                     B = P^T, again S^T's own registers: a lane holds keys
//                     32 u + 4 g + {0..3} and 32 u + 16 + 4 g + {0..3}, g = lane/16)
// The next chunk's K and V loads are in flight during the current chunk's math.
// A workgroup is one (token, kv head): its 4 waves take the chunks in turn (wave w
// chunks w, w + 4, ...) and merge their softmax states through LDS at the end, so
// the longest contexts, which set a decode batch's tail, take a quarter of the
// time, without a second launch.
// V^T row (one dim): 64 keys in 16 units of 8 bytes, unit w of row r at position
// w ^ ((r / 8) % 16), rows 144 bytes apart: both the transpose's 8-byte writes and
// the operand reads take the minimum 2 LDS passes (a 8-byte pad alone: 4 and 3)
constexpr int kFdVRow = 64 * 2 + 16;
// K rows staged row-major in the same buffer first: a 16-byte pad puts the 8 rows
// of a read phase on distinct banks
constexpr int kFdKRow = kFaHd * 2 + 16;
constexpr int kFdWaveLds = kFaHd * kFdVRow;      // per wave
constexpr int kFdLds = 4 * kFdWaveLds;
static_assert(64 * kFdKRow <= kFdWaveLds, "a chunk's K rows fit the wave's V^T buffer");


// A raw buffer over `bytes` bytes at p (32-bit dwords; offsets past the end read zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t attn_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

template <typename T>
struct Mfma16x16;
template <>
struct Mfma16x16<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma16x16<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Decode batches of at most this many tokens without a host order rank their
// tokens in the kernel (each workgroup: tokens^2 / 256 comparisons).
constexpr int64_t kDecSelfOrderMax = 512;

template <typename T, bool SPLIT, bool SKIP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void fa_decode_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kc, const T* __restrict__ vc,
    const int32_t* __restrict__ qseq, const int32_t* __restrict__ qlen, const int32_t* __restrict__ tables,
    int64_t tokens, int q_heads, int kv_heads, int bs, int max_blocks, float scale_log2, int64_t q_stride,
    int split_keys, float* __restrict__ part, const int32_t* __restrict__ order) {
  using M = Mfma16x16<T>;
  using v8 = typename M::v8;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  // order (not with SKIP): the caller's permutation of the tokens over the workgroups
  // (which token each computes; the results do not depend on it)
  // Without SKIP, workgroup x is one (token, kv head): with an order, token index
  // x / kv_heads and kv head x % kv_heads -- one token's kv heads are dispatched
  // together, so a longest-first order reaches every (token, kv head) pair longest
  // first (measured at 256 sequences of U[1, 4096] keys: 186 against 200 us with
  // the kv heads outermost); without one, token x % tokens, kv head x / tokens (a
  // token's kv heads spread over the grid: 210 against 223 us for random lengths).
  const bool self_order = !SKIP && !SPLIT && !order && tokens <= kDecSelfOrderMax;
  const bool tok_major = !SKIP && (order || self_order);
  const int64_t ti = SKIP ? (int64_t)blockIdx.x
                     : tok_major ? (int64_t)blockIdx.x / kv_heads
                                 : (int64_t)blockIdx.x % tokens;
  int64_t t;
  if (self_order) {
    // No order given and few tokens: the workgroup finds its token in longest-first
    // order itself (key count descending, ties by token), dealt as
    // nvf_decode_token_order deals it (slot ti holds rank r * 8 + x, x reversed on
    // odd full rounds r of 8).  Every thread ranks its candidates against all
    // counts, staged in LDS as one distinct 64-bit key per token (the count above
    // the complemented index: a larger key ranks first, ties by token), so a
    // comparison is one compare; the one whose rank is the slot's names it.
    __shared__ int32_t sel;
    int64_t* keys = reinterpret_cast<int64_t*>(lds);
    const int n = (int)tokens;
    for (int i = threadIdx.x; i < n; i += 256) keys[i] = (int64_t)qlen[i] * 4294967296LL + (int64_t)(uint32_t)~i;
    for (int i = n + threadIdx.x; i < ((n + 1) & ~1); i += 256) keys[i] = INT64_MIN;  // pads rank below all
    __syncthreads();
    const int64_t rr = ti / 8, rx = ti % 8;
    const int64_t want = rr * 8 + ((rr & 1) && rr * 8 + 8 <= tokens ? 7 - rx : rx);
    for (int i = threadIdx.x; i < n; i += 256) {
      const int64_t ki = keys[i];
      int rank = 0;
      for (int j2 = 0; j2 < n; j2 += 2) {
        const longlong2 kj = *reinterpret_cast<const longlong2*>(keys + j2);
        rank += (kj.x > ki) + (kj.y > ki);
      }
      if (rank == want) sel = i;
    }
    __syncthreads();
    t = sel;
    __syncthreads();  // the counts' LDS is the waves' buffers below
  } else {
    t = tok_major ? (int64_t)order[ti] : ti;
  }
  if (t < 0 || t >= tokens) return;  // an order entry outside the batch: nothing to compute (uniform)
  // workgroup-uniform: the whole workgroup leaves (fa_prefill_kernel's tile)
  if (SKIP && fa_tile_uniform(qseq, tokens, t / kFaBq)) return;
  // The tiles' second launch (SKIP) has one workgroup per token, so that its many
  // exiting workgroups stay few, and walks the kv heads; otherwise the workgroup's
  // kv head (one trip).
  const int kvh0 = SKIP ? 0 : tok_major ? (int)(blockIdx.x % kv_heads) : (int)(blockIdx.x / tokens);
  const int kvh1 = SKIP ? kv_heads : kvh0 + 1;
  for (int kvh = kvh0; kvh < kvh1; ++kvh) {
    const int G = q_heads / kv_heads;
    const int col = lane & 15, g = lane >> 4;
    const bool head_ok = col < G;
    const int h = kvh * G + col;
    const int L = qlen[t];
    const int64_t seq = qseq[t];
    const int64_t kv_stride = (int64_t)kv_heads * kFaHd;
    const int32_t* tab = tables + seq * max_blocks;
    uint8_t* vt = lds + wave * kFdWaveLds;

    v8 qf[kFaHd / 32];  // B operand: head col, dims 32 s + 8 g
  #pragma unroll
    for (int s = 0; s < kFaHd / 32; ++s) {
      const u32x4 v = head_ok ? ld16(q + t * q_stride + (int64_t)h * kFaHd + 32 * s + 8 * g) : u32x4{0, 0, 0, 0};
      qf[s] = __builtin_bit_cast(v8, v);
    }
    f32x4 o[kFaHd / 16];
  #pragma unroll
    for (int d = 0; d < kFaHd / 16; ++d) o[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    // this wave's chunks: all of the token's, or split blockIdx.z's split_keys keys of them
    int c0 = 0, c1 = L > 0 ? (L + 63) / 64 : 0;
    if constexpr (SPLIT) {
      c0 = (int)blockIdx.z * (split_keys / 64);
      c1 = min(c1, c0 + split_keys / 64);
    }
    // chunk loads, K and V alike: lane l covers dims 8 (l % 16) of keys
    // 16 i + (l / 16) * 4 + {0..3} over i < 4, 16 loads each, so every load
    // instruction reads 4 whole 256-byte head rows.  (K read straight in the MFMA
    // A layout, key 16 kt + col and dims 32 s + 8 g, reads 64-byte pieces of 16 rows
    // per instruction: at 256 sequences of 1..4096 keys 187 against 184 us with the
    // K rows passed through LDS to that layout.)  A chunk's 64 cache rows lie in one
    // block, contiguous: buffer loads over that slab, the lane's part of each
    // address in one VGPR, the rest in the scalar offset, so the 32 loads take no
    // address arithmetic.  V past L is zeroed when the chunk is transposed (only the
    // sequence's last chunk has such keys).
    const uint32_t v_lane = (uint32_t)(((int64_t)4 * g * kv_stride + 8 * col) * sizeof(T));
    const uint32_t slab = (uint32_t)(64 * kv_stride * sizeof(T));
    u32x4 kr[4][4], vr[16];
    auto load_chunk = [&](int c) {
      const int k0 = c * 64;
      const int64_t row0 = (int64_t)tab[k0 / bs] * bs + k0 % bs;
      const __amdgpu_buffer_rsrc_t rk = attn_rsrc(kc + row0 * kv_stride + (int64_t)kvh * kFaHd, slab);
      const __amdgpu_buffer_rsrc_t rv = attn_rsrc(vc + row0 * kv_stride + (int64_t)kvh * kFaHd, slab);
  #pragma unroll
      for (int i = 0; i < 16; ++i)
        kr[i >> 2][i & 3] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        rk, v_lane, (uint32_t)((16 * (i >> 2) + (i & 3)) * kv_stride * sizeof(T)), 0));
  #pragma unroll
      for (int i = 0; i < 16; ++i)
        vr[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rv, v_lane, (uint32_t)((16 * (i >> 2) + (i & 3)) * kv_stride * sizeof(T)), 0));
    };
    if (c0 + wave < c1) load_chunk(c0 + wave);
    for (int c = c0 + wave; c < c1; c += 4) {
      // K rows into the wave's buffer, then back in the MFMA A layout (key 16 kt + col,
      // dims 32 s + 8 g); the V^T transpose below reuses the buffer after these reads
      // (a wave's LDS operations complete in order)
  #pragma unroll
      for (int i = 0; i < 16; ++i)
        *reinterpret_cast<u32x4*>(vt + (16 * (i >> 2) + 4 * g + (i & 3)) * kFdKRow + 16 * col) = kr[i >> 2][i & 3];
      __builtin_amdgcn_wave_barrier();
  #pragma unroll
      for (int kt = 0; kt < 4; ++kt)
  #pragma unroll
        for (int s = 0; s < 4; ++s)
          kr[kt][s] = *reinterpret_cast<const u32x4*>(vt + (16 * kt + col) * kFdKRow + 16 * (4 * s + g));
      __builtin_amdgcn_wave_barrier();
      if (c * 64 + 64 > L) {  // uniform: the last chunk, V of keys past L to zero
  #pragma unroll
        for (int i = 0; i < 16; ++i)
          if (c * 64 + 16 * (i >> 2) + 4 * g + (i & 3) >= L) vr[i] = u32x4{0, 0, 0, 0};
      }
      const int gx = g ^ col;  // (4 i4 + g) ^ col = 4 i4 ^ (g ^ col): i4 only sets bits 2, 3
      // V^T into this wave's LDS: dim 8 col + e, keys 16 i4 + 4 g + {0..3}; the
      // 16-bit values of two keys go into one dword by a byte permute
  #pragma unroll
      for (int i4 = 0; i4 < 4; ++i4)
  #pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;  // high or low halves of (b, a)
          const uint32_t lo = __builtin_amdgcn_perm(vr[4 * i4 + 1][e >> 1], vr[4 * i4][e >> 1], sel);
          const uint32_t hi = __builtin_amdgcn_perm(vr[4 * i4 + 3][e >> 1], vr[4 * i4 + 2][e >> 1], sel);
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          // row 8 col + e, unit 4 i4 + g (keys 16 i4 + 4 g + {0..3})
          *reinterpret_cast<u32x2*>(vt + (8 * col + e) * kFdVRow + 8 * ((4 * i4) ^ gx)) = u32x2{lo, hi};
        }
      // S^T = K . Q^T, 4 tiles of 16 keys
      f32x4 st[4];
  #pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        st[kt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  #pragma unroll
        for (int s = 0; s < 4; ++s) st[kt] = M::mma(__builtin_bit_cast(v8, kr[kt][s]), qf[s], st[kt]);
      }
      if (c + 4 < c1) load_chunk(c + 4);  // in flight during the math below
      __builtin_amdgcn_wave_barrier();
      // online softmax per head (lane column); element j of tile kt is key 64 c + 16 kt + 4 g + j
      float mx = -INFINITY;
  #pragma unroll
      for (int kt = 0; kt < 4; ++kt)
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = c * 64 + 16 * kt + 4 * g + j;
          const float x = key < L ? st[kt][j] * scale_log2 : -INFINITY;
          st[kt][j] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m, mx);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m - m_use);
      float ls = 0.0f;
      v8 pb[2];
  #pragma unroll
      for (int kt = 0; kt < 4; ++kt)
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float p = __builtin_amdgcn_exp2f(st[kt][j] - m_use);
          ls += p;
          pb[kt >> 1][(kt & 1) * 4 + j] = (T)p;
        }
      ls += __shfl_xor(ls, 16);
      ls += __shfl_xor(ls, 32);
      l = l * alpha + ls;
      m = m_new;
      const int gc3 = g ^ (col >> 3);
      // O^T += V^T . P^T: dims 16 d + col, key step u: keys 32 u + 4 g + {0..3}, 32 u + 16 + 4 g + {0..3}
  #pragma unroll
      for (int d = 0; d < kFaHd / 16; ++d) {
        o[d] *= alpha;  // unconditional here: interleaved with the MFMAs it costs less than a wave vote
  #pragma unroll
        for (int u = 0; u < 2; ++u) {
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          // row 16 d + col: units 8 u + g and 8 u + g + 4 (keys 32 u + 4 g + {0..3}, + 16), swizzled
          // by (2 d + col / 8); (8 u + g) ^ (2 d + col / 8) = (8 u ^ 2 d) ^ (g ^ col / 8)
          const uint8_t* r = vt + (16 * d + col) * kFdVRow;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(r + 8 * ((8 * u ^ 2 * d) ^ gc3));
          const u32x2 hi = *reinterpret_cast<const u32x2*>(r + 8 * (((8 * u + 4) ^ 2 * d) ^ gc3));
          o[d] = M::mma(__builtin_bit_cast(v8, u32x4{lo[0], lo[1], hi[0], hi[1]}), pb[u], o[d]);
        }
      }
      __builtin_amdgcn_wave_barrier();  // this chunk's V^T reads before the next chunk's writes
    }
    // Merge the 4 waves' states.  Each wave's V^T area is free now and takes its
    // O^T [128 dims][16 heads] (lane column = head col, dims 16 d + 4 g + j), then
    // m[16] and l[16]; m is in exp2 units, -inf for a wave without keys.
    float* pw = reinterpret_cast<float*>(vt);
  #pragma unroll
    for (int d = 0; d < kFaHd / 16; ++d)
  #pragma unroll
      for (int j = 0; j < 4; ++j) pw[(16 * d + 4 * g + j) * 16 + col] = o[d][j];
    if (g == 0) {
      pw[kFaHd * 16 + col] = m;
      pw[kFaHd * 16 + 16 + col] = l;
    }
    decode_merge_store<T, SPLIT>([&](int w) { return reinterpret_cast<const float*>(lds + w * kFdWaveLds); }, out, part,
                                 t, tokens, q_heads, kvh, G);
    __syncthreads();  // the merge's LDS reads before the next kv head's writes
  }
}

// ---------------------------------------------------------------------------
// Decode-shaped attention for fp32 caches on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32), head_dim 128, at most 16 query heads per kv head:
// one workgroup per (token, kv head) whose 4 waves take the chunks in turn and
// merge in LDS (as fa_decode_kernel), the group's query heads the 16 columns, 16-key
// chunks straight from the cache into registers (the next chunk's loads in
// flight during the current chunk's math; no LDS).
//   S^T = K . Q^T   32 MFMAs; MFMA 4 i + e contracts dim 16 i + 4 (lane / 16) + e,
//                   so a lane's operands are 16-byte runs of its key's K row / q,
//                   and one load instruction takes 64 bytes of each of 16 K rows.
//   O^T += V^T . P^T  MFMA u contracts key 4 (lane / 16) + u, the key S^T's
//                   register u of this lane holds (P^T = those registers); row r
//                   of O^T tile dt is dim 64 (dt / 4) + 4 r + dt % 4, so one
//                   load instruction takes 4 whole 256-byte halves of V rows.
constexpr int kFd32Bk = 16;  // keys per chunk

template <bool SPLIT, bool SKIP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void fa_decode_f32_kernel(
    const float* __restrict__ q, float* __restrict__ out, const float* __restrict__ kc, const float* __restrict__ vc,
    const int32_t* __restrict__ qseq, const int32_t* __restrict__ qlen, const int32_t* __restrict__ tables,
    int64_t tokens, int q_heads, int kv_heads, int bs, int max_blocks, float scale_log2, int64_t q_stride,
    int split_keys, float* __restrict__ part, const int32_t* __restrict__ order) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  __shared__ float merge[4][kDecMergeFloats];
  const bool tok_major = !SKIP && order;  // the workgroup's (token, kv head) as fa_decode_kernel's
  const int64_t ti = SKIP ? (int64_t)blockIdx.x
                     : tok_major ? (int64_t)blockIdx.x / kv_heads
                                 : (int64_t)blockIdx.x % tokens;
  const int64_t t = tok_major ? (int64_t)order[ti] : ti;
  if (t < 0 || t >= tokens) return;
  // workgroup-uniform: the whole workgroup leaves (fa_prefill_f32_kernel's tile)
  if (SKIP && fa_tile_uniform(qseq, tokens, t / kFaBq)) return;
  // as fa_decode_kernel: the tiles' second launch walks the kv heads per token
  const int kvh0 = SKIP ? 0 : tok_major ? (int)(blockIdx.x % kv_heads) : (int)(blockIdx.x / tokens);
  const int kvh1 = SKIP ? kv_heads : kvh0 + 1;
  for (int kvh = kvh0; kvh < kvh1; ++kvh) {
    const int G = q_heads / kv_heads;
    const int col = lane & 15, g = lane >> 4;
    const bool head_ok = col < G;
    const int h = kvh * G + col;
    const int L = qlen[t];
    const int64_t seq = qseq[t];
    const int64_t kv_stride = (int64_t)kv_heads * kFaHd;
    const int32_t* tab = tables + seq * max_blocks;

    f32x4 qf[8];  // B operand: head col, dims 16 i + 4 g + e
  #pragma unroll
    for (int i = 0; i < 8; ++i)
      qf[i] = head_ok ? __builtin_bit_cast(f32x4, ld16(q + t * q_stride + (int64_t)h * kFaHd + 16 * i + 4 * g))
                      : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 o[8];
  #pragma unroll
    for (int d = 0; d < 8; ++d) o[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    // this wave's chunks: all of the token's, or split blockIdx.z's split_keys keys of them
    int c0 = 0, c1 = L > 0 ? (L + kFd32Bk - 1) / kFd32Bk : 0;
    if constexpr (SPLIT) {
      c0 = (int)blockIdx.z * (split_keys / kFd32Bk);
      c1 = min(c1, c0 + split_keys / kFd32Bk);
    }

    // chunk c: K row of key 16 c + col, dims 16 i + 4 g (A operands of S^T); V row
    // of key 16 c + 4 g + u, dims 4 col and 64 + 4 col (A operands of O^T, zero past L)
    auto load = [&](int c, u32x4* kr, u32x4* vr) {
      const int k0 = c * kFd32Bk;
      const int64_t row0 = (int64_t)tab[k0 / bs] * bs + k0 % bs;
      const float* kb = kc + (row0 + col) * kv_stride + (int64_t)kvh * kFaHd + 4 * g;
  #pragma unroll
      for (int i = 0; i < 8; ++i) kr[i] = ld16(kb + 16 * i);
      const float* vb = vc + row0 * kv_stride + (int64_t)kvh * kFaHd + 4 * col;
  #pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int key = 4 * g + u;
        const bool ok = k0 + key < L;
        // (the rows lie inside the chunk's block: unconditional loads, selected values)
        const u32x4 v0 = ld16(vb + (int64_t)key * kv_stride), v1 = ld16(vb + (int64_t)key * kv_stride + 64);
        vr[2 * u] = ok ? v0 : u32x4{0, 0, 0, 0};
        vr[2 * u + 1] = ok ? v1 : u32x4{0, 0, 0, 0};
      }
    };
    auto compute = [&](int c, const u32x4* kr, const u32x4* vr) {
      f32x4 st = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  #pragma unroll
      for (int i = 0; i < 8; ++i) {
        const f32x4 a = __builtin_bit_cast(f32x4, kr[i]);
  #pragma unroll
        for (int e = 0; e < 4; ++e) st = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], qf[i][e], st, 0, 0, 0);
      }
      // online softmax per head (lane column); register v is key 16 c + 4 g + v
      float mx = -INFINITY;
      if ((c + 1) * kFd32Bk <= L) {
  #pragma unroll
        for (int v = 0; v < 4; ++v) mx = fmaxf(mx, st[v]);
      } else {
  #pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float x = c * kFd32Bk + 4 * g + v < L ? st[v] : -INFINITY;
          st[v] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // lazy running max, as in fa_prefill_kernel
      const float m_cand = fmaxf(m, mx * scale_log2);
      if (__any(m_cand > m + kFaLazy)) {
        const float alpha = __builtin_amdgcn_exp2f(m - (m_cand == -INFINITY ? 0.0f : m_cand));
        l *= alpha;
  #pragma unroll
        for (int d = 0; d < 8; ++d) o[d] *= alpha;
        m = m_cand;
      }
      const float m_use = m == -INFINITY ? 0.0f : m;
      float ls = 0.0f;
      // (the product rounded as in the max, not fused into the difference: the key
      // that set m weighs exactly 1, so a single key returns its V row exactly)
  #pragma unroll
      for (int v = 0; v < 4; ++v) {
  #pragma clang fp contract(off)
        st[v] = __builtin_amdgcn_exp2f(st[v] * scale_log2 - m_use);
        ls += st[v];
      }
      ls += __shfl_xor(ls, 16);
      ls += __shfl_xor(ls, 32);
      l += ls;
  #pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f32x4 a0 = __builtin_bit_cast(f32x4, vr[2 * u]), a1 = __builtin_bit_cast(f32x4, vr[2 * u + 1]);
  #pragma unroll
        for (int d = 0; d < 4; ++d) {
          o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[d], st[u], o[d], 0, 0, 0);
          o[4 + d] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[d], st[u], o[4 + d], 0, 0, 0);
        }
      }
    };

    // wave w takes chunks w, w + 4, ...; two per trip, the register sets trading roles
    u32x4 ka[8], va[8], kb_[8], vb_[8];
    if (c0 + wave < c1) load(c0 + wave, ka, va);
    for (int c = c0 + wave; c < c1; c += 8) {
      if (c + 4 < c1) load(c + 4, kb_, vb_);
      compute(c, ka, va);
      if (c + 4 < c1) {
        if (c + 8 < c1) load(c + 8, ka, va);
        compute(c + 4, kb_, vb_);
      }
    }
    // O^T: register v of tile d is dim 64 (d / 4) + 4 (4 g + v) + d % 4 of head col
    float* pw = merge[wave];
  #pragma unroll
    for (int d = 0; d < 8; ++d)
  #pragma unroll
      for (int v = 0; v < 4; ++v) pw[(64 * (d >> 2) + 4 * (4 * g + v) + (d & 3)) * 16 + col] = o[d][v];
    if (g == 0) {
      pw[kFaHd * 16 + col] = m;
      pw[kFaHd * 16 + 16 + col] = l;
    }
    decode_merge_store<float, SPLIT>([&](int w) { return static_cast<const float*>(merge[w]); }, out, part, t, tokens,
                                     q_heads, kvh, G);
    __syncthreads();  // the merge's LDS reads before the next kv head's writes
  }
}

// ---------------------------------------------------------------------------
// One wave per (token, head).  DPL = head dimensions per lane (head_dim <= 64 DPL).
template <typename T, int DPL, bool VEC>
__global__ __launch_bounds__(kAttnWaves * 64) void attn_wave_kernel(
    const T* __restrict__ q, T* __restrict__ out, const T* __restrict__ kc, const T* __restrict__ vc,
    const int32_t* __restrict__ qseq, const int32_t* __restrict__ qlen, const int32_t* __restrict__ tables,
    int64_t tokens, int q_heads, int kv_heads, int hd, int bs, int max_blocks, float scale, int64_t q_stride,
    bool skip_uniform_tiles) {
  constexpr int N = Pack<T>::N;
  __shared__ float q_sh[kAttnWaves][64 * DPL];
  __shared__ float p_sh[kAttnWaves][64];
  __shared__ int64_t row_sh[kAttnWaves][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t gw = (int64_t)blockIdx.x * kAttnWaves + w;
  if (gw >= tokens * q_heads) return;  // whole waves only; no workgroup barrier below
  const int64_t t = gw / q_heads;
  const int h = (int)(gw - t * q_heads);
  if (skip_uniform_tiles && fa_tile_uniform(qseq, tokens, t / kFaBq)) return;  // fa_prefill_kernel's
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

// ---------------------------------------------------------------------------
// Split attention (too little work to fill the GPU: few (token, kv head) pairs or
// few tiles, long contexts): the tile and decode kernels run with blockIdx.z =
// split, each over split_keys keys; every token is written by exactly one of them,
// as an unnormalised
// partial O (fp32, [token][q head][split][128]) and its running max (exp2 units)
// and sum ([token][q head][split][2], after the O block); this kernel merges them:
// out = sum_z 2^(m_z - M) O_z / sum_z 2^(m_z - M) l_z, M = max_z m_z.  One
// workgroup per (token, q head): 4 waves take every 4th split, two dims per lane,
// each merging its splits online in one round of loads, and meet in LDS.
template <typename T>
__global__ __launch_bounds__(256) void attn_split_combine_kernel(const float* __restrict__ part, T* __restrict__ out,
                                                                 int64_t tokens,
                                                                 int q_heads, int nsplit) {
  __shared__ float red[4][2 * 64 + 2];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t t = blockIdx.x;
  const int h = (int)blockIdx.y;
  const int64_t p0 = (t * q_heads + h) * nsplit;
  const float* pml = part + tokens * q_heads * nsplit * kFaHd + 2 * p0;
  // wave w merges splits w, w + 4, ... online (its loads independent of the
  // arithmetic, so they go out together): state (mw, den, a0, a1) relative to its
  // running max mw; an empty split (m = -inf, O = 0, l = 0) weighs 0
  float mw = -INFINITY, den = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll 4
  for (int z = wave; z < nsplit; z += 4) {
    const float mz = pml[2 * z], lz = pml[2 * z + 1];
    const float2 v = *reinterpret_cast<const float2*>(part + (p0 + z) * kFaHd + 2 * lane);
    const float mn = fmaxf(mw, mz);
    const float so = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - mn);
    const float sn = mz == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mz - mn);
    den = den * so + lz * sn;
    a0 = a0 * so + v.x * sn;
    a1 = a1 * so + v.y * sn;
    mw = mn;
  }
  red[wave][2 * lane] = a0;
  red[wave][2 * lane + 1] = a1;
  if (lane == 0) {
    red[wave][128] = mw;
    red[wave][129] = den;
  }
  __syncthreads();
  if (wave != 0) return;
  // the 4 wave states, rescaled to their common max; no keys at all gives zeros,
  // as the unsplit kernels write
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < 4; ++w) mx = fmaxf(mx, red[w][128]);
  float sc[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) sc[w] = red[w][128] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(red[w][128] - mx);
  a0 = (red[0][2 * lane] * sc[0] + red[1][2 * lane] * sc[1]) + (red[2][2 * lane] * sc[2] + red[3][2 * lane] * sc[3]);
  a1 = (red[0][2 * lane + 1] * sc[0] + red[1][2 * lane + 1] * sc[1]) +
       (red[2][2 * lane + 1] * sc[2] + red[3][2 * lane + 1] * sc[3]);
  den = (red[0][129] * sc[0] + red[1][129] * sc[1]) + (red[2][129] * sc[2] + red[3][129] * sc[3]);
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  T* o = out + (t * q_heads + h) * kFaHd + 2 * lane;
  o[0] = from_f32<T>(a0 * inv);
  o[1] = from_f32<T>(a1 * inv);
}

// How an attention call is split: only when its work cannot fill the GPU --
// fewer than 512 tiles (one round of resident tile workgroups) when tiles run,
// else fewer than 1024 (token, kv head) decode waves -- and the context is long;
// then into key ranges (multiples of 64 keys; at least 512 keys per range for
// tiles) for about 1024 tile workgroups or 512 decode waves.  The context bound is
// the block table's width.
constexpr int64_t kSplitMinWaves = 1024;
constexpr int64_t kSplitTargetWaves = 512;  // a decode wave keeps ~32 KB in flight: 512 cover HBM
constexpr int64_t kSplitMinKeys = 256;  // 4 waves per split workgroup, each with whole chunks
constexpr int64_t kSplitMinTiles = 512;
constexpr int64_t kSplitTargetTiles = 1024;
constexpr int64_t kSplitMinTileKeys = 512;
struct SplitPlan {
  int nsplit = 1;
  int keys = 0;
};
inline bool attn_tiles(int64_t tokens, int64_t max_query_len) { return max_query_len != 1 && tokens >= kFaBq; }
inline SplitPlan split_plan(int64_t tokens, int q_heads, int kv_heads, int hd, int bs, int max_blocks,
                            int64_t max_query_len) {
  SplitPlan p;
  const int64_t ctx = (int64_t)bs * max_blocks;
  if (hd != kFaHd || q_heads / kv_heads > 16 || bs % 64 != 0) return p;
  int64_t n;
  if (attn_tiles(tokens, max_query_len)) {
    const int64_t wgs = (tokens + kFaBq - 1) / kFaBq * q_heads;
    if (wgs >= kSplitMinTiles) return p;
    n = std::min<int64_t>((kSplitTargetTiles + wgs - 1) / wgs, ctx / kSplitMinTileKeys);
  } else {
    const int64_t waves = tokens * kv_heads;
    if (waves >= kSplitMinWaves) return p;
    n = std::min<int64_t>((kSplitTargetWaves + waves - 1) / waves, ctx / kSplitMinKeys);
  }
  if (n <= 1) return p;
  int64_t keys = ((ctx + n - 1) / n + 63) / 64 * 64;
  n = (ctx + keys - 1) / keys;
  if (n <= 1 || n > 65535 || keys > INT32_MAX) return p;
  p.nsplit = (int)n;
  p.keys = (int)keys;
  return p;
}
inline int64_t split_bytes(int64_t tokens, int q_heads, const SplitPlan& p) {
  return p.nsplit > 1 ? tokens * q_heads * p.nsplit * (kFaHd + 2) * (int64_t)sizeof(float) : 0;
}

template <typename T, int DPL>
void launch_attn_wave(const void* q, void* out, const void* kc, const void* vc, const int32_t* qseq,
                      const int32_t* qlen, const int32_t* tables, int64_t tokens, int q_heads, int kv_heads, int hd,
                      int bs, int max_blocks, float scale, int64_t q_stride, bool vec, bool skip, hipStream_t st) {
  const int64_t waves = tokens * q_heads;
  const dim3 grid((unsigned)((waves + kAttnWaves - 1) / kAttnWaves)), block(kAttnWaves * 64);
  const T* qt = static_cast<const T*>(q);
  T* ot = static_cast<T*>(out);
  const T* kt = static_cast<const T*>(kc);
  const T* vt = static_cast<const T*>(vc);
  if (vec) {
    attn_wave_kernel<T, DPL, true><<<grid, block, 0, st>>>(qt, ot, kt, vt, qseq, qlen, tables, tokens, q_heads,
                                                           kv_heads, hd, bs, max_blocks, scale, q_stride, skip);
  } else {
    attn_wave_kernel<T, DPL, false><<<grid, block, 0, st>>>(qt, ot, kt, vt, qseq, qlen, tables, tokens, q_heads,
                                                            kv_heads, hd, bs, max_blocks, scale, q_stride, skip);
  }
}

template <typename T>
int attention_dispatch(const void* q, void* out, const void* kc, const void* vc, const int32_t* qseq,
                       const int32_t* qlen, const int32_t* tables, int64_t tokens, int q_heads, int kv_heads, int hd,
                       int bs, int max_blocks, float scale, int64_t q_stride, int64_t max_query_len, void* ws,
                       int64_t ws_bytes, hipStream_t st, bool aligned = false, const int32_t* order = nullptr) {
  // aligned: every sequence starts at a multiple of kFaBq tokens (checked on the host
  // from the caller's cu_seqlens), so every tile is uniform and the tiles' second
  // launch, whose workgroups would all exit, is not made
  constexpr int N = Pack<T>::N;
  if (tokens * kv_heads > INT32_MAX) return fail(NVF_ERR_INVALID, "paged_attention: too many tokens");
  const float sl = scale * 1.4426950408889634f;
  const int64_t ntiles = (tokens + kFaBq - 1) / kFaBq;
  if (ntiles * q_heads > INT32_MAX) return fail(NVF_ERR_INVALID, "paged_attention: too many tiles");
  // Matrix-core paths (head_dim 128, 16-byte rows, scale > 0: the kernels take the
  // running max on unscaled scores).  Tiles: 128 tokens of one sequence, unless the
  // caller promised a decode batch (max_query_len 1) or there are fewer tokens
  // than one tile; the decode kernel takes every other token.  A split (the
  // caller's workspace) runs both over key ranges and merges.
  const bool base = hd == kFaHd && aligned16(q) && aligned16(out) && aligned16(kc) && aligned16(vc) &&
                    q_stride % N == 0 && scale > 0.0f;
  const bool dec = base && q_heads / kv_heads <= 16 && bs % (sizeof(T) == 2 ? kFaBk : kFd32Bk) == 0;
  const bool tiles = base && attn_tiles(tokens, max_query_len) && bs % (sizeof(T) == 2 ? kFaBk : kF32Bk) == 0 &&
                     (sizeof(T) == 4 || dec);
  const SplitPlan sp = split_plan(tokens, q_heads, kv_heads, hd, bs, max_blocks, max_query_len);
  const bool split = dec && sp.nsplit > 1 && ws != nullptr && ws_bytes >= split_bytes(tokens, q_heads, sp);
  const unsigned nz = split ? (unsigned)sp.nsplit : 1u;
  const int skeys = split ? sp.keys : 0;
  float* part = split ? static_cast<float*>(ws) : nullptr;
  const T* qt = static_cast<const T*>(q);
  T* ot = static_cast<T*>(out);
  const T* kt = static_cast<const T*>(kc);
  const T* vt = static_cast<const T*>(vc);
  if (tiles) {
    if constexpr (sizeof(T) == 2) {
      static std::once_flag attr_once;
      std::call_once(attr_once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&fa_prefill_kernel<T, false>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kFaLds);
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&fa_prefill_kernel<T, true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kFaLds);
      });
      const dim3 grid((unsigned)(ntiles * q_heads), 1, nz);
      if (split)
        fa_prefill_kernel<T, true><<<grid, 256, kFaLds, st>>>(qt, ot, kt, vt, qseq, qlen, tables, tokens, q_heads,
                                                              kv_heads, bs, max_blocks, sl, q_stride, ntiles, skeys,
                                                              part);
      else
        fa_prefill_kernel<T, false><<<grid, 256, kFaLds, st>>>(qt, ot, kt, vt, qseq, qlen, tables, tokens, q_heads,
                                                               kv_heads, bs, max_blocks, sl, q_stride, ntiles, 0,
                                                               nullptr);
    } else {
      static std::once_flag f32_once;
      std::call_once(f32_once, [] {
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&fa_prefill_f32_kernel<false>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kF32Lds);
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&fa_prefill_f32_kernel<true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kF32Lds);
      });
      const dim3 grid((unsigned)(ntiles * q_heads), 1, nz);
      if (split)
        fa_prefill_f32_kernel<true><<<grid, 256, kF32Lds, st>>>(qt, ot, kt, vt, qseq, qlen, tables, tokens, q_heads,
                                                                kv_heads, bs, max_blocks, sl, q_stride, ntiles, skeys,
                                                                part);
      else
        fa_prefill_f32_kernel<false><<<grid, 256, kF32Lds, st>>>(qt, ot, kt, vt, qseq, qlen, tables, tokens,
                                                                 q_heads, kv_heads, bs, max_blocks, sl, q_stride,
                                                                 ntiles, 0, nullptr);
    }
    const int rc = launch_status("paged_attention(tiles)");
    if (rc != NVF_OK) return rc;
  }
  if (tiles && aligned) {
    if (!split) return NVF_OK;
    attn_split_combine_kernel<T><<<dim3((unsigned)tokens, (unsigned)q_heads), 256, 0, st>>>(part, ot, tokens,
                                                                                            q_heads, sp.nsplit);
    return launch_status("paged_attention(split merge)");
  }
  if (dec) {
    // one workgroup per (token, kv head); for the tiles' second launch (SKIP), one
    // per token walking the kv heads, since nearly all of its workgroups exit at once
    const dim3 grid((unsigned)(tiles ? tokens : tokens * kv_heads), 1u, nz);
    const int kk = split ? skeys : 0;
    float* pp = split ? part : nullptr;
#define NVF_DEC_LAUNCH_ORD(KERN, LDS, ORD)                                                                     \
  KERN<<<grid, 256, LDS, st>>>(qt, ot, kt, vt, qseq, qlen, tables, tokens, q_heads, kv_heads, bs, max_blocks, sl, \
                               q_stride, kk, pp, ORD)
    if constexpr (sizeof(T) == 2) {
      static std::once_flag dec_once;
      std::call_once(dec_once, [] {
        const void* ks[4] = {reinterpret_cast<const void*>(&fa_decode_kernel<T, false, false>),
                             reinterpret_cast<const void*>(&fa_decode_kernel<T, false, true>),
                             reinterpret_cast<const void*>(&fa_decode_kernel<T, true, false>),
                             reinterpret_cast<const void*>(&fa_decode_kernel<T, true, true>)};
        for (const void* k : ks) (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kFdLds);
      });
      if (split && tiles) NVF_DEC_LAUNCH_ORD((fa_decode_kernel<T, true, true>), kFdLds, nullptr);
      else if (split) NVF_DEC_LAUNCH_ORD((fa_decode_kernel<T, true, false>), kFdLds, order);
      else if (tiles) NVF_DEC_LAUNCH_ORD((fa_decode_kernel<T, false, true>), kFdLds, nullptr);
      else NVF_DEC_LAUNCH_ORD((fa_decode_kernel<T, false, false>), kFdLds, order);
    } else {
      if (split && tiles) NVF_DEC_LAUNCH_ORD((fa_decode_f32_kernel<true, true>), 0, nullptr);
      else if (split) NVF_DEC_LAUNCH_ORD((fa_decode_f32_kernel<true, false>), 0, order);
      else if (tiles) NVF_DEC_LAUNCH_ORD((fa_decode_f32_kernel<false, true>), 0, nullptr);
      else NVF_DEC_LAUNCH_ORD((fa_decode_f32_kernel<false, false>), 0, order);
    }
#undef NVF_DEC_LAUNCH_ORD
    int rc = launch_status("paged_attention(decode)");
    if (rc != NVF_OK || !split) return rc;
    attn_split_combine_kernel<T><<<dim3((unsigned)tokens, (unsigned)q_heads), 256, 0, st>>>(part, ot, tokens,
                                                                                            q_heads, sp.nsplit);
    return launch_status("paged_attention(split merge)");
  }
  // everything else (other head sizes, block sizes or head groups, scale <= 0),
  // leaving the fp32 tiles' tokens alone
  const bool vec = hd % N == 0 && aligned16(kc) && ((int64_t)kv_heads * hd) % N == 0;
  const bool skip = tiles;
  switch ((hd + 63) / 64) {
    case 1: launch_attn_wave<T, 1>(q, out, kc, vc, qseq, qlen, tables, tokens, q_heads, kv_heads, hd, bs, max_blocks,
                                   scale, q_stride, vec, skip, st); break;
    case 2: launch_attn_wave<T, 2>(q, out, kc, vc, qseq, qlen, tables, tokens, q_heads, kv_heads, hd, bs, max_blocks,
                                   scale, q_stride, vec, skip, st); break;
    case 3: launch_attn_wave<T, 3>(q, out, kc, vc, qseq, qlen, tables, tokens, q_heads, kv_heads, hd, bs, max_blocks,
                                   scale, q_stride, vec, skip, st); break;
    default: launch_attn_wave<T, 4>(q, out, kc, vc, qseq, qlen, tables, tokens, q_heads, kv_heads, hd, bs,
                                    max_blocks, scale, q_stride, vec, skip, st); break;
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

static int paged_attention_entry(const void* q, void* out, const void* k_cache, const void* v_cache,
                                 const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                                 int64_t tokens, int q_heads, int kv_heads, int head_dim, int block_size,
                                 int max_blocks, float scale, int64_t q_stride, int64_t max_query_len, void* workspace,
                                 int64_t workspace_bytes, int dtype, void* stream, bool aligned,
                                 const int32_t* order = nullptr) {
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
  if (workspace && !aligned16(workspace))
    return fail(NVF_ERR_INVALID, "nvf_paged_attention: workspace must be 16-byte aligned");
  if ((tokens * q_heads + kAttnWaves - 1) / kAttnWaves > INT32_MAX)
    return fail(NVF_ERR_INVALID, "nvf_paged_attention: too many (token, head) pairs");
  int rc = NVF_OK;
  NVF_DISPATCH_DTYPE(dtype, T, rc = attention_dispatch<T>(q, out, k_cache, v_cache, query_seq, query_key_len,
                                                         block_tables, tokens, q_heads, kv_heads, head_dim, block_size,
                                                         max_blocks, scale, q_stride, max_query_len, workspace,
                                                         workspace_bytes, as_stream(stream), aligned, order));
  return rc;
}

int nvf_paged_attention_ws(const void* q, void* out, const void* k_cache, const void* v_cache,
                           const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                           int64_t tokens, int q_heads, int kv_heads, int head_dim, int block_size, int max_blocks,
                           float scale, int64_t q_stride, int64_t max_query_len, void* workspace,
                           int64_t workspace_bytes, int dtype, void* stream) {
  return paged_attention_entry(q, out, k_cache, v_cache, query_seq, query_key_len, block_tables, tokens, q_heads,
                               kv_heads, head_dim, block_size, max_blocks, scale, q_stride, max_query_len, workspace,
                               workspace_bytes, dtype, stream, false);
}

int nvf_decode_token_order(const int32_t* key_len_host, int64_t tokens, int32_t* order_host) {
  if (tokens < 0 || tokens > INT32_MAX) return fail(NVF_ERR_INVALID, "nvf_decode_token_order: bad token count");
  if (tokens == 0) return NVF_OK;
  if (!key_len_host || !order_host) return fail(NVF_ERR_INVALID, "nvf_decode_token_order: NULL pointer");
  // longest first (ties by token), dealt over the 8 XCDs in snake order: round r of 8
  // workgroups r*8 .. r*8+7 (workgroup id mod 8 is its XCD) takes the next 8 tokens,
  // reversed on odd rounds, so every XCD's sum of key counts is nearly equal; a last
  // partial round stays in order so that every id is below tokens
  std::vector<int32_t> idx((size_t)tokens);
  for (int64_t i = 0; i < tokens; ++i) idx[(size_t)i] = (int32_t)i;
  std::stable_sort(idx.begin(), idx.end(),
                   [&](int32_t a, int32_t b) { return key_len_host[a] > key_len_host[b]; });
  for (int64_t p = 0; p < tokens; ++p) {
    const int64_t r = p / 8, x = p % 8;
    const bool full = r * 8 + 8 <= tokens;
    order_host[r * 8 + ((r & 1) && full ? 7 - x : x)] = idx[(size_t)p];
  }
  return NVF_OK;
}

int nvf_paged_attention_order_ws(const void* q, void* out, const void* k_cache, const void* v_cache,
                                 const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                                 const int32_t* token_order, int64_t tokens, int q_heads, int kv_heads, int head_dim,
                                 int block_size, int max_blocks, float scale, int64_t q_stride, int64_t max_query_len,
                                 void* workspace, int64_t workspace_bytes, int dtype, void* stream) {
  if (!token_order) return fail(NVF_ERR_INVALID, "nvf_paged_attention_order_ws: NULL token_order");
  return paged_attention_entry(q, out, k_cache, v_cache, query_seq, query_key_len, block_tables, tokens, q_heads,
                               kv_heads, head_dim, block_size, max_blocks, scale, q_stride, max_query_len, workspace,
                               workspace_bytes, dtype, stream, false, token_order);
}

int nvf_paged_attention_seqs_ws(const void* q, void* out, const void* k_cache, const void* v_cache,
                                const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                                const int32_t* cu_seqlens_host, int num_seqs, int64_t tokens, int q_heads,
                                int kv_heads, int head_dim, int block_size, int max_blocks, float scale,
                                int64_t q_stride, int64_t max_query_len, void* workspace, int64_t workspace_bytes,
                                int dtype, void* stream) {
  if (!cu_seqlens_host || num_seqs <= 0)
    return fail(NVF_ERR_INVALID, "nvf_paged_attention_seqs_ws: cu_seqlens_host and num_seqs > 0 are required");
  if (cu_seqlens_host[0] != 0 || cu_seqlens_host[num_seqs] != tokens)
    return fail(NVF_ERR_INVALID, "nvf_paged_attention_seqs_ws: cu_seqlens must run from 0 to tokens=%lld",
                (long long)tokens);
  bool aligned = true;
  for (int s = 1; s <= num_seqs; ++s) {
    if (cu_seqlens_host[s] < cu_seqlens_host[s - 1])
      return fail(NVF_ERR_INVALID, "nvf_paged_attention_seqs_ws: cu_seqlens must not decrease");
    if (s < num_seqs && cu_seqlens_host[s] % kFaBq != 0) aligned = false;
  }
  return paged_attention_entry(q, out, k_cache, v_cache, query_seq, query_key_len, block_tables, tokens, q_heads,
                               kv_heads, head_dim, block_size, max_blocks, scale, q_stride, max_query_len, workspace,
                               workspace_bytes, dtype, stream, aligned);
}

int nvf_paged_attention(const void* q, void* out, const void* k_cache, const void* v_cache, const int32_t* query_seq,
                        const int32_t* query_key_len, const int32_t* block_tables, int64_t tokens, int q_heads,
                        int kv_heads, int head_dim, int block_size, int max_blocks, float scale, int64_t q_stride,
                        int64_t max_query_len, int dtype, void* stream) {
  return nvf_paged_attention_ws(q, out, k_cache, v_cache, query_seq, query_key_len, block_tables, tokens, q_heads,
                                kv_heads, head_dim, block_size, max_blocks, scale, q_stride, max_query_len, nullptr, 0,
                                dtype, stream);
}

int64_t nvf_paged_attention_workspace_size(int64_t tokens, int q_heads, int kv_heads, int head_dim, int block_size,
                                           int max_blocks, int64_t max_query_len) {
  if (tokens <= 0 || q_heads <= 0 || kv_heads <= 0 || block_size <= 0 || max_blocks <= 0 || q_heads % kv_heads)
    return 0;
  return split_bytes(tokens, q_heads,
                     split_plan(tokens, q_heads, kv_heads, head_dim, block_size, max_blocks, max_query_len));
}

// ---------------------------------------------------------------------------
// nvf_paged_attention_noalloc: nvf_paged_attention_ws for callers that cannot
// allocate (HIP graph capture, serving loops, harnesses that forbid hipMalloc).
// The split partials go to `scratch`, a file-scope device array of
// kAttnScratchBytes that every GPU this library runs on holds until the process
// ends.  On the host the array's name is only a stand-in for its symbol: its
// device address (one per GPU) comes from hipGetSymbolAddress, taken on the
// entry's first call on each device with that device current, and only that
// address is passed to kernels.  Every call on a GPU shares the one array and
// leaves its contents behind (every split writes all of its partials, so no
// clearing is needed); calls that overlap on one GPU (several streams or
// threads at once) race on it.
// ---------------------------------------------------------------------------
constexpr int64_t kAttnScratchBytes = 32ll << 20;  // split decode needs <= 12.8 MB; short prefill chunks after long contexts more
static __device__ __align__(256) float scratch[kAttnScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// scratch's device address on the current device (NULL + last error on failure)
void* scratch_ptr() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(NVF_ERR_LAUNCH, "nvf_paged_attention_noalloc: no usable current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      fail(NVF_ERR_LAUNCH, "nvf_paged_attention_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
           hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

int64_t nvf_paged_attention_noalloc_max_bytes(void) { return kAttnScratchBytes; }

int nvf_paged_attention_noalloc(const void* q, void* out, const void* k_cache, const void* v_cache,
                                const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                                int64_t tokens, int q_heads, int kv_heads, int head_dim, int block_size,
                                int max_blocks, float scale, int64_t q_stride, int64_t max_query_len, int dtype,
                                void* stream) {
  const int64_t need = nvf_paged_attention_workspace_size(tokens, q_heads, kv_heads, head_dim, block_size, max_blocks,
                                                          max_query_len);
  if (need > kAttnScratchBytes)
    return fail(NVF_ERR_INVALID,
                "nvf_paged_attention_noalloc: this call's split needs %lld bytes of scratch, more than the %lld-byte "
                "static scratch (use nvf_paged_attention_ws with a workspace)",
                (long long)need, (long long)kAttnScratchBytes);
  void* ws = nullptr;
  if (need > 0 && !(ws = scratch_ptr())) return NVF_ERR_LAUNCH;
  return paged_attention_entry(q, out, k_cache, v_cache, query_seq, query_key_len, block_tables, tokens, q_heads,
                               kv_heads, head_dim, block_size, max_blocks, scale, q_stride, max_query_len, ws, need,
                               dtype, stream, false);
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

// The drop-in splits small batches over long contexts through the same static
// scratch as nvf_paged_attention_noalloc, so it allocates nothing, like the
// reference's hip_paged_attention (src/hip_ops.hip:735-744).  A split that would
// need more than the scratch runs unsplit instead (same results within the
// attention tolerance, slower).  Like the reference's ops it assumes one calling
// thread: calls overlapping on one GPU would share the scratch.
void hip_paged_attention(const float* q, float* out, const float* k_cache, const float* v_cache,
                         const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                         int tokens, int q_heads, int kv_heads, int head_dim, int block_size, int max_blocks,
                         float scale) {
  if (tokens <= 0 || q_heads <= 0 || kv_heads <= 0) return;
  int64_t need = nvf_paged_attention_workspace_size(tokens, q_heads, kv_heads, head_dim, block_size, max_blocks, 0);
  void* ws = nullptr;
  if (need > kAttnScratchBytes) need = 0;
  if (need > 0 && !(ws = scratch_ptr())) dropin_check(NVF_ERR_LAUNCH, "hip_paged_attention");
  dropin_check(nvf_paged_attention_ws(q, out, k_cache, v_cache, query_seq, query_key_len, block_tables, tokens,
                                      q_heads, kv_heads, head_dim, block_size, max_blocks, scale,
                                      (int64_t)q_heads * head_dim, 0, ws, need, NVF_F32, nullptr),
               "hip_paged_attention");
}

}  // extern "C"
