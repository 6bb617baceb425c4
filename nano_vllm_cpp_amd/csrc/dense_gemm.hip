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
// Design for gfx950: v_mfma_f32_32x32x2_f32 (fp32 products and sums, 157 TFLOP/s
// dense).  A 256-thread workgroup owns a BM x 128 output tile: BM = 128 as 2 x 2
// waves of 64 x 64, or BM = 32 (m <= 32: decode batches) as 1 x 4 waves of 32 x 32,
// so a small m does not multiply the matrix-core work.  K moves in 16-element
// stages through LDS, double-buffered, with the next stage's loads in flight
// during the current stage's MFMAs:
//   * activation rows, upconverted to fp32 (8 elements per thread);
//   * weight rows, decoded to fp32 by the same element sources as the embedding
//     gathers (weight_formats.hpp; 8 elements per thread, bit-exact values);
//   * LDS rows padded to 20 floats, so the 16 lanes of a ds_read_b128 phase hit
//     16 distinct 4-bank groups.
// Inside a stage the k order is permuted (the dot product does not care): MFMA
// step s contracts k = s on lanes 0-31 and k = 8 + s on lanes 32-63 for both
// operands, so each lane reads its 8 values of a row as two 16-byte LDS reads.
// The sums are fp32 in a different order from the reference's, so results agree
// within the recursive-summation bound the tests state.
//
// A k that is not a multiple of 16 (the reference takes any k) runs the RAGGED
// variant: the same tiles and MFMAs, but every staged value is read on its own,
// k beyond the row's end staged as zero, weights decoded through 4-element aligned
// runs of the same sources (rows no longer start on 8-element boundaries).

#include "nvf_device.hpp"
#include "nvf_host.hpp"
#include "weight_formats.hpp"

namespace nvf {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kDgBN = 128;           // output columns per workgroup
constexpr int kDgKC = 16;            // k elements per LDS stage
constexpr int kDgRow = kDgKC + 4;    // LDS floats per staged row (padded)
constexpr int kDgThreads = 256;
constexpr int kDgXcds = 8;

template <int BM>
constexpr int dg_stage_floats() {
  return (BM + kDgBN) * kDgRow;
}

// Workgroup -> output tile, XCD-aware: workgroups are dealt to the 8 XCDs
// round-robin, and each XCD takes a contiguous range of an order that walks 8
// tile rows at a time column by column, so its resident workgroups share weight
// and activation panels in its L2.
__device__ __forceinline__ void dg_tile(int tiles_n, int64_t& tm, int64_t& tn) {
  const int tiles = (int)gridDim.x;
  const int tiles_m = tiles / tiles_n;
  const int xcd = (int)blockIdx.x % kDgXcds, local = (int)blockIdx.x / kDgXcds;
  const int per = tiles / kDgXcds, extra = tiles % kDgXcds;
  const int id = xcd * per + (xcd < extra ? xcd : extra) + local;
  const int gsz = 8 * tiles_n;
  const int first = (id / gsz) * 8;
  const int rows_g = tiles_m - first < 8 ? tiles_m - first : 8;
  const int in_g = id % gsz;
  tm = first + in_g % rows_g;
  tn = in_g / rows_g;
}

// The 4-element form of an 8-element weight source, for the ragged-k staging.
template <typename S>
struct Narrow;
template <typename T>
struct Narrow<Table<8, T>> {
  using type = Table<4, T>;
  __device__ static type make(const Table<8, T>& s) { return type{s.table}; }
};
template <int L>
struct Narrow<Q4K<8, L>> {
  using type = Q4K<4, L>;
  __device__ static type make(const Q4K<8, L>& s) { return type{s.wq}; }
};
template <>
struct Narrow<Q5K<8>> {
  using type = Q5K<4>;
  __device__ static type make(const Q5K<8>& s) { return type{s.wq}; }
};
template <>
struct Narrow<Q6K<8>> {
  using type = Q6K<4>;
  __device__ static type make(const Q6K<8>& s) { return type{s.wq}; }
};

// Element e of a weight source: K-quants decode the aligned 4-run that holds it
// (inside e's 256-element superblock); plain rows read the element alone, so
// nothing past the table's end is touched.
template <typename S4>
__device__ __forceinline__ float element_at(const S4& s, int64_t e) {
  float v[4];
  s.decode(s.load(e & ~int64_t(3)), v);
  return v[e & 3];
}
template <typename T>
__device__ __forceinline__ float element_at(const Table<4, T>& s, int64_t e) {
  return to_f32(s.table[e]);
}

template <typename TX, typename Src, int BM, typename TO, bool RAGGED>
__global__ __launch_bounds__(kDgThreads) __attribute__((amdgpu_waves_per_eu(2))) void dense_gemm_kernel(
    const TX* __restrict__ x, Src w, TO* __restrict__ out, int64_t m, int64_t n, int64_t k, int tiles_n) {
  constexpr int WN = BM == 128 ? 2 : 4;              // waves along n
  constexpr int TM = BM == 128 ? 2 : 1;              // 32-row MFMA tiles per wave
  constexpr int TN = BM == 128 ? 2 : 1;              // 32-column MFMA tiles per wave
  constexpr int kStage = dg_stage_floats<BM>();
  __shared__ float lds[2 * kStage];
  int64_t tm, tn;
  dg_tile(tiles_n, tm, tn);
  const int64_t row0 = tm * BM, col0 = tn * kDgBN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  // staging roles: thread t moves 8 k-values (half t & 1 of the stage) of activation
  // row t >> 1 (t < 2 BM) and of weight column t >> 1
  const int sr = tid >> 1, sh = (tid & 1) * 8;
  const bool a_role = sr < BM, a_ok = a_role && row0 + sr < m;
  const bool b_ok = col0 + sr < n;
  const Table<8, TX> xs{x};
  typename Table<8, TX>::Raw ar;
  typename Src::Raw br;
  const int64_t a_e0 = (row0 + sr) * k + sh;  // element offsets at stage 0
  const int64_t b_e0 = (col0 + sr) * k + sh;
  int staged = 0;  // RAGGED: the stage the next store writes
  auto load = [&](int st) {
    const int64_t kc = (int64_t)st * kDgKC;
    if constexpr (RAGGED) {
      staged = st;
    } else {
      if (a_ok) ar = xs.load(a_e0 + kc);
      if (b_ok) br = w.load(b_e0 + kc);
    }
  };
  auto store = [&](int buf) {
    float* s = lds + buf * kStage;
    float v[8];
    if constexpr (RAGGED) {
      const int64_t i0 = (int64_t)staged * kDgKC + sh;  // k index of v[0]
      if (a_role) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = a_ok && i0 + i < k ? to_f32(x[a_e0 - sh + i0 + i]) : 0.0f;
        float* d = s + sr * kDgRow + sh;
        st16(d, Pack<float>::pack(v));
        st16(d + 4, Pack<float>::pack(v + 4));
      }
      const auto w4 = Narrow<Src>::make(w);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = b_ok && i0 + i < k ? element_at(w4, b_e0 - sh + i0 + i) : 0.0f;
      float* d = s + (BM + sr) * kDgRow + sh;
      st16(d, Pack<float>::pack(v));
      st16(d + 4, Pack<float>::pack(v + 4));
      return;
    }
    if (a_role) {
      if (a_ok) {
        xs.decode(ar, v);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
      }
      float* d = s + sr * kDgRow + sh;
      st16(d, Pack<float>::pack(v));
      st16(d + 4, Pack<float>::pack(v + 4));
    }
    if (b_ok) {
      w.decode(br, v);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
    float* d = s + (BM + sr) * kDgRow + sh;
    st16(d, Pack<float>::pack(v));
    st16(d + 4, Pack<float>::pack(v + 4));
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = f32x16{};
  // fragment rows: MFMA tile a of this wave covers rows 32 (TM wm + a) + (lane & 31)
  const int half = lane >> 5;
  const int fa = (TM * 32 * wm + (lane & 31)) * kDgRow + 8 * half;
  const int fb = (BM + TN * 32 * wn + (lane & 31)) * kDgRow + 8 * half;

  const int nst = (int)((k + kDgKC - 1) / kDgKC);
  load(0);
  store(0);
  __syncthreads();
#pragma unroll 1
  for (int st = 0; st < nst; ++st) {
    const float* s = lds + (st & 1) * kStage;
    if (st + 1 < nst) load(st + 1);  // in flight during this stage's MFMAs
    f32x4 av[TM][2], bv[TN][2];
#pragma unroll
    for (int a = 0; a < TM; ++a) {
      av[a][0] = __builtin_bit_cast(f32x4, ld16(s + fa + a * 32 * kDgRow));
      av[a][1] = __builtin_bit_cast(f32x4, ld16(s + fa + a * 32 * kDgRow + 4));
    }
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      bv[b][0] = __builtin_bit_cast(f32x4, ld16(s + fb + b * 32 * kDgRow));
      bv[b][1] = __builtin_bit_cast(f32x4, ld16(s + fb + b * 32 * kDgRow + 4));
    }
#pragma unroll
    for (int step = 0; step < 8; ++step)
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a][step >> 2][step & 3], bv[b][step >> 2][step & 3],
                                                         acc[a][b], 0, 0, 0);
    if (st + 1 < nst) {
      store((st + 1) & 1);  // the other buffer: its last readers passed the previous barrier
      __syncthreads();
    }
  }

  // D layout of v_mfma_f32_32x32x2f32: lane l, value j -> column l % 32,
  // row 8 (j / 4) + 4 (l / 32) + j % 4
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int64_t r = row0 + TM * 32 * wm + 32 * a + 8 * (j >> 2) + 4 * half + (j & 3);
      if (r >= m) continue;
#pragma unroll
      for (int b = 0; b < TN; ++b) {
        const int64_t c = col0 + TN * 32 * wn + 32 * b + (lane & 31);
        if (c < n) out[r * n + c] = from_f32<TO>(acc[a][b][j]);
      }
    }
}

// ---------------------------------------------------------------------------
// 32-element group sources for the decode products: one lane decodes a whole
// 32-element group of a K-quant superblock per load (e0 % 32 == 0), so the
// superblock header and the group's scale / min are read and decoded once per 32
// values instead of once per 8.  Values are bit-identical to Q4K / Q5K / Q6K
// (weight_formats.hpp): the same formulas on the same bytes.
template <typename S>
struct RunOf;  // elements one load of a source yields
template <typename T>
struct RunOf<Table<8, T>> {
  static constexpr int value = 8;
};

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
// m <= 2 (dense_gemv_fma_kernel): LPC = 16 (dense) or 8 (K-quants) lanes per
// column; lane l = CPS b + j (CPS = 64 / LPC columns per set) streams run b of
// column j of each of its C column sets (LPC runs: 128 or 256 contiguous k of one
// column per step) with the same k of each of the m rows, accumulating m x C fp32
// sums; the LPC lanes of a column are summed at the end.
//
// 2 < m <= 16 (dense_gemv_mfma_kernel): v_mfma_f32_16x16x4_f32, lane l = 16 s + j
// giving activation row j and weight column j at k slot s.  Lane l streams 16
// (dense: two runs of 8) or 32 consecutive k at offset (16 or 32) s of column j of
// each of C 16-column groups; value i of the lane's span is MFMA step i, with
// k slot s <-> k = span s + i.  The matrix core sums the k slots, so only the
// waves are summed at the end.
constexpr int kGvWaves = 4;
constexpr int kGemvRows = 16;

template <typename TX, int R>
__device__ __forceinline__ void load_x_run(const Table<8, TX>& xs, int64_t e0, typename Table<8, TX>::Raw* xr) {
#pragma unroll
  for (int u = 0; u < R / 8; ++u) xr[u] = xs.load(e0 + 8 * u);
}
template <typename TX, int R>
__device__ __forceinline__ void decode_x_run(const Table<8, TX>& xs, const typename Table<8, TX>::Raw* xr, float* v) {
#pragma unroll
  for (int u = 0; u < R / 8; ++u) xs.decode(xr[u], v + 8 * u);
}

template <typename TX, typename Src, int MR, int C, int S, typename TO>
__global__ __launch_bounds__(kGvWaves * 64) void dense_gemv_fma_kernel(const TX* __restrict__ x, Src w,
                                                                       TO* __restrict__ out, int64_t m, int64_t n,
                                                                       int64_t k) {
  constexpr int R = RunOf<Src>::value, LPC = R == 8 ? 16 : 8, CPS = 64 / LPC, KS = LPC * R;
  constexpr int G = kGvWaves / S;               // column groups per workgroup (S waves split K in each)
  __shared__ float part[kGvWaves][MR][C][CPS];  // [wave][row][set][column]
  const int lane = threadIdx.x & 63, j = lane % CPS, b = lane / CPS;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int grp = wave / S, split = wave % S;
  const int64_t c0 = ((int64_t)blockIdx.x * G + grp) * CPS * C;
  const int64_t nsteps = (k + KS - 1) / KS, full = k / KS;  // steps; steps every lane's run is inside
  const int64_t s_begin = nsteps * split / S, s_end = nsteps * (split + 1) / S;
  const int64_t f_end = s_end < full ? s_end : full;
  const Table<8, TX> xs{x};
  // columns past n read column n - 1 (their sums are never stored): no per-lane
  // branches in the loop
  int64_t wrow[C];
#pragma unroll
  for (int q = 0; q < C; ++q) {
    const int64_t c = c0 + CPS * q + j;
    wrow[q] = (c < n ? c : n - 1) * k + (int64_t)R * b;
  }
  const int64_t xrow = (int64_t)R * b;
  float acc[MR][C];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < C; ++q) acc[r][q] = 0.0f;

  struct Buf {
    typename Src::Raw w[C];
    typename Table<8, TX>::Raw x[MR][R / 8];
  };
  auto load = [&](Buf& f, int64_t st) {
    const int64_t kk = st * KS;
#pragma unroll
    for (int q = 0; q < C; ++q) f.w[q] = w.load(wrow[q] + kk);
#pragma unroll
    for (int r = 0; r < MR; ++r) load_x_run<TX, R>(xs, (int64_t)r * k + xrow + kk, f.x[r]);
  };
  auto compute = [&](const Buf& f) {
    float xv[MR][R];
#pragma unroll
    for (int r = 0; r < MR; ++r) decode_x_run<TX, R>(xs, f.x[r], xv[r]);
#pragma unroll
    for (int q = 0; q < C; ++q) {
      float wv[R];
      w.decode(f.w[q], wv);
#pragma unroll
      for (int i = 0; i < R; ++i)
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[r][q] = __builtin_fmaf(xv[r][i], wv[i], acc[r][q]);
    }
  };
  // full steps, two raw buffers in turn: the next step's loads are in flight
  // while the current one is decoded.  The prefetch is unconditional (the last
  // step reloads itself), so the memory counter waits stay exact: a load that
  // may or may not have been issued makes the compiler wait for all of them.
  Buf fa, fb;
  int64_t st = s_begin;
  if (st < f_end) {
    const int64_t last = f_end - 1;
    load(fa, st);
    while (true) {
      load(fb, st + 1 < last ? st + 1 : last);
      compute(fa);
      if (++st >= f_end) break;
      load(fa, st + 1 < last ? st + 1 : last);
      compute(fb);
      if (++st >= f_end) break;
    }
  }
  // the last, partial step (k not a multiple of the step): lanes past k add nothing
  if (f_end < s_end && xrow + f_end * KS < k) {
    load(fa, f_end);
    compute(fa);
  }

#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < C; ++q) {
      float v = acc[r][q];
#pragma unroll
      for (int d = CPS; d < 64; d *= 2) v += __shfl_xor(v, d, 64);
      if (lane < CPS) part[wave][r][q][j] = v;
    }
  __syncthreads();
  for (int t = (int)threadIdx.x; t < G * MR * C * CPS; t += kGvWaves * 64) {
    const int jj = t % CPS, q = (t / CPS) % C, r = (t / (CPS * C)) % MR, g = t / (CPS * C * MR);
    const int64_t col = ((int64_t)blockIdx.x * G + g) * CPS * C + CPS * q + jj;
    if (r >= m || col >= n) continue;
    float v = part[g * S][r][q][jj];
#pragma unroll
    for (int wv = 1; wv < S; ++wv) v += part[g * S + wv][r][q][jj];
    out[(int64_t)r * n + col] = from_f32<TO>(v);
  }
}

template <typename TX, typename Src, int C, typename TO>
__global__ __launch_bounds__(kGvWaves * 64) void dense_gemv_mfma_kernel(const TX* __restrict__ x, Src w,
                                                                        TO* __restrict__ out, int64_t m, int64_t n,
                                                                        int64_t k) {
  constexpr int R = RunOf<Src>::value, H = R == 8 ? 2 : 1, SPAN = H * R, KS = 4 * SPAN;
  __shared__ float part[kGvWaves][C][16][17];  // [wave][group][row][column] (padded)
  const int lane = threadIdx.x & 63, j = lane & 15, ks = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t c0 = (int64_t)blockIdx.x * 16 * C;
  const int64_t nsteps = (k + KS - 1) / KS;
  const int64_t s_begin = nsteps * wave / kGvWaves, s_end = nsteps * (wave + 1) / kGvWaves;
  const Table<8, TX> xs{x};
  const bool row_ok = j < m;
  bool col_ok[C];
#pragma unroll
  for (int q = 0; q < C; ++q) col_ok[q] = c0 + 16 * q + j < n;
  f32x4 acc[C];
#pragma unroll
  for (int q = 0; q < C; ++q) acc[q] = f32x4{};

  for (int64_t s = s_begin; s < s_end; ++s) {
    const int64_t kk = s * KS + (int64_t)SPAN * ks;
    typename Src::Raw wr[C][H];
    typename Table<8, TX>::Raw xr[H][R / 8];
    bool h_ok[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
      h_ok[h] = kk + R * h < k;
#pragma unroll
      for (int q = 0; q < C; ++q)
        if (h_ok[h] && col_ok[q]) wr[q][h] = w.load((c0 + 16 * q + j) * k + kk + R * h);
      if (h_ok[h] && row_ok) load_x_run<TX, R>(xs, (int64_t)j * k + kk + R * h, xr[h]);
    }
#pragma unroll
    for (int h = 0; h < H; ++h) {
      float xv[R];
      if (h_ok[h] && row_ok) {
        decode_x_run<TX, R>(xs, xr[h], xv);
      } else {
#pragma unroll
        for (int i = 0; i < R; ++i) xv[i] = 0.0f;
      }
#pragma unroll
      for (int q = 0; q < C; ++q) {
        float wv[R];
        if (h_ok[h] && col_ok[q]) {
          w.decode(wr[q][h], wv);
        } else {
#pragma unroll
          for (int i = 0; i < R; ++i) wv[i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < R; ++i) acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[i], wv[i], acc[q], 0, 0, 0);
      }
    }
  }

  // D of v_mfma_f32_16x16x4_f32: lane l, value r -> row 4 (l / 16) + r, column l % 16
#pragma unroll
  for (int q = 0; q < C; ++q)
#pragma unroll
    for (int r = 0; r < 4; ++r) part[wave][q][4 * ks + r][j] = acc[q][r];
  __syncthreads();
  for (int t = (int)threadIdx.x; t < C * 256; t += kGvWaves * 64) {
    const int jj = t & 15, row = (t >> 4) & 15, q = t >> 8;
    const int64_t col = c0 + 16 * q + jj;
    if (row >= m || col >= n) continue;
    float v = part[0][q][row][jj];
#pragma unroll
    for (int wv = 1; wv < kGvWaves; ++wv) v += part[wv][q][row][jj];
    out[(int64_t)row * n + col] = from_f32<TO>(v);
  }
}

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
  if (n >= (int64_t)CPS * CMAX * kGvWaves * 1024)
    dense_gemv_fma_kernel<TX, Src, MR, CMAX, 1, TO><<<grid(CPS * CMAX * kGvWaves), blk, 0, st>>>(x, src, out, m, n, k);
  else if (n >= (int64_t)CPS * CMAX * 1024)
    dense_gemv_fma_kernel<TX, Src, MR, CMAX, 4, TO><<<grid(CPS * CMAX), blk, 0, st>>>(x, src, out, m, n, k);
  else
    dense_gemv_fma_kernel<TX, Src, MR, 1, 4, TO><<<grid(CPS), blk, 0, st>>>(x, src, out, m, n, k);
  return launch_status("dense_gemv_fma");
}

template <typename TX, typename Src, typename TO>
int launch_gemv_mfma(const TX* x, const Src& src, TO* out, int64_t m, int64_t n, int64_t k, hipStream_t st) {
  const dim3 blk(kGvWaves * 64);
  if (n >= 64 * 1024)
    dense_gemv_mfma_kernel<TX, Src, 4, TO><<<dim3((unsigned)((n + 63) / 64)), blk, 0, st>>>(x, src, out, m, n, k);
  else if (n >= 32 * 1024)
    dense_gemv_mfma_kernel<TX, Src, 2, TO><<<dim3((unsigned)((n + 31) / 32)), blk, 0, st>>>(x, src, out, m, n, k);
  else
    dense_gemv_mfma_kernel<TX, Src, 1, TO><<<dim3((unsigned)((n + 15) / 16)), blk, 0, st>>>(x, src, out, m, n, k);
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
    if (ragged)
      dense_gemm_kernel<TX, Src, 32, TO, true><<<g, kDgThreads, 0, st>>>(xp, src, op, m, n, k, tiles_n);
    else
      dense_gemm_kernel<TX, Src, 32, TO, false><<<g, kDgThreads, 0, st>>>(xp, src, op, m, n, k, tiles_n);
  } else {
    const dim3 g((unsigned)(((m + 127) / 128) * tiles_n));
    if (ragged)
      dense_gemm_kernel<TX, Src, 128, TO, true><<<g, kDgThreads, 0, st>>>(xp, src, op, m, n, k, tiles_n);
    else
      dense_gemm_kernel<TX, Src, 128, TO, false><<<g, kDgThreads, 0, st>>>(xp, src, op, m, n, k, tiles_n);
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
