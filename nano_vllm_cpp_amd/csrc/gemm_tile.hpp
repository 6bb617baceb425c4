// The fp32 matrix-core tile kernel shared by the weight GEMM (dense_gemm.hip) and
// the MoE expert products (moe.hip): v_mfma_f32_32x32x2_f32 over BM x 128 output
// tiles (BM = 128: 2 x 2 waves of 64 x 64; BM = 32: 1 x 4 waves of 32 x 32), K in
// 16-element LDS stages, double-buffered with the next stage's loads in flight.
//   * activation rows, upconverted to fp32 (8 elements per thread);
//   * weight rows, decoded to fp32 by the element sources of weight_formats.hpp
//     (8 elements per thread, bit-exact values);
//   * LDS rows padded to 20 floats, so the 16 lanes of a ds_read_b128 phase hit
//     16 distinct 4-bank groups.
// Inside a stage the k order is permuted (the dot product does not care): MFMA
// step s contracts k = s on lanes 0-31 and k = 8 + s on lanes 32-63 for both
// operands, so each lane reads its 8 values of a row as two 16-byte LDS reads.
// A k that is not a multiple of 16, or a misaligned operand, runs the RAGGED
// variant: the same tiles and MFMAs, every staged value read on its own, k beyond
// the row's end staged as zero, weights decoded through 4-element aligned runs.
#pragma once

#include "nvf_device.hpp"
#include "nvf_host.hpp"
#include "weight_formats.hpp"

namespace nvf {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// bf16 weight rows take the split product: each fp32 activation is the exact sum of
// three bf16 pieces (RNE to 8 bits, then the remainder, twice: 24 = 3 x 8 significand
// bits), so the three bf16 matrix-core products x_i . w are exact products summed in
// fp32 -- 3k terms instead of k, at 16 / 3 times the fp32 matrix-core rate.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Whether the decode product double-buffers a source's raw loads: measured per
// source -- it pays for fp16 / bf16 rows and Q4_K / Q5_K groups, and costs more in
// occupancy than it gains for fp32 rows and Q6_K groups (larger raw registers).
template <typename S>
struct GemvPrefetch {
  static constexpr bool value = true;
};
template <>
struct GemvPrefetch<Table<8, float>> {
  static constexpr bool value = false;
};

template <typename S>
struct SplitBf16 {
  static constexpr bool value = false;
};
template <>
struct SplitBf16<Table<8, __bf16>> {
  static constexpr bool value = true;
};
// the tile kernel splits fp16 weights too (two exact bf16 pieces each)
template <typename S>
struct SplitTile {
  static constexpr bool value = false;
};
template <>
struct SplitTile<Table<8, __bf16>> {
  static constexpr bool value = true;
};
template <>
struct SplitTile<Table<8, _Float16>> {
  static constexpr bool value = true;
};
__device__ __forceinline__ void split3(const float* v, bf16x8* p) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // the first piece truncates (the top 16 bits of v): exact, and it cannot round up
    // past the largest bf16 to infinity the way round-to-nearest would near FLT_MAX;
    // an infinite v keeps its infinity in the first piece alone
    const __bf16 a = __builtin_bit_cast(__bf16, (uint16_t)(__builtin_bit_cast(uint32_t, v[i]) >> 16));
    const float r1 = __builtin_isinf(v[i]) ? 0.0f : v[i] - (float)a;  // exact: the bits below a's 8
    const __bf16 b = (__bf16)r1;
    const float r2 = r1 - (float)b;    // exact, and at most 8 significant bits
    p[0][i] = a;
    p[1][i] = b;
    p[2][i] = (__bf16)r2;
  }
}
__device__ __forceinline__ bf16x8 raw_bf16x8(const Table<8, __bf16>::Raw& r) {
  return __builtin_bit_cast(bf16x8, u32x4{r.w[0], r.w[1], r.w[2], r.w[3]});
}
template <typename T>
__device__ __forceinline__ bf16x8 raw_bf16x8(const T&) {  // never called: the split takes bf16 rows only
  return bf16x8{};
}


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

// The tile kernel over a problem policy P, which names the workgroup's tiles and
// the element offsets of their rows and columns, and stores the results.  A
// workgroup takes items blockIdx.x, blockIdx.x + gridDim.x, ... until tile() says
// there are no more (a policy with more tiles than the grid has workgroups):
//   bool tile(int64_t item, int tiles_n, Tile& t)  -- false: no such item
//   static constexpr bool kLoop                    -- false: one item per workgroup
//   int64_t a_row(const Tile&, int r)         -- element offset of tile row r in x, or -1
//   int64_t b_row(const Tile&, int c)         -- element offset of tile column c's weight row, or -1
//   void store(const Tile&, int r, int c, v)  -- result of tile row r, column c
// PlainProb below is the plain GEMM; the MoE expert products supply their own.
template <typename TX, typename Src, int BM, bool RAGGED, typename P>
__global__ __launch_bounds__(kDgThreads) __attribute__((amdgpu_waves_per_eu(2))) void gemm_tile_kernel(
    const TX* __restrict__ x, Src w, P prob, int64_t k, int tiles_n) {
  constexpr int WN = BM == 128 ? 2 : 4;              // waves along n
  constexpr int TM = BM == 128 ? 2 : 1;              // 32-row MFMA tiles per wave
  constexpr int TN = BM == 128 ? 2 : 1;              // 32-column MFMA tiles per wave
  constexpr int kStage = dg_stage_floats<BM>();
  __shared__ float lds[2 * kStage];
  for (int64_t item = blockIdx.x;; item += gridDim.x) {
    typename P::Tile tile;
    if (!prob.tile(item, tiles_n, tile)) break;  // uniform per workgroup
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;

    // staging roles: thread t moves 8 k-values (half t & 1 of the stage) of activation
    // row t >> 1 (t < 2 BM) and of weight column t >> 1
    const int sr = tid >> 1, sh = (tid & 1) * 8;
    const bool a_role = sr < BM;
    const int64_t a_off = a_role ? prob.a_row(tile, sr) : -1, b_off = prob.b_row(tile, sr);
    const bool a_ok = a_off >= 0, b_ok = b_off >= 0;
    const Table<8, TX> xs{x};
    typename Table<8, TX>::Raw ar;
    typename Src::Raw br;
    const int64_t a_e0 = a_off + sh;  // element offsets at stage 0
    const int64_t b_e0 = b_off + sh;
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
        const int r = TM * 32 * wm + 32 * a + 8 * (j >> 2) + 4 * half + (j & 3);
#pragma unroll
        for (int b = 0; b < TN; ++b) prob.store(tile, r, TN * 32 * wn + 32 * b + (lane & 31), acc[a][b][j]);
      }
    if constexpr (!P::kLoop) break;  // one item per workgroup
    __syncthreads();                 // LDS is reused by the next item
  }
}

// fp16 / bf16 weight rows on the bf16 matrix cores (BM = 128, k % 16 == 0,
// vector-aligned operands): the tile kernel's structure with each staged activation
// split into three bf16 pieces (split3: exact) and each weight staged as it is (bf16)
// or as two bf16 pieces (fp16: 11 significand bits = 8 + the exact remainder), so
// 3 x WP v_mfma_f32_32x32x16_bf16 per 16-k stage and 32 x 32 tile sum exact products
// in fp32 (3 WP k terms instead of k).  LDS per stage: three activation planes and WP
// weight planes, rows of 16 bf16 padded to 48 bytes (the 16 rows of a ds_read_b128
// phase hit distinct bank groups: 3 r mod 16).  Lane l reads 8 bf16 of row l % 32 at
// k slot 8 (l / 32) for both operands, so the instruction contracts matching k.
constexpr int kSpRow = 24;  // bf16 per staged row (16 + padding)
template <typename TX, typename TW, typename P>
__global__ __launch_bounds__(kDgThreads) __attribute__((amdgpu_waves_per_eu(2))) void gemm_tile_split_kernel(
    const TX* __restrict__ x, Table<8, TW> w, P prob, int64_t k, int tiles_n) {
  constexpr int BM = 128, WN = 2, TM = 2, TN = 2;
  constexpr int WP = __is_same(TW, __bf16) ? 1 : 2;                 // weight pieces
  constexpr int kPlane = BM * kSpRow, kStage = (3 + WP) * kPlane;  // activation planes + weight planes (bf16)
  __shared__ __attribute__((aligned(16))) __bf16 lds[2 * kStage];
  for (int64_t item = blockIdx.x;; item += gridDim.x) {
    typename P::Tile tile;
    if (!prob.tile(item, tiles_n, tile)) break;  // uniform per workgroup
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    // staging: thread t moves 8 k-values (half t & 1 of the stage) of activation row
    // t >> 1 and of weight column t >> 1
    const int sr = tid >> 1, sh = (tid & 1) * 8;
    const int64_t a_off = prob.a_row(tile, sr), b_off = prob.b_row(tile, sr);
    const bool a_ok = a_off >= 0, b_ok = b_off >= 0;
    const Table<8, TX> xs{x};
    typename Table<8, TX>::Raw ar;
    typename Table<8, TW>::Raw br;
    auto load = [&](int st) {
      const int64_t kc = (int64_t)st * kDgKC + sh;
      if (a_ok) ar = xs.load(a_off + kc);
      if (b_ok) br = w.load(b_off + kc);
    };
    auto store = [&](int buf) {
      __bf16* s = lds + buf * kStage;
      float v[8];
      if (a_ok) {
        xs.decode(ar, v);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
      }
      bf16x8 p[3];
      split3(v, p);
#pragma unroll
      for (int pc = 0; pc < 3; ++pc) st16(s + pc * kPlane + sr * kSpRow + sh, __builtin_bit_cast(u32x4, p[pc]));
      if constexpr (WP == 1) {
        st16(s + 3 * kPlane + sr * kSpRow + sh, b_ok ? u32x4{br.w[0], br.w[1], br.w[2], br.w[3]} : u32x4{});
      } else {
        float wv[8];
        if (b_ok) {
          w.decode(br, wv);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) wv[i] = 0.0f;
        }
        bf16x8 q[3];
        split3(wv, q);  // an fp16 value: q[2] is 0
        st16(s + 3 * kPlane + sr * kSpRow + sh, __builtin_bit_cast(u32x4, q[0]));
        st16(s + 4 * kPlane + sr * kSpRow + sh, __builtin_bit_cast(u32x4, q[1]));
      }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b) acc[a][b] = f32x16{};
    const int half = lane >> 5;
    const int fa = (TM * 32 * wm + (lane & 31)) * kSpRow + 8 * half;
    const int fb = (TN * 32 * wn + (lane & 31)) * kSpRow + 8 * half;

    const int nst = (int)(k / kDgKC);
    load(0);
    store(0);
    __syncthreads();
#pragma unroll 1
    for (int st = 0; st < nst; ++st) {
      const __bf16* s = lds + (st & 1) * kStage;
      if (st + 1 < nst) load(st + 1);  // in flight during this stage's MFMAs
#pragma unroll
      for (int wq = WP - 1; wq >= 0; --wq) {  // the smallest pieces first
        bf16x8 bv[TN];
#pragma unroll
        for (int b = 0; b < TN; ++b)
          bv[b] = __builtin_bit_cast(bf16x8, ld16(s + (3 + wq) * kPlane + fb + b * 32 * kSpRow));
#pragma unroll
        for (int pc = 2; pc >= 0; --pc) {
          bf16x8 av[TM];
#pragma unroll
          for (int a = 0; a < TM; ++a)
            av[a] = __builtin_bit_cast(bf16x8, ld16(s + pc * kPlane + fa + a * 32 * kSpRow));
#pragma unroll
          for (int a = 0; a < TM; ++a)
#pragma unroll
            for (int b = 0; b < TN; ++b)
              acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
      }
      if (st + 1 < nst) {
        store((st + 1) & 1);  // the other buffer: its last readers passed the previous barrier
        __syncthreads();
      }
    }

    // D layout of the 32 x 32 MFMAs: lane l, value j -> column l % 32,
    // row 8 (j / 4) + 4 (l / 32) + j % 4
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int r = TM * 32 * wm + 32 * a + 8 * (j >> 2) + 4 * half + (j & 3);
#pragma unroll
        for (int b = 0; b < TN; ++b) prob.store(tile, r, TN * 32 * wn + 32 * b + (lane & 31), acc[a][b][j]);
      }
    if constexpr (!P::kLoop) break;  // one item per workgroup
    __syncthreads();                 // LDS is reused by the next item
  }
}

// The plain GEMM: out[m][n] (row-major, TO) = x[m][k] . W[n][k]^T, tiles in dg_tile's
// XCD-aware order.
template <int BM, typename TO>
struct PlainProb {
  static constexpr bool kLoop = false;
  TO* out;
  int64_t m, n, k;
  struct Tile {
    int64_t row0, col0;
  };
  __device__ bool tile(int64_t item, int tiles_n, Tile& t) const {
    if (item != blockIdx.x) return false;  // one tile per workgroup
    int64_t tm, tn;
    dg_tile(tiles_n, tm, tn);
    t.row0 = tm * BM;
    t.col0 = tn * kDgBN;
    return true;
  }
  __device__ int64_t a_row(const Tile& t, int r) const { return t.row0 + r < m ? (t.row0 + r) * k : -1; }
  __device__ int64_t b_row(const Tile& t, int c) const { return t.col0 + c < n ? (t.col0 + c) * k : -1; }
  __device__ void store(const Tile& t, int r, int c, float v) const {
    const int64_t rr = t.row0 + r, cc = t.col0 + c;
    if (rr < m && cc < n) out[rr * n + cc] = from_f32<TO>(v);
  }
};

// ---------------------------------------------------------------------------
// Decode-shaped product on v_mfma_f32_16x16x4_f32 (m <= 16 rows): lane l = 16 s + j
// gives activation row j and weight column j at k slot s.  Lane l streams 16
// (dense: two runs of 8) or 32 consecutive k at offset (16 or 32) s of column j of
// each of C 16-column groups; value i of the lane's span is MFMA step i, with
// k slot s <-> k = span s + i.  The matrix core sums the k slots; the 4 waves of a
// workgroup split K and meet in LDS, summed in wave order.  The problem policy P
// names the columns of work item `item` (items blockIdx.x, blockIdx.x + gridDim.x,
// ... until it answers false) and the element offsets of its rows and columns:
//   bool tile(int64_t item, int cols, Tile& t), a_row(t, j), b_row(t, c), store(t, r, c, v).
constexpr int kGvWaves = 4;

template <typename S>
struct RunOf;  // elements one load of a source yields
template <typename T>
struct RunOf<Table<8, T>> {
  static constexpr int value = 8;
};


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

template <typename TX, typename Src, int C, typename P>
__global__ __launch_bounds__(kGvWaves * 64) void gemv_mfma_kernel(const TX* __restrict__ x, Src w, P prob,
                                                                  int64_t k) {
  constexpr int R = RunOf<Src>::value, H = R == 8 ? 2 : 1, SPAN = H * R, KS = 4 * SPAN;
  constexpr bool kSplit = SplitBf16<Src>::value;
  __shared__ float part[kGvWaves][C][16][17];  // [wave][group][row][column] (padded)
  const int lane = threadIdx.x & 63, j = lane & 15, ks = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const Table<8, TX> xs{x};
  struct Buf {  // one step's raw loads
    typename Src::Raw w[C][H];
    typename Table<8, TX>::Raw x[H][R / 8];
  };
  for (int64_t item = blockIdx.x;; item += gridDim.x) {
    typename P::Tile tile;
    if (!prob.tile(item, 16 * C, tile)) break;  // uniform per workgroup
    const int64_t nsteps = (k + KS - 1) / KS, full = k / KS;  // steps; steps every lane's runs are inside
    const int64_t s_begin = nsteps * wave / kGvWaves, s_end = nsteps * (wave + 1) / kGvWaves;
    const int64_t f_end = s_end < full ? s_end : full;
    // a row or column outside the problem reads row 0 of its operand instead (valid
    // memory; its results are never stored), so the loop has no per-lane branches
    int64_t x_off = prob.a_row(tile, j);
    const bool row_ok = x_off >= 0;
    if (!row_ok) x_off = 0;
    int64_t w_off[C];
    bool col_ok[C];
#pragma unroll
    for (int q = 0; q < C; ++q) {
      w_off[q] = prob.b_row(tile, 16 * q + j);
      col_ok[q] = w_off[q] >= 0;
      if (!col_ok[q]) w_off[q] = 0;
    }
    f32x4 acc[C];
#pragma unroll
    for (int q = 0; q < C; ++q) acc[q] = f32x4{};

    // lane runs h of step st: k = st KS + SPAN ks + R h .. + R; `lim` masks the runs
    // of a partial last step (every run is inside on a full step)
    auto load = [&](Buf& f, int64_t st, bool partial) {
      const int64_t kk = st * KS + (int64_t)SPAN * ks;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        if (partial && kk + R * h >= k) continue;
#pragma unroll
        for (int q = 0; q < C; ++q) f.w[q][h] = w.load(w_off[q] + kk + R * h);
        // without the prefetch every step waits for all its loads, so a row outside the
        // problem may skip its load (its lanes' results are not stored)
        if (GemvPrefetch<Src>::value || row_ok) load_x_run<TX, R>(xs, x_off + kk + R * h, f.x[h]);
      }
    };
    auto compute = [&](const Buf& f, int64_t st, bool partial) {
      const int64_t kk = st * KS + (int64_t)SPAN * ks;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const bool in = !partial || kk + R * h < k;
        float xv[R];
        if (in) {
          decode_x_run<TX, R>(xs, f.x[h], xv);
        } else {
#pragma unroll
          for (int i = 0; i < R; ++i) xv[i] = 0.0f;
        }
        if constexpr (kSplit) {
          // x = x1 + x2 + x3 exactly in bf16; each piece times a bf16 weight is exact in fp32
          bf16x8 xp[3];
          split3(xv, xp);
#pragma unroll
          for (int q = 0; q < C; ++q) {
            const bf16x8 wb = in ? raw_bf16x8(f.w[q][h]) : bf16x8{};
#pragma unroll
            for (int pc = 2; pc >= 0; --pc)  // the smallest pieces first
              acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xp[pc], wb, acc[q], 0, 0, 0);
          }
        } else {
#pragma unroll
          for (int q = 0; q < C; ++q) {
            float wv[R];
            if (in) {
              w.decode(f.w[q][h], wv);
            } else {
#pragma unroll
              for (int i = 0; i < R; ++i) wv[i] = 0.0f;
            }
#pragma unroll
            for (int i = 0; i < R; ++i) acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[i], wv[i], acc[q], 0, 0, 0);
          }
        }
      }
    };
    // full steps; with GemvPrefetch, two raw buffers in turn with the next step's loads
    // in flight, the prefetch unconditional (the last step reloads itself), which keeps
    // the memory-counter waits exact
    Buf fa;
    int64_t st = s_begin;
    if constexpr (GemvPrefetch<Src>::value) {
      Buf fb;
      if (st < f_end) {
        const int64_t last = f_end - 1;
        load(fa, st, false);
        while (true) {
          load(fb, st + 1 < last ? st + 1 : last, false);
          compute(fa, st, false);
          if (++st >= f_end) break;
          load(fa, st + 1 < last ? st + 1 : last, false);
          compute(fb, st, false);
          if (++st >= f_end) break;
        }
      }
    } else {
      for (; st < f_end; ++st) {
        load(fa, st, false);
        compute(fa, st, false);
      }
    }
    if (f_end < s_end) {  // the partial last step
      load(fa, f_end, true);
      compute(fa, f_end, true);
    }

    // D of v_mfma_f32_16x16x4_f32 and 16x16x32_bf16: lane l, value r -> row 4 (l / 16) + r, column l % 16
#pragma unroll
    for (int q = 0; q < C; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[wave][q][4 * ks + r][j] = acc[q][r];
    __syncthreads();
    for (int t = (int)threadIdx.x; t < C * 256; t += kGvWaves * 64) {
      const int jj = t & 15, row = (t >> 4) & 15, q = t >> 8;
      float v = part[0][q][row][jj];
#pragma unroll
      for (int wv = 1; wv < kGvWaves; ++wv) v += part[wv][q][row][jj];
      prob.store(tile, row, 16 * q + jj, v);
    }
    if constexpr (!P::kLoop) break;  // one item per workgroup
    __syncthreads();                 // LDS is reused by the next item
  }
}

// ---------------------------------------------------------------------------
// Decode-shaped product with plain FMAs (m <= MR rows, MR = 1 or 2): LPC = 16 (dense
// rows) or 8 (K-quant groups) lanes per column; lane l = CPS b + j (CPS = 64 / LPC
// columns per set) streams run b of column j of each of its C column sets (LPC runs:
// 128 or 256 contiguous k of one column per step) with the same k of each row,
// accumulating MR x C fp32 sums; the LPC lanes of a column are summed at the end.  S
// waves of the workgroup split K (S = 4), or each wave owns its own columns (S = 1,
// wide outputs).  Full steps double-buffer the raw loads with an unconditional
// prefetch (the last step reloads itself), which keeps the memory-counter waits
// exact.  A row or column outside the problem reads row 0 (valid memory; its results
// are never stored).  The policy names the workgroup's G C CPS columns per item.
// LPCX (optional): lanes per column instead (64: a load instruction covers 1 KB of one
// weight row).
template <typename TX, typename Src, int MR, int C, int S, typename P, int LPCX = 0>
__global__ __launch_bounds__(kGvWaves * 64) void gemv_fma_kernel(const TX* __restrict__ x, Src w, P prob,
                                                                 int64_t k) {
  constexpr int R = RunOf<Src>::value, LPC = LPCX ? LPCX : (R == 8 ? 16 : 8), CPS = 64 / LPC, KS = LPC * R;
  constexpr int G = kGvWaves / S;               // column groups per workgroup (S waves split K in each)
  __shared__ float part[kGvWaves][MR][C][CPS];  // [wave][row][set][column]
  const int lane = threadIdx.x & 63, j = lane % CPS, b = lane / CPS;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int grp = wave / S, split = wave % S;
  const Table<8, TX> xs{x};
  struct Buf {
    typename Src::Raw w[C];
    typename Table<8, TX>::Raw x[MR][R / 8];
  };
  for (int64_t item = blockIdx.x;; item += gridDim.x) {
    typename P::Tile tile;
    if (!prob.tile(item, G * CPS * C, tile)) break;  // uniform per workgroup
    const int64_t nsteps = (k + KS - 1) / KS, full = k / KS;  // steps; steps every lane's run is inside
    const int64_t s_begin = nsteps * split / S, s_end = nsteps * (split + 1) / S;
    const int64_t f_end = s_end < full ? s_end : full;
    const int64_t kb = (int64_t)R * b;  // this lane's run inside a step
    int64_t wrow[C];
#pragma unroll
    for (int q = 0; q < C; ++q) {
      const int64_t o = prob.b_row(tile, grp * CPS * C + CPS * q + j);
      wrow[q] = (o >= 0 ? o : 0) + kb;
    }
    int64_t xrow[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      const int64_t o = prob.a_row(tile, r);
      xrow[r] = (o >= 0 ? o : 0) + kb;
    }
    float acc[MR][C];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int q = 0; q < C; ++q) acc[r][q] = 0.0f;

    auto load = [&](Buf& f, int64_t st) {
      const int64_t kk = st * KS;
#pragma unroll
      for (int q = 0; q < C; ++q) f.w[q] = w.load(wrow[q] + kk);
#pragma unroll
      for (int r = 0; r < MR; ++r) load_x_run<TX, R>(xs, xrow[r] + kk, f.x[r]);
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
    if (f_end < s_end && kb + f_end * KS < k) {
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
      float v = part[g * S][r][q][jj];
#pragma unroll
      for (int wv = 1; wv < S; ++wv) v += part[g * S + wv][r][q][jj];
      prob.store(tile, r, g * CPS * C + CPS * q + jj, v);
    }
    if constexpr (!P::kLoop) break;  // one item per workgroup
    __syncthreads();                 // LDS is reused by the next item
  }
}

// The plain decode product: out[m][n] = x[m][k] . W[n][k]^T, m <= 16, workgroup b
// on columns [b 16 C, (b + 1) 16 C).
template <typename TO>
struct PlainGemvProb {
  static constexpr bool kLoop = false;
  TO* out;
  int64_t m, n, k;
  struct Tile {
    int64_t col0;
  };
  __device__ bool tile(int64_t item, int cols, Tile& t) const {
    if (item != blockIdx.x) return false;  // one column group per workgroup
    t.col0 = item * cols;
    return true;
  }
  __device__ int64_t a_row(const Tile&, int j) const { return j < m ? (int64_t)j * k : -1; }
  __device__ int64_t b_row(const Tile& t, int c) const { return t.col0 + c < n ? (t.col0 + c) * k : -1; }
  __device__ void store(const Tile& t, int r, int c, float v) const {
    if (r < m && t.col0 + c < n) out[(int64_t)r * n + t.col0 + c] = from_f32<TO>(v);
  }
};


}  // namespace nvf
