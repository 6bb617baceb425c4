// Mixture-of-experts routing and expert FFN, and the two elementwise helpers of
// the shared-expert path.
//
// Reference: hip_moe_route (moe_route_kernel, src/hip_ops.hip:813-844), hip_moe_ffn
// (moe_ffn_kernel :861-893, launcher :901-912), hip_add_inplace (:914-923) and
// hip_scale_rows_sigmoid (:925-939), called from src/model.cpp:797-828 for a layer
// with experts.  The reference runs one thread per row for the routing and one
// workgroup per token for the FFN, with a scalar dot product per weight row.
//
// Routing (moe_route_kernel): one wave per row, the reference's arithmetic in
// double in its order -- the maximum and the sums by one lane in index order, the
// exponentials in parallel, and the top-K selection as the reference's selection
// sort: each round takes the largest value at positions >= i (a tie goes to the
// smallest position: its strict-greater scan) and swaps it to position i.  So the
// experts chosen and their order, ties included, are the reference's, and the
// scores are its doubles rounded once to fp32.  (NaN logits are outside this: the
// reference's result then depends on its scan order.)
//
// Expert FFN: out[t] += sum_k w[t,k] * down_e(silu(gate_e(x[t])) * up_e(x[t])),
// e = slot_of[idx[t,k]], for w != 0.  On the GPU the (token, k) pairs are grouped by
// expert slot, and each slot's pairs run as one matrix product on the fp32 matrix
// cores (the tile kernel of gemm_tile.hpp with a gathering problem policy):
//   1. count the pairs per slot, scan, and list each slot's 32- or 128-row tiles;
//   2. scatter the pairs into slot order;
//   3. gate/up: [pairs of slot s] x gu[s]^T -> GU (fp32, 2I per pair);
//   4. SwiGLU (nvf_silu_and_mul on fp32: the reference's g / (1 + expf(-g)) * u);
//   5. down: Y x dn[s]^T -> V, stored by pair;
//   6. combine: res = sum over k in k order of w * V[t, k] (skipping w == 0), out += res,
//      the reference's accumulation order, so the result does not depend on the
//      scatter order and no atomics touch the output.
// The products' fp32 sums run in another order than the reference's block_dot, so
// results agree within the bound the tests state, not bit for bit.
#include <mutex>

#include "gemm_tile.hpp"

namespace nvf {

// ---------------------------------------------------------------------------
// routing
constexpr int kMoeMaxExperts = 4096;

__global__ __launch_bounds__(64) void moe_route_kernel(const float* __restrict__ logits, int E, int K, int norm,
                                                      int32_t* __restrict__ idx, float* __restrict__ score) {
  extern __shared__ __attribute__((aligned(16))) double rsm[];
  double* pr = rsm;                                   // [E] values, permuted by the selection
  int* ix = reinterpret_cast<int*>(rsm + E);          // [E] expert ids, permuted alike
  __shared__ double s_max, s_inv;
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x;
  const float* lg = logits + t * E;
  if (lane == 0) {  // the reference's running maximum, in index order
    double m = -1e300;
    for (int i = 0; i < E; ++i) {
      const double v = (double)lg[i];
      m = m > v ? m : v;
    }
    s_max = m;
  }
  __syncthreads();
  const double maxv = s_max;
  for (int i = lane; i < E; i += 64) pr[i] = exp((double)lg[i] - maxv);
  __syncthreads();
  if (lane == 0) {
    double sum = 0.0;
    for (int i = 0; i < E; ++i) sum += pr[i];
    s_inv = 1.0 / sum;
  }
  __syncthreads();
  const double inv = s_inv;
  for (int i = lane; i < E; i += 64) {
    pr[i] *= inv;
    ix[i] = i;
  }
  __syncthreads();
  for (int i = 0; i < K; ++i) {
    // largest value at positions >= i; a tie goes to the smaller position.  Every
    // lane starts from position i itself, as the reference's scan does (best = i),
    // so a NaN there keeps i (nothing compares greater) and NaNs elsewhere never win.
    double bv = pr[i];
    int bp = i;
    for (int j = i + 1 + lane; j < E; j += 64)
      if (pr[j] > bv) {
        bv = pr[j];
        bp = j;
      }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
      const double ov = __shfl_xor(bv, d, 64);
      const int op = __shfl_xor(bp, d, 64);
      if (ov > bv || (ov == bv && op < bp)) {
        bv = ov;
        bp = op;
      }
    }
    if (lane == 0) {
      const double tp = pr[i];
      pr[i] = pr[bp];
      pr[bp] = tp;
      const int ti = ix[i];
      ix[i] = ix[bp];
      ix[bp] = ti;
      idx[t * K + i] = ix[i];
      score[t * K + i] = (float)pr[i];
    }
    __syncthreads();
  }
  if (norm && lane == 0) {
    double s = 0.0;
    for (int i = 0; i < K; ++i) s += pr[i];
    const double sinv = 1.0 / s;
    for (int i = 0; i < K; ++i) score[t * K + i] = (float)(pr[i] * sinv);
  }
}

// ---------------------------------------------------------------------------
// elementwise helpers (fp32, 16-byte vectors where the pointers allow)
__global__ void add_inplace_kernel(float* __restrict__ dst, const float* __restrict__ src, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] += src[i];
}
__global__ void add_inplace_vec_kernel(float* __restrict__ dst, const float* __restrict__ src, int64_t n4) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    f32x4 a = __builtin_bit_cast(f32x4, ld16(dst + 4 * i));
    const f32x4 b = __builtin_bit_cast(f32x4, ld16(src + 4 * i));
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] += b[j];
    st16(dst + 4 * i, __builtin_bit_cast(u32x4, a));
  }
}

// dst[t, c] *= 1 / (1 + expf(-s[t])): one workgroup per row, the factor formed as
// the reference forms it (so each element's product is the reference's)
__global__ __launch_bounds__(256) void scale_rows_sigmoid_kernel(float* __restrict__ dst, const float* __restrict__ s,
                                                                 int64_t cols) {
  const int64_t t = blockIdx.x;
  const float g = s[t];
  const float f = 1.0f / (1.0f + expf(-g));
  float* row = dst + t * cols;
  for (int64_t c = threadIdx.x; c < cols; c += 256) row[c] *= f;
}

// ---------------------------------------------------------------------------
// expert FFN
constexpr int kMoeMaxSlots = 65536;

struct MoeLayout {  // workspace regions (byte offsets, 256-aligned)
  int64_t counts, cursor, offsets, tile_slot, tile_pos, tile_end, ntiles, list, gu, y, v, total;
  int64_t max_tiles;
  static int64_t up(int64_t b) { return (b + 255) & ~int64_t(255); }
  MoeLayout(int64_t pairs, int64_t H, int64_t I, int64_t slots, int bm) {
    max_tiles = (pairs + bm - 1) / bm + (pairs < slots ? pairs : slots);
    int64_t o = 0;
    counts = o;
    o += up(4 * slots);
    cursor = o;
    o += up(4 * slots);
    offsets = o;
    o += up(4 * (slots + 1));
    tile_slot = o;
    o += up(4 * max_tiles);
    tile_pos = o;
    o += up(4 * max_tiles);
    tile_end = o;
    o += up(4 * max_tiles);
    ntiles = o;
    o += 256;
    list = o;
    o += up(4 * pairs);
    gu = o;
    o += up(8 * pairs * I);
    y = o;
    o += up(4 * pairs * I);
    v = o;
    o += up(4 * pairs * H);
    total = o;
  }
};

__global__ void moe_clear_kernel(int32_t* __restrict__ counts, int32_t* __restrict__ cursor, int64_t slots) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < slots; i += (int64_t)gridDim.x * blockDim.x) {
    counts[i] = 0;
    cursor[i] = 0;
  }
}

// a pair takes part when its weight is nonzero and its expert has a slot in [0, slots)
__device__ __forceinline__ int pair_slot(const int32_t* idx, const float* score, const int32_t* slot_of, int64_t p,
                                         int64_t slots) {
  if (score[p] == 0.0f) return -1;
  const int32_t s = slot_of[idx[p]];
  return s >= 0 && s < slots ? s : -1;
}

__global__ void moe_count_kernel(const int32_t* __restrict__ idx, const float* __restrict__ score,
                                 const int32_t* __restrict__ slot_of, int64_t pairs, int64_t slots,
                                 int32_t* __restrict__ counts) {
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < pairs; p += (int64_t)gridDim.x * blockDim.x) {
    const int s = pair_slot(idx, score, slot_of, p, slots);
    if (s >= 0) atomicAdd(counts + s, 1);
  }
}

// One workgroup: exclusive scans of the counts (row offsets) and of each slot's
// tile count, then the tile list (slot, first row) and its length.
constexpr int kScanThreads = 1024;
__global__ __launch_bounds__(kScanThreads) void moe_scan_kernel(const int32_t* __restrict__ counts, int64_t slots,
                                                                int bm, int32_t* __restrict__ offsets,
                                                                int32_t* __restrict__ tile_slot,
                                                                int32_t* __restrict__ tile_pos,
                                                                int32_t* __restrict__ tile_end,
                                                                int32_t* __restrict__ ntiles) {
  __shared__ int32_t part_rows[kScanThreads], part_tiles[kScanThreads];
  const int tid = threadIdx.x;
  const int64_t per = (slots + kScanThreads - 1) / kScanThreads;
  const int64_t s0 = tid * per, s1 = s0 + per < slots ? s0 + per : slots;
  int32_t rows = 0, tiles = 0;
  for (int64_t s = s0; s < s1; ++s) {
    rows += counts[s];
    tiles += (counts[s] + bm - 1) / bm;
  }
  part_rows[tid] = rows;
  part_tiles[tid] = tiles;
  __syncthreads();
  for (int d = 1; d < kScanThreads; d <<= 1) {  // inclusive scan (Hillis-Steele)
    const int32_t a = tid >= d ? part_rows[tid - d] : 0, b = tid >= d ? part_tiles[tid - d] : 0;
    __syncthreads();
    part_rows[tid] += a;
    part_tiles[tid] += b;
    __syncthreads();
  }
  int32_t r = part_rows[tid] - rows, tl = part_tiles[tid] - tiles;
  for (int64_t s = s0; s < s1; ++s) {
    offsets[s] = r;
    const int32_t c = counts[s];
    for (int32_t i = 0; i < c; i += bm) {
      tile_slot[tl] = (int32_t)s;
      tile_pos[tl] = r + i;
      tile_end[tl] = r + c;
      ++tl;
    }
    r += c;
  }
  if (tid == kScanThreads - 1) {
    offsets[slots] = part_rows[tid];
    *ntiles = part_tiles[tid];
  }
}

__global__ void moe_scatter_kernel(const int32_t* __restrict__ idx, const float* __restrict__ score,
                                   const int32_t* __restrict__ slot_of, int64_t pairs, int64_t slots,
                                   const int32_t* __restrict__ offsets, int32_t* __restrict__ cursor,
                                   int32_t* __restrict__ list) {
  for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < pairs; p += (int64_t)gridDim.x * blockDim.x) {
    const int s = pair_slot(idx, score, slot_of, p, slots);
    if (s >= 0) list[offsets[s] + atomicAdd(cursor + s, 1)] = (int32_t)p;
  }
}

// Up to 4096 pairs: one workgroup sorts the (slot, pair) keys in LDS (bitonic),
// then the first position of each slot's run walks to the run's end and lists its
// tiles.  Needs no slot range (the counting path above scans every slot) and is
// one launch instead of four.
constexpr int kSortMax = 4096;
__global__ __launch_bounds__(1024) void moe_sort_small_kernel(const int32_t* __restrict__ idx,
                                                              const float* __restrict__ score,
                                                              const int32_t* __restrict__ slot_of, int pairs, int n2,
                                                              int64_t slots, int bm, int32_t* __restrict__ list,
                                                              int32_t* __restrict__ tile_slot,
                                                              int32_t* __restrict__ tile_pos,
                                                              int32_t* __restrict__ tile_end,
                                                              int32_t* __restrict__ ntiles) {
  __shared__ uint32_t key[kSortMax];
  __shared__ int32_t count;
  const int tid = threadIdx.x;
  if (tid == 0) count = 0;
  for (int i = tid; i < n2; i += 1024) {
    const int s = i < pairs ? pair_slot(idx, score, slot_of, i, slots) : -1;
    key[i] = s >= 0 ? ((uint32_t)s << 12) | (uint32_t)i : 0xffffffffu;  // slot < 2^16, pair < 2^12
  }
  __syncthreads();
  for (int size = 2; size <= n2; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < n2; i += 1024) {
        const int j = i ^ stride;
        if (j > i) {
          const uint32_t a = key[i], b = key[j];
          if ((a > b) == ((i & size) == 0)) {
            key[i] = b;
            key[j] = a;
          }
        }
      }
      __syncthreads();
    }
  for (int i = tid; i < pairs; i += 1024) {
    const uint32_t ki = key[i];
    if (ki == 0xffffffffu) continue;
    list[i] = (int32_t)(ki & 0xfffu);
    const uint32_t slot = ki >> 12;
    if (i > 0 && (key[i - 1] >> 12) == slot) continue;  // not the run's first position
    int end = i + 1;
    while (end < pairs && key[end] != 0xffffffffu && (key[end] >> 12) == slot) ++end;
    for (int p = i; p < end; p += bm) {
      const int t = atomicAdd(&count, 1);
      tile_slot[t] = (int32_t)slot;
      tile_pos[t] = p;
      tile_end[t] = end;
    }
  }
  __syncthreads();
  if (tid == 0) *ntiles = count;
}

// The expert products as tile-kernel problems: tile = (slot, first list row,
// first column); rows past the slot's last pair, or columns past n, are empty.
struct MoeTiles {
  static constexpr bool kLoop = true;
  const int32_t* tile_slot;
  const int32_t* tile_pos;
  const int32_t* tile_end;
  const int32_t* ntiles;
  const int32_t* list;
  int64_t cols;    // output columns per workgroup
  int64_t n_cols;  // output columns of the product
  struct Tile {
    int64_t slot, pos0, pos_end, col0;
  };
  __device__ bool pick(int64_t item, Tile& t) const {  // item = tile x column groups + column group
    const int64_t groups = (n_cols + cols - 1) / cols;
    const int64_t tm = item / groups;
    if (tm >= *ntiles) return false;
    t.slot = tile_slot[tm];
    t.pos0 = tile_pos[tm];
    t.pos_end = tile_end[tm];
    t.col0 = (item % groups) * cols;
    return true;
  }
};

// gate/up: rows are the pairs' tokens' x rows; columns the slot's 2I weight rows
struct MoeGateUp : MoeTiles {
  int64_t K, H, I;
  float* gu_out;  // [list row][2I]
  using Tile = MoeTiles::Tile;
  __device__ bool tile(int64_t item, int, Tile& t) const { return pick(item, t); }
  __device__ int64_t a_row(const Tile& t, int r) const {
    const int64_t pos = t.pos0 + r;
    return pos < t.pos_end ? (int64_t)(list[pos] / K) * H : -1;
  }
  __device__ int64_t b_row(const Tile& t, int c) const {
    const int64_t col = t.col0 + c;
    return col < 2 * I ? (t.slot * 2 * I + col) * H : -1;
  }
  __device__ void store(const Tile& t, int r, int c, float v) const {
    const int64_t pos = t.pos0 + r, col = t.col0 + c;
    if (pos < t.pos_end && col < 2 * I) gu_out[pos * 2 * I + col] = v;
  }
};

// down: rows are the SwiGLU rows in list order; columns the slot's H weight rows;
// results stored by pair
struct MoeDown : MoeTiles {
  int64_t H, I;
  float* v_out;  // [pair][H]
  using Tile = MoeTiles::Tile;
  __device__ bool tile(int64_t item, int, Tile& t) const { return pick(item, t); }
  __device__ int64_t a_row(const Tile& t, int r) const {
    const int64_t pos = t.pos0 + r;
    return pos < t.pos_end ? pos * I : -1;
  }
  __device__ int64_t b_row(const Tile& t, int c) const {
    const int64_t col = t.col0 + c;
    return col < H ? (t.slot * H + col) * I : -1;
  }
  __device__ void store(const Tile& t, int r, int c, float v) const {
    const int64_t pos = t.pos0 + r, col = t.col0 + c;
    if (pos < t.pos_end && col < H) v_out[(int64_t)list[pos] * H + col] = v;
  }
};

// out[t] += sum over k in k order of w[t,k] * V[t,k] (pairs that took part only):
// one workgroup per token; the token's weights (0 for a pair that did not take
// part) go to LDS once, then each thread sums its columns.
constexpr int kCombineMaxK = 256;
template <typename TO>
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ v, const int32_t* __restrict__ idx,
                                                          const float* __restrict__ score,
                                                          const int32_t* __restrict__ slot_of, int64_t K, int64_t H,
                                                          int64_t slots, TO* __restrict__ out) {
  __shared__ float wk[kCombineMaxK];
  const int64_t t = blockIdx.x;
  for (int64_t k = threadIdx.x; k < K; k += 256)
    wk[k] = pair_slot(idx, score, slot_of, t * K + k, slots) >= 0 ? score[t * K + k] : 0.0f;
  __syncthreads();
  const float* vt = v + t * K * H;
  // 4 columns per thread when the rows are whole 16-byte vectors; 8 k-values' loads
  // are issued before they are added (in k order), so their latencies overlap
  const bool vec = H % 4 == 0;  // v is 256-byte aligned in the workspace
  const int64_t step = vec ? 4 : 1;
  for (int64_t o = threadIdx.x * step; o < H; o += 256 * step) {
    float res[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t k0 = 0; k0 < K; k0 += 8) {
      f32x4 vals[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t k = k0 + u;
        if (k < K && wk[k] != 0.0f) {
          if (vec) {
            vals[u] = __builtin_bit_cast(f32x4, ld16(vt + k * H + o));
          } else {
            vals[u] = f32x4{vt[k * H + o], 0.0f, 0.0f, 0.0f};
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t k = k0 + u;
        if (k < K && wk[k] != 0.0f)
#pragma unroll
          for (int c = 0; c < 4; ++c) res[c] += wk[k] * vals[u][c];
      }
    }
    for (int c = 0; c < (int)step; ++c) out[t * H + o + c] = from_f32<TO>(to_f32(out[t * H + o + c]) + res[c]);
  }
}

// How a call runs: up to 4096 pairs are grouped by the one-launch sort, more by
// counting; rows per expert tile are 16 on the decode product (the grouped form of
// the weight-streaming GEMV, when rows are whole 8-element runs and aligned), else
// 32 or 128 on the tile kernel.
struct MoePlan {
  bool sort, gemv;
  int bm, gemv_c;
  MoePlan(int64_t pairs, int64_t slots, bool vec_rows) {
    gemv = pairs <= kSortMax && vec_rows;
    // the one-launch sort for few pairs, or when counting would scan too many slots
    sort = pairs <= kSortMax && (pairs <= 512 || slots > kSortMax);
    bm = gemv ? 16 : pairs >= 4096 ? 128 : 32;
    // 64 columns per workgroup once there are enough tiles: each workgroup gathers its
    // tile's activation rows once for 4x the weight columns
    gemv_c = pairs >= 256 ? 4 : 1;
  }
};

// The grid: every (tile, column group) item of the bound, capped at 8 workgroups
// per CU; workgroups loop over the items (most of the bound is empty: the number of
// tiles is known only on the device).
inline dim3 moe_grid(int64_t max_tiles, int64_t groups) {
  const int64_t items = max_tiles * groups, cap = 8 * 256;
  return dim3((unsigned)(items < cap ? items : cap));
}

template <typename TX, typename TW, typename Prob>
int moe_product(const TX* a, const TW* w, Prob prob, int64_t k, const MoePlan& plan, bool vec, int64_t max_tiles,
                hipStream_t st) {
  const Table<8, TW> src{w};
  if (plan.gemv) {
    prob.cols = 16 * plan.gemv_c;
    const dim3 g = moe_grid(max_tiles, (prob.n_cols + prob.cols - 1) / prob.cols);
    if (plan.gemv_c == 4)
      gemv_mfma_kernel<TX, Table<8, TW>, 4><<<g, kGvWaves * 64, 0, st>>>(a, src, prob, k);
    else
      gemv_mfma_kernel<TX, Table<8, TW>, 1><<<g, kGvWaves * 64, 0, st>>>(a, src, prob, k);
  } else {
    prob.cols = kDgBN;
    const int tiles_n = (int)((prob.n_cols + kDgBN - 1) / kDgBN);
    const dim3 g = moe_grid(max_tiles, tiles_n);
    if constexpr (SplitTile<Table<8, TW>>::value) {  // the split product on the bf16 matrix cores
      if (plan.bm == 128 && vec) {
        gemm_tile_split_kernel<TX><<<g, kDgThreads, 0, st>>>(a, src, prob, k, tiles_n);
        return launch_status("moe expert product (split)");
      }
    }
    if (plan.bm == 128)
      vec ? gemm_tile_kernel<TX, Table<8, TW>, 128, false><<<g, kDgThreads, 0, st>>>(a, src, prob, k, tiles_n)
          : gemm_tile_kernel<TX, Table<8, TW>, 128, true><<<g, kDgThreads, 0, st>>>(a, src, prob, k, tiles_n);
    else
      vec ? gemm_tile_kernel<TX, Table<8, TW>, 32, false><<<g, kDgThreads, 0, st>>>(a, src, prob, k, tiles_n)
          : gemm_tile_kernel<TX, Table<8, TW>, 32, true><<<g, kDgThreads, 0, st>>>(a, src, prob, k, tiles_n);
  }
  return launch_status("moe expert product");
}

template <typename TX, typename TW>
int launch_moe_ffn(const TX* x, const int32_t* idx, const float* score, const TW* gu, const TW* dn,
                   const int32_t* slot_of, int64_t rows, int64_t H, int64_t I, int64_t K, int64_t slots, void* out,
                   int out_dtype, uint8_t* work, hipStream_t st) {
  const int64_t pairs = rows * K;
  const bool aligned = aligned16(x) && aligned16(gu) && aligned16(dn);
  const MoePlan plan(pairs, slots, aligned && H % 8 == 0 && I % 8 == 0);
  const bool vec = aligned && H % kDgKC == 0 && I % kDgKC == 0;  // the tile kernel's vector staging
  const MoeLayout L(pairs, H, I, slots, plan.bm);
  int32_t* counts = reinterpret_cast<int32_t*>(work + L.counts);
  int32_t* cursor = reinterpret_cast<int32_t*>(work + L.cursor);
  int32_t* offsets = reinterpret_cast<int32_t*>(work + L.offsets);
  int32_t* tile_slot = reinterpret_cast<int32_t*>(work + L.tile_slot);
  int32_t* tile_pos = reinterpret_cast<int32_t*>(work + L.tile_pos);
  int32_t* tile_end = reinterpret_cast<int32_t*>(work + L.tile_end);
  int32_t* ntiles = reinterpret_cast<int32_t*>(work + L.ntiles);
  int32_t* list = reinterpret_cast<int32_t*>(work + L.list);
  float* gu_rows = reinterpret_cast<float*>(work + L.gu);
  float* y_rows = reinterpret_cast<float*>(work + L.y);
  float* v_rows = reinterpret_cast<float*>(work + L.v);
  if (plan.sort) {
    int n2 = 1;
    while (n2 < pairs) n2 <<= 1;
    moe_sort_small_kernel<<<1, 1024, 0, st>>>(idx, score, slot_of, (int)pairs, n2, slots, plan.bm, list, tile_slot,
                                              tile_pos, tile_end, ntiles);
  } else {
    const unsigned pb = (unsigned)((pairs + 255) / 256 < 4096 ? (pairs + 255) / 256 : 4096);
    const int64_t cb = (slots + 255) / 256;
    moe_clear_kernel<<<(unsigned)(cb < 1024 ? cb : 1024), 256, 0, st>>>(counts, cursor, slots);
    moe_count_kernel<<<pb, 256, 0, st>>>(idx, score, slot_of, pairs, slots, counts);
    moe_scan_kernel<<<1, kScanThreads, 0, st>>>(counts, slots, plan.bm, offsets, tile_slot, tile_pos, tile_end,
                                                ntiles);
    moe_scatter_kernel<<<pb, 256, 0, st>>>(idx, score, slot_of, pairs, slots, offsets, cursor, list);
  }
  int rc = launch_status("moe pair grouping");
  if (rc != NVF_OK) return rc;

  const MoeTiles base{tile_slot, tile_pos, tile_end, ntiles, list, 0, 0};
  {
    MoeGateUp prob;
    static_cast<MoeTiles&>(prob) = base;
    prob.n_cols = 2 * I;
    prob.K = K;
    prob.H = H;
    prob.I = I;
    prob.gu_out = gu_rows;
    rc = moe_product(x, gu, prob, H, plan, vec, L.max_tiles, st);
    if (rc != NVF_OK) return rc;
  }
  rc = nvf_silu_and_mul(gu_rows, y_rows, pairs, I, NVF_F32, st);
  if (rc != NVF_OK) return rc;
  {
    MoeDown prob;
    static_cast<MoeTiles&>(prob) = base;
    prob.n_cols = H;
    prob.H = H;
    prob.I = I;
    prob.v_out = v_rows;
    rc = moe_product(static_cast<const float*>(y_rows), dn, prob, I, plan, vec, L.max_tiles, st);
    if (rc != NVF_OK) return rc;
  }
  NVF_DISPATCH_DTYPE(out_dtype, TO,
                     (moe_combine_kernel<TO><<<(unsigned)rows, 256, 0, st>>>(v_rows, idx, score, slot_of, K, H, slots,
                                                                              static_cast<TO*>(out))));
  return launch_status("moe combine");
}

// The drop-in's workspace: a static device array (one per GPU, address from
// hipGetSymbolAddress), rows taken in chunks that fit it.
constexpr int64_t kMoeScratchBytes = 64ll << 20;
static __device__ __align__(256) uint8_t moe_scratch[kMoeScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_moe_mu;
void* g_moe_ptr[kMaxDevices] = {};

void* moe_scratch_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(NVF_ERR_LAUNCH, "hip_moe_ffn: no usable current device");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_moe_mu);
  if (!g_moe_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(moe_scratch));
    if (e != hipSuccess) {
      fail(NVF_ERR_LAUNCH, "hip_moe_ffn: hipGetSymbolAddress(moe_scratch) failed on device %d: %s", dev,
           hipGetErrorString(e));
      return nullptr;
    }
    g_moe_ptr[dev] = p;
  }
  return g_moe_ptr[dev];
}

int moe_check(const void* x, const int32_t* idx, const float* score, const void* gu, const void* dn,
              const int32_t* slot_of, int64_t rows, int64_t H, int64_t I, int64_t K, int64_t slots, void* out,
              const char* who) {
  if (rows < 0 || H <= 0 || I <= 0 || K <= 0 || slots <= 0)
    return fail(NVF_ERR_INVALID, "%s: bad sizes rows=%lld H=%lld I=%lld K=%lld slots=%lld", who, (long long)rows,
                (long long)H, (long long)I, (long long)K, (long long)slots);
  if (slots > kMoeMaxSlots) return fail(NVF_ERR_INVALID, "%s: more than %d expert slots", who, kMoeMaxSlots);
  if (K > kCombineMaxK) return fail(NVF_ERR_INVALID, "%s: more than %d experts per token", who, kCombineMaxK);
  if (rows * K > INT32_MAX / 2) return fail(NVF_ERR_INVALID, "%s: too many (token, expert) pairs", who);
  if (rows > 0 && (!x || !idx || !score || !gu || !dn || !slot_of || !out))
    return fail(NVF_ERR_INVALID, "%s: NULL pointer", who);
  return NVF_OK;
}

}  // namespace nvf

using namespace nvf;

extern "C" {

int nvf_moe_route(const float* logits, int64_t rows, int64_t E, int64_t K, int norm, int32_t* idx, float* score,
                  void* stream) {
  if (rows < 0 || E <= 0 || K <= 0 || K > E || E > kMoeMaxExperts)
    return fail(NVF_ERR_INVALID, "nvf_moe_route: bad sizes rows=%lld E=%lld K=%lld (E <= %d, K <= E)",
                (long long)rows, (long long)E, (long long)K, kMoeMaxExperts);
  if (rows > INT32_MAX) return fail(NVF_ERR_INVALID, "nvf_moe_route: rows=%lld exceed one launch", (long long)rows);
  if (rows == 0) return NVF_OK;
  if (!logits || !idx || !score) return fail(NVF_ERR_INVALID, "nvf_moe_route: NULL pointer");
  moe_route_kernel<<<(unsigned)rows, 64, (size_t)E * (sizeof(double) + sizeof(int)), as_stream(stream)>>>(
      logits, (int)E, (int)K, norm ? 1 : 0, idx, score);
  return launch_status("moe_route_kernel");
}

int64_t nvf_moe_ffn_workspace_size(int64_t rows, int64_t H, int64_t I, int64_t K, int64_t slots) {
  if (rows <= 0 || H <= 0 || I <= 0 || K <= 0 || slots <= 0) return 0;
  return MoeLayout(rows * K, H, I, slots, 16).total;  // the most tiles any plan lists (16-row tiles)
}

int nvf_moe_ffn_ws(const void* x, int x_dtype, const int32_t* idx, const float* score, const void* gu,
                   const void* dn, int w_bf16, const int32_t* slot_of, int64_t rows, int64_t H, int64_t I, int64_t K,
                   int64_t slots, void* out, int out_dtype, void* work, int64_t work_bytes, void* stream) {
  static const char* who = "nvf_moe_ffn_ws";
  if (!dtype_ok(x_dtype) || !dtype_ok(out_dtype)) return fail(NVF_ERR_INVALID, "%s: bad dtype", who);
  int rc = moe_check(x, idx, score, gu, dn, slot_of, rows, H, I, K, slots, out, who);
  if (rc != NVF_OK || rows == 0) return rc;
  const int64_t need = nvf_moe_ffn_workspace_size(rows, H, I, K, slots);
  if (!work || work_bytes < need || !aligned16(work))
    return fail(NVF_ERR_INVALID, "%s: needs a 16-byte aligned workspace of %lld bytes (got %lld)", who,
                (long long)need, (long long)work_bytes);
  uint8_t* wb = static_cast<uint8_t*>(work);
  hipStream_t st = as_stream(stream);
  NVF_DISPATCH_DTYPE(x_dtype, TX,
                     (rc = w_bf16 ? launch_moe_ffn<TX, __bf16>(static_cast<const TX*>(x), idx, score,
                                                              static_cast<const __bf16*>(gu),
                                                              static_cast<const __bf16*>(dn), slot_of, rows, H, I, K,
                                                              slots, out, out_dtype, wb, st)
                                 : launch_moe_ffn<TX, _Float16>(static_cast<const TX*>(x), idx, score,
                                                                static_cast<const _Float16*>(gu),
                                                                static_cast<const _Float16*>(dn), slot_of, rows, H, I,
                                                                K, slots, out, out_dtype, wb, st)));
  return rc;
}

// Drop-ins: include/nanovllm/hip_ops.hpp:37-40 / src/hip_ops.hip:895-939 (fp32, null
// stream).  hip_moe_ffn takes expert slots below 65536 (a pair whose slot_of entry
// is negative or beyond that is skipped; the reference would read outside its slot
// arrays) and runs its rows in chunks through the static device scratch, so it
// allocates nothing; calls overlapping on one GPU from other threads or streams
// would share that scratch.
void hip_moe_route(const float* logits, int rows, int E, int K, bool norm, int32_t* idx, float* score) {
  if (rows <= 0) return;
  dropin_check(nvf_moe_route(logits, rows, E, K, norm ? 1 : 0, idx, score, nullptr), "hip_moe_route");
}

void hip_moe_ffn(const float* x, const int32_t* idx, const float* score, const uint16_t* gu, const uint16_t* dn,
                 const int32_t* slot_of, int rows, int H, int I, int K, bool bf16, float* out) {
  if (rows <= 0) return;
  const int64_t slots = kMoeMaxSlots;
  dropin_check(moe_check(x, idx, score, gu, dn, slot_of, rows, H, I, K, slots, out, "hip_moe_ffn"), "hip_moe_ffn");
  uint8_t* ws = static_cast<uint8_t*>(moe_scratch_ptr());
  if (!ws) dropin_check(NVF_ERR_LAUNCH, "hip_moe_ffn");
  // largest row chunk whose workspace fits the scratch
  int64_t chunk = rows;
  while (chunk > 1 && nvf_moe_ffn_workspace_size(chunk, H, I, K, slots) > kMoeScratchBytes) chunk = (chunk + 1) / 2;
  if (nvf_moe_ffn_workspace_size(chunk, H, I, K, slots) > kMoeScratchBytes)
    dropin_check(fail(NVF_ERR_INVALID, "hip_moe_ffn: one row needs more than the %lld-byte scratch",
                      (long long)kMoeScratchBytes),
                 "hip_moe_ffn");
  for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
    const int64_t rc = rows - r0 < chunk ? rows - r0 : chunk;
    dropin_check(nvf_moe_ffn_ws(x + r0 * H, NVF_F32, idx + r0 * K, score + r0 * K, gu, dn, bf16 ? 1 : 0, slot_of, rc,
                                H, I, K, slots, out + r0 * H, NVF_F32, ws, kMoeScratchBytes, nullptr),
                 "hip_moe_ffn");
  }
}

int nvf_add_inplace(float* dst, const float* src, int64_t n, void* stream) {
  if (n < 0) return fail(NVF_ERR_INVALID, "nvf_add_inplace: negative size");
  if (n == 0) return NVF_OK;
  if (!dst || !src) return fail(NVF_ERR_INVALID, "nvf_add_inplace: NULL pointer");
  hipStream_t st = as_stream(stream);
  if (aligned16(dst) && aligned16(src) && n % 4 == 0) {
    const int64_t b = (n / 4 + 255) / 256;
    add_inplace_vec_kernel<<<(unsigned)(b < 4096 ? b : 4096), 256, 0, st>>>(dst, src, n / 4);
  } else {
    const int64_t b = (n + 255) / 256;
    add_inplace_kernel<<<(unsigned)(b < 4096 ? b : 4096), 256, 0, st>>>(dst, src, n);
  }
  return launch_status("add_inplace");
}

int nvf_scale_rows_sigmoid(float* dst, const float* s, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols < 0) return fail(NVF_ERR_INVALID, "nvf_scale_rows_sigmoid: negative size");
  if (rows > INT32_MAX)
    return fail(NVF_ERR_INVALID, "nvf_scale_rows_sigmoid: rows=%lld exceed one launch", (long long)rows);
  if (rows == 0 || cols == 0) return NVF_OK;
  if (!dst || !s) return fail(NVF_ERR_INVALID, "nvf_scale_rows_sigmoid: NULL pointer");
  scale_rows_sigmoid_kernel<<<(unsigned)rows, 256, 0, as_stream(stream)>>>(dst, s, cols);
  return launch_status("scale_rows_sigmoid");
}

void hip_add_inplace(float* dst, const float* src, size_t n) {
  if (n == 0) return;
  dropin_check(nvf_add_inplace(dst, src, (int64_t)n, nullptr), "hip_add_inplace");
}

void hip_scale_rows_sigmoid(float* dst, const float* s, int rows, int cols) {
  if (rows <= 0) return;
  dropin_check(nvf_scale_rows_sigmoid(dst, s, rows, cols, nullptr), "hip_scale_rows_sigmoid");
}

}  // extern "C"
