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
// Decode-shaped products (m <= 16 rows, k % 8 == 0): bound by streaming the
// weights once from HBM.  Every fp32 matrix-core shape consumes at most 64 weight
// elements per 32 cycles per SIMD (8 per clock per CU), below what HBM delivers
// for K-quant weights (~23 elements per clock per CU for Q4_K), so the smallest
// batches use plain FMAs.  The 4 waves of a workgroup split K (contiguous ranges
// of steps) and meet in LDS, summed in wave order.  The activations are read from
// global memory (L2-resident: every workgroup reads the same m rows).
//
// m <= 2 (dense_gemv_fma_kernel): lane l = 4 b + j streams 8 consecutive weights
// of column j of each of its C column quads at k offset 8 b (16 lanes read 128
// contiguous k of one column per step) with the same 8 k of each of the m rows,
// and accumulates m x C fp32 sums; the 16 lanes of a column are summed at the end.
//
// 2 < m <= 16 (dense_gemv_mfma_kernel): v_mfma_f32_16x16x4_f32, lane l = 16 s + j
// giving activation row j and weight column j at k slot s.  Lane l streams 16
// consecutive k (two 8-runs) at offset 16 s of column j of each of C 16-column
// groups (64 contiguous k per column per step); run h, value i is MFMA step
// 8 h + i with k slot s <-> k = 16 s + 8 h + i.  The matrix core sums the k slots,
// so only the waves are summed at the end.
constexpr int kGvWaves = 4;
constexpr int kGemvRows = 16;

template <typename TX, typename Src, int MR, int C, typename TO>
__global__ __launch_bounds__(kGvWaves * 64) void dense_gemv_fma_kernel(const TX* __restrict__ x, Src w,
                                                                       TO* __restrict__ out, int64_t m, int64_t n,
                                                                       int64_t k) {
  __shared__ float part[kGvWaves][MR][C][4];  // [wave][row][quad][column]
  const int lane = threadIdx.x & 63, j = lane & 3, b = lane >> 2;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t c0 = (int64_t)blockIdx.x * 4 * C;
  const int64_t nsteps = (k + 127) / 128;
  const int64_t s_begin = nsteps * wave / kGvWaves, s_end = nsteps * (wave + 1) / kGvWaves;
  const Table<8, TX> xs{x};
  float acc[MR][C];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < C; ++q) acc[r][q] = 0.0f;
  bool col_ok[C];
#pragma unroll
  for (int q = 0; q < C; ++q) col_ok[q] = c0 + 4 * q + j < n;

  for (int64_t s = s_begin; s < s_end; ++s) {
    const int64_t kk = s * 128 + 8 * b;  // this lane's 8 k (k % 8 == 0: all or none are inside)
    if (kk >= k) continue;
    typename Src::Raw wr[C];
    typename Table<8, TX>::Raw xr[MR];
#pragma unroll
    for (int q = 0; q < C; ++q)
      if (col_ok[q]) wr[q] = w.load((c0 + 4 * q + j) * k + kk);
#pragma unroll
    for (int r = 0; r < MR; ++r)
      if (r < m) xr[r] = xs.load((int64_t)r * k + kk);
    float xv[MR][8];
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      if (r < m) {
        xs.decode(xr[r], xv[r]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[r][i] = 0.0f;
      }
    }
#pragma unroll
    for (int q = 0; q < C; ++q) {
      float wv[8];
      if (col_ok[q]) {
        w.decode(wr[q], wv);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) wv[i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[r][q] = __builtin_fmaf(xv[r][i], wv[i], acc[r][q]);
    }
  }

#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < C; ++q) {
      float v = acc[r][q];
#pragma unroll
      for (int d = 0; d < 4; ++d) v += __shfl_xor(v, 4 << d, 64);
      if (lane < 4) part[wave][r][q][j] = v;
    }
  __syncthreads();
  for (int t = (int)threadIdx.x; t < MR * C * 4; t += kGvWaves * 64) {
    const int jj = t & 3, q = (t >> 2) % C, r = (t >> 2) / C;
    const int64_t col = c0 + 4 * q + jj;
    if (r >= m || col >= n) continue;
    float v = part[0][r][q][jj];
#pragma unroll
    for (int wv = 1; wv < kGvWaves; ++wv) v += part[wv][r][q][jj];
    out[(int64_t)r * n + col] = from_f32<TO>(v);
  }
}

template <typename TX, typename Src, int C, typename TO>
__global__ __launch_bounds__(kGvWaves * 64) void dense_gemv_mfma_kernel(const TX* __restrict__ x, Src w,
                                                                        TO* __restrict__ out, int64_t m, int64_t n,
                                                                        int64_t k) {
  __shared__ float part[kGvWaves][C][16][17];  // [wave][group][row][column] (padded)
  const int lane = threadIdx.x & 63, j = lane & 15, ks = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t c0 = (int64_t)blockIdx.x * 16 * C;
  const int64_t nsteps = (k + 63) / 64;
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
    const int64_t kk = s * 64 + 16 * ks;
    typename Src::Raw wr[C][2];
    typename Table<8, TX>::Raw xr[2];
    bool h_ok[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      h_ok[h] = kk + 8 * h < k;
#pragma unroll
      for (int q = 0; q < C; ++q)
        if (h_ok[h] && col_ok[q]) wr[q][h] = w.load((c0 + 16 * q + j) * k + kk + 8 * h);
      if (h_ok[h] && row_ok) xr[h] = xs.load((int64_t)j * k + kk + 8 * h);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float xv[8];
      if (h_ok[h] && row_ok) {
        xs.decode(xr[h], xv);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = 0.0f;
      }
#pragma unroll
      for (int q = 0; q < C; ++q) {
        float wv[8];
        if (h_ok[h] && col_ok[q]) {
          w.decode(wr[q][h], wv);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) wv[i] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[q] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[i], wv[i], acc[q], 0, 0, 0);
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

// Column quads / groups per wave: 4 when that leaves >= ~1000 workgroups, fewer
// for narrow outputs.
template <typename TX, typename Src, int MR, typename TO>
int launch_gemv_fma(const TX* x, const Src& src, TO* out, int64_t m, int64_t n, int64_t k, hipStream_t st) {
  if (n >= 16 * 1024)
    dense_gemv_fma_kernel<TX, Src, MR, 4, TO><<<dim3((unsigned)((n + 15) / 16)), kGvWaves * 64, 0, st>>>(x, src, out, m, n, k);
  else if (n >= 8 * 1024)
    dense_gemv_fma_kernel<TX, Src, MR, 2, TO><<<dim3((unsigned)((n + 7) / 8)), kGvWaves * 64, 0, st>>>(x, src, out, m, n, k);
  else
    dense_gemv_fma_kernel<TX, Src, MR, 1, TO><<<dim3((unsigned)((n + 3) / 4)), kGvWaves * 64, 0, st>>>(x, src, out, m, n, k);
  return launch_status("dense_gemv_fma");
}

template <typename TX, typename Src, typename TO>
int launch_gemv_mfma(const TX* x, const Src& src, TO* out, int64_t m, int64_t n, int64_t k, hipStream_t st) {
  if (n >= 64 * 1024)
    dense_gemv_mfma_kernel<TX, Src, 4, TO><<<dim3((unsigned)((n + 63) / 64)), kGvWaves * 64, 0, st>>>(x, src, out, m, n, k);
  else if (n >= 32 * 1024)
    dense_gemv_mfma_kernel<TX, Src, 2, TO><<<dim3((unsigned)((n + 31) / 32)), kGvWaves * 64, 0, st>>>(x, src, out, m, n, k);
  else
    dense_gemv_mfma_kernel<TX, Src, 1, TO><<<dim3((unsigned)((n + 15) / 16)), kGvWaves * 64, 0, st>>>(x, src, out, m, n, k);
  return launch_status("dense_gemv_mfma");
}

template <typename TX, typename Src, typename TO>
int launch_dense(const void* x, const Src& src, void* out, int64_t m, int64_t n, int64_t k, bool vec,
                 hipStream_t st) {
  const int tiles_n = (int)((n + kDgBN - 1) / kDgBN);
  const TX* xp = static_cast<const TX*>(x);
  TO* op = static_cast<TO*>(out);
  if (vec && m <= kGemvRows && k % 8 == 0) {
    if (m == 1) return launch_gemv_fma<TX, Src, 1, TO>(xp, src, op, m, n, k, st);
    if (m == 2) return launch_gemv_fma<TX, Src, 2, TO>(xp, src, op, m, n, k, st);
    return launch_gemv_mfma<TX, Src, TO>(xp, src, op, m, n, k, st);
  }
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
