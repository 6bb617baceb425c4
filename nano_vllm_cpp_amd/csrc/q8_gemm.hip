// Q8_0 GEMM on the int8 matrix cores, and the activation quantizer that feeds it.
//
// Reference: hip_matmul_q8 (src/hip_ops.hip:639-686), used for every Q8_0 weight
// by matmul_dispatch (src/model.cpp:665-672).  The reference quantizes each
// activation row to int8 with scale 127/max|x| (q8_row_scale_kernel, :205-217;
// quantizer :244-245), takes int8 dot products against the split-plane weights
// (w8 [n][k] int8, ws [n][k/32] fp16) and applies the weight block scale per
// 16-element slice (:221-312) or per 4-element lane chunk (:317-364, m <= 8), then
// multiplies by 1/scale_row.
//
// Here the arithmetic is regrouped for CDNA4's v_mfma_i32_32x32x32_i8, whose K of
// 32 is exactly one Q8_0 block:
//   I[r][c][b] = sum_{i in block b} xq[r][i] * w8[c][i]             (exact int32)
//   out[r][c]  = (sum_b float(ws[c][b]) * float(I[r][c][b])) * (1/scale[r])
// The integer block dot is exact in both implementations; only the fp32 summation
// order of the block terms differs (the reference sums 16-element halves, this
// sums whole blocks), so results agree within the recursive-summation bound the
// tests state.
//
// Tiling: a 256-thread workgroup owns a 128 x 128 output tile; each of its four
// waves owns 64 x 64 (2 x 2 MFMA tiles of 32 x 32).  The K loop stages
// kGemmKC-byte slices of the 128 activation rows and the 128 weight rows through
// LDS (double-buffered, rows padded to 16 B past the slice so that the 16 lanes
// of a ds_read_b128 phase hit 16 distinct 4-bank groups).  Per block and wave:
// 4 MFMAs and 64 (cvt + fma) per lane to apply the block scale -- the scale
// application, not the MFMA, bounds this kernel (VALU : MFMA time is about 4:1).
#include <hip/hip_runtime.h>

#include <mutex>

#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int kGemmBM = 128;                 // output rows per workgroup
constexpr int kGemmBN = 128;                 // output columns per workgroup
constexpr int kGemmKC = 128;                 // bytes of K per LDS stage (4 Q8_0 blocks)
constexpr int kGemmRow = kGemmKC + 16;       // padded LDS row
constexpr int kGemmBlk = kGemmKC / 32;       // Q8_0 blocks per stage
constexpr int kGemmStage = (kGemmBM + kGemmBN) * kGemmRow + kGemmBN * kGemmBlk * 4;  // + fp32 block scales
constexpr int kGemmLds = 2 * kGemmStage;     // double-buffered
constexpr int kGemmThreads = 256;

// ---------------------------------------------------------------------------
// Row quantizer: scale[r] = 127 / max|x[r,:]| (0 for max <= 1e-8) and
// xq[r,i] = (int8) min(127, max(-127, x[r,i] * scale[r])) (truncation), the
// reference's q8_row_scale_kernel (src/hip_ops.hip:205-217) and its GEMMs'
// quantizer (:244-245, :340-344).  One 256-thread workgroup per row; the row is
// read twice (the second pass hits L2).
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void q8_quantize_rows_kernel(const T* __restrict__ x, float* __restrict__ scale,
                                                               int8_t* __restrict__ xq, int64_t k) {
  const int64_t r = blockIdx.x;
  const T* row = x + r * k;
  int8_t* qrow = xq + r * k;
  __shared__ float part[4];
  float mx = 0.0f;
  constexpr int N = Pack<T>::N;
  if constexpr (VEC) {
    for (int64_t c = threadIdx.x; c < k / N; c += 256) {
      float v[N];
      Pack<T>::unpack(ld16(row + c * N), v);
#pragma unroll
      for (int e = 0; e < N; ++e) mx = fmaxf(mx, fabsf(v[e]));
    }
  } else {
    for (int64_t i = threadIdx.x; i < k; i += 256) mx = fmaxf(mx, fabsf((float)row[i]));
  }
  mx = wave_max(mx);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
  const float s = q8_row_scale(mx);
  if (threadIdx.x == 0) scale[r] = s;
  if constexpr (VEC) {
    for (int64_t c = threadIdx.x; c < k / N; c += 256) {
      float v[N];
      Pack<T>::unpack(ld16(row + c * N), v);
      uint32_t w[N / 4];
#pragma unroll
      for (int d = 0; d < N / 4; ++d) {
        w[d] = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[d] |= (uint32_t)(q8_quantize(v[4 * d + e], s) & 0xff) << (8 * e);
      }
      if constexpr (N == 8) {
        *reinterpret_cast<uint2*>(qrow + c * N) = make_uint2(w[0], w[1]);
      } else {
        *reinterpret_cast<uint32_t*>(qrow + c * N) = w[0];
      }
    }
  } else {
    for (int64_t i = threadIdx.x; i < k; i += 256) qrow[i] = (int8_t)q8_quantize((float)row[i], s);
  }
}

// ---------------------------------------------------------------------------
__device__ __forceinline__ float fp16_bits_to_float(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// One thread's share of a stage's global loads: 16 bytes from each of 4 rows
// (rows (t >> 3) + 32 * i of the tile, bytes (t & 7) * 16 of the K slice).  Every
// load is unconditional: a row past the end is clamped to the last row and a K
// offset past the end to the last 16 bytes, and the data are zeroed by a select,
// so the loop has no branches and no early vmcnt waits.
struct SliceLoader {
  const int8_t* ptr[4];  // row base + this thread's byte offset in the slice
  bool row_ok[4];
  int64_t kb;            // K offset of this thread's 16 bytes in the current slice
  bool k_ok;             // kb < k for the slice in flight
  i32x4 r[4];            // raw data in flight (masked when stored)

  __device__ __forceinline__ void init(const int8_t* base, int64_t row0, int64_t rows, int64_t k) {
    const int t = threadIdx.x;
    kb = (t & 7) * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t row = row0 + (t >> 3) + 32 * i;
      row_ok[i] = row < rows;
      ptr[i] = base + (row_ok[i] ? row : rows - 1) * k;
    }
  }
  __device__ __forceinline__ void load(int64_t k) {
    k_ok = kb < k;
    const int64_t off = k_ok ? kb : k - 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = *reinterpret_cast<const i32x4*>(ptr[i] + off);
  }
  // Writes the slice in flight to LDS rows (t >> 3) + 32 * i, zeroing rows and
  // bytes outside the matrix.
  __device__ __forceinline__ void store(uint8_t* lds) const {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = k_ok && row_ok[i];
      const i32x4 v = i32x4{ok ? r[i][0] : 0, ok ? r[i][1] : 0, ok ? r[i][2] : 0, ok ? r[i][3] : 0};
      *reinterpret_cast<i32x4*>(lds + ((t >> 3) + 32 * i) * kGemmRow + (t & 7) * 16) = v;
    }
  }
};

template <typename TO>
__device__ __forceinline__ void gemm_store_out(TO* p, float v) {
  if constexpr (sizeof(TO) == 4) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = (TO)v;
  }
}

// out[m][n] (row-major) = dequantized Q8_0 product; see the file header.
// Grid: one workgroup per 128 x 128 output tile, tiles_n tiles per tile row.
//
// Per stage a wave issues 16 MFMAs (4 blocks x 2 x 2 tiles) through a ring of two
// result registers: MFMA t+1 is issued before the scale of MFMA t is applied, so
// the matrix core works while the VALU converts and accumulates.  The LDS
// fragments of block b+1 are read while block b is applied.
template <typename TO>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2))) void q8_gemm_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ rscale, const int8_t* __restrict__ w8,
    const uint16_t* __restrict__ ws, TO* __restrict__ out, int64_t m, int64_t n, int64_t k, int tiles_n) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ float inv_row[kGemmBM];

  const int tile = blockIdx.x;
  const int64_t row0 = (int64_t)(tile / tiles_n) * kGemmBM;
  const int64_t col0 = (int64_t)(tile % tiles_n) * kGemmBN;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t nblk = k / 32;

  if (threadIdx.x < kGemmBM) {
    const int64_t r = row0 + threadIdx.x;
    const float s = r < m ? rscale[r] : 0.0f;
    inv_row[threadIdx.x] = s > 0.0f ? 1.0f / s : 0.0f;  // the reference's adq (:309)
  }

  float acc[2][2][16];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.0f;

  SliceLoader la, lb;
  la.init(xq, row0, m, k);
  lb.init(w8, col0, n, k);
  // Block scales: thread t loads column col0 + (t & 127), blocks 2 * (t >> 7) + {0, 1}
  // of each stage (clamped + selected like the slices), stored as fp32 [block][column].
  const int sc_c = threadIdx.x & (kGemmBN - 1);
  const int sc_b = 2 * (threadIdx.x >> 7);
  const bool sc_col_ok = col0 + sc_c < n;
  const uint16_t* sc_ptr = ws + (sc_col_ok ? col0 + sc_c : n - 1) * nblk;
  uint16_t sc_raw[2];
  bool sc_ok[2];
  auto load_scales = [&](int64_t blk0) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int64_t b = blk0 + sc_b + e;
      sc_ok[e] = sc_col_ok && b < nblk;
      sc_raw[e] = sc_ptr[sc_ok[e] ? b : nblk - 1];
    }
  };
  auto store_scales = [&](uint8_t* stage) {
    float* s = reinterpret_cast<float*>(stage + (kGemmBM + kGemmBN) * kGemmRow);
#pragma unroll
    for (int e = 0; e < 2; ++e) s[(sc_b + e) * kGemmBN + sc_c] = sc_ok[e] ? fp16_bits_to_float(sc_raw[e]) : 0.0f;
  };

  const int nstages = (int)((k + kGemmKC - 1) / kGemmKC);
  la.load(k);
  lb.load(k);
  load_scales(0);
  la.store(lds);
  lb.store(lds + kGemmBM * kGemmRow);
  store_scales(lds);
  __syncthreads();

  const int a_off = (wm * 64 + (lane & 31)) * kGemmRow + (lane >> 5) * 16;
  const int b_off = kGemmBM * kGemmRow + (wn * 64 + (lane & 31)) * kGemmRow + (lane >> 5) * 16;
  const int s_off = (kGemmBM + kGemmBN) * kGemmRow + (wn * 64 + (lane & 31)) * 4;

  // Fragments of one block g: stage buffer (g / kGemmBlk) & 1, block g % kGemmBlk.
  i32x4 fa0, fa1, fb0, fb1;
  float s0, s1;
  auto read_frags = [&](int g) {
    const uint8_t* buf = lds + ((g / kGemmBlk) & 1) * kGemmStage;
    const int bi = g % kGemmBlk;
    fa0 = *reinterpret_cast<const i32x4*>(buf + a_off + bi * 32);
    fa1 = *reinterpret_cast<const i32x4*>(buf + a_off + 32 * kGemmRow + bi * 32);
    fb0 = *reinterpret_cast<const i32x4*>(buf + b_off + bi * 32);
    fb1 = *reinterpret_cast<const i32x4*>(buf + b_off + 32 * kGemmRow + bi * 32);
    s0 = *reinterpret_cast<const float*>(buf + s_off + bi * kGemmBN * 4);
    s1 = *reinterpret_cast<const float*>(buf + s_off + bi * kGemmBN * 4 + 32 * 4);
  };
  auto apply = [](float (&c)[16], const i32x16& d, float sc) {
#pragma unroll
    for (int j = 0; j < 16; ++j) c[j] = fmaf(sc, (float)d[j], c[j]);
  };

  // One iteration per Q8_0 block.  The first MFMA of block g + 1 is issued
  // inside iteration g, so every result is ready when its scale is applied; a
  // stage's global loads go out at its first block and land in LDS at its last.
  const int nb = nstages * kGemmBlk;
  read_frags(0);
  i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0, fb0, i32x16{}, 0, 0, 0);
#pragma unroll 1
  for (int g = 0; g < nb; ++g) {
    const int bi = g % kGemmBlk;
    const int st = g / kGemmBlk;
    const bool more = st + 1 < nstages;
    if (bi == 0 && more) {
      la.kb += kGemmKC;
      lb.kb += kGemmKC;
      la.load(k);
      lb.load(k);
      load_scales((int64_t)(st + 1) * kGemmBlk);
    }
    const i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0, fb1, i32x16{}, 0, 0, 0);
    const i32x16 d2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa1, fb0, i32x16{}, 0, 0, 0);
    const i32x16 d3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa1, fb1, i32x16{}, 0, 0, 0);
    const float c0 = s0, c1 = s1;
    apply(acc[0][0], d0, c0);
    apply(acc[0][1], d1, c1);
    apply(acc[1][0], d2, c0);
    if (bi == kGemmBlk - 1) {
      if (more) {
        uint8_t* nxt = lds + ((st + 1) & 1) * kGemmStage;
        la.store(nxt);
        lb.store(nxt + kGemmBM * kGemmRow);
        store_scales(nxt);
      }
      __syncthreads();
    }
    if (g + 1 < nb) {
      read_frags(g + 1);
      d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0, fb0, i32x16{}, 0, 0, 0);
    }
    apply(acc[1][1], d3, c1);
  }

  // D layout of v_mfma_*_32x32: lane l, value j -> column l % 32,
  // row 8 * (j / 4) + 4 * (l / 32) + j % 4.
  int64_t col[2];
  bool col_ok[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    col[f] = col0 + wn * 64 + f * 32 + (lane & 31);
    col_ok[f] = col[f] < n;
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int rl = wm * 64 + a * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
      const int64_t r = row0 + rl;
      if (r >= m) continue;
      const float inv = inv_row[rl];
#pragma unroll
      for (int b = 0; b < 2; ++b)
        if (col_ok[b]) gemm_store_out(out + r * n + col[b], acc[a][b][j] * inv);
    }
}

}  // namespace nvf

using namespace nvf;

namespace {

int check_gemm(const void* xq, const float* rscale, const void* w8, const void* ws, int64_t m, int64_t n, int64_t k,
               const void* out, int dtype, const char* who) {
  if (m < 0 || n < 0 || k < 0) return fail(NVF_ERR_INVALID, "%s: negative size", who);
  if (k % 32 != 0) return fail(NVF_ERR_INVALID, "%s: k=%lld is not a multiple of the Q8_0 block (32)", who, (long long)k);
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "%s: bad out dtype %d", who, dtype);
  if (m == 0 || n == 0 || k == 0) return NVF_OK;
  if (!xq || !rscale || !w8 || !ws || !out) return fail(NVF_ERR_INVALID, "%s: null pointer", who);
  if (!aligned16(xq) || !aligned16(w8))
    return fail(NVF_ERR_INVALID, "%s: xq and w8 must be 16-byte aligned", who);
  if ((reinterpret_cast<uintptr_t>(ws) & 1u) != 0) return fail(NVF_ERR_INVALID, "%s: ws must be 2-byte aligned", who);
  const int64_t tiles = ((m + kGemmBM - 1) / kGemmBM) * ((n + kGemmBN - 1) / kGemmBN);
  if (tiles > INT32_MAX) return fail(NVF_ERR_INVALID, "%s: %lld output tiles exceed the grid", who, (long long)tiles);
  return NVF_OK;
}

template <typename TO>
int launch_gemm(const int8_t* xq, const float* rscale, const int8_t* w8, const uint16_t* ws, TO* out, int64_t m,
                int64_t n, int64_t k, hipStream_t stream) {
  static std::once_flag attr_once;
  std::call_once(attr_once, [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&q8_gemm_kernel<TO>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
  });
  const int tiles_n = (int)((n + kGemmBN - 1) / kGemmBN);
  const int64_t tiles = ((m + kGemmBM - 1) / kGemmBM) * tiles_n;
  q8_gemm_kernel<TO><<<dim3((unsigned)tiles), dim3(kGemmThreads), kGemmLds, stream>>>(xq, rscale, w8, ws, out, m, n,
                                                                                      k, tiles_n);
  return launch_status("q8_gemm_kernel");
}

template <typename T>
void launch_quantize(const void* x, float* scale, int8_t* xq, int64_t rows, int64_t k, bool vec, hipStream_t stream) {
  const T* xt = static_cast<const T*>(x);
  if (vec) {
    q8_quantize_rows_kernel<T, true><<<dim3((unsigned)rows), dim3(256), 0, stream>>>(xt, scale, xq, k);
  } else {
    q8_quantize_rows_kernel<T, false><<<dim3((unsigned)rows), dim3(256), 0, stream>>>(xt, scale, xq, k);
  }
}

int quantize_rows(const void* x, int dtype, float* scale, int8_t* xq, int64_t rows, int64_t k, hipStream_t stream) {
  if (rows > INT32_MAX) return fail(NVF_ERR_INVALID, "q8_quantize_rows: rows=%lld exceeds the grid", (long long)rows);
  const bool vec = aligned16(x) && k % 8 == 0 && (reinterpret_cast<uintptr_t>(xq) & 7u) == 0;
  NVF_DISPATCH_DTYPE(dtype, T, launch_quantize<T>(x, scale, xq, rows, k, vec, stream));
  return launch_status("q8_quantize_rows_kernel");
}

// Grow-only device scratch for the drop-in's quantized activations and row scales,
// the same policy as the reference's static `arow` buffer (src/hip_ops.hip:642-648):
// not thread-safe, like the reference's single-threaded engine.
struct DropinScratch {
  void* p = nullptr;
  size_t cap = 0;
  int device = -1;
};
DropinScratch g_scratch;

}  // namespace

extern "C" {

int nvf_q8_quantize_rows(const void* x, float* row_scale, int8_t* xq, int64_t rows, int64_t k, int dtype,
                         void* stream) {
  if (rows < 0 || k < 0) return fail(NVF_ERR_INVALID, "q8_quantize_rows: negative size");
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "q8_quantize_rows: bad dtype %d", dtype);
  if (rows == 0) return NVF_OK;
  if (!x || !row_scale || !xq) return fail(NVF_ERR_INVALID, "q8_quantize_rows: null pointer");
  return quantize_rows(x, dtype, row_scale, xq, rows, k, as_stream(stream));
}

int nvf_matmul_q8_0(const int8_t* xq, const float* row_scale, const uint8_t* w8, const uint16_t* ws, int64_t m,
                    int64_t n, int64_t k, void* out, int out_dtype, void* stream) {
  const int st = check_gemm(xq, row_scale, w8, ws, m, n, k, out, out_dtype, "matmul_q8_0");
  if (st != NVF_OK || m == 0 || n == 0 || k == 0) return st;
  const int8_t* w = reinterpret_cast<const int8_t*>(w8);
  int rc = NVF_OK;
  NVF_DISPATCH_DTYPE(out_dtype, TO, rc = launch_gemm<TO>(xq, row_scale, w, ws, static_cast<TO*>(out), m, n, k,
                                                        as_stream(stream)));
  return rc;
}

// Drop-in for src/hip_ops.hip:639-686 (declared at include/nanovllm/hip_ops.hpp:10):
// fp32 activations and output on the null stream.  Quantizes x into the grow-only
// scratch, then runs the int8 GEMM.
void hip_matmul_q8(const float* x, const uint8_t* w8, const uint16_t* ws, int m, int n, int k, float* out) {
  if (m <= 0 || n <= 0 || k <= 0) return;
  int dev = 0;
  dropin_check(hipGetDevice(&dev) == hipSuccess ? NVF_OK : fail(NVF_ERR_LAUNCH, "hipGetDevice failed"),
               "hip_matmul_q8");
  const size_t q_bytes = ((size_t)m * (size_t)k + 255) & ~(size_t)255;
  const size_t need = q_bytes + (size_t)m * sizeof(float);
  if (need > g_scratch.cap || dev != g_scratch.device) {
    if (g_scratch.p) (void)hipFree(g_scratch.p);
    g_scratch.p = nullptr;
    g_scratch.cap = 0;
    if (hipMalloc(&g_scratch.p, need) != hipSuccess)
      dropin_check(fail(NVF_ERR_LAUNCH, "hip_matmul_q8: scratch allocation of %zu bytes failed", need),
                   "hip_matmul_q8");
    g_scratch.cap = need;
    g_scratch.device = dev;
  }
  int8_t* xq = static_cast<int8_t*>(g_scratch.p);
  float* rs = reinterpret_cast<float*>(static_cast<uint8_t*>(g_scratch.p) + q_bytes);
  dropin_check(nvf_q8_quantize_rows(x, rs, xq, m, k, NVF_F32, nullptr), "hip_matmul_q8");
  dropin_check(nvf_matmul_q8_0(xq, rs, w8, ws, m, n, k, out, NVF_F32, nullptr), "hip_matmul_q8");
}

}  // extern "C"
