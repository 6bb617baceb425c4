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
// LDS (double-buffered, 16-byte chunks XOR-swizzled by row so that the 16 lanes
// of a ds_read_b128 phase hit 16 distinct 4-bank groups).  Per block and wave:
// 4 MFMAs and 64 (cvt + fma) per lane to apply the block scale -- the scale
// application, not the MFMA, bounds this kernel (VALU : MFMA time is about 4:1).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "nvf_device.hpp"
#include "nvf_host.hpp"

namespace nvf {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmBM = 128;                 // output rows per workgroup
constexpr int kGemmBN = 128;                 // output columns per workgroup
constexpr int kGemmKC = 64;                  // bytes of K per LDS stage (2 Q8_0 blocks)
constexpr int kGemmCPR = kGemmKC / 16;       // 16-byte chunks per LDS row
constexpr int kGemmRPI = 1024 / kGemmKC;     // rows per 1 KB wave DMA transfer
constexpr int kGemmSwz = 256 / kGemmKC;      // rows sharing a bank offset
constexpr int kGemmBlk = kGemmKC / 32;       // Q8_0 blocks per stage
// + the block scales: fp16 values in 4-byte slots (an LDS DMA of 2 bytes per lane
// fills one dword per lane, zero-extended)
constexpr int kGemmStage = (kGemmBM + kGemmBN) * kGemmKC + kGemmBN * kGemmBlk * 4;
constexpr int kGemmLds = 2 * kGemmStage;     // double-buffered
constexpr int kGemmThreads = 256;
constexpr int kGemmGroupM = 8;               // tile rows per group of the tile order
constexpr int kXcds = 8;                     // accelerator dies of an MI355X

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

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  // raw buffer, 32-bit dwords; offsets at or past `bytes` read as zero
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

constexpr uint32_t kOob = 0x80000000u;  // a buffer offset past every tile: reads zero
// Cache policy of a load read exactly once (the decode GEMV's weights and scales):
// non-temporal.  An LDS DMA stream of 136 MB runs 10% faster with it (22.1 against
// 24.6 us, the rate of plain register loads).
constexpr int kNt = 2;

// LDS rows hold kGemmKC bytes (kGemmCPR chunks of 16 B) with chunk c of row r at
// position c ^ ((r / kGemmSwz) % kGemmCPR): rows kGemmKC bytes apart fall on
// kGemmSwz distinct bank offsets, and the swizzle spreads the rest, so the 16
// lanes of a ds_read_b128 phase (16 consecutive rows, one chunk) cover all 64
// banks once.
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row / kGemmSwz) % kGemmCPR); }

template <typename TO>
__device__ __forceinline__ void gemm_store_out(TO* p, float v) {
  if constexpr (sizeof(TO) == 4) {
    __builtin_nontemporal_store(v, p);
  } else {
    *p = (TO)v;
  }
}

// out[m][n] (row-major) = dequantized Q8_0 product; see the file header.
// Grid: one workgroup per 128 x 128 output tile, tiles_n tiles per tile row;
// with SPLIT, blockIdx.y is a range of st_per_split K stages whose fp32 partial
// sums go to part [split][m][n] (q8_gemm_reduce_kernel finishes them).
//
// Stage loads go straight from HBM to LDS (buffer_load ... lds): each wave moves
// 32 activation rows and 32 weight rows per stage in 1 KB transfers, through
// buffer resources spanning only this tile's rows, so rows past the matrix read
// as zero; the stage's K offset rides in the scalar offset, so a full stage costs
// no VALU.  Only a partial last stage (k not a multiple of kGemmKC) checks each
// chunk against k.  The block scales come by LDS DMA too (fp16 in 4-byte slots).
//
// One loop iteration per Q8_0 block; the first MFMA of block g + 1 is issued
// while block g is applied, so each result is ready when its scale is applied.
// PL: k is not a multiple of the 64-byte stage, so the last stage is partial (known
// at launch; without it the loop carries none of the partial stage's address selects).
template <typename TO, bool SPLIT, bool PL = true>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(3))) void q8_gemm_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ rscale, const int8_t* __restrict__ w8,
    const uint16_t* __restrict__ ws, TO* __restrict__ out, int64_t m, int64_t n, int64_t k, int tiles_n,
    int st_per_split, float* __restrict__ part) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ float inv_row[kGemmBM];

  // XCD-aware tile order.  Workgroups are dealt to the 8 XCDs round-robin
  // (blockIdx % 8); each XCD gets a contiguous range of a grouped tile order
  // (kGemmGroupM tile rows at a time, column by column), so the workgroups
  // resident on one XCD share activation and weight panels in its L2.
  const int tiles = (int)gridDim.x;
  const int tiles_m = tiles / tiles_n;
  const int xcd = (int)blockIdx.x % kXcds, local = (int)blockIdx.x / kXcds;
  const int per = tiles / kXcds, extra = tiles % kXcds;
  const int id = xcd * per + (xcd < extra ? xcd : extra) + local;
  const int gsz = kGemmGroupM * tiles_n;
  const int first = (id / gsz) * kGemmGroupM;
  const int rows_g = tiles_m - first < kGemmGroupM ? tiles_m - first : kGemmGroupM;
  const int in_g = id % gsz;
  const int64_t row0 = (int64_t)(first + in_g % rows_g) * kGemmBM;
  const int64_t col0 = (int64_t)(in_g / rows_g) * kGemmBN;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
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

  // tile-local buffer resources (rows past m / n fall outside and read zero)
  const int64_t a_rows = m - row0 < kGemmBM ? m - row0 : kGemmBM;
  const int64_t b_rows = n - col0 < kGemmBN ? n - col0 : kGemmBN;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(xq + row0 * k, a_rows * k);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(w8 + col0 * k, b_rows * k);
  const __amdgpu_buffer_rsrc_t rsc = make_rsrc(ws + col0 * nblk, b_rows * nblk * 2);

  // This lane's DMA rows: wave w moves tile rows 32 w + kGemmRPI i + lane / kGemmCPR,
  // fetching the chunk that belongs at LDS position lane % kGemmCPR of each.
  constexpr int kDma = 32 / kGemmRPI;  // 1 KB transfers per wave and matrix per stage
  uint32_t dma_off[kDma];
  int dma_chunk[kDma];
#pragma unroll
  for (int i = 0; i < kDma; ++i) {
    const int row = 32 * wave + kGemmRPI * i + lane / kGemmCPR;
    dma_chunk[i] = swz(row, lane % kGemmCPR);
    dma_off[i] = (uint32_t)(row * k) + (uint32_t)(dma_chunk[i] * 16);
  }
  // Block scales: [block][column] after the tiles, by LDS DMA as well (2 bytes per
  // lane, landing in 4-byte slots): thread t moves column t % 128 of block t / 128.
  static_assert(kGemmBlk * kGemmBN == kGemmThreads, "one scale per thread and stage");
  const int sc_c = threadIdx.x & (kGemmBN - 1);
  const int sc_b = threadIdx.x >> 7;
  const uint32_t sc_off = (uint32_t)((sc_c * nblk + sc_b) * 2);

  const int nstages = (int)((k + kGemmKC - 1) / kGemmKC);
  // this workgroup's K stages: all, or split blockIdx.y's st_per_split of them (every
  // split is non-empty: the host sizes the split count so)
  const int st0 = SPLIT ? (int)blockIdx.y * st_per_split : 0;
  const int st1 = SPLIT ? min(nstages, st0 + st_per_split) : nstages;
  const bool partial_last = PL && k % kGemmKC != 0;
  // Loads stage st into LDS buffer `buf`, all by DMA.
  auto issue = [&](int st, int buf) {  // st: absolute stage; buf: its double-buffer slot
    uint8_t* stage = lds + buf * kGemmStage;
    const uint32_t kc = (uint32_t)st * kGemmKC;
    uint8_t* sc_dst = stage + (kGemmBM + kGemmBN) * kGemmKC + wave * 256;  // this wave's 64 scale slots
    if (partial_last && st == nstages - 1) {  // uniform, at most once per tile
#pragma unroll
      for (int i = 0; i < kDma; ++i) {
        const uint32_t off = (int64_t)kc + dma_chunk[i] * 16 < k ? dma_off[i] + kc : kOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ra, (__attribute__((address_space(3))) void*)(stage + (32 * wave + kGemmRPI * i) * kGemmKC), 16, off, 0,
            0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rb,
            (__attribute__((address_space(3))) void*)(stage + kGemmBM * kGemmKC +
                                                      (32 * wave + kGemmRPI * i) * kGemmKC),
            16, off, 0, 0, 0);
      }
      const int64_t b = (int64_t)st * kGemmBlk + sc_b;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsc, (__attribute__((address_space(3))) void*)sc_dst, 2,
                                               b < nblk ? sc_off + st * kGemmBlk * 2 : kOob, 0, 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < kDma; ++i) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ra, (__attribute__((address_space(3))) void*)(stage + (32 * wave + kGemmRPI * i) * kGemmKC), 16,
            dma_off[i], kc, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rb,
            (__attribute__((address_space(3))) void*)(stage + kGemmBM * kGemmKC +
                                                      (32 * wave + kGemmRPI * i) * kGemmKC),
            16, dma_off[i], kc, 0, 0);
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsc, (__attribute__((address_space(3))) void*)sc_dst, 2, sc_off,
                                               (uint32_t)st * kGemmBlk * 2, 0, 0);
    }
  };
  // This wave's LDS DMA must land before the barrier that publishes a stage.
  auto publish = [&] {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
  };

  // fragment LDS offsets: tile row r = wm*64 + (lane & 31) (+32 for the second
  // tile) and weight row wn*64 + (lane & 31), chunk 2*bi + (lane >> 5), swizzled.
  // Block bi's offsets are block 0's with bit 5 flipped per bi bit (the chunk
  // index moves by 2 bi under the xor swizzle).
  const int fr = wm * 64 + (lane & 31);
  const int fcol = wn * 64 + (lane & 31);
  const int cx0 = swz(fr, lane >> 5) << 4;  // the weight row fcol has the same swizzle
  const int fa_addr0 = fr * kGemmKC + cx0;
  const int fb_addr0 = kGemmBM * kGemmKC + fcol * kGemmKC + cx0;
  const int fs_addr0 = (kGemmBM + kGemmBN) * kGemmKC + fcol * 4;

  i32x4 fa0, fa1, fb0, fb1;
  float s0, s1;
  auto read_frags = [&](int g) {
    const uint8_t* base = lds + ((g / kGemmBlk) & 1) * kGemmStage;
    const int bi = g % kGemmBlk;
    const int fa_addr = fa_addr0 ^ (bi << 5), fb_addr = fb_addr0 ^ (bi << 5);
    fa0 = *reinterpret_cast<const i32x4*>(base + fa_addr);
    fa1 = *reinterpret_cast<const i32x4*>(base + fa_addr + 32 * kGemmKC);
    fb0 = *reinterpret_cast<const i32x4*>(base + fb_addr);
    fb1 = *reinterpret_cast<const i32x4*>(base + fb_addr + 32 * kGemmKC);
    s0 = fp16_bits_to_float(*reinterpret_cast<const uint16_t*>(base + fs_addr0 + bi * kGemmBN * 4));
    s1 = fp16_bits_to_float(*reinterpret_cast<const uint16_t*>(base + fs_addr0 + bi * kGemmBN * 4 + 32 * 4));
  };
  auto apply = [](float (&c)[16], const i32x16& d, float sc) {
#pragma unroll
    for (int j = 0; j < 16; ++j) c[j] = fmaf(sc, (float)d[j], c[j]);
  };

  issue(st0, 0);
  publish();
  const int nb = (st1 - st0) * kGemmBlk;  // blocks g = 0 .. nb - 1 of this workgroup's stages
  read_frags(0);
  i32x16 d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0, fb0, i32x16{}, 0, 0, 0);
  // One iteration per Q8_0 block, 0 .. nb-2; the last block is peeled so that
  // the loop body has no conditional MFMA (a conditional result costs register
  // copies every iteration).  A stage's successor is loaded at its first block
  // and published (scales stored, DMA drained, barrier) after its MFMAs of the
  // last block are issued.
#pragma unroll 1
  for (int g = 0; g < nb - 1; ++g) {
    const int bi = g % kGemmBlk;
    const int st = g / kGemmBlk;
    if (bi == 0) issue(st0 + st + 1, (st + 1) & 1);  // uniform; g < nb - 1 implies a successor
    const i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0, fb1, i32x16{}, 0, 0, 0);
    const i32x16 d2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa1, fb0, i32x16{}, 0, 0, 0);
    const i32x16 d3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa1, fb1, i32x16{}, 0, 0, 0);
    const float c0 = s0, c1 = s1;
    if (bi == kGemmBlk - 1) publish();
    read_frags(g + 1);  // LDS latency hides behind the first two applies
    apply(acc[0][0], d0, c0);
    apply(acc[0][1], d1, c1);
    d0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0, fb0, i32x16{}, 0, 0, 0);
    apply(acc[1][0], d2, c0);
    apply(acc[1][1], d3, c1);
  }
  {
    const i32x16 d1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa0, fb1, i32x16{}, 0, 0, 0);
    const i32x16 d2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa1, fb0, i32x16{}, 0, 0, 0);
    const i32x16 d3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa1, fb1, i32x16{}, 0, 0, 0);
    apply(acc[0][0], d0, s0);
    apply(acc[0][1], d1, s1);
    apply(acc[1][0], d2, s0);
    apply(acc[1][1], d3, s1);
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
      if constexpr (SPLIT) {  // fp32 partial sums of this split; the reduction scales
#pragma unroll
        for (int b = 0; b < 2; ++b)
          if (col_ok[b]) part[((int64_t)blockIdx.y * m + r) * n + col[b]] = acc[a][b][j];
        continue;
      }
      const float inv = inv_row[rl];
#pragma unroll
      for (int b = 0; b < 2; ++b)
        if (col_ok[b]) gemm_store_out(out + r * n + col[b], acc[a][b][j] * inv);
    }
}

// ---------------------------------------------------------------------------
// Decode-shaped product (m <= kGemvMaxM rows): bound by streaming the weights
// once from HBM, so the layout serves the loads.
//
// A wave owns 16 weight columns (or 32: CG = 2 groups of 16 sharing each
// activation fragment) and a contiguous range of K; S waves of a workgroup
// share a column group (splitting K) and meet in LDS at the end, summed in split
// order; a workgroup holds W / S column groups.  The weights go
// HBM -> LDS by DMA in 256-byte runs per column (one 1 KB transfer = 4 columns x
// 256 B, the K offset in the scalar offset, so a stage costs no VALU), into a
// wave-private double buffer: the next stage is in flight while the current one
// is computed.  16-byte chunk c of column j sits at position c ^ (j % 16), so the
// 16 columns' reads of one chunk hit 16 distinct bank groups.  The block scales
// of the workgroup's columns are staged in LDS once.
//
// Per block pair (64 bytes of K) lane l = 16 q + j holds 16 bytes, k in
// [16 q, 16 q + 16), of weight column j and of activation row j -- the operand
// layout of v_mfma_i32_16x16x64_i8.  Lanes q = 0, 1 hold the pair's first block,
// q = 2, 3 its second; the block scales differ, so each pair takes two MFMAs,
// each with the activation lanes of the other block zeroed (the K = 64
// instruction then sums exactly one block).  MFMA time is idle capacity here.
//
// The activations come one of two ways.  With XL (K split over the waves) the workgroup's m rows are
// staged in LDS once, by DMA in the prologue (rows padded by 16 bytes, so the 16
// rows of a ds_read_b128 phase fall in distinct banks).  The loop then holds LDS
// reads only, and its vmcnt waits are the explicit ones, which leave the next
// weight stage in flight.  Without XL (when those rows would cost the launch
// resident workgroups) they are register loads per stage; the compiler does not
// count LDS DMA in its own vmcnt waits for those registers, so they also drain
// part of the next stage.
constexpr int kGemvMaxM = 16;
constexpr int kGvKC = 256;                        // bytes of K per stage (4 block pairs)
constexpr int kGvWaveBuf = 16 * kGvKC;            // one stage of one wave's 16 columns
constexpr int kGemvScaleLds = 32768;              // bytes of LDS for the staged scales
constexpr int kGemvXLdsMax = 65536;               // bytes of LDS for staged activation rows
constexpr int64_t kLdsPerCu = 160 * 1024;

template <int W, int S, int CG = 1>
constexpr int gemv_cols() { return W / S * 16 * CG; }  // columns per workgroup of W waves

// XF (fused activation quantizer, needs XL): the m rows arrive as 16-bit or fp32
// activations in TO (xf, row stride xf_ld elements) instead of int8 rows + scales;
// each workgroup quantizes them into its staged LDS rows itself, exactly as
// nvf_q8_quantize_rows (XF = 1) or nvf_silu_and_mul_q8 over [gate | up] rows
// (XF = 2) would: the row maximum is order-independent and each value is quantized
// alone, so the int8 rows and scales are bit-identical to the separate pass's.
// XF = 3: residual-add + RMSNorm over the rows first, exactly as nvf_rms_norm_q8
// (xres, when given, is the residual: the rows become round(x + xres), which
// workgroup 0 stores to xres_out; then round(v * inv_rms * xg)).  Bit-identity
// needs the norm's own sum of squares: a first pass sums each row's squares in the
// norm kernel's layout (rms_waves_per_row) and order, one (row, sub-wave) per wave.
//
// H8 (m <= 8): both blocks of a pair in one MFMA.  Lane (j, q) takes activation row
// j % 8, and only for j < 8 with q < 2 (the pair's first block) or j >= 8 with q >= 2
// (its second); other lanes hold zero (their loads fall outside the buffer).  D rows
// 0-7 are then the first block's dots of rows 0-7 and D rows 8-15 the second block's,
// so lane (j, q) applies one scale, block 2 p + q / 2 of column j, and the two halves
// of a row meet in the final sum.  Half the MFMAs and half the applies of the
// two-MFMA form, none of them on padding rows.
// vmcnt(4 CG): every load but the last weight stage's 4 CG transfers
template <int CG>
__device__ __forceinline__ void gemv_wait_but_stage() {
  static_assert(CG == 1 || CG == 2, "one or two column groups per wave");
  if constexpr (CG == 2)
    __builtin_amdgcn_s_waitcnt(0x0F78);
  else
    __builtin_amdgcn_s_waitcnt(0x0F74);
}

// CG: 16-column groups per wave (2: each activation fragment feeds two MFMAs, half
// the activation loads per weight byte).
template <typename TO, int W, int S, bool XL, int XF = 0, bool H8 = false, int CG = 1>
__global__ __launch_bounds__(W * 64) __attribute__((amdgpu_waves_per_eu(2))) void q8_gemv_kernel(const int8_t* __restrict__ xq,
                                                         const float* __restrict__ rscale,
                                                         const int8_t* __restrict__ w8,
                                                         const uint16_t* __restrict__ ws,
                                                         TO* __restrict__ out, int64_t m, int64_t n, int64_t k,
                                                         int sc_bytes, const TO* __restrict__ xf = nullptr,
                                                         int64_t xf_ld = 0, const TO* __restrict__ xres = nullptr,
                                                         TO* __restrict__ xres_out = nullptr,
                                                         const TO* __restrict__ xg = nullptr, float eps = 0.0f) {
  static_assert(XF == 0 || XL, "the fused quantizer writes the staged LDS rows");
  constexpr int kCols = gemv_cols<W, S, CG>();
  constexpr int kWaveBuf = CG * kGvWaveBuf;  // one stage of one wave's columns
  constexpr int kGvDmaLds = W * 2 * kWaveBuf;
  // [DMA buffers][scales][activation rows (XL)]; after the loop each wave's partial
  // sums reuse its own DMA buffers
  extern __shared__ __attribute__((aligned(16))) uint8_t dyn[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int grp = wave / S, split = wave % S;
  const int j = lane & 15, q = lane >> 4;
  const int64_t wg_c0 = (int64_t)blockIdx.x * kCols;
  const int64_t nblk = k / 32, npairs = (nblk + 1) / 2;
  const int64_t wg_cols = n - wg_c0 < kCols ? n - wg_c0 : kCols;
  uint16_t* sc_lds = reinterpret_cast<uint16_t*>(dyn + kGvDmaLds);
  uint8_t* x_lds = dyn + kGvDmaLds + sc_bytes;
  // XF: per-wave row maxima and the rows' scales, after the staged rows (dynamic LDS
  // only, so the kernel may take the whole 160 KiB)
  float* xf_max = reinterpret_cast<float*>(x_lds + ((m * (k + 16) + 15) & ~int64_t(15)));
  float* xf_scale = xf_max + W * kGemvMaxM;
  float* xf_ss = xf_scale + kGemvMaxM;  // XF 3: [row][sub-wave] sums of squares
  const int64_t xrow = k + 16;  // LDS bytes per staged activation row

  const int64_t c0 = wg_c0 + (int64_t)grp * 16 * CG;  // this wave's first column
  const int64_t cols = n - c0 < 16 * CG ? n - c0 : 16 * CG;
  const int64_t p_begin = npairs * split / S, p_end = npairs * (split + 1) / S;
  const bool active = cols > 0 && p_end > p_begin;  // uniform per wave
  float acc[CG][4] = {};

  // rows past m / columns past n fall outside these resources and read zero
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w8 + (active ? c0 * k : 0), active ? cols * k : 0);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xq, m * k);
  uint8_t* wbuf = dyn + wave * 2 * kWaveBuf;
  // DMA lane l of transfer i: column 4 i + l / 16, LDS position l % 16, fetching chunk (l % 16) ^ column
  // (loop bounds that do not depend on CG: the host compilation pass otherwise
  // drops the kernel's instantiation, and its launch stub, without a diagnostic)
  uint32_t dma_off[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int col = 4 * i + (lane >> 4);
    dma_off[i] = (uint32_t)(col * k) + 16u * (uint32_t)((lane & 15) ^ (col & 15));
  }
  const int64_t kb0 = 64 * p_begin;
  const int nst = (int)((p_end - p_begin + 3) / 4);
  auto issue = [&](int st) {
    uint8_t* dst = wbuf + (st & 1) * kWaveBuf;
    const uint32_t soff = (uint32_t)(kb0 + (int64_t)st * kGvKC);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < 4 * CG)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (__attribute__((address_space(3))) void*)(dst + i * 1024), 16,
                                               dma_off[i], soff, 0, kNt);
  };
  const int xr = H8 ? (j & 7) : j;                          // the activation row lane (j, q) holds
  const bool x_half_ok = !H8 || ((j < 8) == (q < 2));       // H8: this lane's block of the pair
  const uint32_t x_off = (uint32_t)(xr * k) + 16u * q;
  // Register path (no XL): the activations of stage st + 1 are loaded at the top of
  // stage st into the other half of a register double buffer.  These loads are
  // invisible to the compiler (inline asm): its own vmcnt waits, which do not count
  // the LDS DMA, would otherwise drain the next weight stage wherever the registers
  // are read.  The stage-end vmcnt wait covers them; x_ready() then ties the
  // registers to that wait, so no read of them can be scheduled before it.
  const i32x4 x_desc = {(int)(uint32_t)reinterpret_cast<uintptr_t>(xq),
                        (int)(uint32_t)((reinterpret_cast<uintptr_t>(xq) >> 32) & 0xffffu), (int)(m * k), 0x00020000};
  i32x4 xa[4], xb[4];
  auto load_x = [&](i32x4 (&xv)[4], int st) {  // 16 bytes of each of stage st's 4 pairs (zero past k)
    const int64_t pst = p_begin + 4 * st;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const int64_t p = pst + pp;
      const bool ok = x_half_ok && p < p_end && 64 * p + 16 * q < k;
      const uint32_t off = ok ? x_off + (uint32_t)(64 * p) : kOob;
      asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(xv[pp]) : "v"(off), "s"(x_desc) : "memory");
    }
  };
  auto x_ready = [&](i32x4 (&xv)[4]) {
    asm volatile("" : "+v"(xv[0]), "+v"(xv[1]), "+v"(xv[2]), "+v"(xv[3]));
  };
  (void)rx;
  // Issue order: weight stage 0, the scales (and XL rows), stage 0's register
  // activations, weight stage 1.  vmcnt counts in issue order, so vmcnt(4) waits
  // for everything but stage 1, which stays in flight; the prologue's HBM
  // latencies overlap.  LDS DMA lane l of a transfer fills 4 (or 16) bytes at
  // base + 4 l (16 l).
  if (active) issue(0);
  {
    // the block scales: wg_cols rows of nblk fp16 values, whole 4-byte words, then
    // an odd last value by itself (a 4-byte load that straddles the end of the
    // slab reads as zero entirely, so that word is never loaded whole)
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(ws + wg_c0 * nblk, wg_cols * nblk * 2);
    const int64_t cnt = wg_cols * nblk;
    uint32_t* dst = reinterpret_cast<uint32_t*>(sc_lds);
    for (int64_t i0 = 0; i0 < cnt / 2; i0 += W * 64) {
      const int64_t i = i0 + threadIdx.x;
      if (i < cnt / 2)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void*)(dst + i0 + 64 * wave), 4, (uint32_t)(4 * i), 0, 0, kNt);
    }
    if constexpr (XL && XF == 0) {  // m rows of k bytes (k % 32 == 0), 1 KB transfers spread over the waves
      const int per_row = (int)((k + 1023) / 1024);
      for (int t = wave; t < m * per_row; t += W) {
        const int r = t / per_row, c = t % per_row;
        const int64_t kb = 1024 * (int64_t)c + 16 * lane;
        if (kb < k)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rx, (__attribute__((address_space(3))) void*)(x_lds + r * xrow + 1024 * c), 16,
              (uint32_t)(r * k + kb), 0, 0, 0);
      }
    }
    // XF: the fp rows' loads go out here too, so their latency overlaps weight stage 0
    // (not after the wait below): a single row's values for the thread (hold), and for
    // XF 3 each wave's rows in the norm's layout (npre)
    constexpr int N = Pack<TO>::N;
    const int64_t nv = k / N;
    constexpr int kHold = XF == 3 ? 4 : 8;  // a single row of up to kHold vectors per thread stays in registers
    constexpr int kNormPre = 4;             // norm-layout vectors per lane preloaded
    const bool hold = XF != 0 && m == 1 && nv <= (int64_t)kHold * W * 64;
    // (fp32 rows of XF 1 / 2 are loaded after the wait: preloaded they take ~230 VGPRs)
    constexpr bool kPre = sizeof(TO) == 2 || XF == 3;
    const int wpr = rms_waves_per_row(nv);
    const int vpl = (int)((nv + (int64_t)wpr * 64 - 1) / ((int64_t)wpr * 64));
    const bool npre = XF == 3 && m * wpr <= W && vpl <= kNormPre;
    u32x4 ha[kHold], hb[kHold], hg[kHold];  // x; up (XF 2) or residual (XF 3); norm weight (XF 3)
    u32x4 na[kNormPre], nb[kNormPre];
    if constexpr (XF != 0) {
      if (kPre && hold) {
#pragma unroll
        for (int i = 0; i < kHold; ++i) {
          const int64_t c = threadIdx.x + (int64_t)i * W * 64;
          if (c < nv) {
            ha[i] = ld16(xf + c * N);
            if constexpr (XF == 2) hb[i] = ld16(xf + k + c * N);
            if constexpr (XF == 3) {
              if (xres) hb[i] = ld16(xres + c * N);
              hg[i] = ld16(xg + c * N);
            }
          }
        }
      }
      if (npre && wave < m * wpr) {
        const int64_t r = wave / wpr;
        const int sub = wave % wpr;
#pragma unroll
        for (int i = 0; i < kNormPre; ++i) {
          const int64_t c = ((int64_t)i * wpr + sub) * 64 + lane;
          if (i < vpl && c < nv) {
            na[i] = ld16(xf + r * xf_ld + c * N);
            if (xres) nb[i] = ld16(xres + r * k + c * N);
          }
        }
      }
    }
    if (active) {
      if constexpr (!XL) load_x(xa, 0);
      if (nst > 1) issue(1);
    }
    if (active && nst > 1)
      gemv_wait_but_stage<CG>();  // all but weight stage 1
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    if constexpr (!XL) {
      if (active) x_ready(xa);
    }
    if ((cnt & 1) && threadIdx.x == 0)
      sc_lds[cnt - 1] = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (uint32_t)(2 * (cnt - 1)), 0, 0);
    if constexpr (XF != 0) {
      // Pass 1: each row's max |value| (wave maxima to LDS); pass 2, after a barrier:
      // the scale, then every value quantized into the staged row (the values are
      // computed twice rather than held: up to 16 rows of k).  Weight stage 1 stays
      // in flight meanwhile.
      // XF 3: the row value round(x + residual) (or x), as the norm stores it
      auto res_raw = [&](const u32x4& xv4, const u32x4& rv4, float* v) {
        Pack<TO>::unpack(xv4, v);
        if (xres) {
          float a[N];
          Pack<TO>::unpack(rv4, a);
#pragma unroll
          for (int e = 0; e < N; ++e) v[e] += a[e];
          Pack<TO>::unpack(Pack<TO>::pack(v), v);
        }
      };
      // the raw vectors of row r, vector c
      auto load_raw = [&](int64_t r, int64_t c, u32x4& a, u32x4& b, u32x4& gg) {
        a = ld16(xf + r * xf_ld + c * N);
        if constexpr (XF == 2) b = ld16(xf + r * xf_ld + k + c * N);
        if constexpr (XF == 3) {
          if (xres) b = ld16(xres + r * k + c * N);
          gg = ld16(xg + c * N);
        }
      };
      if constexpr (XF == 3) {  // pass 0: the norm's sums of squares, in its layout and order
        auto sum_row = [&](auto&& vec_at) {
          float ss = 0.0f;
          for (int i = 0; i < vpl; ++i) {
            float v[N];
            if (vec_at(i, v)) {
#pragma unroll
              for (int e = 0; e < N; ++e) ss = fmaf(v[e], v[e], ss);
            }
          }
          return wave_sum(ss);
        };
        if (npre) {
          if (wave < m * wpr) {
            const int64_t r = wave / wpr;
            const int sub = wave % wpr;
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < kNormPre; ++i) {
              const int64_t c = ((int64_t)i * wpr + sub) * 64 + lane;
              if (i < vpl && c < nv) {
                float v[N];
                res_raw(na[i], nb[i], v);
#pragma unroll
                for (int e = 0; e < N; ++e) ss = fmaf(v[e], v[e], ss);
              }
            }
            ss = wave_sum(ss);
            if (lane == 0) xf_ss[r * 4 + sub] = ss;
          }
        } else {
          for (int64_t it = wave; it < m * wpr; it += W) {
            const int64_t r = it / wpr;
            const int sub = (int)(it % wpr);
            const float ss = sum_row([&](int i, float* v) {
              const int64_t c = ((int64_t)i * wpr + sub) * 64 + lane;
              if (c >= nv) return false;
              u32x4 a, b, gg;
              load_raw(r, c, a, b, gg);
              res_raw(a, b, v);
              return true;
            });
            if (lane == 0) xf_ss[r * 4 + sub] = ss;
          }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      auto row_inv = [&](int64_t r) {  // the norm's 1/rms of row r
        float ss = xf_ss[r * 4];
        if (wpr > 1) {
          ss = 0.0f;
          for (int s4 = 0; s4 < wpr; ++s4) ss += xf_ss[r * 4 + s4];
        }
        return rsqrtf(ss / (float)k + eps);
      };
      // the quantizer's input values from the raw vectors; pass 1 stores the residual
      // row (workgroup 0 only), pass 2 only recomputes
      auto finish = [&](int64_t r, int64_t c, const u32x4& a, const u32x4& b, const u32x4& gg, float* v, float inv,
                        bool store_res) {
        if constexpr (XF == 3) {
          float g[N], o[N];
          res_raw(a, b, v);
          if (store_res && xres && blockIdx.x == 0) st16(xres_out + r * k + c * N, Pack<TO>::pack(v));
          Pack<TO>::unpack(gg, g);
#pragma unroll
          for (int e = 0; e < N; ++e) o[e] = v[e] * inv * g[e];
          Pack<TO>::unpack(Pack<TO>::pack(o), v);  // the stored (rounded) normalised value
        } else {
          Pack<TO>::unpack(a, v);
          if constexpr (XF == 2) {
            float u[N];
            Pack<TO>::unpack(b, u);
#pragma unroll
            for (int e = 0; e < N; ++e) v[e] = to_f32(from_f32<TO>(silu_mul<TO>(v[e], u[e])));  // the stored value
          }
        }
      };
      auto act = [&](int64_t r, int64_t c, float* v, float inv, bool store_res) {
        u32x4 a, b, gg;
        load_raw(r, c, a, b, gg);
        finish(r, c, a, b, gg, v, inv, store_res);
      };
      float hv[kHold][N];
      if (hold) {
        float mx = 0.0f;
        const float inv0 = XF == 3 ? row_inv(0) : 0.0f;
#pragma unroll
        for (int i = 0; i < kHold; ++i) {
          const int64_t c = threadIdx.x + (int64_t)i * W * 64;
          if (c < nv) {
            if constexpr (kPre)
              finish(0, c, ha[i], hb[i], hg[i], hv[i], inv0, true);
            else
              act(0, c, hv[i], inv0, true);
#pragma unroll
            for (int e = 0; e < N; ++e) mx = fmaxf(mx, fabsf(hv[i][e]));
          }
        }
        mx = wave_max(mx);
        if (lane == 0) xf_max[wave * kGemvMaxM] = mx;
      }
      for (int64_t r = 0; r < (hold ? 0 : m); ++r) {
        float mx = 0.0f;
        const float inv = XF == 3 ? row_inv(r) : 0.0f;
        for (int64_t c = threadIdx.x; c < nv; c += W * 64) {
          float v[N];
          act(r, c, v, inv, true);
#pragma unroll
          for (int e = 0; e < N; ++e) mx = fmaxf(mx, fabsf(v[e]));
        }
        mx = wave_max(mx);
        if (lane == 0) xf_max[wave * kGemvMaxM + r] = mx;
      }
      // publish the maxima: a bare barrier (no workgroup fence, whose vmcnt(0) wait
      // the loads above have already forced anyway)
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      auto quant_store = [&](int64_t r, int64_t c, const float* v, float sc) {
        uint32_t q4[N / 4];
#pragma unroll
        for (int d = 0; d < N / 4; ++d) {
          q4[d] = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) q4[d] |= (uint32_t)(q8_quantize(v[4 * d + e], sc) & 0xff) << (8 * e);
        }
#pragma unroll
        for (int d = 0; d < N / 4; ++d) reinterpret_cast<uint32_t*>(x_lds + r * xrow + c * N)[d] = q4[d];
      };
      if (hold) {
        float mx = xf_max[0];
#pragma unroll
        for (int w = 1; w < W; ++w) mx = fmaxf(mx, xf_max[w * kGemvMaxM]);
        const float sc = q8_row_scale(mx);
        if (threadIdx.x == 0) xf_scale[0] = sc;
#pragma unroll
        for (int i = 0; i < kHold; ++i) {
          const int64_t c = threadIdx.x + (int64_t)i * W * 64;
          if (c < nv) quant_store(0, c, hv[i], sc);
        }
      }
      for (int64_t r = 0; r < (hold ? 0 : m); ++r) {
        float mx = xf_max[r];
#pragma unroll
        for (int w = 1; w < W; ++w) mx = fmaxf(mx, xf_max[w * kGemvMaxM + r]);
        const float sc = q8_row_scale(mx);
        if (threadIdx.x == 0) xf_scale[r] = sc;
        const float inv = XF == 3 ? row_inv(r) : 0.0f;
        for (int64_t c = threadIdx.x; c < nv; c += W * 64) {
          float v[N];
          act(r, c, v, inv, false);
          quant_store(r, c, v, sc);
        }
      }
    }
    // Every wave's DMA writes are complete (its vmcnt wait above) and the one LDS
    // store is waited by lgkmcnt(0), so a bare barrier publishes the scales; a
    // workgroup-scope fence here would add a vmcnt(0) and drain weight stage 1.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  if (active) {
    const uint16_t* sc_col = sc_lds + ((int64_t)grp * 16 * CG + j) * nblk;  // (+ 16 nblk per group)
    // XL: lane (j, q) reads row xr (rows past m, and under H8 the other block's
    // lanes, hold zero: the address is clamped to row 0 and the value selected away)
    const bool x_row_ok = xr < m && x_half_ok;
    const uint8_t* x_src = x_lds + (x_row_ok ? xr : 0) * xrow + 16 * q;
    // xa holds the stage's register activations, xb receives the next stage's and
    // is copied into xa after the stage-end wait (a copy before it would read
    // registers the loads have not yet written)
    for (int st = 0; st < nst; ++st) {
      i32x4 (&xc)[4] = xa;
      i32x4 (&xn)[4] = xb;
      // weight stage st (and its register activations) are here; stage st + 1 is in flight
      if constexpr (!XL) {
        if (st + 1 < nst) load_x(xn, st + 1);
      }
      const int64_t pst = p_begin + 4 * st;
      const int npp = p_end - pst < 4 ? (int)(p_end - pst) : 4;
      const uint8_t* src = wbuf + (st & 1) * kWaveBuf + j * kGvKC;
      // one block pair: operands from LDS (or registers), then its MFMA(s) and applies
      struct Operands {
        i32x4 wv[CG], x;
        float s_lo[CG], s_hi[CG];
      };
      auto fetch = [&](int pp) {
        const int64_t p = pst + pp;
        const int64_t b = 2 * p;
        Operands o;
#pragma unroll
        for (int g = 0; g < CG; ++g)
          o.wv[g] = *reinterpret_cast<const i32x4*>(src + g * 16 * kGvKC + 16 * ((4 * pp + q) ^ j));
        if constexpr (XL) {
          const i32x4 xl = *reinterpret_cast<const i32x4*>(x_src + 64 * p);
          o.x = x_row_ok && 64 * p + 16 * q < k ? xl : i32x4{0, 0, 0, 0};
        } else {
          o.x = xc[pp];
        }
#pragma unroll
        for (int g = 0; g < CG; ++g) {
          const uint16_t* scg = sc_col + g * 16 * nblk;
          if constexpr (H8) {  // this lane's block: b or b + 1 (scale 0 past the last block)
            const int64_t bq = b + (q >> 1);
            const float sv = fp16_bits_to_float(scg[bq < nblk ? bq : b]);  // read unconditionally
            o.s_lo[g] = bq < nblk ? sv : 0.0f;
            o.s_hi[g] = 0.0f;
          } else {
            o.s_lo[g] = fp16_bits_to_float(scg[b]);
            const float s1 = fp16_bits_to_float(scg[b + 1 < nblk ? b + 1 : b]);  // read unconditionally
            o.s_hi[g] = b + 1 < nblk ? s1 : 0.0f;
          }
        }
        return o;
      };
      auto apply = [&](const Operands& o) {
        const i32x4 z = {0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < CG; ++g) {
          if constexpr (H8) {
            const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.x, o.wv[g], z, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[g][v] = fmaf(o.s_lo[g], (float)d[v], acc[g][v]);
          } else {
            const i32x4 x_lo = q < 2 ? o.x : z;  // first block of the pair
            const i32x4 x_hi = q < 2 ? z : o.x;  // second block
            const i32x4 d_lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(x_lo, o.wv[g], z, 0, 0, 0);
            const i32x4 d_hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(x_hi, o.wv[g], z, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              acc[g][v] = fmaf(o.s_lo[g], (float)d_lo[v], acc[g][v]);
              acc[g][v] = fmaf(o.s_hi[g], (float)d_hi[v], acc[g][v]);
            }
          }
        }
      };
      if (npp == 4) {  // uniform: a full stage reads all its operands first, then computes
        Operands o[4];
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) o[pp] = fetch(pp);
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) apply(o[pp]);
      } else {
#pragma unroll
        for (int pp = 0; pp < 4; ++pp)
          if (pp < npp) apply(fetch(pp));
      }
      if (st + 1 < nst) {
        // weight stage st + 2 into the buffer just read (its values are in
        // registers); vmcnt(4) leaves that one in flight and completes stage st + 1
        // and its register activations
        if (st + 2 < nst) {
          issue(st + 2);
          gemv_wait_but_stage<CG>();
        } else {
          __builtin_amdgcn_s_waitcnt(0x0F70);
        }
        if constexpr (!XL) {
          x_ready(xn);
#pragma unroll
          for (int pp = 0; pp < 4; ++pp) xc[pp] = xn[pp];
        }
      }
    }
  }
  // D layout of v_mfma_*_16x16: lane l, value v -> column l % 16, row 4 * (l / 16) + v.
  // Partial sums [wave][column group][16 rows][17] in the wave's own DMA buffers
  // (all its transfers completed at its last vmcnt wait).
  auto part = [&](int w, int cg, int r, int c) -> float& {
    return reinterpret_cast<float*>(dyn + w * 2 * kWaveBuf)[(cg * 16 + r) * 17 + c];
  };
#pragma unroll
  for (int g = 0; g < CG; ++g)
#pragma unroll
    for (int v = 0; v < 4; ++v) part(wave, g, 4 * q + v, j) = acc[g][v];
  __syncthreads();
  for (int o = threadIdx.x; o < kCols * 16; o += W * 64) {
    const int c = o % kCols, r = o / kCols;  // consecutive threads -> consecutive columns
    const int g = c / (16 * CG), cg = (c / 16) % CG, cj = c % 16;
    const int64_t col = wg_c0 + c;
    if (r < m && col < n) {
      float sum = 0.0f;
#pragma unroll
      for (int sp = 0; sp < S; ++sp) {
        sum += part(g * S + sp, cg, r, cj);
        if constexpr (H8) sum += part(g * S + sp, cg, r + 8, cj);  // the pairs' second blocks
      }
      const float sc = XF != 0 ? xf_scale[r] : rscale[r];
      const float inv = sc > 0.0f ? 1.0f / sc : 0.0f;  // the reference's adq (:358)
      gemm_store_out(out + r * n + col, sum * inv);
    }
  }
}

// Launches the GEMV with W waves per workgroup and K split S; false if the
// staged scales would not fit.  The activation rows go to LDS (XL) when they fit
// and cost no resident workgroups the launch can use.
template <typename TO, int W, int S, int CG = 1>
bool try_gemv(const int8_t* xq, const float* rscale, const int8_t* w8, const uint16_t* ws, TO* out, int64_t m,
              int64_t n, int64_t k, hipStream_t stream) {
  constexpr int kCols = gemv_cols<W, S, CG>();
  constexpr int kDma = W * 2 * kGvWaveBuf * CG;
  const int64_t sc_bytes = (kCols * (k / 32) * 2 + 15) & ~15;
  if (sc_bytes > kGemvScaleLds) return false;
  const int64_t x_bytes = m * (k + 16);
  const int64_t wgs = (n + kCols - 1) / kCols;
  const int64_t cus = 256;
  auto resident = [&](int64_t lds) {  // workgroups per CU, by LDS and by wave slots (8 per SIMD)
    return std::min<int64_t>(kLdsPerCu / lds, 32 / W);
  };
  const int64_t need = (wgs + cus - 1) / cus;  // workgroups per CU the launch can use
  const int64_t lds_r = kDma + sc_bytes, lds_x = lds_r + x_bytes;
  // (S = 1: a wave's long run of stages keeps enough in flight; its register
  // activations measured faster than the extra LDS reads)
  const bool xl = S > 1 && x_bytes <= kGemvXLdsMax &&
                  std::min(resident(lds_x), need) >= std::min(resident(lds_r), need);
  static std::once_flag attr_once;
  std::call_once(attr_once, [] {
    const int lds_reg = kDma + kGemvScaleLds;
    const int lds_xl = (int)std::min<int64_t>(kLdsPerCu, kDma + kGemvScaleLds + kGemvXLdsMax);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&q8_gemv_kernel<TO, W, S, false, 0, false, CG>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds_reg);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&q8_gemv_kernel<TO, W, S, false, 0, true, CG>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds_reg);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&q8_gemv_kernel<TO, W, S, true, 0, false, CG>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds_xl);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&q8_gemv_kernel<TO, W, S, true, 0, true, CG>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds_xl);
  });
  const dim3 grid((unsigned)wgs), block(W * 64);
  const bool h8 = m <= 8;
  if (xl && h8)
    q8_gemv_kernel<TO, W, S, true, 0, true, CG><<<grid, block, (size_t)lds_x, stream>>>(xq, rscale, w8, ws, out, m, n,
                                                                                   k, (int)sc_bytes);
  else if (xl)
    q8_gemv_kernel<TO, W, S, true, 0, false, CG><<<grid, block, (size_t)lds_x, stream>>>(xq, rscale, w8, ws, out, m, n,
                                                                                    k, (int)sc_bytes);
  else if (h8)
    q8_gemv_kernel<TO, W, S, false, 0, true, CG><<<grid, block, (size_t)lds_r, stream>>>(xq, rscale, w8, ws, out, m, n,
                                                                                    k, (int)sc_bytes);
  else
    q8_gemv_kernel<TO, W, S, false, 0, false, CG><<<grid, block, (size_t)lds_r, stream>>>(xq, rscale, w8, ws, out, m, n,
                                                                                     k, (int)sc_bytes);
  return true;
}

// The GEMV with the fused activation quantizer (XF 1 or 2): always the staged-row
// form; false when the rows or the scales would not fit the workgroup's LDS.
// The fused norm's operands (XF 3).
template <typename TO>
struct RmsOperands {
  const TO* res = nullptr;
  TO* res_out = nullptr;
  const TO* g = nullptr;
  float eps = 0.0f;
};

template <typename TO, int W, int S, int XF>
bool try_gemv_act(const TO* xf, int64_t xf_ld, const int8_t* w8, const uint16_t* ws, TO* out, int64_t m, int64_t n,
                  int64_t k, hipStream_t stream, const RmsOperands<TO>& rn) {
  constexpr int kDma = W * 2 * kGvWaveBuf;
  constexpr int kCols = gemv_cols<W, S>();
  const int64_t sc_bytes = (kCols * (k / 32) * 2 + 15) & ~15;
  // rows, then maxima, scales and the norm's sums of squares
  const int64_t x_bytes = ((m * (k + 16) + 15) & ~int64_t(15)) + (W + 1 + 4) * kGemvMaxM * 4;
  if (sc_bytes > kGemvScaleLds || x_bytes > kGemvXLdsMax || kDma + sc_bytes + x_bytes > kLdsPerCu) return false;
  static std::once_flag attr_once;
  std::call_once(attr_once, [] {
    const int lds = (int)std::min<int64_t>(kLdsPerCu, kDma + kGemvScaleLds + kGemvXLdsMax);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&q8_gemv_kernel<TO, W, S, true, XF, false>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&q8_gemv_kernel<TO, W, S, true, XF, true>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  });
  const int64_t wgs = (n + kCols - 1) / kCols;
  const dim3 grid((unsigned)wgs), block(W * 64);
  const size_t lds = (size_t)(kDma + sc_bytes + x_bytes);
  if (m <= 8)
    q8_gemv_kernel<TO, W, S, true, XF, true><<<grid, block, lds, stream>>>(
        nullptr, nullptr, w8, ws, out, m, n, k, (int)sc_bytes, xf, xf_ld, rn.res, rn.res_out, rn.g, rn.eps);
  else
    q8_gemv_kernel<TO, W, S, true, XF, false><<<grid, block, lds, stream>>>(
        nullptr, nullptr, w8, ws, out, m, n, k, (int)sc_bytes, xf, xf_ld, rn.res, rn.res_out, rn.g, rn.eps);
  return true;
}

// Split-K reduction: out[r][c] = (sum over splits, in order, of part[split][r][c]) /
// row_scale[r] (0 where the scale is 0, as the tile kernel), in the output dtype.
// Four consecutive columns per thread where the row allows.
template <typename TO>
__global__ __launch_bounds__(256) void q8_gemm_reduce_kernel(const float* __restrict__ part,
                                                             const float* __restrict__ rscale, TO* __restrict__ out,
                                                             int64_t m, int64_t n, int splits) {
  const int64_t nq = (n + 3) / 4;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= m * nq) return;
  const int64_t r = i / nq, c0 = (i % nq) * 4;
  const float s = rscale[r];
  const float inv = s > 0.0f ? 1.0f / s : 0.0f;
  const int64_t mn = m * n;
  const float* p = part + r * n + c0;
  if (n % 4 == 0) {  // 16-byte rows: one vector load per split
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int z = 0; z < splits; ++z) acc += __builtin_bit_cast(f32x4, ld16(p + z * mn));
#pragma unroll
    for (int e = 0; e < 4; ++e) gemm_store_out(out + r * n + c0 + e, acc[e] * inv);
    return;
  }
  for (int64_t c = 0; c < 4 && c0 + c < n; ++c) {
    float acc = 0.0f;
    for (int z = 0; z < splits; ++z) acc += p[z * mn + c];
    gemm_store_out(out + r * n + c0 + c, acc * inv);
  }
}

// Split-K plan for the tile GEMM: when the output has fewer than kGemmSplitBelow
// tiles (half a round of the 768 resident workgroups), K is cut into ranges of
// whole stages (at least 8) for about kGemmSplitTarget workgroups.  (At 592 tiles
// the partial-sum traffic costs more than the idle CUs: measured.)
constexpr int64_t kGemmSplitBelow = 384;
constexpr int64_t kGemmSplitTarget = 768;
constexpr int64_t kGemmSplitMinStages = 8;
struct GemmSplit {
  int splits = 1;
  int st_per_split = 0;
};
inline GemmSplit gemm_split_plan(int64_t m, int64_t n, int64_t k) {
  GemmSplit p;
  if (m <= kGemvMaxM || k % 32 != 0 || k > ((int64_t)1 << 24)) return p;
  const int64_t tiles = ((m + kGemmBM - 1) / kGemmBM) * ((n + kGemmBN - 1) / kGemmBN);
  const int64_t nstages = (k + kGemmKC - 1) / kGemmKC;
  if (tiles >= kGemmSplitBelow) return p;
  int64_t s = std::min<int64_t>((kGemmSplitTarget + tiles - 1) / tiles, nstages / kGemmSplitMinStages);
  if (s <= 1) return p;
  const int64_t per = (nstages + s - 1) / s;
  s = (nstages + per - 1) / per;  // every split non-empty
  if (s <= 1 || s > 65535) return p;
  p.splits = (int)s;
  p.st_per_split = (int)per;
  return p;
}
inline int64_t gemm_split_bytes(int64_t m, int64_t n, const GemmSplit& p) {
  return p.splits > 1 ? p.splits * m * n * (int64_t)sizeof(float) : 0;
}

}  // namespace nvf

using namespace nvf;

namespace {

int check_gemm(const void* xq, const float* rscale, const void* w8, const void* ws, int64_t m, int64_t n, int64_t k,
               const void* out, int dtype, const char* who) {
  if (m < 0 || n < 0 || k < 0) return fail(NVF_ERR_INVALID, "%s: negative size", who);
  if (k % 32 != 0) return fail(NVF_ERR_INVALID, "%s: k=%lld is not a multiple of the Q8_0 block (32)", who, (long long)k);
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "%s: bad out dtype %d", who, dtype);
  if (k > (int64_t)1 << 24)  // buffer offsets within a 128-row tile stay below 2^31
    return fail(NVF_ERR_INVALID, "%s: k=%lld exceeds 2^24", who, (long long)k);
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
                int64_t n, int64_t k, void* work, int64_t work_bytes, hipStream_t stream) {
  if (m <= kGemvMaxM) {
    // fewest K splits that still give >= ~2048 waves (16 columns each); more splits
    // when the staged scales of a wider column set would not fit
    const int64_t groups = (n + 15) / 16;
    bool ok = false;
    // (wide outputs: one-wave workgroups of 32 columns, so one activation fragment feeds
    // two MFMAs and the many small workgroups spread evenly over the CUs, 4 or 5 each;
    // measured at the gate_up shape, m = 8: 25.7-26.0 us against 28.1-28.4 for 2 waves
    // of 32 columns (2 or 3 workgroups per CU), 30.8 for 4 waves of 16 columns and 30.3
    // for 1 wave of 64; capping residency at 5 one-wave workgroups per CU: 36.4)
    if (groups >= 2048) ok = try_gemv<TO, 1, 1, 2>(xq, rscale, w8, ws, out, m, n, k, stream);
    if (!ok && groups >= 1024) ok = try_gemv<TO, 4, 2>(xq, rscale, w8, ws, out, m, n, k, stream);
    if (!ok && groups >= 512) ok = try_gemv<TO, 4, 4>(xq, rscale, w8, ws, out, m, n, k, stream);
    if (!ok) ok = try_gemv<TO, 8, 8>(xq, rscale, w8, ws, out, m, n, k, stream);
    if (ok) return launch_status("q8_gemv_kernel");
  }
  static std::once_flag attr_once;
  std::call_once(attr_once, [] {
    for (const void* f : {reinterpret_cast<const void*>(&q8_gemm_kernel<TO, false, true>),
                          reinterpret_cast<const void*>(&q8_gemm_kernel<TO, true, true>),
                          reinterpret_cast<const void*>(&q8_gemm_kernel<TO, false, false>),
                          reinterpret_cast<const void*>(&q8_gemm_kernel<TO, true, false>)})
      (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
  });
  const int tiles_n = (int)((n + kGemmBN - 1) / kGemmBN);
  const int64_t tiles = ((m + kGemmBM - 1) / kGemmBM) * tiles_n;
  const GemmSplit sp = gemm_split_plan(m, n, k);
  if (sp.splits > 1 && work && work_bytes >= gemm_split_bytes(m, n, sp)) {
    float* part = static_cast<float*>(work);
    const dim3 grid((unsigned)tiles, (unsigned)sp.splits);
    if (k % kGemmKC != 0)
      q8_gemm_kernel<TO, true, true><<<grid, dim3(kGemmThreads), kGemmLds, stream>>>(
          xq, rscale, w8, ws, out, m, n, k, tiles_n, sp.st_per_split, part);
    else
      q8_gemm_kernel<TO, true, false><<<grid, dim3(kGemmThreads), kGemmLds, stream>>>(
          xq, rscale, w8, ws, out, m, n, k, tiles_n, sp.st_per_split, part);
    const int rc = launch_status("q8_gemm_kernel(split)");
    if (rc != NVF_OK) return rc;
    const int64_t threads = m * ((n + 3) / 4);
    q8_gemm_reduce_kernel<TO><<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream>>>(part, rscale, out, m,
                                                                                                 n, sp.splits);
    return launch_status("q8_gemm_reduce_kernel");
  }
  if (k % kGemmKC != 0)
    q8_gemm_kernel<TO, false, true><<<dim3((unsigned)tiles), dim3(kGemmThreads), kGemmLds, stream>>>(
        xq, rscale, w8, ws, out, m, n, k, tiles_n, 0, nullptr);
  else
    q8_gemm_kernel<TO, false, false><<<dim3((unsigned)tiles), dim3(kGemmThreads), kGemmLds, stream>>>(
        xq, rscale, w8, ws, out, m, n, k, tiles_n, 0, nullptr);
  return launch_status("q8_gemm_kernel");
}

// The decode GEMV (m <= 16) on fp activations, quantized in its prologue (XF 1:
// rows [m, k]; XF 2: SwiGLU over [gate | up] rows [m, 2k]).  The same (W, S)
// choice as launch_gemm; NVF_ERR_INVALID when no GEMV form fits.
template <typename TO, int XF>
int launch_gemv_act(const TO* xf, int64_t xf_ld, const int8_t* w8, const uint16_t* ws, TO* out, int64_t m, int64_t n,
                    int64_t k, hipStream_t stream, const RmsOperands<TO>& rn = {}) {
  const int64_t groups = (n + 15) / 16;
  bool ok = false;
  if (groups >= 2048) ok = try_gemv_act<TO, 4, 1, XF>(xf, xf_ld, w8, ws, out, m, n, k, stream, rn);
  if (!ok && groups >= 1024) ok = try_gemv_act<TO, 4, 2, XF>(xf, xf_ld, w8, ws, out, m, n, k, stream, rn);
  if (!ok && groups >= 512) ok = try_gemv_act<TO, 4, 4, XF>(xf, xf_ld, w8, ws, out, m, n, k, stream, rn);
  if (!ok) ok = try_gemv_act<TO, 8, 8, XF>(xf, xf_ld, w8, ws, out, m, n, k, stream, rn);
  if (!ok)
    return fail(NVF_ERR_INVALID, "matmul_q8_0_act: m=%lld rows of k=%lld do not fit the GEMV's LDS (quantize "
                "separately and use nvf_matmul_q8_0)", (long long)m, (long long)k);
  return launch_status("q8_gemv_kernel(act)");
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

int nvf_matmul_q8_0_ws(const int8_t* xq, const float* row_scale, const uint8_t* w8, const uint16_t* ws, int64_t m,
                       int64_t n, int64_t k, void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
                       void* stream) {
  const int st = check_gemm(xq, row_scale, w8, ws, m, n, k, out, out_dtype, "matmul_q8_0");
  if (st != NVF_OK || m == 0 || n == 0 || k == 0) return st;
  if (workspace && !aligned16(workspace))
    return fail(NVF_ERR_INVALID, "matmul_q8_0: workspace must be 16-byte aligned");
  if (m * ((n + 3) / 4) / 256 >= INT32_MAX) return fail(NVF_ERR_INVALID, "matmul_q8_0: output too large");
  const int8_t* w = reinterpret_cast<const int8_t*>(w8);
  int rc = NVF_OK;
  NVF_DISPATCH_DTYPE(out_dtype, TO, rc = launch_gemm<TO>(xq, row_scale, w, ws, static_cast<TO*>(out), m, n, k,
                                                        workspace, workspace_bytes, as_stream(stream)));
  return rc;
}

int nvf_matmul_q8_0(const int8_t* xq, const float* row_scale, const uint8_t* w8, const uint16_t* ws, int64_t m,
                    int64_t n, int64_t k, void* out, int out_dtype, void* stream) {
  return nvf_matmul_q8_0_ws(xq, row_scale, w8, ws, m, n, k, out, out_dtype, nullptr, 0, stream);
}

int nvf_matmul_q8_0_act(const void* x, int64_t x_stride, int act, const uint8_t* w8, const uint16_t* ws, int64_t m,
                        int64_t n, int64_t k, void* out, int dtype, void* stream) {
  static const char* who = "matmul_q8_0_act";
  if (m < 0 || n < 0 || k < 0) return fail(NVF_ERR_INVALID, "%s: negative size", who);
  if (k % 32 != 0) return fail(NVF_ERR_INVALID, "%s: k=%lld is not a multiple of the Q8_0 block (32)", who, (long long)k);
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "%s: bad dtype %d", who, dtype);
  if (act != 0 && act != 1) return fail(NVF_ERR_INVALID, "%s: act=%d (0: rows, 1: SwiGLU over gate | up)", who, act);
  if (m > kGemvMaxM)
    return fail(NVF_ERR_INVALID, "%s: m=%lld > %d rows (the decode GEMV's; quantize separately and use "
                "nvf_matmul_q8_0)", who, (long long)m, kGemvMaxM);
  if (x_stride < (act ? 2 : 1) * k) return fail(NVF_ERR_INVALID, "%s: x_stride=%lld too small", who, (long long)x_stride);
  if (m == 0 || n == 0 || k == 0) return NVF_OK;
  if (!x || !w8 || !ws || !out) return fail(NVF_ERR_INVALID, "%s: null pointer", who);
  if (!aligned16(x) || !aligned16(w8) || (x_stride * dtype_bytes(dtype)) % 16 != 0)
    return fail(NVF_ERR_INVALID, "%s: x (and its rows) and w8 must be 16-byte aligned", who);
  if ((reinterpret_cast<uintptr_t>(ws) & 1u) != 0) return fail(NVF_ERR_INVALID, "%s: ws must be 2-byte aligned", who);
  if (bytes_overlap(out, m * n * dtype_bytes(dtype), x, ((m - 1) * x_stride + (act ? 2 : 1) * k) * dtype_bytes(dtype)))
    return fail(NVF_ERR_INVALID, "%s: out must not overlap x (every workgroup reads x while others write out)", who);
  const int8_t* w = reinterpret_cast<const int8_t*>(w8);
  int rc = NVF_OK;
  if (act == 0)
    NVF_DISPATCH_DTYPE(dtype, T, rc = (launch_gemv_act<T, 1>(static_cast<const T*>(x), x_stride, w, ws,
                                                            static_cast<T*>(out), m, n, k, as_stream(stream))));
  else
    NVF_DISPATCH_DTYPE(dtype, T, rc = (launch_gemv_act<T, 2>(static_cast<const T*>(x), x_stride, w, ws,
                                                            static_cast<T*>(out), m, n, k, as_stream(stream))));
  return rc;
}

int nvf_matmul_q8_0_rms(const void* x, int64_t x_stride, const void* residual, void* residual_out,
                        const void* norm_weight, float eps, const uint8_t* w8, const uint16_t* ws, int64_t m, int64_t n,
                        int64_t k, void* out, int dtype, void* stream) {
  static const char* who = "matmul_q8_0_rms";
  if (m < 0 || n < 0 || k < 0) return fail(NVF_ERR_INVALID, "%s: negative size", who);
  if (k % 32 != 0) return fail(NVF_ERR_INVALID, "%s: k=%lld is not a multiple of the Q8_0 block (32)", who, (long long)k);
  if (!dtype_ok(dtype)) return fail(NVF_ERR_INVALID, "%s: bad dtype %d", who, dtype);
  if (m > kGemvMaxM)
    return fail(NVF_ERR_INVALID, "%s: m=%lld > %d rows (the decode GEMV's; use nvf_rms_norm_q8 and "
                "nvf_matmul_q8_0)", who, (long long)m, kGemvMaxM);
  const int64_t eb = dtype_bytes(dtype);
  const int64_t nvec = k * eb / 16;
  if (nvec > (int64_t)kRmsMaxVpl * 4 * 64)
    return fail(NVF_ERR_INVALID, "%s: k=%lld exceeds the register-resident norm row (use nvf_rms_norm_q8 and "
                "nvf_matmul_q8_0)", who, (long long)k);
  if (x_stride < k) return fail(NVF_ERR_INVALID, "%s: x_stride=%lld too small", who, (long long)x_stride);
  if ((residual == nullptr) != (residual_out == nullptr))
    return fail(NVF_ERR_INVALID, "%s: residual and residual_out go together", who);
  if (m == 0 || n == 0 || k == 0) return NVF_OK;
  if (!x || !norm_weight || !w8 || !ws || !out) return fail(NVF_ERR_INVALID, "%s: null pointer", who);
  if (!aligned16(x) || !aligned16(w8) || !aligned16(norm_weight) || (x_stride * eb) % 16 != 0 ||
      (residual && (!aligned16(residual) || !aligned16(residual_out))))
    return fail(NVF_ERR_INVALID, "%s: x (and its rows), residual, residual_out, norm_weight and w8 must be 16-byte "
                "aligned", who);
  if ((reinterpret_cast<uintptr_t>(ws) & 1u) != 0) return fail(NVF_ERR_INVALID, "%s: ws must be 2-byte aligned", who);
  {
    // every workgroup reads x and residual in its prologue while workgroup 0 writes
    // residual_out and every workgroup writes its columns of out
    const int64_t rb = m * k * eb, xb = ((m - 1) * x_stride + k) * eb, ob = m * n * eb;
    if (residual && (bytes_overlap(residual_out, rb, residual, rb) || bytes_overlap(residual_out, rb, x, xb)))
      return fail(NVF_ERR_INVALID, "%s: residual_out must not overlap residual or x", who);
    if (bytes_overlap(out, ob, x, xb) || (residual && (bytes_overlap(out, ob, residual, rb) ||
                                                       bytes_overlap(out, ob, residual_out, rb))))
      return fail(NVF_ERR_INVALID, "%s: out must not overlap x, residual or residual_out", who);
  }
  const int8_t* w = reinterpret_cast<const int8_t*>(w8);
  int rc = NVF_OK;
  NVF_DISPATCH_DTYPE(dtype, T, (rc = launch_gemv_act<T, 3>(
                                    static_cast<const T*>(x), x_stride, w, ws, static_cast<T*>(out), m, n, k,
                                    as_stream(stream),
                                    RmsOperands<T>{static_cast<const T*>(residual), static_cast<T*>(residual_out),
                                                   static_cast<const T*>(norm_weight), eps})));
  return rc;
}

int64_t nvf_matmul_q8_0_workspace_size(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  return gemm_split_bytes(m, n, gemm_split_plan(m, n, k));
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
  const size_t s_bytes = ((size_t)m * sizeof(float) + 255) & ~(size_t)255;
  const size_t w_bytes = (size_t)nvf_matmul_q8_0_workspace_size(m, n, k);  // split-K partials (0: unsplit)
  const size_t need = q_bytes + s_bytes + w_bytes;
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
  void* work = w_bytes ? static_cast<uint8_t*>(g_scratch.p) + q_bytes + s_bytes : nullptr;
  dropin_check(nvf_matmul_q8_0_ws(xq, rs, w8, ws, m, n, k, out, NVF_F32, work, (int64_t)w_bytes, nullptr),
               "hip_matmul_q8");
}

}  // extern "C"
