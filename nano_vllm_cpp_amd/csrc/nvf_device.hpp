// Device-side building blocks shared by the fused-op kernels (gfx950, wave64).
//
//  * Storage types: float, _Float16 and __bf16.  Loads upcast exactly; stores
//    round to nearest even (clang fptrunc, v_cvt_pk_* on gfx950).
//  * Pack<T>: one 16-byte vector (global_load/store_dwordx4) as N floats.
//  * wave/group sums built from DPP row ops and one ds_swizzle, no LDS memory.
//  * FastDiv: 32-bit divide by a launch-constant divisor (mul-hi + shift).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nvf {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// 16-byte packs
// ---------------------------------------------------------------------------
template <typename T>
struct Pack;

template <>
struct Pack<float> {
  static constexpr int N = 4;
  static __device__ __forceinline__ void unpack(const u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = v[i];  // bit_cast of a vector-element lvalue reads element 0: copy first
      f[i] = __builtin_bit_cast(float, w);
    }
  }
  static __device__ __forceinline__ u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = f[i];
      v[i] = __builtin_bit_cast(uint32_t, x);
    }
    return v;
  }
};

template <>
struct Pack<_Float16> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void unpack(const u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = v[i];
      const f16x2 h = __builtin_bit_cast(f16x2, w);
      f[2 * i] = (float)h[0];
      f[2 * i + 1] = (float)h[1];
    }
  }
  static __device__ __forceinline__ u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x2 p = {f[2 * i], f[2 * i + 1]};
      v[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(p, f16x2));
    }
    return v;
  }
};

template <>
struct Pack<__bf16> {
  static constexpr int N = 8;
  static __device__ __forceinline__ void unpack(const u32x4 v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __builtin_bit_cast(float, v[i] << 16);
      f[2 * i + 1] = __builtin_bit_cast(float, v[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ u32x4 pack(const float* f) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x2 p = {f[2 * i], f[2 * i + 1]};
      v[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2));
    }
    return v;
  }
};

// Scalar element access for the generic (unaligned / odd-shape) kernels.
template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return (float)v;
}
template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return (T)v;
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
// Streaming variants: data touched exactly once (no reuse in L2/MALL).
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16_nt(void* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// ---------------------------------------------------------------------------
// Wavefront reductions (wave64).  DPP controls:
//   0xb1  quad_perm [1,0,3,2]      0x4e  quad_perm [2,3,0,1]
//   0x141 row_half_mirror (i <-> 7-i inside 8 lanes)
//   0x140 row_mirror      (i <-> 15-i inside 16 lanes)
// then ds_swizzle bit-mode xor 16 (offset 0x401f: and 0x1f, or 0, xor 0x10)
// crosses 16-lane rows, and readlane 0 + readlane 32 joins the two halves.
// Every step adds two equal-magnitude partials in a fixed order, so all lanes
// of a group end with the bit-identical sum.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Sum over aligned groups of G lanes (G in 1,2,4,8,16,32); result in every lane of the group.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32, "group size");
  if constexpr (G >= 2) v += dpp_mov<0xb1>(v);
  if constexpr (G >= 4) v += dpp_mov<0x4e>(v);
  if constexpr (G >= 8) v += dpp_mov<0x141>(v);
  if constexpr (G >= 16) v += dpp_mov<0x140>(v);
  if constexpr (G >= 32)
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f));
  return v;
}

// Max over aligned groups of G lanes, same lane pattern as group_sum.
template <int G>
__device__ __forceinline__ float group_max(float v) {
  static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32, "group size");
  if constexpr (G >= 2) v = fmaxf(v, dpp_mov<0xb1>(v));
  if constexpr (G >= 4) v = fmaxf(v, dpp_mov<0x4e>(v));
  if constexpr (G >= 8) v = fmaxf(v, dpp_mov<0x141>(v));
  if constexpr (G >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
  if constexpr (G >= 32)
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f)));
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = group_max<32>(v);
  return fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)),
               __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32)));
}

// Sum over the full wave; wave-uniform result.  EXEC must be full.
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<32>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
}

// SiLU(g) * u, the reference's g / (1 + expf(-g)) * u (src/hip_ops.hip:419-429).
// fp32 keeps the exact expression (IEEE divide, precise expf); fp16/bf16 use
// v_exp_f32 + v_rcp_f32 (a few fp32 ulp, far below one 16-bit ulp).  Every
// kernel that computes SwiGLU (the SwiGLU kernels, the decode GEMV's fused
// prologue) calls this one function, so they all produce the same bits.
template <typename T>
__device__ __forceinline__ float silu_mul(float g, float u) {
  if constexpr (sizeof(T) == 4) {
    return g / (1.0f + expf(-g)) * u;
  } else {
    const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
    float v = g * __builtin_amdgcn_rcpf(1.0f + e) * u;
    // The fp32 product is the value: an empty asm keeps the compiler from folding
    // the last multiply into the 16-bit conversion (v_fma_mix rounds once where
    // multiply-then-convert rounds twice), so every kernel stores the same bits.
    asm("" : "+v"(v));
    return v;
  }
}

// Q8 activation quantizer of the reference's INT8 GEMM path: per-row scale
// 127 / max|x| (0 for an all-~zero row) and q = (int8)clamp(x * scale, +-127)
// with C truncation (src/hip_ops.hip:205-217, :244-245).
// RMSNorm row layout (rms_norm.hip, and the decode GEMV's fused norm, which must sum
// the squares in the same order to give a bit-identical 1/rms): a row of nvec
// 16-byte vectors goes to rms_waves_per_row(nvec) waves; vector i of lane l in
// sub-wave s is (i * wpr + s) * 64 + l; each lane sums its squares by fmaf in
// (i, element) order, then wave_sum, then the sub-waves' sums in order s = 0, 1, ...
__host__ __device__ constexpr int rms_waves_per_row(int64_t nvec) { return nvec >= 256 ? 4 : (nvec >= 128 ? 2 : 1); }
constexpr int kRmsMaxVpl = 16;  // vectors per lane of the register-resident 4-wave row

__device__ __forceinline__ float q8_row_scale(float max_abs) { return max_abs > 1e-8f ? 127.0f / max_abs : 0.0f; }
__device__ __forceinline__ int q8_quantize(float v, float scale) {
  return (int)(int8_t)fminf(127.0f, fmaxf(-127.0f, v * scale));
}

// ---------------------------------------------------------------------------
// n / d for n < 2^32 and a divisor fixed at launch (Granlund-Montgomery).
// ---------------------------------------------------------------------------
struct FastDiv {
  uint32_t d, m, s;
  FastDiv() = default;
  __host__ explicit FastDiv(uint32_t div) : d(div) {
    s = 0;
    while ((1ull << s) < div) ++s;
    m = (uint32_t)(((1ull << 32) * ((1ull << s) - div)) / div + 1);
  }
  // (n * m) >> 32 is v_mul_hi_u32 on the device; the same code runs on the host
  // for the unit test.
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
    const uint32_t hi = (uint32_t)(((uint64_t)n * m) >> 32);
    return (uint32_t)(((uint64_t)hi + n) >> s);
  }
};

}  // namespace nvf
