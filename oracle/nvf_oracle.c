/*
 * nvf_oracle.c -- scalar C restatement of Nano_vLLM_cpp's fused per-layer ops.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  See nvf_oracle.h
 * for the pin of every function.  Citations are Nano_vLLM_cpp source paths.
 */
#include "nvf_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- storage codecs ----------------------------------------------------- */

/* include/nanovllm/common.hpp:28-54: exact fp16 decode, subnormals included. */
float orc_fp16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t ex = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (ex == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      /* value = man * 2^-24; normalise the mantissa */
      int e = 127 - 14;
      while (!(man & 0x400u)) {
        man <<= 1;
        --e;
      }
      bits = sign | ((uint32_t)e << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (ex == 0x1fu) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((ex + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* include/nanovllm/common.hpp:65-91: round-to-nearest-even, overflow -> Inf.
 * NaN keeps a quiet NaN (the reference maps NaN to Inf; no path here makes one). */
uint16_t orc_f32_to_fp16(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  uint32_t sign = (b >> 16) & 0x8000u;
  uint32_t absb = b & 0x7fffffffu;
  if (absb > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  int32_t ex = (int32_t)(absb >> 23) - 127 + 15;
  uint32_t man = absb & 0x7fffffu;
  if (ex >= 31) return (uint16_t)(sign | 0x7c00u);
  if (ex <= 0) {
    if (ex < -10) return (uint16_t)sign;
    man |= 0x800000u;
    uint32_t sh = (uint32_t)(14 - ex);
    uint32_t m = man >> sh;
    uint32_t rem = man & ((1u << sh) - 1u);
    uint32_t halfway = 1u << (sh - 1);
    if (rem > halfway || (rem == halfway && (m & 1u))) ++m;
    return (uint16_t)(sign | m); /* m may carry into the exponent field: correct */
  }
  uint32_t m = man >> 13;
  uint32_t rem = man & 0x1fffu;
  uint32_t out = ((uint32_t)ex << 10) | m;
  if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) ++out; /* carry is correct */
  if (out >= 0x7c00u) out = 0x7c00u;
  return (uint16_t)(sign | out);
}

/* include/nanovllm/common.hpp:56-61 */
float orc_bf16_to_f32(uint16_t h) {
  uint32_t b = (uint32_t)h << 16;
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* round-to-nearest-even fp32 -> bf16, quiet NaN preserved */
uint16_t orc_f32_to_bf16(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40u);
  uint32_t lsb = (b >> 16) & 1u;
  b += 0x7fffu + lsb;
  return (uint16_t)(b >> 16);
}

float orc_load(const void* p, int64_t i, int dtype) {
  if (dtype == ORC_F32) return ((const float*)p)[i];
  uint16_t h = ((const uint16_t*)p)[i];
  return dtype == ORC_F16 ? orc_fp16_to_f32(h) : orc_bf16_to_f32(h);
}

void orc_store(void* p, int64_t i, float v, int dtype) {
  if (dtype == ORC_F32)
    ((float*)p)[i] = v;
  else
    ((uint16_t*)p)[i] = dtype == ORC_F16 ? orc_f32_to_fp16(v) : orc_f32_to_bf16(v);
}

/* src/model.cpp:416-420: inv_freq in double, rounded to float. */
void orc_inv_freq(double theta, int head_dim, float* out) {
  for (int i = 0; i < head_dim / 2; ++i) out[i] = (float)(1.0 / pow(theta, (2.0 * i) / head_dim));
}

/* ---- K-quant superblocks ----------------------------------------------- */

/* 6-bit (scale, min) of group j from the 12-byte table:
 * src/gguf.cpp:482-489 == src/hip_ops.hip:116-128 */
static void q4k_scale_min(const uint8_t* s12, int j, uint32_t* sc, uint32_t* mn) {
  if (j < 4) {
    *sc = s12[j] & 63;
    *mn = s12[j + 4] & 63;
  } else {
    *sc = (s12[j + 4] & 0xF) | ((s12[j - 4] >> 6) << 4);
    *mn = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4);
  }
}

/* Q4_K, 144 B: [fp16 d][fp16 dmin][12 B scales][128 B qs].
 * GGML layout: src/gguf.cpp:477-496 (also tools/ref_top5.cpp:140-165):
 *   group j reads bytes qs[(j>>1)*32 + kk], nibble (j&1)*4.
 * HIP_LEGACY layout: src/hip_ops.hip:130-140 (qk_w_q4):
 *   group j reads bytes qs[j*16 + (e&15)], low nibble when e < 16. */
void orc_dequant_q4k_block(const uint8_t* blk, float* y, int layout) {
  float d = orc_fp16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
  float dmin = orc_fp16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
  for (int j = 0; j < 8; ++j) {
    uint32_t sc, mn;
    q4k_scale_min(blk + 4, j, &sc, &mn);
    float d1 = d * (float)sc, m1 = dmin * (float)mn;
    for (int e = 0; e < 32; ++e) {
      int q;
      if (layout == ORC_QK_LAYOUT_GGML) {
        q = (blk[16 + (j >> 1) * 32 + e] >> ((j & 1) * 4)) & 0xF;
      } else {
        uint8_t qb = blk[16 + j * 16 + (e & 15)];
        q = e < 16 ? (qb & 0xF) : (qb >> 4);
      }
      y[j * 32 + e] = d1 * (float)q - m1;
    }
  }
}

/* Q5_K, 176 B: [fp16 d][fp16 dmin][12 B scales][32 B qh][128 B ql].
 * tools/ref_top5.cpp:166-186 == src/hip_ops.hip:142-155 (qk_w_q5). */
void orc_dequant_q5k_block(const uint8_t* blk, float* y) {
  float d = orc_fp16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
  float dmin = orc_fp16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
  const uint8_t* qh = blk + 16;
  const uint8_t* ql = blk + 48;
  for (int group = 0; group < 4; ++group) {
    for (int slot = 0; slot < 2; ++slot) {
      int j = group * 2 + slot;
      uint32_t sc, mn;
      q4k_scale_min(blk + 4, j, &sc, &mn);
      float d1 = d * (float)sc, m1 = dmin * (float)mn;
      uint32_t hmask = (slot == 0 ? 1u : 2u) << (group * 2);
      for (int l = 0; l < 32; ++l) {
        int q = slot == 0 ? (ql[group * 32 + l] & 0xF) : (ql[group * 32 + l] >> 4);
        if (qh[l] & hmask) q += 16;
        y[group * 64 + slot * 32 + l] = d1 * (float)q - m1;
      }
    }
  }
}

/* Q6_K, 210 B: [128 B ql][64 B qh][16 x int8 scales][fp16 d].
 * src/gguf.cpp:500-518 == src/hip_ops.hip:157-182 (qk_w_q6); (d*sc)*(q-32). */
void orc_dequant_q6k_block(const uint8_t* blk, float* y) {
  float d = orc_fp16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
  for (int half = 0; half < 2; ++half) {
    const uint8_t* ql = blk + half * 64;
    const uint8_t* qh = blk + 128 + half * 32;
    const int8_t* sc = (const int8_t*)(blk + 192 + half * 8);
    for (int l = 0; l < 32; ++l) {
      int is = l >> 4;
      int q1 = (ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4);
      int q2 = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4);
      int q3 = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
      int q4 = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
      y[half * 128 + l] = d * (float)sc[is + 0] * (float)(q1 - 32);
      y[half * 128 + l + 32] = d * (float)sc[is + 2] * (float)(q2 - 32);
      y[half * 128 + l + 64] = d * (float)sc[is + 4] * (float)(q3 - 32);
      y[half * 128 + l + 96] = d * (float)sc[is + 6] * (float)(q4 - 32);
    }
  }
}

/* ---- embedding gathers -------------------------------------------------- */

/* src/hip_ops.hip:565-574 over the split planes of src/model.cpp:394-404:
 * out[t,c] = fp16(ws[e>>5]) * int8(w8[e]), e = ids[t]*H + c.  Exact in fp32. */
void orc_embedding_q8_split(const int64_t* ids, const uint8_t* w8, const uint16_t* ws, int64_t tokens,
                            int64_t hidden, void* out, int out_dtype) {
  for (int64_t t = 0; t < tokens; ++t)
    for (int64_t c = 0; c < hidden; ++c) {
      int64_t e = ids[t] * hidden + c;
      float v = orc_fp16_to_f32(ws[e >> 5]) * (float)(int8_t)w8[e];
      orc_store(out, t * hidden + c, v, out_dtype);
    }
}

/* The same gather over interleaved 34-byte GGUF Q8_0 blocks
 * (src/gguf.cpp:353-362; decode as tools/ref_top5.cpp:121-136). */
void orc_embedding_q8_blocks(const int64_t* ids, const uint8_t* blocks, int64_t tokens, int64_t hidden,
                             void* out, int out_dtype) {
  for (int64_t t = 0; t < tokens; ++t)
    for (int64_t c = 0; c < hidden; ++c) {
      int64_t e = ids[t] * hidden + c;
      const uint8_t* b = blocks + (e >> 5) * 34;
      float s = orc_fp16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
      float v = s * (float)(int8_t)b[2 + (e & 31)];
      orc_store(out, t * hidden + c, v, out_dtype);
    }
}

/* src/model.cpp:396-405 (upload_q8_split): block b's first two bytes are its
 * fp16 scale (little-endian), the next 32 its int8 values. */
void orc_q8_0_split_blocks(const uint8_t* blocks, int64_t nblocks, int8_t* w8, uint16_t* ws) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const uint8_t* p = blocks + b * 34;
    ws[b] = (uint16_t)(p[0] | (p[1] << 8));
    for (int i = 0; i < 32; ++i) w8[b * 32 + i] = (int8_t)p[2 + i];
  }
}

/* src/hip_ops.hip:600-609 (+ qk_w :184-193): element e = ids[t]*H + c lives in
 * superblock e>>8 at offset e&255; kinds 12/13/14 = Q4_K/Q5_K/Q6_K. */
void orc_embedding_qk(const int64_t* ids, const uint8_t* wq, int64_t tokens, int64_t hidden, int kind,
                      int layout, void* out, int out_dtype) {
  int64_t bb = kind == 12 ? 144 : (kind == 13 ? 176 : 210);
  float y[256];
  int64_t cached = -1;
  for (int64_t t = 0; t < tokens; ++t)
    for (int64_t c = 0; c < hidden; ++c) {
      int64_t e = ids[t] * hidden + c;
      int64_t b = e >> 8;
      if (b != cached) {
        const uint8_t* blk = wq + b * bb;
        if (kind == 12)
          orc_dequant_q4k_block(blk, y, layout);
        else if (kind == 13)
          orc_dequant_q5k_block(blk, y);
        else
          orc_dequant_q6k_block(blk, y);
        cached = b;
      }
      orc_store(out, t * hidden + c, y[e & 255], out_dtype);
    }
}

/* src/hip_ops.hip:553-563 (embedding_kernel<uint16_t>) */
void orc_embedding_u16(const int64_t* ids, const uint16_t* table, int64_t tokens, int64_t hidden,
                       int table_bf16, void* out, int out_dtype) {
  for (int64_t t = 0; t < tokens; ++t)
    for (int64_t c = 0; c < hidden; ++c) {
      uint16_t h = table[ids[t] * hidden + c];
      float v = table_bf16 ? orc_bf16_to_f32(h) : orc_fp16_to_f32(h);
      orc_store(out, t * hidden + c, v, out_dtype);
    }
}

/* ---- norms -------------------------------------------------------------- */

/* tools/ref_top5.cpp:243-252 (double accumulation; inv rounded to float);
 * operation order of src/hip_ops.hip:373-393: out = (x * inv) * w. */
static void rms_row(const float* xr, const void* w, float* o, int64_t hidden, float eps, int dtype) {
  double s = 0.0;
  for (int64_t i = 0; i < hidden; ++i) s += (double)xr[i] * xr[i];
  float inv = (float)(1.0 / sqrt(s / (double)hidden + (double)eps));
  for (int64_t i = 0; i < hidden; ++i) o[i] = xr[i] * inv * orc_load(w, i, dtype);
}

void orc_rms_norm(const void* x, const void* w, void* out, int64_t rows, int64_t hidden, float eps,
                  int dtype) {
  float* xr = (float*)malloc(sizeof(float) * (size_t)hidden * 2);
  float* o = xr + hidden;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < hidden; ++i) xr[i] = orc_load(x, r * hidden + i, dtype);
    rms_row(xr, w, o, hidden, eps, dtype);
    for (int64_t i = 0; i < hidden; ++i) orc_store(out, r * hidden + i, o[i], dtype);
  }
  free(xr);
}

/* src/hip_ops.hip:395-417 + tools/ref_top5.cpp:346-348: residual <- x + residual
 * (stored, i.e. rounded to the storage dtype), then RMSNorm of the stored row. */
void orc_rms_norm_add(const void* x, void* residual, const void* w, void* out, int64_t rows,
                      int64_t hidden, float eps, int dtype) {
  float* rr = (float*)malloc(sizeof(float) * (size_t)hidden * 2);
  float* o = rr + hidden;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < hidden; ++i) {
      float v = orc_load(x, r * hidden + i, dtype) + orc_load(residual, r * hidden + i, dtype);
      orc_store(residual, r * hidden + i, v, dtype);
      rr[i] = orc_load(residual, r * hidden + i, dtype);
    }
    rms_row(rr, w, o, hidden, eps, dtype);
    for (int64_t i = 0; i < hidden; ++i) orc_store(out, r * hidden + i, o[i], dtype);
  }
  free(rr);
}

/* ---- SwiGLU ------------------------------------------------------------- */

/* src/hip_ops.hip:419-429 and tools/ref_top5.cpp:576:
 * out[r,c] = g / (1 + expf(-g)) * u, g = gu[r, c], u = gu[r, I + c]. */
void orc_silu_and_mul(const void* gate_up, void* out, int64_t rows, int64_t inter, int dtype) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < inter; ++c) {
      float g = orc_load(gate_up, r * 2 * inter + c, dtype);
      float u = orc_load(gate_up, r * 2 * inter + inter + c, dtype);
      orc_store(out, r * inter + c, g / (1.0f + expf(-g)) * u, dtype);
    }
}

/* ---- RoPE --------------------------------------------------------------- */

/* NeoX rotate-half on one head held in fp32, src/hip_ops.hip:431-450 and
 * tools/ref_top5.cpp:409-426: angle = float(pos) * inv_freq[d]. */
static void rope_head(float* hv, float pos, const float* inv_freq, int head_dim) {
  int half = head_dim / 2;
  for (int d = 0; d < half; ++d) {
    float fr = pos * inv_freq[d];
    float c = cosf(fr), s = sinf(fr);
    float x1 = hv[d], x2 = hv[d + half];
    hv[d] = x1 * c - x2 * s;
    hv[d + half] = x2 * c + x1 * s;
  }
}

void orc_rope(void* data, const int64_t* positions, int64_t tokens, int heads, int head_dim,
              int64_t stride, const float* inv_freq, int dtype) {
  float* hv = (float*)malloc(sizeof(float) * (size_t)head_dim);
  for (int64_t t = 0; t < tokens; ++t)
    for (int h = 0; h < heads; ++h) {
      int64_t base = t * stride + (int64_t)h * head_dim;
      for (int d = 0; d < head_dim; ++d) hv[d] = orc_load(data, base + d, dtype);
      rope_head(hv, (float)positions[t], inv_freq, head_dim);
      for (int d = 0; d < head_dim; ++d) orc_store(data, base + d, hv[d], dtype);
    }
  free(hv);
}

/* Qwen3 QK-norm then RoPE, src/model.cpp:774-778 (rms_norm rows = T*heads,
 * hidden = head_dim, tools/ref_top5.cpp:398-407), then rope as above.  The
 * normalised head stays fp32 between the two steps; one rounding at the end.
 * A NULL gamma skips the norm for that tensor. */
static void qk_one(void* buf, const int64_t* positions, const void* gw, const float* inv_freq,
                   int64_t tokens, int heads, int head_dim, int64_t stride, float eps, int dtype,
                   const float* bias) {
  float* hv = (float*)malloc(sizeof(float) * (size_t)head_dim * 2);
  float* nv = hv + head_dim;
  for (int64_t t = 0; t < tokens; ++t)
    for (int h = 0; h < heads; ++h) {
      int64_t base = t * stride + (int64_t)h * head_dim;
      for (int d = 0; d < head_dim; ++d) hv[d] = orc_load(buf, base + d, dtype);
      if (bias)
        for (int d = 0; d < head_dim; ++d) hv[d] += bias[(int64_t)h * head_dim + d];
      if (gw) {
        rms_row(hv, gw, nv, head_dim, eps, dtype);
        memcpy(hv, nv, sizeof(float) * (size_t)head_dim);
      }
      rope_head(hv, (float)positions[t], inv_freq, head_dim);
      for (int d = 0; d < head_dim; ++d) orc_store(buf, base + d, hv[d], dtype);
    }
  free(hv);
}

void orc_qk_norm_rope(void* q, void* k, const int64_t* positions, const void* q_w, const void* k_w,
                      const float* inv_freq, int64_t tokens, int q_heads, int kv_heads, int head_dim,
                      int64_t q_stride, int64_t k_stride, float eps, int dtype) {
  if (q && q_heads > 0) qk_one(q, positions, q_w, inv_freq, tokens, q_heads, head_dim, q_stride, eps, dtype, NULL);
  if (k && kv_heads > 0) qk_one(k, positions, k_w, inv_freq, tokens, kv_heads, head_dim, k_stride, eps, dtype, NULL);
}

/* ---- qkv bias ------------------------------------------------------------- */

/* src/hip_ops.hip:366-371 (add_bias_kernel, called by hip_add_bias_inplace :688-692):
 * x[r, c] += bias[c], fp32 bias, one rounding to the storage type. */
void orc_add_bias(void* x, const float* bias, int64_t rows, int64_t cols, int64_t stride, int dtype) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c)
      orc_store(x, r * stride + c, orc_load(x, r * stride + c, dtype) + bias[c], dtype);
}

/* src/model.cpp:768-778 then hip_store_kv (:780-781): qkv bias on q, k and v, QK-norm
 * (gammas optional), RoPE, then the KV store, as one op.  The biased head stays fp32
 * through the norm and the rotation (in fp32 storage the reference's separate passes
 * give the same bits); v + v_bias is rounded once into v_cache and v is not written.
 * bias: fp32 [q_heads*hd | kv_heads*hd | kv_heads*hd] or NULL. */
void orc_qkv_bias_qk_norm_rope_store_kv(void* q, void* k, const void* v, const float* bias,
                                        const int64_t* positions, const void* q_w, const void* k_w,
                                        const float* inv_freq, int64_t tokens, int q_heads, int kv_heads,
                                        int head_dim, int64_t q_stride, int64_t k_stride, int64_t v_stride,
                                        float eps, void* k_cache, void* v_cache, const int32_t* slot_mapping,
                                        int dtype) {
  const int64_t qn = (int64_t)q_heads * head_dim, kn = (int64_t)kv_heads * head_dim;
  if (q && q_heads > 0)
    qk_one(q, positions, q_w, inv_freq, tokens, q_heads, head_dim, q_stride, eps, dtype, bias);
  qk_one(k, positions, k_w, inv_freq, tokens, kv_heads, head_dim, k_stride, eps, dtype, bias ? bias + qn : NULL);
  for (int64_t t = 0; t < tokens; ++t) {
    const int32_t slot = slot_mapping[t];
    if (slot < 0) continue;
    for (int64_t c = 0; c < kn; ++c) {
      orc_store(k_cache, (int64_t)slot * kn + c, orc_load(k, t * k_stride + c, dtype), dtype);
      const float vv = orc_load(v, t * v_stride + c, dtype) + (bias ? bias[qn + kn + c] : 0.0f);
      orc_store(v_cache, (int64_t)slot * kn + c, vv, dtype);
    }
  }
}

/* ---- Q8 activation row scale (for the Q8_0 GEMM) ------------------------ */

/* src/hip_ops.hip:205-217: max |x| over the row, scale = 127 / max or 0. */
void orc_q8_row_scale(const void* x, float* scale, int64_t rows, int64_t hidden, int dtype) {
  for (int64_t r = 0; r < rows; ++r) {
    float mx = 0.0f;
    for (int64_t i = 0; i < hidden; ++i) mx = fmaxf(mx, fabsf(orc_load(x, r * hidden + i, dtype)));
    scale[r] = mx > 1e-8f ? 127.0f / mx : 0.0f;
  }
}

/* src/hip_ops.hip:244-245: (int8_t)fminf(127, fmaxf(-127, v * as)), a C cast
 * (truncation toward zero). */
void orc_q8_quantize(const void* x, const float* scale, int8_t* q, int64_t rows, int64_t hidden, int dtype) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t i = 0; i < hidden; ++i) {
      const float v = orc_load(x, r * hidden + i, dtype) * scale[r];
      q[r * hidden + i] = (int8_t)fminf(127.0f, fmaxf(-127.0f, v));
    }
}

/* ---- Q8_0 GEMM ------------------------------------------------------------ */

/* src/hip_ops.hip:639-686 (hip_matmul_q8).  With I[r,c,b] the exact integer dot
 * of block b, I = sum_{i in b} xq[r,i] * w8[c,i], and adq[r] = 1.0f / scale[r]
 * (0 when scale[r] is 0, :309 and :358), the reference's tile kernel (:221-312)
 * and GEMV (:317-364) both compute
 *     out[r,c] = (sum_b ws[c,b] * I[r,c,b]) * adq[r]
 * in fp32, summing the block terms in different orders (16-element halves in the
 * tile kernel, 4-element lane chunks then 32 lanes in the GEMV).  This function
 * returns that value in double, where each term ws*I is exact (11 x 20 bits) and
 * the sum carries at most a 2^-53 relative error, together with
 *     err[r,c] = (k/32 + 4) * 2^-24 * sum_b |ws[c,b] * I[r,c,b]| * adq[r],
 * a bound on the error of any fp32 recursive summation of the 2*k/32 half-block
 * terms followed by the adq product: the tolerance for a fp32 implementation. */
void orc_matmul_q8_i8(const int8_t* xq, const float* scale, const uint8_t* w8, const uint16_t* ws, int64_t m,
                      int64_t n, int64_t k, double* out, double* err) {
  const int64_t nblk = k / 32;
  for (int64_t r = 0; r < m; ++r) {
    const float adq = scale[r] > 0.0f ? 1.0f / scale[r] : 0.0f;
    for (int64_t c = 0; c < n; ++c) {
      double sum = 0.0, mag = 0.0;
      for (int64_t b = 0; b < nblk; ++b) {
        int32_t dot = 0;
        for (int i = 0; i < 32; ++i)
          dot += (int32_t)xq[r * k + b * 32 + i] * (int32_t)(int8_t)w8[c * k + b * 32 + i];
        const double t = (double)orc_fp16_to_f32(ws[c * nblk + b]) * (double)dot;
        sum += t;
        mag += fabs(t);
      }
      out[r * n + c] = sum * (double)adq;
      err[r * n + c] = (double)(nblk + 4) * ldexp(1.0, -24) * mag * (double)adq;
    }
  }
}

/* The weight element w(c, i) = element c*k + i of the flat weight array, decoded
 * exactly to fp32: fp32 rows (src/hip_ops.hip:43-64 matmul_kernel<float>), fp16/bf16
 * rows widened (matmul_kernel<uint16_t>, wt_load :38-41), or K-quant superblocks over
 * the flat index (matmul_qk_kernel :577-598 via qk_w :184-193; Q4_K in `layout`). */
static void dense_weight_row(const void* w, int w_format, int layout, int64_t c, int64_t k, float* row) {
  if (w_format == 0) {
    for (int64_t i = 0; i < k; ++i) row[i] = ((const float*)w)[c * k + i];
  } else if (w_format == 1 || w_format == 2) {
    for (int64_t i = 0; i < k; ++i) {
      const uint16_t h = ((const uint16_t*)w)[c * k + i];
      row[i] = w_format == 2 ? orc_bf16_to_f32(h) : orc_fp16_to_f32(h);
    }
  } else {
    const int64_t bb = w_format == 12 ? 144 : (w_format == 13 ? 176 : 210);
    float y[256];
    int64_t cached = -1;
    for (int64_t i = 0; i < k; ++i) {
      const int64_t e = c * k + i, b = e >> 8;
      if (b != cached) {
        const uint8_t* blk = (const uint8_t*)w + b * bb;
        if (w_format == 12)
          orc_dequant_q4k_block(blk, y, layout);
        else if (w_format == 13)
          orc_dequant_q5k_block(blk, y);
        else
          orc_dequant_q6k_block(blk, y);
        cached = b;
      }
      row[i] = y[e & 255];
    }
  }
}

/* hip_matmul / hip_matmul_u16 / hip_matmul_qk (src/hip_ops.hip:746-777):
 * out[r][c] = sum_i x[r][i] * w(c, i), x [m,k] in x_dtype.  The reference sums the
 * fp32 products in k order (16-element tiles, one output per thread); this sums
 * them in double, and err[r][c] = (k + 2) u sum_i |x w| bounds every fp32 summation
 * order (one rounding per product and per addition). */
void orc_matmul_w(const void* x, int x_dtype, const void* w, int w_format, int layout, int64_t m, int64_t n,
                  int64_t k, double* out, double* err) {
  float* row = (float*)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1));
  float* xr = (float*)malloc(sizeof(float) * (size_t)(m * k > 0 ? m * k : 1));
  for (int64_t i = 0; i < m * k; ++i) xr[i] = orc_load(x, i, x_dtype);
  for (int64_t c = 0; c < n; ++c) {
    dense_weight_row(w, w_format, layout, c, k, row);
    for (int64_t r = 0; r < m; ++r) {
      double sum = 0.0, mag = 0.0;
      for (int64_t i = 0; i < k; ++i) {
        const double t = (double)xr[r * k + i] * (double)row[i];
        sum += t;
        mag += fabs(t);
      }
      out[r * n + c] = sum;
      err[r * n + c] = (double)(k + 2) * ldexp(1.0, -24) * mag;
    }
  }
  free(row);
  free(xr);
}

/* src/hip_ops.hip:611-619 (gather_rows_kernel): out[r][c] = rows[indices[r]][c], a copy
 * in the storage dtype. */
void orc_gather_rows(const void* rows, const int32_t* indices, int64_t cols, int64_t out_rows, void* out,
                     int dtype) {
  const size_t e = dtype == ORC_F32 ? 4 : 2;
  for (int64_t r = 0; r < out_rows; ++r)
    memcpy((char*)out + (size_t)(r * cols) * e, (const char*)rows + (size_t)((int64_t)indices[r] * cols) * e,
           (size_t)cols * e);
}

/* The reference's whole hip_matmul_q8 on activations x [m,k] in `dtype`: row
 * scales (:205-217), quantization (:244-245), then orc_matmul_q8_i8.  scale_out
 * [m] and xq_out [m,k] receive the intermediate values when not NULL. */
void orc_matmul_q8(const void* x, int dtype, const uint8_t* w8, const uint16_t* ws, int64_t m, int64_t n, int64_t k,
                   double* out, double* err, float* scale_out, int8_t* xq_out) {
  float* sc = scale_out ? scale_out : (float*)malloc(sizeof(float) * (size_t)(m > 0 ? m : 1));
  int8_t* q = xq_out ? xq_out : (int8_t*)malloc((size_t)(m * k > 0 ? m * k : 1));
  orc_q8_row_scale(x, sc, m, k, dtype);
  orc_q8_quantize(x, sc, q, m, k, dtype);
  orc_matmul_q8_i8(q, sc, w8, ws, m, n, k, out, err);
  if (!xq_out) free(q);
  if (!scale_out) free(sc);
}

/* ---- KV cache store and paged attention ----------------------------------- */

/* src/hip_ops.hip:452-466 (store_kv_kernel): for each token t with
 * slot = slot_mapping[t] >= 0, k_cache[slot, :] = key[t, :] and
 * v_cache[slot, :] = value[t, :] (kv_heads * head_dim values, a plain copy in
 * the storage dtype); slots < 0 are skipped. */
void orc_store_kv(const void* key, const void* value, void* k_cache, void* v_cache, const int32_t* slot_mapping,
                  int64_t tokens, int kv_heads, int head_dim, int dtype) {
  const int64_t d = (int64_t)kv_heads * head_dim;
  const size_t e = dtype == ORC_F32 ? 4 : 2;
  for (int64_t t = 0; t < tokens; ++t) {
    const int32_t slot = slot_mapping[t];
    if (slot < 0) continue;
    memcpy((char*)k_cache + (size_t)slot * d * e, (const char*)key + (size_t)t * d * e, (size_t)d * e);
    memcpy((char*)v_cache + (size_t)slot * d * e, (const char*)value + (size_t)t * d * e, (size_t)d * e);
  }
}

/* src/hip_ops.hip:473-550 (paged_attention_kernel).  For query token t and head
 * h: seq = query_seq[t], L = query_key_len[t], kv head h / (q_heads / kv_heads);
 * key j < L lives at cache row block_tables[seq * max_blocks + j / block_size] *
 * block_size + j % block_size (rows of kv_heads * head_dim values, :468-471);
 * out = softmax_j(scale * q . K_j) . V, and 0 when L <= 0 (:488-491).  The
 * reference accumulates an online softmax over 64-key chunks in fp32; this
 * computes the same quantity in double (max-subtracted exp, one division) and
 * rounds once to `dtype`.  out_exact (optional) receives the double values and
 * vmax (optional) max |V| over the attended keys per (t, h), the scale of the
 * tolerances. */
void orc_paged_attention(const void* q, void* out, const void* k_cache, const void* v_cache, const int32_t* query_seq,
                         const int32_t* query_key_len, const int32_t* block_tables, int64_t tokens, int q_heads,
                         int kv_heads, int head_dim, int block_size, int max_blocks, float scale, int dtype,
                         double* out_exact, float* vmax) {
  const int group = q_heads / kv_heads;
  const int64_t kv_stride = (int64_t)kv_heads * head_dim, q_stride = (int64_t)q_heads * head_dim;
  int64_t cap = 64;
  double* sc = (double*)malloc(sizeof(double) * (size_t)cap);
  double* acc = (double*)malloc(sizeof(double) * (size_t)head_dim);
  for (int64_t t = 0; t < tokens; ++t) {
    const int32_t L = query_key_len[t];
    const int32_t seq = query_seq[t];
    if (L > cap) {
      cap = L;
      sc = (double*)realloc(sc, sizeof(double) * (size_t)cap);
    }
    for (int h = 0; h < q_heads; ++h) {
      const int kvh = h / group;
      const int64_t qo = t * q_stride + (int64_t)h * head_dim;
      double m = -INFINITY, vm = 0.0;
      for (int32_t j = 0; j < L; ++j) {
        const int64_t row = (int64_t)block_tables[(int64_t)seq * max_blocks + j / block_size] * block_size +
                            j % block_size;
        double dot = 0.0;
        for (int d = 0; d < head_dim; ++d)
          dot += (double)orc_load(q, qo + d, dtype) * (double)orc_load(k_cache, row * kv_stride + kvh * head_dim + d, dtype);
        sc[j] = dot * (double)scale;
        if (sc[j] > m) m = sc[j];
      }
      double sum = 0.0;
      for (int d = 0; d < head_dim; ++d) acc[d] = 0.0;
      for (int32_t j = 0; j < L; ++j) {
        const int64_t row = (int64_t)block_tables[(int64_t)seq * max_blocks + j / block_size] * block_size +
                            j % block_size;
        const double p = exp(sc[j] - m);
        sum += p;
        for (int d = 0; d < head_dim; ++d) {
          const double v = (double)orc_load(v_cache, row * kv_stride + kvh * head_dim + d, dtype);
          acc[d] += p * v;
          if (fabs(v) > vm) vm = fabs(v);
        }
      }
      for (int d = 0; d < head_dim; ++d) {
        const double o = L > 0 ? acc[d] / sum : 0.0;
        orc_store(out, qo + d, (float)o, dtype);
        if (out_exact) out_exact[qo + d] = o;
      }
      if (vmax) vmax[t * q_heads + h] = (float)vm;
    }
  }
  free(acc);
  free(sc);
}

/* ---- layer-0 embedding + residual-add + RMSNorm -------------------------- */

void orc_embedding_rms_norm(const int64_t* ids, int format, const void* table, const void* scales, int64_t tokens,
                            int64_t hidden, const void* w, void* residual, void* out, float eps, int dtype) {
  float* emb = (float*)malloc(sizeof(float) * (size_t)(tokens * hidden));
  if (format == 0)
    orc_embedding_q8_split(ids, (const uint8_t*)table, (const uint16_t*)scales, tokens, hidden, emb, ORC_F32);
  else
    orc_embedding_q8_blocks(ids, (const uint8_t*)table, tokens, hidden, emb, ORC_F32);
  /* the gather's value in the storage dtype, then the layer-0 add onto zeros */
  void* x = malloc((size_t)(tokens * hidden) * (dtype == ORC_F32 ? 4 : 2));
  for (int64_t i = 0; i < tokens * hidden; ++i) {
    orc_store(x, i, emb[i], dtype);
    orc_store(residual, i, 0.0f, dtype);
  }
  orc_rms_norm_add(x, residual, w, out, tokens, hidden, eps, dtype);
  free(x);
  free(emb);
}

/* src/hip_ops.hip:813-844 (moe_route_kernel), one row at a time as the reference's
 * single thread does it. */
void orc_moe_route(const float* logits, int64_t rows, int E, int K, int norm, int32_t* idx, float* score) {
  double* pr = (double*)malloc(sizeof(double) * (size_t)E);
  int* ix = (int*)malloc(sizeof(int) * (size_t)E);
  for (int64_t t = 0; t < rows; ++t) {
    const float* lg = logits + t * E;
    double maxv = -1e300;
    for (int i = 0; i < E; ++i) maxv = maxv > (double)lg[i] ? maxv : (double)lg[i];
    double sum = 0.0;
    for (int i = 0; i < E; ++i) {
      pr[i] = exp((double)lg[i] - maxv);
      sum += pr[i];
    }
    const double inv = 1.0 / sum;
    for (int i = 0; i < E; ++i) {
      pr[i] *= inv;
      ix[i] = i;
    }
    for (int i = 0; i < K; ++i) {
      int best = i;
      for (int j = i + 1; j < E; ++j)
        if (pr[j] > pr[best]) best = j;
      const double tp = pr[i];
      pr[i] = pr[best];
      pr[best] = tp;
      const int ti = ix[i];
      ix[i] = ix[best];
      ix[best] = ti;
      idx[t * K + i] = ix[i];
      score[t * K + i] = (float)pr[i];
    }
    if (norm) {
      double s = 0.0;
      for (int i = 0; i < K; ++i) s += pr[i];
      const double sinv = 1.0 / s;
      for (int i = 0; i < K; ++i) score[t * K + i] = (float)(pr[i] * sinv);
    }
  }
  free(pr);
  free(ix);
}

/* src/hip_ops.hip:861-893 (moe_ffn_kernel) in double, with a first-order fp32 bound. */
void orc_moe_ffn(const void* x, int x_dtype, const int32_t* idx, const float* score, const uint16_t* gu,
                 const uint16_t* dn, int w_bf16, const int32_t* slot_of, int64_t rows, int64_t H, int64_t I,
                 int64_t K, int64_t slots, const double* out_in, double* out, double* err) {
  const double u = 1.0 / 16777216.0; /* 2^-24 */
  double* xv = (double*)malloc(sizeof(double) * (size_t)H);
  double* y = (double*)malloc(sizeof(double) * (size_t)I);
  double* ey = (double*)malloc(sizeof(double) * (size_t)I);
  double* res = (double*)malloc(sizeof(double) * (size_t)H);
  double* eres = (double*)malloc(sizeof(double) * (size_t)H);
  double* wv = (double*)malloc(sizeof(double) * (size_t)H);
#define ORC_W(p, i) ((double)(w_bf16 ? orc_bf16_to_f32((p)[i]) : orc_fp16_to_f32((p)[i])))
  for (int64_t t = 0; t < rows; ++t) {
    for (int64_t i = 0; i < H; ++i) {
      xv[i] = (double)orc_load(x, t * H + i, x_dtype);
      res[i] = 0.0;
      eres[i] = 0.0;
      wv[i] = 0.0;
    }
    for (int64_t k = 0; k < K; ++k) {
      const double w = (double)score[t * K + k];
      if (w == 0.0) continue;
      const int32_t sl = slot_of[idx[t * K + k]];
      if (sl < 0 || sl >= slots) continue;
      const uint16_t* g = gu + (int64_t)sl * 2 * I * H;
      const uint16_t* d = dn + (int64_t)sl * H * I;
      for (int64_t j = 0; j < I; ++j) {
        double gg = 0.0, uu = 0.0, ag = 0.0, au = 0.0;
        for (int64_t i = 0; i < H; ++i) {
          const double a = xv[i] * ORC_W(g, j * H + i), b = xv[i] * ORC_W(g, (I + j) * H + i);
          gg += a;
          uu += b;
          ag += fabs(a);
          au += fabs(b);
        }
        const double eg = (double)(H + 2) * u * ag, eu = (double)(H + 2) * u * au;
        const double sg = 1.0 / (1.0 + exp(-gg));
        const double silu = gg * sg;
        const double dsilu = sg * (1.0 + gg * (1.0 - sg));
        y[j] = silu * uu;
        ey[j] = fabs(dsilu * uu) * eg + fabs(silu) * eu + 8.0 * u * fabs(y[j]);
      }
      for (int64_t o = 0; o < H; ++o) {
        double v = 0.0, av = 0.0, prop = 0.0;
        for (int64_t j = 0; j < I; ++j) {
          const double dw = ORC_W(d, o * I + j);
          v += y[j] * dw;
          av += fabs(y[j] * dw);
          prop += fabs(dw) * ey[j];
        }
        const double ev = (double)(I + 2) * u * av + prop;
        res[o] += w * v;
        eres[o] += fabs(w) * ev;
        wv[o] += fabs(w * v);
      }
    }
    for (int64_t o = 0; o < H; ++o) {
      const double r = out_in[t * H + o] + res[o];
      out[t * H + o] = r;
      err[t * H + o] = eres[o] + (double)(K + 1) * u * wv[o] + u * (fabs(r) + fabs(res[o]));
    }
  }
#undef ORC_W
  free(xv);
  free(y);
  free(ey);
  free(res);
  free(eres);
  free(wv);
}
