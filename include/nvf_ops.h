/*
 * nvf_ops.h -- C ABI of the MI355X (gfx950) fused per-layer ops library
 * (libnvf_ops.so).  Plain pointers and sizes only.
 *
 * Two families of entry points:
 *
 *  1. Drop-in replacements with the exact names and parameter lists of the
 *     Nano_vLLM_cpp op interface (include/nanovllm/hip_ops.hpp), given C
 *     linkage.  Semantics kept: fp32 activations, device pointers owned by the
 *     caller, launches on the legacy null stream, early return for a zero or
 *     negative size, and on a launch failure a message on stderr followed by
 *     exit(1) (the reference's HIP_CHECK, include/nanovllm/common.hpp:14-23).
 *
 *  2. Typed entry points (nvf_*): fp32 / fp16 / bf16 storage (NVF_F32 /
 *     NVF_F16 / NVF_BF16), an explicit stream (a hipStream_t passed as void*;
 *     NULL = null stream) and an int status (NVF_OK or a negative code;
 *     nvf_last_error() describes the last failure of the calling thread).
 *     Math is fp32 on upcast inputs, rounded once to the storage type.
 *
 * No entry point allocates device memory or synchronises the stream.
 * Calls are asynchronous; concurrent calls on different streams are safe.
 */
#ifndef NVF_OPS_H
#define NVF_OPS_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum nvf_dtype { NVF_F32 = 0, NVF_F16 = 1, NVF_BF16 = 2 };

/* Nibble order inside a Q4_K superblock.  GGML is the GGUF on-disk order
 * (src/gguf.cpp:477-496, tools/ref_top5.cpp:140-165,
 * shaders/vulkan/embedding_qk.comp:54-55).  HIP_LEGACY reproduces the
 * reference's device decoder qk_w_q4 (src/hip_ops.hip:130-140). */
enum nvf_qk_layout { NVF_QK_LAYOUT_GGML = 0, NVF_QK_LAYOUT_HIP_LEGACY = 1 };

/* K-quant kinds, the GGML type ids the reference passes (src/model.cpp:163). */
enum nvf_qk_kind { NVF_Q4_K = 12, NVF_Q5_K = 13, NVF_Q6_K = 14 };

/* Weight formats of nvf_matmul (row-major [n][k] element arrays; the K-quants are
 * 256-element superblocks over the flat element index, src/hip_ops.hip:184-193). */
enum nvf_w_format {
  NVF_W_F32 = 0,
  NVF_W_F16 = 1,
  NVF_W_BF16 = 2,
  NVF_W_Q4_K = 12,
  NVF_W_Q5_K = 13,
  NVF_W_Q6_K = 14
};

/* Table formats of the fused embedding entry point. */
enum nvf_emb_format {
  NVF_EMB_Q8_0 = 0,        /* split planes: table = int8 [V*H], scales = fp16 [V*H/32] */
  NVF_EMB_Q8_0_BLOCKS = 1, /* 34-byte GGUF blocks */
  NVF_EMB_Q4_K = 12,       /* GGML nibble order */
  NVF_EMB_Q5_K = 13,
  NVF_EMB_Q6_K = 14
};

enum nvf_status {
  NVF_OK = 0,
  NVF_ERR_INVALID = -1, /* bad size, dtype, kind, layout or NULL pointer */
  NVF_ERR_LAUNCH = -2   /* the HIP launch failed */
};

/* ---- 1. drop-in replacements (include/nanovllm/hip_ops.hpp) ------------- */

/* hip_ops.hpp:14 -- out = x * rsqrt(mean(x^2) + eps) * weight per row.
 * out == x allowed (Qwen3 QK-norm in place, src/model.cpp:774-775). */
void hip_rms_norm(const float* x, const float* weight, float* out, int rows, int hidden, float eps);

/* hip_ops.hpp:15 -- residual <- x + residual; out = RMSNorm(residual) * weight. */
void hip_rms_norm_add(const float* x, float* residual, const float* weight, float* out, int rows, int hidden,
                      float eps);

/* hip_ops.hpp:12 -- x[r,c] += bias[c] over rows x cols (the Qwen2.5 qkv bias,
 * src/model.cpp:768-772; kernel src/hip_ops.hip:366-371). */
void hip_add_bias_inplace(float* x, const float* bias, int rows, int cols);

/* hip_ops.hpp:17 -- out[r,c] = silu(gate_up[r,c]) * gate_up[r,I+c]. */
void hip_silu_and_mul(const float* gate_up, float* out, int rows, int intermediate);

/* hip_ops.hpp:19-20 -- NeoX RoPE in place on data[t*stride + h*head_dim + d]. */
void hip_rope_inplace(float* data, const int64_t* positions, int tokens, int heads, int head_dim, int64_t stride,
                      const float* inv_freq);

/* hip_ops.hpp:30 -- fp32 table gather. */
void hip_embedding(const int64_t* ids, const float* table, int tokens, int hidden, float* out);

/* hip_ops.hpp:31 -- F16 / BF16 table gather to fp32. */
void hip_embedding_u16(const int64_t* ids, const uint16_t* table, int tokens, int hidden, float* out,
                       bool table_bf16);

/* hip_ops.hpp:32 -- Q8_0 gather from split planes (int8 w8 + fp16 scale plane ws,
 * src/model.cpp:394-404) to fp32; bit-exact. */
void hip_embedding_q8(const int64_t* ids, const uint8_t* w8, const uint16_t* ws, int tokens, int hidden,
                      float* out);

/* hip_ops.hpp:33 -- K-quant gather (kind 12/13/14) to fp32.  Q4_K in GGML (GGUF) order by
 * default, which differs from the reference's device decoder (src/hip_ops.hip:130-140);
 * nvf_set_dropin_q4k_layout(NVF_QK_LAYOUT_HIP_LEGACY) makes it read the reference's order. */
void hip_embedding_qk(const int64_t* ids, const uint8_t* wq, int tokens, int hidden, float* out, int kind);

/* hip_ops.hpp:8 -- out[m,n] = x[m,k] . w[n,k]^T, fp32 weights. */
void hip_matmul(const float* x, const float* w, int m, int n, int k, float* out);

/* hip_ops.hpp:9 -- as hip_matmul with fp16 (w_bf16 false) or bf16 weights, widened exactly. */
void hip_matmul_u16(const float* x, const uint16_t* w, int m, int n, int k, float* out, bool w_bf16);

/* hip_ops.hpp:11 -- as hip_matmul with K-quant weights (kind 12/13/14: Q4_K/Q5_K/Q6_K
 * superblocks over the flat [n][k] element index), decoded exactly.  Q4_K nibble order
 * as hip_embedding_qk (nvf_set_dropin_q4k_layout).  Needs n*k a multiple of 256. */
void hip_matmul_qk(const float* x, const uint8_t* wq, int m, int n, int k, float* out, int kind);

/* hip_ops.hpp:34 -- out[r,:] = rows[indices[r],:] for r < out_rows (the last-token rows
 * ahead of the LM head, src/model.cpp:839).  rows_count > 0 bounds the indices: an index
 * outside [0, rows_count) gives a NaN row (the reference ignores rows_count and reads it). */
void hip_gather_rows(const float* rows, const int32_t* indices, int rows_count, int cols, int out_rows, float* out);

/* hip_ops.hpp:37 -- top-K experts per row of fp32 router logits [rows, E]: softmax in
 * double, the reference's selection sort (its tie order), optional renormalisation of the
 * K scores; idx [rows, K] int32, score [rows, K] fp32.  E <= 4096. */
void hip_moe_route(const float* logits, int rows, int E, int K, bool norm, int32_t* idx, float* score);

/* hip_ops.hpp:38-40 -- out[t] += sum_k score[t,k] * down(silu(gate(x[t])) * up(x[t])) for the
 * expert slot slot_of[idx[t,k]] (gu slot [2I, H] gate rows then up rows, dn slot [H, I],
 * fp16 or bf16), pairs with score 0 skipped.  Expert slots below 65536; a pair whose slot
 * is negative or beyond is skipped (the reference would read outside its slot arrays).
 * Runs through a static 64 MiB device scratch in row chunks: allocates nothing. */
void hip_moe_ffn(const float* x, const int32_t* idx, const float* score, const uint16_t* gu, const uint16_t* dn,
                 const int32_t* slot_of, int rows, int H, int I, int K, bool bf16, float* out);

/* hip_ops.hpp:41 -- dst[i] += src[i], fp32. */
void hip_add_inplace(float* dst, const float* src, size_t n);

/* hip_ops.hpp:42 -- dst[t, c] *= 1 / (1 + expf(-s[t])), fp32 (Qwen2-MoE shared-expert gate). */
void hip_scale_rows_sigmoid(float* dst, const float* s, int rows, int cols);

/* No reference counterpart: selects the Q4_K nibble order hip_embedding_qk reads,
 * process-wide (NVF_QK_LAYOUT_GGML, the default, or NVF_QK_LAYOUT_HIP_LEGACY). */
int nvf_set_dropin_q4k_layout(int layout);

/* hip_ops.hpp:10 -- Q8_0 GEMM, out[m,n] = x[m,k] * dequant(w8, ws)^T in fp32, with
 * the reference's per-row int8 activation quantization (hip_ops.hip:639-686).
 * k must be a multiple of 32; the quantized rows go to a grow-only device scratch
 * (the reference's own policy, hip_ops.hip:642-648). */
void hip_matmul_q8(const float* x, const uint8_t* w8, const uint16_t* ws, int m, int n, int k, float* out);

/* hip_ops.hpp:22-23 -- k_cache[slot_mapping[t], :] = key[t, :], same for values
 * (rows of kv_heads * head_dim fp32 values); slots < 0 are skipped. */
void hip_store_kv(const float* key, const float* value, float* k_cache, float* v_cache, const int32_t* slot_mapping,
                  int tokens, int kv_heads, int head_dim);

/* hip_ops.hpp:25-28 -- paged attention over the fp32 cache [blocks * block_size,
 * kv_heads, head_dim]: token t attends the first query_key_len[t] keys of
 * sequence query_seq[t] (block_tables[seq * max_blocks + j / block_size]);
 * out = softmax(scale * q . K) . V per head, 0 when query_key_len[t] <= 0.
 * head_dim <= 256.  Like the reference's kernel, this trusts its metadata: the
 * table entries a query reaches must name cache blocks, and query_key_len <=
 * block_size * max_blocks (the caller's prepare_prefill/prepare_decode builds them so). */
void hip_paged_attention(const float* q, float* out, const float* k_cache, const float* v_cache,
                         const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                         int tokens, int q_heads, int kv_heads, int head_dim, int block_size, int max_blocks,
                         float scale);

/* ---- 2. typed entry points ---------------------------------------------- */

/* Residual-add + RMSNorm (replaces hip_rms_norm_add, hip_ops.hpp:15).  All four
 * tensors in `dtype`; residual is read and written back rounded to `dtype`,
 * and the norm is taken over that stored row. */
int nvf_rms_norm_add(const void* x, void* residual, const void* weight, void* out, int64_t rows, int64_t hidden,
                     float eps, int dtype, void* stream);

/* RMSNorm (replaces hip_rms_norm, hip_ops.hpp:14); out == x allowed. */
int nvf_rms_norm(const void* x, const void* weight, void* out, int64_t rows, int64_t hidden, float eps, int dtype,
                 void* stream);

/* RMSNorm (residual NULL) or residual-add + RMSNorm (residual given) that also
 * writes the Q8_0 GEMM's activation quantizer outputs, fused: row_scale[r] =
 * 127 / max|out[r,:]| (0 when that max <= 1e-8) -- the reference computes it
 * in a separate pass, q8_row_scale_kernel (src/hip_ops.hip:205-217, called by
 * hip_matmul_q8 :639-686) -- and, when q_out is given, the int8 row
 * q = (int8)clamp(out * row_scale, +-127) (truncation, :244-245).  out may be
 * NULL when q_out is given.  row_scale: fp32 [rows]; q_out: int8 [rows, hidden]. */
int nvf_rms_norm_q8(const void* x, void* residual, const void* weight, void* out, float* row_scale, int8_t* q_out,
                    int64_t rows, int64_t hidden, float eps, int dtype, void* stream);

/* SiLU(gate) * up over gate_up [rows, 2*inter] -> out [rows, inter]
 * (replaces hip_silu_and_mul, hip_ops.hpp:17). */
int nvf_silu_and_mul(const void* gate_up, void* out, int64_t rows, int64_t inter, int dtype, void* stream);

/* Fused Qwen3 QK-norm + NeoX RoPE on q and k in one launch (composition of
 * hip_rms_norm at src/model.cpp:774-775 and hip_rope_inplace at :777-778).
 * q: [tokens, q_stride], heads at h*head_dim; k: [tokens, k_stride].  q_w / k_w
 * are [head_dim] gammas in `dtype`; pass both NULL for plain RoPE.  k may be NULL
 * when kv_heads == 0.  inv_freq: device fp32 [head_dim/2].  The normalised head
 * stays fp32 until the rotated value is stored. */
int nvf_qk_norm_rope(void* q, void* k, const int64_t* positions, const void* q_w, const void* k_w,
                     const float* inv_freq, int64_t tokens, int q_heads, int kv_heads, int head_dim,
                     int64_t q_stride, int64_t k_stride, float eps, int dtype, void* stream);

/* nvf_qk_norm_rope followed by nvf_store_kv(k, v, ...) in one launch where the shape
 * allows (head_dim 64/128/256, 16-byte aligned rows, kv_heads * head_dim <= 4096), the
 * two launches otherwise; the results are those of the pair.  The reference calls the
 * RoPE (src/model.cpp:777-778) and then the store (hip_store_kv, hip_ops.hpp:22-23)
 * on the same k and v; this fuses that sequence, so it has no single counterpart.
 * k is rotated in place as well as stored; slot < 0 skips a token's store. */
int nvf_qk_norm_rope_store_kv(void* q, void* k, const void* v, const int64_t* positions, const void* q_w,
                              const void* k_w, const float* inv_freq, int64_t tokens, int q_heads, int kv_heads,
                              int head_dim, int64_t q_stride, int64_t k_stride, int64_t v_stride, float eps,
                              void* k_cache, void* v_cache, const int32_t* slot_mapping, int dtype, void* stream);

/* nvf_qk_norm_rope_store_kv with the Qwen2.5 qkv bias added first: the reference's
 * src/model.cpp:768-778 sequence (hip_add_bias_inplace on q, k and v, then QK-norm,
 * RoPE and hip_store_kv) in one launch where the shape allows.  qkv_bias: device fp32
 * [q_heads*head_dim | kv_heads*head_dim | kv_heads*head_dim] (16-byte aligned for the
 * fused launch); NULL = no bias (then exactly nvf_qk_norm_rope_store_kv).  The bias
 * is added in fp32 to the loaded value, which stays fp32 through the norm and the
 * rotation (one rounding at the store; in fp32 storage this equals the reference's
 * separate passes bit for bit).  q and k hold the biased, rotated heads afterwards;
 * v + v_bias goes to v_cache and the v tensor itself is left unchanged. */
int nvf_qkv_bias_qk_norm_rope_store_kv(void* q, void* k, const void* v, const float* qkv_bias,
                                       const int64_t* positions, const void* q_w, const void* k_w,
                                       const float* inv_freq, int64_t tokens, int q_heads, int kv_heads, int head_dim,
                                       int64_t q_stride, int64_t k_stride, int64_t v_stride, float eps, void* k_cache,
                                       void* v_cache, const int32_t* slot_mapping, int dtype, void* stream);

/* x[r*stride + c] += bias[c] for r < rows, c < cols (replaces hip_add_bias_inplace,
 * hip_ops.hpp:12): x in `dtype`, bias fp32 [cols], one rounding per element. */
int nvf_add_bias(void* x, const float* bias, int64_t rows, int64_t cols, int64_t stride, int dtype, void* stream);

/* GEMM on dense or K-quant weights (replaces hip_matmul, hip_matmul_u16 and
 * hip_matmul_qk, hip_ops.hpp:8-11): out[m,n] (out_dtype) = x[m,k] (x_dtype) . w^T with
 * w in `w_format` (nvf_w_format; Q4_K nibble order `qk_layout`) decoded exactly to fp32,
 * fp32 products and sums on the matrix cores.  Any k; K-quants: n*k a multiple of 256,
 * Q4_K/Q5_K blocks 16-byte aligned, Q6_K 2-byte.  Vector loads when x and dense
 * weights are 16-byte aligned, element-wise staging otherwise. */
int nvf_matmul(const void* x, int x_dtype, const void* w, int w_format, int qk_layout, int64_t m, int64_t n,
               int64_t k, void* out, int out_dtype, void* stream);

/* Row gather (replaces hip_gather_rows, hip_ops.hpp:34): out[r,:] = rows[indices[r],:]
 * for r < out_rows, cols wide, rows and out in `dtype` (a bit-exact copy).
 * rows_count > 0: an index outside [0, rows_count) gives a NaN row instead of a
 * read; rows_count <= 0: indices are trusted, as the reference does. */
int nvf_gather_rows(const void* rows, const int32_t* indices, int64_t rows_count, int64_t cols, int64_t out_rows,
                    void* out, int dtype, void* stream);

/* MoE routing (replaces hip_moe_route, hip_ops.hpp:37) on `stream`; E <= 4096, K <= E. */
int nvf_moe_route(const float* logits, int64_t rows, int64_t E, int64_t K, int norm, int32_t* idx, float* score,
                  void* stream);

/* Workspace bytes nvf_moe_ffn_ws needs for rows x K (token, expert) pairs. */
int64_t nvf_moe_ffn_workspace_size(int64_t rows, int64_t H, int64_t I, int64_t K, int64_t slots);

/* MoE expert FFN (replaces hip_moe_ffn, hip_ops.hpp:38-40): x [rows, H] in x_dtype, out
 * [rows, H] in out_dtype (out += ...), expert weights fp16 (w_bf16 0) or bf16, expert slots
 * in [0, slots) (slots <= 65536; other pairs and pairs with score 0 are skipped).  The pairs
 * are grouped by slot and run as matrix products on the fp32 matrix cores; the k results of
 * a token are summed in k order.  `work`: 16-byte aligned, nvf_moe_ffn_workspace_size bytes. */
int nvf_moe_ffn_ws(const void* x, int x_dtype, const int32_t* idx, const float* score, const void* gu,
                   const void* dn, int w_bf16, const int32_t* slot_of, int64_t rows, int64_t H, int64_t I, int64_t K,
                   int64_t slots, void* out, int out_dtype, void* work, int64_t work_bytes, void* stream);

/* dst[i] += src[i] (replaces hip_add_inplace, hip_ops.hpp:41), fp32, on `stream`. */
int nvf_add_inplace(float* dst, const float* src, int64_t n, void* stream);

/* dst[t, c] *= 1 / (1 + expf(-s[t])) (replaces hip_scale_rows_sigmoid, hip_ops.hpp:42). */
int nvf_scale_rows_sigmoid(float* dst, const float* s, int64_t rows, int64_t cols, void* stream);

/* Q8_0 gather, split planes (as hip_embedding_q8) -> out in out_dtype.
 * vocab > 0: ids outside [0, vocab) produce a NaN row instead of a read;
 * vocab <= 0: ids are trusted (the reference validates them on the host,
 * src/model.cpp:712-716). */
int nvf_embedding_q8_0(const int64_t* ids, const uint8_t* w8, const uint16_t* ws, int64_t tokens, int64_t hidden,
                       int64_t vocab, void* out, int out_dtype, void* stream);

/* Q8_0 gather straight from interleaved 34-byte GGUF blocks
 * ([fp16 d][32 x int8], src/gguf.cpp:353-362) -> out in out_dtype. */
int nvf_embedding_q8_0_blocks(const int64_t* ids, const uint8_t* blocks, int64_t tokens, int64_t hidden,
                              int64_t vocab, void* out, int out_dtype, void* stream);

/* K-quant gather (replaces hip_embedding_qk, hip_ops.hpp:33): kind NVF_Q4_K /
 * NVF_Q5_K / NVF_Q6_K, layout applies to Q4_K only. */
int nvf_embedding_qk(const int64_t* ids, const uint8_t* wq, int64_t tokens, int64_t hidden, int64_t vocab,
                     int kind, int layout, void* out, int out_dtype, void* stream);

/* Plain table gather: table in table_dtype, out in out_dtype
 * (replaces hip_embedding / hip_embedding_u16, hip_ops.hpp:30-31). */
int nvf_embedding(const int64_t* ids, const void* table, int64_t tokens, int64_t hidden, int64_t vocab,
                  int table_dtype, void* out, int out_dtype, void* stream);

/* Layer-0 embedding gather fused with residual-add + RMSNorm: the reference
 * gathers into `hidden` (src/model.cpp:756) and then calls
 * hip_rms_norm_add(hidden, residual, input_layernorm, norm) on its zero-filled
 * residual (:762).  Here residual <- emb + 0 and out <- RMSNorm(residual) * weight
 * are written directly; the gathered row never goes to memory.  residual, out
 * and weight in `dtype`; hidden <= 16 * 64 * (16 / element size). */
int nvf_embedding_rms_norm(const int64_t* ids, int format, const void* table, const void* scales, int64_t tokens,
                           int64_t hidden, int64_t vocab, const void* weight, void* residual, void* out, float eps,
                           int dtype, void* stream);

/* SwiGLU (as nvf_silu_and_mul, replacing hip_silu_and_mul, hip_ops.hpp:17) that also
 * writes the Q8_0 down projection's quantized input: row_scale[r] = 127 / max|v[r,:]|
 * (0 when the maximum is <= 1e-8) and q_out[r,i] = (int8) min(127, max(-127,
 * v[r,i] * row_scale[r])), v the SwiGLU output as stored in `dtype` -- the
 * reference's q8_row_scale_kernel and quantizer (hip_ops.hip:205-217, :244-245)
 * applied to silu_and_mul's output (hip_ops.hip:419-429).  out may be NULL. */
int nvf_silu_and_mul_q8(const void* gate_up, void* out, float* row_scale, int8_t* q_out, int64_t rows,
                        int64_t inter, int dtype, void* stream);

/* Splits nblocks interleaved 34-byte GGUF Q8_0 blocks (fp16 scale, then 32
 * int8 values; the bytes GGUFLoader::load_q8_0 reads, src/gguf.cpp:353-362) into
 * the planes nvf_matmul_q8_0 and nvf_embedding_q8_0 read: w8 [nblocks*32] and
 * ws [nblocks] fp16 bits.  Replaces the host loop upload_q8_split
 * (src/model.cpp:396-405), so the raw GGUF bytes are uploaded as they are.
 * blocks and w8 16-byte aligned, ws 4-byte aligned. */
int nvf_q8_0_split_blocks(const uint8_t* blocks, int64_t nblocks, int8_t* w8, uint16_t* ws, void* stream);

/* Per-row int8 quantization of activations for the Q8_0 GEMM: row_scale[r] =
 * 127 / max|x[r,:]| (0 when the maximum is <= 1e-8) and xq[r,i] = (int8)
 * min(127, max(-127, x[r,i] * row_scale[r])), truncating -- q8_row_scale_kernel
 * (hip_ops.hip:205-217) and its GEMMs' quantizer (hip_ops.hip:244-245). */
int nvf_q8_quantize_rows(const void* x, float* row_scale, int8_t* xq, int64_t rows, int64_t k, int dtype,
                         void* stream);

/* Q8_0 GEMM on pre-quantized activations (replaces hip_matmul_q8, hip_ops.hpp:10,
 * after nvf_q8_quantize_rows or nvf_rms_norm_q8): out[r,c] = (sum_b ws[c,b] *
 * sum_{i in b} xq[r,i] * w8[c,i]) / row_scale[r] (0 where row_scale is 0), written
 * as out_dtype.  w8 [n,k] int8 and xq [m,k] 16-byte aligned; ws [n,k/32] fp16;
 * k a multiple of 32. */
int nvf_matmul_q8_0(const int8_t* xq, const float* row_scale, const uint8_t* w8, const uint16_t* ws, int64_t m,
                    int64_t n, int64_t k, void* out, int out_dtype, void* stream);

/* nvf_matmul_q8_0 with a caller workspace for split-K (no counterpart in the
 * reference; its hip_matmul_q8 tiles the output only): when the output has too
 * few 128 x 128 tiles to fill the GPU (e.g. decode batches of a few hundred rows
 * against 3584-wide outputs), K is cut into ranges whose fp32 partial sums are
 * summed in order by a reduction.  workspace (16-byte aligned) of workspace_bytes
 * >= nvf_matmul_q8_0_workspace_size(m, n, k) enables it; NULL or too small runs
 * unsplit.  Same results within the fp32 summation bound. */
int nvf_matmul_q8_0_ws(const int8_t* xq, const float* row_scale, const uint8_t* w8, const uint16_t* ws, int64_t m,
                       int64_t n, int64_t k, void* out, int out_dtype, void* workspace, int64_t workspace_bytes,
                       void* stream);

/* Bytes of workspace nvf_matmul_q8_0_ws uses for this shape (0: it would not split). */
/* Decode GEMV (m <= 16 rows) on fp activations, no separate quantize pass: out [m, n]
 * (dtype) = the Q8_0 product of the rows quantized as nvf_q8_quantize_rows would
 * (act 0: x [m, k]) or as nvf_silu_and_mul_q8 would (act 1: x = [gate | up] rows
 * [m, 2k], the SwiGLU taken first).  Each workgroup quantizes the rows into its own
 * LDS while the weights stream in, so the int8 rows and scales, and the result, are
 * bit-identical to the separate quantize launch followed by nvf_matmul_q8_0.  This
 * fuses what the reference does in one call, hip_matmul_q8's quantizer and GEMV
 * (src/hip_ops.hip:205-217, :317-364), and for act 1 also hip_silu_and_mul before it
 * (src/model.cpp:830).  x: 16-byte aligned rows, x_stride elements apart (>= k, or
 * 2k for act 1); out must not overlap x.  m > 16, overlapping out, or rows too long
 * for the workgroup's LDS: NVF_ERR_INVALID. */
int nvf_matmul_q8_0_act(const void* x, int64_t x_stride, int act, const uint8_t* w8, const uint16_t* ws, int64_t m,
                        int64_t n, int64_t k, void* out, int dtype, void* stream);

/* Decode GEMV (m <= 16 rows) with residual-add + RMSNorm + quantizer in its prologue:
 * out [m, n] = the Q8_0 product of the rows nvf_rms_norm_q8 would produce, bit for bit.
 * With residual [m, k]: v = round(x + residual), written to residual_out [m, k]
 * (which must not overlap x or residual: every workgroup reads them); without
 * (both NULL): v = x.  out must not overlap x, residual or residual_out.  Then round(v / rms(v) * norm_weight) quantized per row.  Each
 * workgroup repeats the norm in its prologue, its sum of squares in nvf_rms_norm_q8's
 * own order.  This fuses the reference's hip_rms_norm_add then the next Q8_0 matmul
 * (src/model.cpp:762 then :764, :787 then :829; src/hip_ops.hip:395-417, :639-680) into
 * one launch; the in-place residual becomes a second buffer (alternate two across the
 * layer's two norms).  x rows x_stride elements apart; all pointers 16-byte aligned
 * (ws 2); k % 32 == 0 and k * dtype bytes <= 64 KiB; else NVF_ERR_INVALID. */
int nvf_matmul_q8_0_rms(const void* x, int64_t x_stride, const void* residual, void* residual_out,
                        const void* norm_weight, float eps, const uint8_t* w8, const uint16_t* ws, int64_t m, int64_t n,
                        int64_t k, void* out, int dtype, void* stream);

int64_t nvf_matmul_q8_0_workspace_size(int64_t m, int64_t n, int64_t k);

/* KV store (replaces hip_store_kv, hip_ops.hpp:22-23) with the cache in `dtype`;
 * key / value rows are key_stride / value_stride elements apart (>= kv_heads *
 * head_dim), so views into a packed qkv row work. */
int nvf_store_kv(const void* key, const void* value, void* k_cache, void* v_cache, const int32_t* slot_mapping,
                 int64_t tokens, int kv_heads, int head_dim, int64_t key_stride, int64_t value_stride, int dtype,
                 void* stream);

/* Paged attention (replaces hip_paged_attention, hip_ops.hpp:25-28) with q, out and
 * the cache in `dtype` (fp32 math, one rounding of the output).  q rows are
 * q_stride elements apart (>= q_heads * head_dim); out is [tokens, q_heads *
 * head_dim].  q_heads % kv_heads == 0, head_dim <= 256.  max_query_len is a
 * scheduling hint: 1 promises one query token per sequence (a decode batch) and
 * skips the prefill tiles; 0 (unknown) or any other value runs both paths. */
int nvf_paged_attention(const void* q, void* out, const void* k_cache, const void* v_cache, const int32_t* query_seq,
                        const int32_t* query_key_len, const int32_t* block_tables, int64_t tokens, int q_heads,
                        int kv_heads, int head_dim, int block_size, int max_blocks, float scale, int64_t q_stride,
                        int64_t max_query_len, int dtype, void* stream);

/* nvf_paged_attention with a caller workspace for split attention (no counterpart
 * in the reference, whose kernel -- hip_ops.hip:452-550 -- walks each (token,
 * head)'s keys in one workgroup): when the call has too little work to fill the
 * GPU -- few decode (token, kv head) pairs, or few 128-token prefill tiles, over
 * long contexts -- each one's keys are split into ranges processed in parallel
 * and merged.  workspace (16-byte aligned) of workspace_bytes >=
 * nvf_paged_attention_workspace_size(...) enables it; NULL or too small runs
 * unsplit.  Same results to fp32 rounding. */
int nvf_paged_attention_ws(const void* q, void* out, const void* k_cache, const void* v_cache,
                           const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                           int64_t tokens, int q_heads, int kv_heads, int head_dim, int block_size, int max_blocks,
                           float scale, int64_t q_stride, int64_t max_query_len, void* workspace,
                           int64_t workspace_bytes, int dtype, void* stream);

/* nvf_paged_attention_ws for a batch whose token layout the caller also holds on the
 * host: cu_seqlens_host [num_seqs + 1] (0, then each sequence's end; the last entry is
 * tokens), the packing that query_seq describes on the device (the reference's
 * cu_seqlens_q, include/nanovllm/context.hpp:8-25, built on the host by
 * ModelRunner::prepare_prefill, src/model_runner.cpp:43-128).  When every sequence
 * starts at a multiple of 128 tokens, every 128-token tile holds one sequence and the
 * launch for tokens of mixed tiles is not made.  Results equal nvf_paged_attention_ws's.
 * Contract: cu_seqlens_host must describe exactly the packing of query_seq (token t
 * belongs to sequence s iff cu_seqlens_host[s] <= t < cu_seqlens_host[s + 1]).  Only
 * its monotonicity and end points are checked; if it claims 128-aligned sequences
 * that query_seq does not have, the tokens of the mixed tiles are left unwritten. */
int nvf_paged_attention_seqs_ws(const void* q, void* out, const void* k_cache, const void* v_cache,
                                const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                                const int32_t* cu_seqlens_host, int num_seqs, int64_t tokens, int q_heads,
                                int kv_heads, int head_dim, int block_size, int max_blocks, float scale,
                                int64_t q_stride, int64_t max_query_len, void* workspace, int64_t workspace_bytes,
                                int dtype, void* stream);

/* nvf_paged_attention_ws with the caller's schedule for the decode kernel (no
 * counterpart in the reference): token_order (device int32 [tokens], a permutation of
 * 0 .. tokens-1) names the token each decode workgroup computes.  Results equal
 * nvf_paged_attention_ws's; only the time depends on it.  (Not a permutation: an entry
 * outside 0 .. tokens-1 computes nothing and reads or writes no memory for it; the
 * output of a token the order does not name is unspecified.)  For a decode batch with
 * ragged contexts, nvf_decode_token_order gives one that balances the GPU's 8 XCDs
 * (workgroup id mod 8 is its XCD); the engine holds the key counts on the host
 * (src/model_runner.cpp:122) and uploads the order with them.  The prefill tiles
 * ignore it. */
int nvf_paged_attention_order_ws(const void* q, void* out, const void* k_cache, const void* v_cache,
                                 const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                                 const int32_t* token_order, int64_t tokens, int q_heads, int kv_heads, int head_dim,
                                 int block_size, int max_blocks, float scale, int64_t q_stride, int64_t max_query_len,
                                 void* workspace, int64_t workspace_bytes, int dtype, void* stream);

/* Host only: order_host [tokens] = the tokens sorted by key_len_host (descending, ties
 * by index) and dealt over 8 XCDs in snake order, for nvf_paged_attention_order_ws. */
int nvf_decode_token_order(const int32_t* key_len_host, int64_t tokens, int32_t* order_host);

/* Bytes of workspace nvf_paged_attention_ws uses for this shape and max_query_len
 * hint (0: it would not split).  The context bound is block_size * max_blocks. */
int64_t nvf_paged_attention_workspace_size(int64_t tokens, int q_heads, int kv_heads, int head_dim, int block_size,
                                           int max_blocks, int64_t max_query_len);

/* No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  nvf_paged_attention_ws with the split workspace taken from a static
 * device scratch of nvf_paged_attention_noalloc_max_bytes() (32 MiB) that each GPU
 * holds until the process ends; nothing is allocated.  A call whose split needs more
 * (nvf_paged_attention_workspace_size > that) fails with NVF_ERR_INVALID.  Results
 * equal nvf_paged_attention_ws's with a workspace.  All calls on one GPU share the
 * scratch: calls that overlap on one GPU (several streams or threads) race. */
int nvf_paged_attention_noalloc(const void* q, void* out, const void* k_cache, const void* v_cache,
                                const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                                int64_t tokens, int q_heads, int kv_heads, int head_dim, int block_size,
                                int max_blocks, float scale, int64_t q_stride, int64_t max_query_len, int dtype,
                                void* stream);
int64_t nvf_paged_attention_noalloc_max_bytes(void);

/* Host helper: inv_freq[i] = (float)(1 / theta^(2i/head_dim)) in double, the
 * table Qwen3Model builds in its constructor (src/model.cpp:416-420).
 * out is HOST memory of head_dim/2 floats. */
int nvf_rope_inv_freq(double theta, int head_dim, float* out);

/* Copies `bytes` (a multiple of 16; 16-byte aligned pointers) with the same
 * 16-byte non-temporal loads/stores the op kernels use.  No counterpart in the
 * reference: it is the attainable-bandwidth and traffic-counter reference that
 * the op kernels' HBM figures are calibrated against. */
int nvf_stream_copy(void* dst, const void* src, int64_t bytes, void* stream);

/* Measurement reference with the Q8_0 gather's read:write mix (no reference
 * counterpart): dst[16 i .. 16 i + 15] = src[8 i .. 8 i + 7] twice, for
 * src_bytes / 8 items (dst holds 2 * src_bytes; 16-byte aligned dst, 8-byte src). */
int nvf_stream_expand(void* dst, const void* src, int64_t src_bytes, void* stream);

/* Text of the calling thread's last failure ("" if none). */
const char* nvf_last_error(void);

/* ABI version, bumped on any signature change. */
int nvf_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* NVF_OPS_H */
