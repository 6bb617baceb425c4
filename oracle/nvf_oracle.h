/*
 * nvf_oracle.h -- CPU restatement of Nano_vLLM_cpp's fused per-layer ops.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP kernels in
 * nano_vllm_cpp_amd/csrc.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product library never links it
 * and has no CPU fallback.
 *
 * Every function states the reference file:line whose loop it restates
 * (paths relative to the Nano_vLLM_cpp source tree).  All arithmetic is scalar,
 * single-threaded C compiled -O2 (the reference's own -O2, CMakeLists.txt:33),
 * with fp32 math on upcast inputs and one rounding to the storage dtype.
 *
 * Parity pins (each checked in tests/test_oracle.py):
 *   fp16/bf16 codecs ......... exhaustive 65536-code round trip vs numpy + RNE
 *                              midpoint cases
 *   Q8_0 ..................... hand vector vulkanised/test_gguf2vk.py:77-83;
 *                              split-plane == 34 B-block equivalence;
 *                              block split: hand-built block bytes and the
 *                              split -> join round trip
 *   Q4_K / Q6_K .............. bytes produced by the reference's own
 *                              gguf.cpp dequant (oracle/_ref, tests/golden)
 *   Q5_K ..................... closed forms on hand-built blocks (the
 *                              reference's host Q5_K decoder lives inside
 *                              tools/ref_top5.cpp's main program and cannot
 *                              be linked); on the GPU box also compared with
 *                              the reference's own hip_embedding_qk kind 13
 *   RMSNorm (+add) ........... closed form test/test_basic.cpp:23-31,
 *                              homogeneity and gamma-linearity invariants
 *   RoPE / QK-norm ........... pos=0 identity, pair-norm preservation,
 *                              rotate(p) then rotate(-p) identity, composition
 *   qkv bias ................. closed form x + b (one rounding); the fused bias +
 *                              norm + RoPE + store equals, in fp32 storage, the
 *                              composition add_bias -> qk_norm_rope -> store_kv,
 *                              and with a zero bias the unbiased op
 *   SiLU*up .................. silu(0)=0, silu(g)-silu(-g)=g, double-exp
 *                              brute force
 *   Q8 row scale / quantize .. closed forms (the row maximum maps to +-127,
 *                              zero rows give scale 0), truncation toward zero
 *   embedding + layer-0 norm . equal to the composition gather ->
 *                              rms_norm_add with a zero residual
 *   paged attention .......... one key -> that V row; q = 0 -> the mean of the
 *                              attended V rows; L = 0 -> zeros; invariant under a
 *                              permutation of physical blocks; equal to a dense
 *                              numpy softmax(q K^T) V; on the GPU box within the
 *                              tolerance of the reference's hip_paged_attention
 *   KV store ................. a copy: rows land at their slots, slot -1 skipped
 *   dense / K-quant GEMM ..... exact on power-of-two weights and small integers
 *                              (every partial sum exact); equal to a textbook
 *                              matmul of the dequantized weights (numpy); on the
 *                              GPU box the reference's own hip_matmul* lie within
 *                              the bound
 *   row gather ............... a copy: equal to numpy fancy indexing
 *   Q8_0 GEMM ................ exact on power-of-two scales against a textbook
 *                              matmul of the dequantized weights; the error bound
 *                              holds for fp32 sums in every order; on the GPU box
 *                              the reference's own hip_matmul_q8 lies within it
 */
#ifndef NVF_ORACLE_H
#define NVF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2 };
enum { ORC_QK_LAYOUT_GGML = 0, ORC_QK_LAYOUT_HIP_LEGACY = 1 };

float orc_fp16_to_f32(uint16_t h);
uint16_t orc_f32_to_fp16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);

/* element loads/stores through a dtype tag (storage -> fp32 -> storage) */
float orc_load(const void* p, int64_t i, int dtype);
void orc_store(void* p, int64_t i, float v, int dtype);

void orc_inv_freq(double theta, int head_dim, float* out);

void orc_dequant_q4k_block(const uint8_t* blk, float* y, int layout);
void orc_dequant_q5k_block(const uint8_t* blk, float* y);
void orc_dequant_q6k_block(const uint8_t* blk, float* y);

void orc_embedding_q8_split(const int64_t* ids, const uint8_t* w8, const uint16_t* ws, int64_t tokens,
                            int64_t hidden, void* out, int out_dtype);
void orc_embedding_q8_blocks(const int64_t* ids, const uint8_t* blocks, int64_t tokens, int64_t hidden,
                             void* out, int out_dtype);
/* src/model.cpp:396-405 (upload_q8_split): 34-byte blocks -> w8 [nblocks*32], ws [nblocks]. */
void orc_q8_0_split_blocks(const uint8_t* blocks, int64_t nblocks, int8_t* w8, uint16_t* ws);
void orc_embedding_qk(const int64_t* ids, const uint8_t* wq, int64_t tokens, int64_t hidden, int kind,
                      int layout, void* out, int out_dtype);
void orc_embedding_u16(const int64_t* ids, const uint16_t* table, int64_t tokens, int64_t hidden,
                       int table_bf16, void* out, int out_dtype);

void orc_rms_norm(const void* x, const void* w, void* out, int64_t rows, int64_t hidden, float eps,
                  int dtype);
void orc_rms_norm_add(const void* x, void* residual, const void* w, void* out, int64_t rows,
                      int64_t hidden, float eps, int dtype);
void orc_silu_and_mul(const void* gate_up, void* out, int64_t rows, int64_t inter, int dtype);
void orc_rope(void* data, const int64_t* positions, int64_t tokens, int heads, int head_dim,
              int64_t stride, const float* inv_freq, int dtype);
void orc_qk_norm_rope(void* q, void* k, const int64_t* positions, const void* q_w, const void* k_w,
                      const float* inv_freq, int64_t tokens, int q_heads, int kv_heads, int head_dim,
                      int64_t q_stride, int64_t k_stride, float eps, int dtype);

/* src/hip_ops.hip:366-371 (add_bias_kernel): x[r*stride + c] += bias[c], one rounding.
 * orc_qkv_bias_qk_norm_rope_store_kv: src/model.cpp:768-781 (bias on q, k, v; QK-norm;
 * RoPE; KV store) as one op with the biased head kept in fp32 until its store. */
void orc_add_bias(void* x, const float* bias, int64_t rows, int64_t cols, int64_t stride, int dtype);
void orc_qkv_bias_qk_norm_rope_store_kv(void* q, void* k, const void* v, const float* bias,
                                        const int64_t* positions, const void* q_w, const void* k_w,
                                        const float* inv_freq, int64_t tokens, int q_heads, int kv_heads,
                                        int head_dim, int64_t q_stride, int64_t k_stride, int64_t v_stride,
                                        float eps, void* k_cache, void* v_cache, const int32_t* slot_mapping,
                                        int dtype);

/* src/hip_ops.hip:205-217 (q8_row_scale_kernel): scale[r] = 127 / max|x[r,:]|,
 * 0 when the maximum is <= 1e-8; and the int8 values its GEMM forms from them,
 * src/hip_ops.hip:244-245: q = (int8)min(127, max(-127, x * scale)) (truncation). */
void orc_q8_row_scale(const void* x, float* scale, int64_t rows, int64_t hidden, int dtype);
void orc_q8_quantize(const void* x, const float* scale, int8_t* q, int64_t rows, int64_t hidden, int dtype);

/* Q8_0 GEMM, src/hip_ops.hip:639-686: out[r,c] = (sum_b ws[c,b] * I[r,c,b]) /
 * scale[r] with exact integer block dots I, in double, and err[r,c], the fp32
 * recursive-summation bound (k/32 + 4) * 2^-24 * sum_b |ws*I| / scale[r]. */
void orc_matmul_q8_i8(const int8_t* xq, const float* scale, const uint8_t* w8, const uint16_t* ws, int64_t m,
                      int64_t n, int64_t k, double* out, double* err);
void orc_matmul_q8(const void* x, int dtype, const uint8_t* w8, const uint16_t* ws, int64_t m, int64_t n, int64_t k,
                   double* out, double* err, float* scale_out, int8_t* xq_out);

/* Dense / K-quant weight GEMM, src/hip_ops.hip:43-64 and :577-598 (qk_w :184-193):
 * out[r,c] = sum_i x[r,i] * w(c,i), w decoded exactly (fp32 / fp16 / bf16 rows, Q4_K in
 * `layout`, Q5_K, Q6_K), in double; err[r,c] = (k + 2) * 2^-24 * sum_i |x w|, which covers
 * fp32 sums of the products in any order. */
void orc_matmul_w(const void* x, int x_dtype, const void* w, int w_format, int layout, int64_t m, int64_t n,
                  int64_t k, double* out, double* err);

/* src/hip_ops.hip:611-619 (gather_rows_kernel): out[r,:] = rows[indices[r],:]. */
void orc_gather_rows(const void* rows, const int32_t* indices, int64_t cols, int64_t out_rows, void* out,
                     int dtype);

/* src/hip_ops.hip:813-844 (moe_route_kernel): softmax of each logits row in double, the
 * top K by the reference's selection sort (swaps included), scores rounded to fp32,
 * renormalised over the K when `norm`. */
void orc_moe_route(const float* logits, int64_t rows, int E, int K, int norm, int32_t* idx, float* score);

/* src/hip_ops.hip:861-893 (moe_ffn_kernel): out[t,o] = out_in[t,o] + sum_k w_k v_k[o] with
 * v = dn_e . (silu(gu_e[:I] . x) * (gu_e[I:] . x)), e = slot_of[idx[t,k]], for w != 0 and
 * 0 <= e < slots; in double over the exact inputs.  err[t,o]: a first-order bound on an fp32
 * evaluation in any summation order -- each product's (n + 2) 2^-24 sum |terms|, carried
 * through SiLU(g) * u by its derivatives plus 8 2^-24 |y| for expf and the divide, through
 * the down product, the k-sum (K 2^-24 sum |w v|) and the final add. */
void orc_moe_ffn(const void* x, int x_dtype, const int32_t* idx, const float* score, const uint16_t* gu,
                 const uint16_t* dn, int w_bf16, const int32_t* slot_of, int64_t rows, int64_t H, int64_t I,
                 int64_t K, int64_t slots, const double* out_in, double* out, double* err);

/* KV store (src/hip_ops.hip:452-466) and paged attention (:468-550): see the
 * definitions for the exact indexing; attention is computed in double and
 * rounded once to dtype (out_exact / vmax optional). */
void orc_store_kv(const void* key, const void* value, void* k_cache, void* v_cache, const int32_t* slot_mapping,
                  int64_t tokens, int kv_heads, int head_dim, int dtype);
void orc_paged_attention(const void* q, void* out, const void* k_cache, const void* v_cache, const int32_t* query_seq,
                         const int32_t* query_key_len, const int32_t* block_tables, int64_t tokens, int q_heads,
                         int kv_heads, int head_dim, int block_size, int max_blocks, float scale, int dtype,
                         double* out_exact, float* vmax);

/* Layer-0 embedding + residual-add + RMSNorm (src/model.cpp:756 then :762 with
 * the zero-filled residual): residual = emb + 0, out = RMSNorm(residual) * w.
 * format: 0 = Q8_0 split planes (table = w8, scales = ws), 1 = Q8_0 blocks. */
void orc_embedding_rms_norm(const int64_t* ids, int format, const void* table, const void* scales, int64_t tokens,
                            int64_t hidden, const void* w, void* residual, void* out, float eps, int dtype);

#ifdef __cplusplus
}
#endif
#endif
