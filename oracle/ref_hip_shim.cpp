// C-ABI shim over the reference's own HIP launchers (src/hip_ops.hip, C++
// linkage, include/nanovllm/hip_ops.hpp:10-34), compiled for gfx950 from the
// reference sources where they lie (see Makefile) into oracle/_ref/.
// TEST INFRASTRUCTURE ONLY: GPU parity tests use it as a second checker beside
// the C oracle.  Each wrapper launches on the null stream like the reference
// and synchronises so the caller can read the result.
#include <cstdint>

#include "nanovllm/hip_ops.hpp"

extern "C" {
void ref_hip_rms_norm(const float* x, const float* w, float* out, int rows, int hidden, float eps) {
  hip_rms_norm(x, w, out, rows, hidden, eps);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_rms_norm_add(const float* x, float* residual, const float* w, float* out, int rows, int hidden,
                          float eps) {
  hip_rms_norm_add(x, residual, w, out, rows, hidden, eps);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_silu_and_mul(const float* gate_up, float* out, int rows, int inter) {
  hip_silu_and_mul(gate_up, out, rows, inter);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_rope_inplace(float* data, const int64_t* positions, int tokens, int heads, int head_dim,
                          int64_t stride, const float* inv_freq) {
  hip_rope_inplace(data, positions, tokens, heads, head_dim, stride, inv_freq);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_embedding_q8(const int64_t* ids, const uint8_t* w8, const uint16_t* ws, int tokens, int hidden,
                          float* out) {
  hip_embedding_q8(ids, w8, ws, tokens, hidden, out);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_embedding_qk(const int64_t* ids, const uint8_t* wq, int tokens, int hidden, float* out, int kind) {
  hip_embedding_qk(ids, wq, tokens, hidden, out, kind);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_matmul_q8(const float* x, const uint8_t* w8, const uint16_t* ws, int m, int n, int k, float* out) {
  hip_matmul_q8(x, w8, ws, m, n, k, out);
  HIP_CHECK(hipDeviceSynchronize());
}
// No synchronisation: for timing the reference's GEMM with events.
void ref_hip_matmul_q8_async(const float* x, const uint8_t* w8, const uint16_t* ws, int m, int n, int k,
                             float* out) {
  hip_matmul_q8(x, w8, ws, m, n, k, out);
}
void ref_hip_matmul(const float* x, const float* w, int m, int n, int k, float* out) {
  hip_matmul(x, w, m, n, k, out);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_matmul_u16(const float* x, const uint16_t* w, int m, int n, int k, float* out, bool w_bf16) {
  hip_matmul_u16(x, w, m, n, k, out, w_bf16);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_matmul_qk(const float* x, const uint8_t* wq, int m, int n, int k, float* out, int kind) {
  hip_matmul_qk(x, wq, m, n, k, out, kind);
  HIP_CHECK(hipDeviceSynchronize());
}
// No synchronisation, for timing: w_format 0 fp32, 1 fp16, 2 bf16, 12/13/14 K-quants.
void ref_hip_matmul_any_async(int w_format, const float* x, const void* w, int m, int n, int k, float* out) {
  if (w_format == 0)
    hip_matmul(x, static_cast<const float*>(w), m, n, k, out);
  else if (w_format == 1 || w_format == 2)
    hip_matmul_u16(x, static_cast<const uint16_t*>(w), m, n, k, out, w_format == 2);
  else
    hip_matmul_qk(x, static_cast<const uint8_t*>(w), m, n, k, out, w_format);
}
void ref_hip_gather_rows(const float* rows, const int32_t* indices, int rows_count, int cols, int out_rows,
                         float* out) {
  hip_gather_rows(rows, indices, rows_count, cols, out_rows, out);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_moe_route(const float* logits, int rows, int E, int K, bool norm, int32_t* idx, float* score) {
  hip_moe_route(logits, rows, E, K, norm, idx, score);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_moe_ffn(const float* x, const int32_t* idx, const float* score, const uint16_t* gu, const uint16_t* dn,
                     const int32_t* slot_of, int rows, int H, int I, int K, bool bf16, float* out) {
  hip_moe_ffn(x, idx, score, gu, dn, slot_of, rows, H, I, K, bf16, out);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_add_inplace(float* dst, const float* src, size_t n) {
  hip_add_inplace(dst, src, n);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_scale_rows_sigmoid(float* dst, const float* s, int rows, int cols) {
  hip_scale_rows_sigmoid(dst, s, rows, cols);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_store_kv(const float* key, const float* value, float* k_cache, float* v_cache, const int32_t* slots,
                      int tokens, int kv_heads, int head_dim) {
  hip_store_kv(key, value, k_cache, v_cache, slots, tokens, kv_heads, head_dim);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_add_bias_inplace(float* x, const float* bias, int rows, int cols) {
  hip_add_bias_inplace(x, bias, rows, cols);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_paged_attention(const float* q, float* out, const float* k_cache, const float* v_cache,
                             const int32_t* query_seq, const int32_t* query_key_len, const int32_t* block_tables,
                             int tokens, int q_heads, int kv_heads, int head_dim, int block_size, int max_blocks,
                             float scale) {
  hip_paged_attention(q, out, k_cache, v_cache, query_seq, query_key_len, block_tables, tokens, q_heads, kv_heads,
                      head_dim, block_size, max_blocks, scale);
  HIP_CHECK(hipDeviceSynchronize());
}
void ref_hip_embedding_u16(const int64_t* ids, const uint16_t* table, int tokens, int hidden, float* out,
                           int table_bf16) {
  hip_embedding_u16(ids, table, tokens, hidden, out, table_bf16 != 0);
  HIP_CHECK(hipDeviceSynchronize());
}
}
