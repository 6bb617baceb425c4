// C++ caller of the drop-in entry points, in the order Qwen3Model::forward_logits
// calls them (src/model.cpp:756-835), on a Qwen3-0.6B-like layer at 64 tokens.
// It includes only include/nvf_ops.h (the C ABI) and hip_runtime, exactly as
// model.cpp would after the switch, and checks each stage against the C oracle
// (test infrastructure).  Exit code 0 = every stage within its bound.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "../../include/nvf_ops.h"
#include "../../oracle/nvf_oracle.h"

#define CHECK_HIP(x)                                                                          \
  do {                                                                                        \
    hipError_t e_ = (x);                                                                      \
    if (e_ != hipSuccess) {                                                                   \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(2);                                                                           \
    }                                                                                         \
  } while (0)

template <class T>
struct Dev {  // the reference's DeviceBuf/DevVec role: caller-owned device memory
  T* d = nullptr;
  size_t n = 0;
  explicit Dev(const std::vector<T>& h) : n(h.size()) {
    CHECK_HIP(hipMalloc(&d, n * sizeof(T)));
    CHECK_HIP(hipMemcpy(d, h.data(), n * sizeof(T), hipMemcpyHostToDevice));
  }
  explicit Dev(size_t count) : n(count) {
    CHECK_HIP(hipMalloc(&d, n * sizeof(T)));
    CHECK_HIP(hipMemset(d, 0, n * sizeof(T)));  // DeviceBuf zero-fills (common.hpp:126-153)
  }
  ~Dev() { (void)hipFree(d); }
  std::vector<T> host() const {
    std::vector<T> h(n);
    CHECK_HIP(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
  }
};

static int failures = 0;

static void expect(const char* what, const std::vector<float>& got, const std::vector<float>& ref, bool exact,
                   float floor = 0.f) {
  size_t bad = 0;
  double worst = 0;
  for (size_t i = 0; i < ref.size(); ++i) {
    const float g = got[i], r = ref[i];
    if (exact) {
      uint32_t a, b;
      std::memcpy(&a, &g, 4);
      std::memcpy(&b, &r, 4);
      if (a != b) ++bad;
      continue;
    }
    const double tol = std::fmax(std::fmax(1e-5 * std::fabs(r), std::nextafter(std::fabs(r), INFINITY) - std::fabs(r)),
                                 (double)floor);
    const double err = std::fabs((double)g - (double)r);
    if (!(err <= tol)) ++bad;
    worst = std::fmax(worst, err);
  }
  std::printf("%-34s %s  (%zu / %zu outside, max abs err %.3g)\n", what, bad ? "FAIL" : "ok", bad, ref.size(), worst);
  if (bad) ++failures;
}

int main() {
  const int T = 64, H = 1024, I = 3072, V = 4096, heads = 16, kv_heads = 8, hd = 128;
  const int q_size = heads * hd, kv_size = kv_heads * hd;
  const float eps = 1e-6f;
  std::mt19937_64 rng(2024);
  std::normal_distribution<float> n01(0.f, 1.f), g01(1.f, 0.1f);
  std::uniform_real_distribution<float> us(1e-3f, 1e-2f);
  std::uniform_int_distribution<int> q8(-127, 127);
  std::uniform_int_distribution<int64_t> vid(0, V - 1);

  // weights: Q8_0 embedding split planes (model.cpp:394-404), norms, inv_freq
  std::vector<uint8_t> w8((size_t)V * H);
  std::vector<uint16_t> ws((size_t)V * H / 32);
  for (auto& b : w8) b = (uint8_t)(int8_t)q8(rng);
  for (auto& s : ws) s = orc_f32_to_fp16(us(rng));
  std::vector<float> in_ln(H), post_ln(H), q_norm(hd), k_norm(hd), final_ln(H), inv(hd / 2);
  for (auto* v : {&in_ln, &post_ln, &final_ln, &q_norm, &k_norm})
    for (auto& x : *v) x = g01(rng);
  if (nvf_rope_inv_freq(1e6, hd, inv.data()) != NVF_OK) return 2;  // model.cpp:416-420
  std::vector<int64_t> ids(T), pos(T);
  for (int t = 0; t < T; ++t) ids[t] = vid(rng), pos[t] = t;
  // stand-ins for the GEMM outputs between the ops (random, seeded)
  std::vector<float> attn_out((size_t)T * H), q((size_t)T * q_size), k((size_t)T * kv_size), mlp_in((size_t)T * 2 * I),
      down_out((size_t)T * H);
  for (auto* v : {&attn_out, &q, &k, &mlp_in, &down_out})
    for (auto& x : *v) x = n01(rng);

  Dev<uint8_t> d_w8(w8);
  Dev<uint16_t> d_ws(ws);
  Dev<float> d_in_ln(in_ln), d_post_ln(post_ln), d_final_ln(final_ln), d_qn(q_norm), d_kn(k_norm), d_inv(inv);
  Dev<int64_t> d_ids(ids), d_pos(pos);
  Dev<float> hidden((size_t)T * H), residual((size_t)T * H), norm((size_t)T * H);
  Dev<float> d_q(q), d_k(k), d_gate(mlp_in), mlp((size_t)T * I);

  // ---- the forward's op sequence, as model.cpp issues it ----
  hip_embedding_q8(d_ids.d, d_w8.d, d_ws.d, T, H, hidden.d);                            // :756 via :689-696
  hip_rms_norm_add(hidden.d, residual.d, d_in_ln.d, norm.d, T, H, eps);                 // :762 (residual = 0)
  hip_rms_norm(d_q.d, d_qn.d, d_q.d, T * heads, hd, eps);                               // :774 QK-norm, in place
  hip_rms_norm(d_k.d, d_kn.d, d_k.d, T * kv_heads, hd, eps);                            // :775
  hip_rope_inplace(d_q.d, d_pos.d, T, heads, hd, q_size, d_inv.d);                      // :777
  hip_rope_inplace(d_k.d, d_pos.d, T, kv_heads, hd, kv_size, d_inv.d);                  // :778
  std::vector<float> emb_gpu = hidden.host(), res1 = residual.host(), norm1 = norm.host();
  CHECK_HIP(hipMemcpy(hidden.d, attn_out.data(), attn_out.size() * 4, hipMemcpyHostToDevice));  // o_proj stand-in
  hip_rms_norm_add(hidden.d, residual.d, d_post_ln.d, norm.d, T, H, eps);               // :787
  std::vector<float> res2 = residual.host(), norm2 = norm.host();
  hip_silu_and_mul(d_gate.d, mlp.d, T, I);                                              // :830
  CHECK_HIP(hipMemcpy(hidden.d, down_out.data(), down_out.size() * 4, hipMemcpyHostToDevice));  // down stand-in
  hip_rms_norm_add(hidden.d, residual.d, d_final_ln.d, norm.d, T, H, eps);              // :835 final norm
  CHECK_HIP(hipDeviceSynchronize());
  std::vector<float> q_gpu = d_q.host(), k_gpu = d_k.host(), mlp_gpu = mlp.host(), res3 = residual.host(),
                     norm3 = norm.host();

  // ---- the same sequence on the oracle ----
  std::vector<float> r_emb((size_t)T * H), r_res((size_t)T * H, 0.f), r_norm((size_t)T * H), r_q = q, r_k = k,
                     r_mlp((size_t)T * I);
  orc_embedding_q8_split(ids.data(), w8.data(), ws.data(), T, H, r_emb.data(), ORC_F32);
  expect("embedding (bit-exact)", emb_gpu, r_emb, true);
  orc_rms_norm_add(r_emb.data(), r_res.data(), in_ln.data(), r_norm.data(), T, H, eps, ORC_F32);
  expect("layer-0 residual (bit-exact)", res1, r_res, true);
  expect("input_layernorm", norm1, r_norm, false);
  std::vector<float> nq(r_q.size()), nk(r_k.size());
  orc_rms_norm(r_q.data(), q_norm.data(), nq.data(), (int64_t)T * heads, hd, eps, ORC_F32);
  orc_rms_norm(r_k.data(), k_norm.data(), nk.data(), (int64_t)T * kv_heads, hd, eps, ORC_F32);
  orc_rope(nq.data(), pos.data(), T, heads, hd, q_size, inv.data(), ORC_F32);
  orc_rope(nk.data(), pos.data(), T, kv_heads, hd, kv_size, inv.data(), ORC_F32);
  expect("q: QK-norm then RoPE", q_gpu, nq, false, 1e-6f);
  expect("k: QK-norm then RoPE", k_gpu, nk, false, 1e-6f);
  orc_rms_norm_add(attn_out.data(), r_res.data(), post_ln.data(), r_norm.data(), T, H, eps, ORC_F32);
  expect("post-attention residual (bit-exact)", res2, r_res, true);
  expect("post_attention_layernorm", norm2, r_norm, false);
  orc_silu_and_mul(mlp_in.data(), r_mlp.data(), T, I, ORC_F32);
  expect("silu_and_mul", mlp_gpu, r_mlp, false);
  orc_rms_norm_add(down_out.data(), r_res.data(), final_ln.data(), r_norm.data(), T, H, eps, ORC_F32);
  expect("final residual (bit-exact)", res3, r_res, true);
  expect("final norm", norm3, r_norm, false);
  std::printf(failures ? "DROPIN CHAIN FAILED\n" : "DROPIN CHAIN OK\n");
  return failures ? 1 : 0;
}
