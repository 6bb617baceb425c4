// C++ caller of the drop-in entry points, in the order Qwen3Model::forward_logits
// calls them (src/model.cpp:756-844), on one Qwen3-0.6B-like layer: two 32-token
// prefill sequences over a paged KV cache, every projection a Q8_0 GEMM, then the
// final norm, the last rows gathered and the tied lm_head on them (Q8_0, Q4_K and bf16
// tables and heads).  Beside it, on the same activations: Qwen2.5's qkv bias and the
// mixture-of-experts branch (router, routing, shared expert with its gate, routed experts).
// It includes only include/nvf_ops.h (the C ABI) and hip_runtime, exactly as
// model.cpp would after the switch, and checks each stage against the C oracle
// (test infrastructure), each stage fed the GPU's own input to that stage.
// Exit code 0 = every stage within its bound.
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

// |got - ref| <= max(1e-5 |ref|, 1 fp32 ulp, floor), or bit-exact
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
  std::printf("%-40s %s  (%zu / %zu outside, max abs err %.3g)\n", what, bad ? "FAIL" : "ok", bad, ref.size(), worst);
  if (bad) ++failures;
}

// |got - ideal| <= bound (elementwise), for the GEMM (the oracle's fp32 summation
// bound) and attention (a fraction of max |V|)
static void expect_within(const char* what, const std::vector<float>& got, const std::vector<double>& ideal,
                          const std::vector<double>& bound) {
  size_t bad = 0;
  double worst = 0;
  for (size_t i = 0; i < ideal.size(); ++i) {
    const double err = std::fabs((double)got[i] - ideal[i]);
    if (!(err <= bound[i] + 1e-30)) ++bad;
    worst = std::fmax(worst, err / (bound[i] + 1e-30));
  }
  std::printf("%-40s %s  (%zu / %zu outside, worst err/bound %.3g)\n", what, bad ? "FAIL" : "ok", bad, ideal.size(),
              worst);
  if (bad) ++failures;
}

struct Q8W {  // a Q8_0 weight [n, k] as split planes (model.cpp:394-404)
  std::vector<uint8_t> w8;
  std::vector<uint16_t> ws;
};

static Q8W make_q8(std::mt19937_64& rng, int64_t n, int64_t k) {
  std::uniform_int_distribution<int> q8(-127, 127);
  std::uniform_real_distribution<float> us(1e-3f, 1e-2f);
  Q8W w;
  w.w8.resize((size_t)(n * k));
  w.ws.resize((size_t)(n * k / 32));
  for (auto& b : w.w8) b = (uint8_t)(int8_t)q8(rng);
  for (auto& s : w.ws) s = orc_f32_to_fp16(us(rng));
  return w;
}

// The oracle's GEMM on the GPU's own input x [m, k]: ideal values and bounds.
static void oracle_gemm(const std::vector<float>& x, const uint8_t* w8, const uint16_t* ws, int64_t m, int64_t n,
                        int64_t k, std::vector<double>& ideal, std::vector<double>& bound) {
  ideal.assign((size_t)(m * n), 0.0);
  bound.assign((size_t)(m * n), 0.0);
  orc_matmul_q8(x.data(), ORC_F32, w8, ws, m, n, k, ideal.data(), bound.data(), nullptr, nullptr);
}

// The oracle's product with fp32 / fp16 / bf16 weights on the GPU's own input: ideal
// values and bounds, the bound scaled by `factor` (3 for bf16 weights: the prefill
// kernels sum exact bf16 piece products, three terms per product)
static void oracle_matmul_w(const std::vector<float>& x, const void* w, int w_format, int64_t m, int64_t n, int64_t k,
                            double factor, std::vector<double>& ideal, std::vector<double>& bound) {
  ideal.assign((size_t)(m * n), 0.0);
  bound.assign((size_t)(m * n), 0.0);
  orc_matmul_w(x.data(), ORC_F32, w, w_format, ORC_QK_LAYOUT_GGML, m, n, k, ideal.data(), bound.data());
  for (auto& b : bound) b *= factor;
}

int main() {
  // a Qwen3-0.6B-like layer (head_dim 128, GQA 16/8, QK-norm), 2 sequences x 32 prefill tokens
  const int S = 2, per = 32, T = S * per, H = 1024, I = 3072, V = 4096, heads = 16, kv_heads = 8, hd = 128;
  const int q_size = heads * hd, kv_size = kv_heads * hd, bs = 16, max_blocks = per / bs, num_blocks = 8;
  const float eps = 1e-6f, scale = 1.0f / std::sqrt((float)hd);
  std::mt19937_64 rng(2024);
  std::normal_distribution<float> g01(1.f, 0.1f);
  std::uniform_int_distribution<int64_t> vid(0, V - 1);

  // weights: Q8_0 embedding (tied lm_head) and projections, norms, inv_freq
  Q8W emb = make_q8(rng, V, H), wqkv = make_q8(rng, q_size + 2 * kv_size, H), wo = make_q8(rng, H, q_size),
      wgu = make_q8(rng, 2 * I, H), wdn = make_q8(rng, H, I);
  std::vector<float> in_ln(H), post_ln(H), q_norm(hd), k_norm(hd), final_ln(H), inv(hd / 2);
  for (auto* v : {&in_ln, &post_ln, &final_ln, &q_norm, &k_norm})
    for (auto& x : *v) x = g01(rng);
  if (nvf_rope_inv_freq(1e6, hd, inv.data()) != NVF_OK) return 2;  // model.cpp:416-420
  // the prefill context (model_runner.cpp:43-98): positions, query_seq, key lengths,
  // block tables over permuted physical blocks, slot mapping
  std::vector<int64_t> ids(T), pos(T);
  std::vector<int32_t> qseq(T), qlen(T), slots(T), tables(S * max_blocks);
  const int32_t perm[num_blocks] = {5, 2, 7, 0, 3, 6, 1, 4};
  for (int s = 0; s < S; ++s)
    for (int b = 0; b < max_blocks; ++b) tables[s * max_blocks + b] = perm[s * max_blocks + b];
  for (int t = 0; t < T; ++t) {
    const int s = t / per, p = t % per;
    ids[t] = vid(rng), pos[t] = p, qseq[t] = s, qlen[t] = p + 1;
    slots[t] = tables[s * max_blocks + p / bs] * bs + p % bs;
  }

  Dev<uint8_t> d_emb8(emb.w8), d_qkv8(wqkv.w8), d_o8(wo.w8), d_gu8(wgu.w8), d_dn8(wdn.w8);
  Dev<uint16_t> d_embs(emb.ws), d_qkvs(wqkv.ws), d_os(wo.ws), d_gus(wgu.ws), d_dns(wdn.ws);
  Dev<float> d_in_ln(in_ln), d_post_ln(post_ln), d_final_ln(final_ln), d_qn(q_norm), d_kn(k_norm), d_inv(inv);
  Dev<int64_t> d_ids(ids), d_pos(pos);
  Dev<int32_t> d_qseq(qseq), d_qlen(qlen), d_slots(slots), d_tables(tables);
  Dev<float> hidden((size_t)T * H), residual((size_t)T * H), norm((size_t)T * H), d_q((size_t)T * q_size),
      d_k((size_t)T * kv_size), d_v((size_t)T * kv_size), attn((size_t)T * q_size), gate((size_t)T * 2 * I),
      mlp((size_t)T * I);
  Dev<float> k_cache((size_t)num_blocks * bs * kv_size), v_cache((size_t)num_blocks * bs * kv_size);
  auto sync = [] { CHECK_HIP(hipDeviceSynchronize()); };
  std::vector<double> ideal, bound;

  // ---- the forward's op sequence, as model.cpp issues it, checked stage by stage ----
  hip_embedding_q8(d_ids.d, d_emb8.d, d_embs.d, T, H, hidden.d);  // :756 via :689-696
  sync();
  std::vector<float> x = hidden.host(), r_emb((size_t)T * H);
  orc_embedding_q8_split(ids.data(), emb.w8.data(), emb.ws.data(), T, H, r_emb.data(), ORC_F32);
  expect("embedding (bit-exact)", x, r_emb, true);

  auto norm_add = [&](const char* tag, const std::vector<float>& w, Dev<float>& wdev) {
    std::vector<float> h = hidden.host(), r = residual.host(), n((size_t)T * H);
    hip_rms_norm_add(hidden.d, residual.d, wdev.d, norm.d, T, H, eps);  // :762 / :787 / :835
    sync();
    orc_rms_norm_add(h.data(), r.data(), w.data(), n.data(), T, H, eps, ORC_F32);
    char buf[96];
    std::snprintf(buf, sizeof buf, "%s residual (bit-exact)", tag);
    expect(buf, residual.host(), r, true);
    std::snprintf(buf, sizeof buf, "%s norm", tag);
    expect(buf, norm.host(), n, false);
  };
  norm_add("input_layernorm", in_ln, d_in_ln);

  // qkv projections: one fused weight, row slices (:764-767)
  std::vector<float> nx = norm.host();
  hip_matmul_q8(norm.d, d_qkv8.d, d_qkvs.d, T, q_size, H, d_q.d);
  hip_matmul_q8(norm.d, d_qkv8.d + (size_t)q_size * H, d_qkvs.d + (size_t)q_size * H / 32, T, kv_size, H, d_k.d);
  hip_matmul_q8(norm.d, d_qkv8.d + (size_t)(q_size + kv_size) * H, d_qkvs.d + (size_t)(q_size + kv_size) * H / 32, T,
                kv_size, H, d_v.d);
  sync();
  oracle_gemm(nx, wqkv.w8.data(), wqkv.ws.data(), T, q_size, H, ideal, bound);
  expect_within("q projection (Q8_0 GEMM)", d_q.host(), ideal, bound);
  oracle_gemm(nx, wqkv.w8.data() + (size_t)q_size * H, wqkv.ws.data() + (size_t)q_size * H / 32, T, kv_size, H, ideal,
              bound);
  expect_within("k projection (row slice)", d_k.host(), ideal, bound);
  oracle_gemm(nx, wqkv.w8.data() + (size_t)(q_size + kv_size) * H,
              wqkv.ws.data() + (size_t)(q_size + kv_size) * H / 32, T, kv_size, H, ideal, bound);
  expect_within("v projection (row slice)", d_v.host(), ideal, bound);

  // QK-norm then RoPE (:774-778)
  std::vector<float> q = d_q.host(), k = d_k.host(), v = d_v.host();
  hip_rms_norm(d_q.d, d_qn.d, d_q.d, T * heads, hd, eps);
  hip_rms_norm(d_k.d, d_kn.d, d_k.d, T * kv_heads, hd, eps);
  hip_rope_inplace(d_q.d, d_pos.d, T, heads, hd, q_size, d_inv.d);
  hip_rope_inplace(d_k.d, d_pos.d, T, kv_heads, hd, kv_size, d_inv.d);
  sync();
  std::vector<float> nq(q.size()), nk(k.size());
  orc_rms_norm(q.data(), q_norm.data(), nq.data(), (int64_t)T * heads, hd, eps, ORC_F32);
  orc_rms_norm(k.data(), k_norm.data(), nk.data(), (int64_t)T * kv_heads, hd, eps, ORC_F32);
  orc_rope(nq.data(), pos.data(), T, heads, hd, q_size, inv.data(), ORC_F32);
  orc_rope(nk.data(), pos.data(), T, kv_heads, hd, kv_size, inv.data(), ORC_F32);
  expect("q: QK-norm then RoPE", d_q.host(), nq, false, 1e-6f);
  expect("k: QK-norm then RoPE", d_k.host(), nk, false, 1e-6f);

  // KV store, then paged attention (:780-784)
  std::vector<float> qg = d_q.host(), kg = d_k.host();
  hip_store_kv(d_k.d, d_v.d, k_cache.d, v_cache.d, d_slots.d, T, kv_heads, hd);
  sync();
  std::vector<float> kc_ref(k_cache.n, 0.f), vc_ref(v_cache.n, 0.f);
  orc_store_kv(kg.data(), v.data(), kc_ref.data(), vc_ref.data(), slots.data(), T, kv_heads, hd, ORC_F32);
  expect("k cache (bit-exact)", k_cache.host(), kc_ref, true);
  expect("v cache (bit-exact)", v_cache.host(), vc_ref, true);
  hip_paged_attention(d_q.d, attn.d, k_cache.d, v_cache.d, d_qseq.d, d_qlen.d, d_tables.d, T, heads, kv_heads, hd, bs,
                      max_blocks, scale);
  sync();
  {
    std::vector<float> ao((size_t)T * q_size), vmax((size_t)T * heads);
    std::vector<double> ex((size_t)T * q_size), tol((size_t)T * q_size);
    orc_paged_attention(qg.data(), ao.data(), kc_ref.data(), vc_ref.data(), qseq.data(), qlen.data(), tables.data(), T,
                        heads, kv_heads, hd, bs, max_blocks, scale, ORC_F32, ex.data(), vmax.data());
    for (size_t i = 0; i < tol.size(); ++i) tol[i] = 1e-4 * vmax[i / hd] + 1e-7;
    expect_within("paged attention", attn.host(), ex, tol);
  }

  // o_proj, post-attention norm (:786-787)
  std::vector<float> ax = attn.host();
  hip_matmul_q8(attn.d, d_o8.d, d_os.d, T, H, q_size, hidden.d);
  sync();
  oracle_gemm(ax, wo.w8.data(), wo.ws.data(), T, H, q_size, ideal, bound);
  expect_within("o projection", hidden.host(), ideal, bound);
  norm_add("post_attention_layernorm", post_ln, d_post_ln);

  // MLP (:828-830)
  nx = norm.host();
  hip_matmul_q8(norm.d, d_gu8.d, d_gus.d, T, 2 * I, H, gate.d);
  sync();
  oracle_gemm(nx, wgu.w8.data(), wgu.ws.data(), T, 2 * I, H, ideal, bound);
  expect_within("gate_up projection", gate.host(), ideal, bound);
  std::vector<float> gu = gate.host(), r_mlp((size_t)T * I);
  hip_silu_and_mul(gate.d, mlp.d, T, I);
  sync();
  orc_silu_and_mul(gu.data(), r_mlp.data(), T, I, ORC_F32);
  expect("silu_and_mul", mlp.host(), r_mlp, false);
  std::vector<float> mx = mlp.host();
  hip_matmul_q8(mlp.d, d_dn8.d, d_dns.d, T, H, I, hidden.d);
  sync();
  oracle_gemm(mx, wdn.w8.data(), wdn.ws.data(), T, H, I, ideal, bound);
  expect_within("down projection", hidden.host(), ideal, bound);

  // Qwen2.5's qkv bias (:768-772; this layer is Qwen3-like and takes QK-norm instead), on a
  // copy of the projected q: bit-exact (one fp32 add)
  {
    std::vector<float> bias(q_size);
    for (auto& b : bias) b = g01(rng) - 1.f;
    Dev<float> qb(q), d_bias(bias);
    hip_add_bias_inplace(qb.d, d_bias.d, T, q_size);
    sync();
    std::vector<float> r_qb = q;
    orc_add_bias(r_qb.data(), bias.data(), T, q_size, q_size, ORC_F32);
    expect("qkv bias (bit-exact)", qb.host(), r_qb, true);
  }

  // a mixture-of-experts FFN in the dense MLP's place (:789-826, Qwen2-MoE-like), on the same
  // post-attention norm output: router (fp32 weights), top-K routing, the shared expert
  // (bf16) with its sigmoid gate, then the routed bf16 experts added on top
  {
    const int E = 16, K = 4, Ie = 256, SI = 512;
    std::normal_distribution<float> w05(0.f, 0.05f);
    auto bf16_weights = [&](size_t count) {
      std::vector<uint16_t> w(count);
      for (auto& e : w) e = orc_f32_to_bf16(w05(rng));
      return w;
    };
    std::vector<float> router((size_t)E * H);
    for (auto& e : router) e = w05(rng);
    const std::vector<uint16_t> sh_gu = bf16_weights((size_t)2 * SI * H), sh_dn = bf16_weights((size_t)H * SI),
                                sh_gate = bf16_weights(H), ex_gu = bf16_weights((size_t)E * 2 * Ie * H),
                                ex_dn = bf16_weights((size_t)E * H * Ie);
    std::vector<int32_t> slot_of(E);
    for (int e = 0; e < E; ++e) slot_of[e] = (e * 7) % E;  // experts placed in permuted slots (moe_place)
    Dev<float> d_router(router), route((size_t)T * E), d_sc((size_t)T * K), sgate((size_t)T * 2 * SI),
        smlp((size_t)T * SI), moe((size_t)T * H), shs((size_t)T);
    Dev<uint16_t> d_shgu(sh_gu), d_shdn(sh_dn), d_shg(sh_gate), d_exgu(ex_gu), d_exdn(ex_dn);
    Dev<int32_t> d_slot(slot_of), d_idx((size_t)T * K);
    const std::vector<float> nx2 = norm.host();

    hip_matmul(norm.d, d_router.d, T, E, H, route.d);  // :797
    sync();
    oracle_matmul_w(nx2, router.data(), NVF_W_F32, T, E, H, 1.0, ideal, bound);
    expect_within("MoE router logits (fp32 weights)", route.host(), ideal, bound);
    const std::vector<float> lg = route.host();
    hip_moe_route(route.d, T, E, K, true, d_idx.d, d_sc.d);  // :798
    sync();
    std::vector<int32_t> r_idx((size_t)T * K);
    std::vector<float> r_sc((size_t)T * K);
    orc_moe_route(lg.data(), T, E, K, 1, r_idx.data(), r_sc.data());
    const bool ids_ok = d_idx.host() == r_idx;
    std::printf("%-40s %s\n", "MoE routing: expert ids (exact)", ids_ok ? "ok" : "FAIL");
    if (!ids_ok) ++failures;
    expect("MoE routing: scores (bit-exact)", d_sc.host(), r_sc, true);

    hip_matmul_u16(norm.d, d_shgu.d, T, 2 * SI, H, sgate.d, true);  // shared expert, :802-804
    sync();
    oracle_matmul_w(nx2, sh_gu.data(), NVF_W_BF16, T, 2 * SI, H, 3.0, ideal, bound);
    expect_within("shared expert gate_up (bf16 weights)", sgate.host(), ideal, bound);
    const std::vector<float> sg = sgate.host();
    std::vector<float> r_sm((size_t)T * SI);
    hip_silu_and_mul(sgate.d, smlp.d, T, SI);
    sync();
    orc_silu_and_mul(sg.data(), r_sm.data(), T, SI, ORC_F32);
    expect("shared expert silu_and_mul", smlp.host(), r_sm, false);
    const std::vector<float> sm = smlp.host();
    hip_matmul_u16(smlp.d, d_shdn.d, T, H, SI, moe.d, true);
    sync();
    oracle_matmul_w(sm, sh_dn.data(), NVF_W_BF16, T, H, SI, 3.0, ideal, bound);
    expect_within("shared expert down", moe.host(), ideal, bound);
    hip_matmul_u16(norm.d, d_shg.d, T, 1, H, shs.d, true);  // its gate, :805-809
    sync();
    oracle_matmul_w(nx2, sh_gate.data(), NVF_W_BF16, T, 1, H, 3.0, ideal, bound);
    expect_within("shared expert gate logit", shs.host(), ideal, bound);
    const std::vector<float> mo = moe.host(), sv = shs.host();
    std::vector<float> r_gated(mo.size());
    for (int t = 0; t < T; ++t)
      for (int c = 0; c < H; ++c)
        r_gated[(size_t)t * H + c] = mo[(size_t)t * H + c] * (1.0f / (1.0f + std::exp(-sv[t])));
    hip_scale_rows_sigmoid(moe.d, shs.d, T, H);
    sync();
    expect("shared expert sigmoid gate", moe.host(), r_gated, false);

    const std::vector<float> base = moe.host();  // the routed experts add to it (:817-825)
    const std::vector<double> base_d(base.begin(), base.end());
    const std::vector<int32_t> hidx = d_idx.host();
    const std::vector<float> hsc = d_sc.host();
    hip_moe_ffn(norm.d, d_idx.d, d_sc.d, d_exgu.d, d_exdn.d, d_slot.d, T, H, Ie, K, true, moe.d);
    sync();
    std::vector<double> m_ideal((size_t)T * H), m_err((size_t)T * H);
    orc_moe_ffn(nx2.data(), ORC_F32, hidx.data(), hsc.data(), ex_gu.data(), ex_dn.data(), 1, slot_of.data(), T, H, Ie,
                K, E, base_d.data(), m_ideal.data(), m_err.data());
    for (auto& e : m_err) e *= 6.0;  // bf16 experts on the split products (as the MoE GPU tests)
    expect_within("routed experts (hip_moe_ffn, added)", moe.host(), m_ideal, m_err);
  }

  // final norm (:835), each sequence's last row gathered (:837-839), the tied lm_head on
  // them (:841-843; m = 2, the decode GEMV)
  norm_add("final norm", final_ln, d_final_ln);
  const std::vector<int32_t> last_idx = {per - 1, T - 1};  // ctx.last_indices
  Dev<int32_t> d_last(last_idx);
  Dev<float> selected((size_t)2 * H), logits2((size_t)2 * V);
  const std::vector<float> nf = norm.host();
  hip_gather_rows(norm.d, d_last.d, T, H, 2, selected.d);
  sync();
  std::vector<float> r_sel((size_t)2 * H);
  orc_gather_rows(nf.data(), last_idx.data(), H, 2, r_sel.data(), ORC_F32);
  expect("last rows gathered (bit-exact)", selected.host(), r_sel, true);
  hip_matmul_q8(selected.d, d_emb8.d, d_embs.d, 2, V, H, logits2.d);
  sync();
  oracle_gemm(r_sel, emb.w8.data(), emb.ws.data(), 2, V, H, ideal, bound);
  expect_within("lm_head logits (Q8_0, m = 2)", logits2.host(), ideal, bound);

  // the other table and head formats embedding_dispatch / matmul_dispatch take
  // (:665-696): a Q4_K table (GGUF nibble order, the drop-in's default) and a bf16 one,
  // each gathered for the prompt and used as the tied head on the gathered rows
  {
    std::vector<uint8_t> q4k((size_t)V * H / 256 * 144);
    std::uniform_int_distribution<int> byte(0, 255);
    std::uniform_real_distribution<float> us(1e-3f, 1e-2f);
    for (size_t b = 0; b < q4k.size() / 144; ++b) {
      uint8_t* blk = q4k.data() + b * 144;
      const uint16_t d = orc_f32_to_fp16(us(rng)), dmin = orc_f32_to_fp16(us(rng));
      std::memcpy(blk, &d, 2);
      std::memcpy(blk + 2, &dmin, 2);
      for (int i = 4; i < 144; ++i) blk[i] = (uint8_t)byte(rng);  // any 12 bytes are valid 6-bit scales / mins
    }
    std::normal_distribution<float> n01(0.f, 1.f);
    std::vector<uint16_t> tbf((size_t)V * H);
    for (auto& e : tbf) e = orc_f32_to_bf16(n01(rng) * 0.05f);
    Dev<uint8_t> d_q4k(q4k);
    Dev<uint16_t> d_tbf(tbf);
    Dev<float> e_out((size_t)T * H);
    std::vector<float> r_e((size_t)T * H);

    hip_embedding_qk(d_ids.d, d_q4k.d, T, H, e_out.d, NVF_Q4_K);  // :691
    sync();
    orc_embedding_qk(ids.data(), q4k.data(), T, H, NVF_Q4_K, ORC_QK_LAYOUT_GGML, r_e.data(), ORC_F32);
    expect("Q4_K embedding (bit-exact)", e_out.host(), r_e, true);
    hip_embedding_u16(d_ids.d, d_tbf.d, T, H, e_out.d, true);  // :695
    sync();
    orc_embedding_u16(ids.data(), tbf.data(), T, H, 1, r_e.data(), ORC_F32);
    expect("bf16 embedding (bit-exact)", e_out.host(), r_e, true);

    hip_matmul_qk(selected.d, d_q4k.d, 2, V, H, logits2.d, NVF_Q4_K);  // :667
    sync();
    oracle_matmul_w(r_sel, q4k.data(), NVF_W_Q4_K, 2, V, H, 1.0, ideal, bound);
    expect_within("lm_head logits (Q4_K, m = 2)", logits2.host(), ideal, bound);
    hip_matmul_u16(selected.d, d_tbf.d, 2, V, H, logits2.d, true);  // :671
    sync();
    oracle_matmul_w(r_sel, tbf.data(), NVF_W_BF16, 2, V, H, 3.0, ideal, bound);
    expect_within("lm_head logits (bf16, m = 2)", logits2.host(), ideal, bound);
  }

  // a decode step over a longer cache (model_runner.cpp:100-128: one query per
  // sequence, key_len = its context) in 64-key blocks: few (token, kv head) pairs,
  // so the drop-in splits the keys over its own workspace and merges
  {
    const int ds = 2, dbs = 64, dmax = 12;
    const int ctx[ds] = {300, 700};
    const int rows = ds * dmax * dbs;
    std::vector<float> dq((size_t)ds * q_size), dk((size_t)rows * kv_size), dv((size_t)rows * kv_size);
    std::normal_distribution<float> n01(0.f, 1.f);
    for (auto* a : {&dq, &dk, &dv})
      for (auto& e : *a) e = n01(rng);
    std::vector<int32_t> dqs(ds), dql(ds), dtab((size_t)ds * dmax);
    for (int s2 = 0; s2 < ds; ++s2) {
      dqs[s2] = s2, dql[s2] = ctx[s2];
      for (int b = 0; b < dmax; ++b) dtab[s2 * dmax + b] = (s2 * dmax + b * 5) % (ds * dmax);  // a permutation
    }
    if (nvf_paged_attention_workspace_size(ds, heads, kv_heads, hd, dbs, dmax, 0) <= 0) {
      std::printf("decode step: expected a split plan\n");
      ++failures;
    }
    Dev<float> g_q(dq), g_k(dk), g_v(dv), g_o((size_t)ds * q_size);
    Dev<int32_t> g_qs(dqs), g_ql(dql), g_tab(dtab);
    hip_paged_attention(g_q.d, g_o.d, g_k.d, g_v.d, g_qs.d, g_ql.d, g_tab.d, ds, heads, kv_heads, hd, dbs, dmax, scale);
    sync();
    std::vector<float> ao((size_t)ds * q_size), vmax((size_t)ds * heads);
    std::vector<double> ex((size_t)ds * q_size), tol((size_t)ds * q_size);
    orc_paged_attention(dq.data(), ao.data(), dk.data(), dv.data(), dqs.data(), dql.data(), dtab.data(), ds, heads,
                        kv_heads, hd, dbs, dmax, scale, ORC_F32, ex.data(), vmax.data());
    for (size_t i = 0; i < tol.size(); ++i) tol[i] = 1e-4 * vmax[i / hd] + 1e-7;
    expect_within("decode step: split paged attention", g_o.host(), ex, tol);
  }

  std::printf(failures ? "DROPIN CHAIN FAILED\n" : "DROPIN CHAIN OK\n");
  return failures ? 1 : 0;
}
