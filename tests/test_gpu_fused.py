"""GPU parity for the fusions with the path's neighbours:

* nvf_rms_norm_q8 -- RMSNorm (+ residual add) that also emits the Q8_0 GEMM's
  activation row scale and int8 row (the reference's q8_row_scale_kernel pass,
  src/hip_ops.hip:205-217, and its GEMM's quantizer, :244-245);
* nvf_embedding_rms_norm -- layer-0 gather + residual-add onto zeros + RMSNorm
  (src/model.cpp:756 then :762);
* nvf_silu_and_mul_q8 -- SwiGLU (src/hip_ops.hip:419-429) emitting the down
  projection's row scale and int8 rows.

Bars: the row scale and int8 row bit-exact against the oracle's quantizer
applied to the kernel's own stored output (the quantizer is exact arithmetic on
that row); the stored output within the RMSNorm tolerance of the oracle; the
fused residual bit-exact (emb + 0).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_vllm_cpp_amd import ops
from tests import harness as H

pytestmark = pytest.mark.gpu

DTYPES = [H.F32, H.F16, H.BF16]
DT_IDS = ["f32", "f16", "bf16"]


def case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("add", [True, False], ids=["add", "plain"])
@pytest.mark.parametrize("rows,hidden", [(64, 3584), (33, 896), (5, 999), (7, 4096)])
def test_rms_norm_q8(gpu, dt, add, rows, hidden):
    o = H.oracle()
    r = H.rng(rows * hidden + dt + 7 * add)
    x, res = H.gen_act(r, (rows, hidden), dt), H.gen_act(r, (rows, hidden), dt)
    x[1] = H.to_storage(np.zeros(hidden, np.float32), dt)  # an all-zero input row (scale 0 when plain)
    w = H.gen_act(r, (hidden,), dt, 1.0, 0.1)
    ref_res, ref_out = res.copy(), np.empty_like(x)
    if add:
        o.orc_rms_norm_add(H.ptr(x), H.ptr(ref_res), H.ptr(w), H.ptr(ref_out), rows, hidden, 1e-6, dt)
    else:
        o.orc_rms_norm(H.ptr(x), H.ptr(w), H.ptr(ref_out), rows, hidden, 1e-6, dt)
    d_res = H.to_dev(res, gpu, dt)
    case(f"rms_norm_q8 add={add} rows={rows} hidden={hidden} dt={dt}")
    out, scale, q = ops.rms_norm_q8(H.to_dev(x, gpu, dt), H.to_dev(w, gpu, dt), 1e-6, d_res if add else None)
    got_out, got_scale, got_q = H.to_host(out), scale.cpu().numpy(), q.cpu().numpy()
    if add:
        H.assert_bitexact(H.to_host(d_res), ref_res, "residual")
    H.assert_close(got_out, ref_out, dt, what="out")
    exp_scale = np.empty(rows, np.float32)
    o.orc_q8_row_scale(H.ptr(got_out), H.ptr(exp_scale), rows, hidden, dt)
    H.assert_bitexact(got_scale, exp_scale, "row scale")
    exp_q = np.empty((rows, hidden), np.int8)
    o.orc_q8_quantize(H.ptr(got_out), H.ptr(exp_scale), exp_q.ctypes.data, rows, hidden, dt)
    H.assert_bitexact(got_q, exp_q, "int8 row")
    if not add:
        assert got_scale[1] == 0.0 and not got_q[1].any()
    # the same call without the fp output: identical scale and int8 row
    d_res2 = H.to_dev(res, gpu, dt)
    case("rms_norm_q8 without out")
    none, scale2, q2 = ops.rms_norm_q8(H.to_dev(x, gpu, dt), H.to_dev(w, gpu, dt), 1e-6, d_res2 if add else None,
                                       want_out=False)
    assert none is None
    H.assert_bitexact(scale2.cpu().numpy(), got_scale, "row scale (no out)")
    H.assert_bitexact(q2.cpu().numpy(), got_q, "int8 row (no out)")


def _emb_reference(o, fmt, ids, table, scales, T, Hd, dt):
    """The gathered rows in the storage dtype (oracle)."""
    emb = np.empty((T, Hd), H.NP_STORAGE[dt])
    if fmt == ops.EMB_Q8_0:
        o.orc_embedding_q8_split(H.ptr(ids), H.ptr(table), H.ptr(scales), T, Hd, H.ptr(emb), dt)
    elif fmt == ops.EMB_Q8_0_BLOCKS:
        o.orc_embedding_q8_blocks(H.ptr(ids), H.ptr(table), T, Hd, H.ptr(emb), dt)
    else:
        o.orc_embedding_qk(H.ptr(ids), H.ptr(table), T, Hd, fmt, H.GGML, H.ptr(emb), dt)
    return emb


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("fmt", [ops.EMB_Q8_0, ops.EMB_Q8_0_BLOCKS, ops.EMB_Q4_K, ops.EMB_Q5_K, ops.EMB_Q6_K],
                         ids=["q8_0", "q8_0_blocks", "q4_k", "q5_k", "q6_k"])
# (row splits at these 70 rows: 256 one wave per row, the others four)
@pytest.mark.parametrize("hidden", [3584, 1024, 256, 12288])
def test_embedding_rms_norm(gpu, dt, fmt, hidden):
    o = H.oracle()
    r = H.rng(hidden + fmt * 3 + dt)
    V, T = 300, 70
    scales = None
    if fmt in (ops.EMB_Q8_0, ops.EMB_Q8_0_BLOCKS):
        w8, ws = H.gen_q8_0(r, V, hidden)
        table, scales = (w8, ws) if fmt == ops.EMB_Q8_0 else (H.q8_split_to_blocks(w8, ws), None)
    else:
        bb, offs = {ops.EMB_Q4_K: (144, (0, 2)), ops.EMB_Q5_K: (176, (0, 2)), ops.EMB_Q6_K: (210, (208,))}[fmt]
        table = H.gen_raw_blocks(r, V * hidden // 256, bb, offs)
    ids = r.integers(0, V, T).astype(np.int64)
    ids[:2] = [V - 1, 0]
    w = H.gen_act(r, (hidden,), dt, 1.0, 0.1)
    emb = _emb_reference(o, fmt, ids, table, scales, T, hidden, dt)
    ref_res = H.to_storage(np.zeros((T, hidden), np.float32), dt)
    ref_out = np.empty_like(emb)
    o.orc_rms_norm_add(H.ptr(emb), H.ptr(ref_res), H.ptr(w), H.ptr(ref_out), T, hidden, 1e-6, dt)
    case(f"embedding_rms_norm fmt={fmt} hidden={hidden} dt={dt}")
    res, out = ops.embedding_rms_norm(H.to_dev(ids, gpu), fmt, H.to_dev(table, gpu),
                                      H.to_dev(scales, gpu) if scales is not None else None, hidden,
                                      H.to_dev(w, gpu, dt), 1e-6, V)
    H.assert_bitexact(H.to_host(res), ref_res, "fused residual")
    H.assert_close(H.to_host(out), ref_out, dt, what="fused norm")


@pytest.mark.parametrize("fmt", [ops.EMB_Q8_0, ops.EMB_Q8_0_BLOCKS], ids=["q8_0", "q8_0_blocks"])
def test_embedding_rms_norm_many_rows(gpu, fmt):
    """16384 rows: the 8-bit tables' two-waves-per-row split."""
    o = H.oracle()
    dt, hidden, V, T = H.F16, 3584, 300, 16384
    r = H.rng(fmt + 4242)
    w8, ws = H.gen_q8_0(r, V, hidden)
    table, scales = (w8, ws) if fmt == ops.EMB_Q8_0 else (H.q8_split_to_blocks(w8, ws), None)
    ids = r.integers(0, V, T).astype(np.int64)
    w = H.gen_act(r, (hidden,), dt, 1.0, 0.1)
    emb = _emb_reference(o, fmt, ids, table, scales, T, hidden, dt)
    ref_res = H.to_storage(np.zeros((T, hidden), np.float32), dt)
    ref_out = np.empty_like(emb)
    o.orc_rms_norm_add(H.ptr(emb), H.ptr(ref_res), H.ptr(w), H.ptr(ref_out), T, hidden, 1e-6, dt)
    case(f"embedding_rms_norm fmt={fmt} rows={T}")
    res, out = ops.embedding_rms_norm(H.to_dev(ids, gpu), fmt, H.to_dev(table, gpu),
                                      H.to_dev(scales, gpu) if scales is not None else None, hidden,
                                      H.to_dev(w, gpu, dt), 1e-6, V)
    H.assert_bitexact(H.to_host(res), ref_res, "fused residual")
    H.assert_close(H.to_host(out), ref_out, dt, what="fused norm")


def test_embedding_rms_norm_bad_ids_and_args(gpu):
    r = H.rng(5)
    V, hidden = 40, 512
    w8, ws = H.gen_q8_0(r, V, hidden)
    ids = np.array([3, V, -2], np.int64)
    w = torch.ones(hidden, dtype=torch.float16, device=gpu)
    case("embedding_rms_norm out-of-range ids")
    res, out = ops.embedding_rms_norm(H.to_dev(ids, gpu), ops.EMB_Q8_0, H.to_dev(w8, gpu), H.to_dev(ws, gpu), hidden,
                                      w, 1e-6, V)
    o = out.float().cpu().numpy()
    assert np.isfinite(o[0]).all() and np.isnan(o[1:]).all()
    with pytest.raises(ops.NvfError, match="hidden"):
        ops.embedding_rms_norm(H.to_dev(ids, gpu), ops.EMB_Q4_K, H.to_dev(w8, gpu), None, 500, w[:500], 1e-6, V)


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("rows,inter", [(64, 18944), (33, 4864), (7, 999), (5, 12288), (3, 40)])
def test_silu_and_mul_q8(gpu, dt, rows, inter):
    """SwiGLU + the down projection's quantizer: the fp output is bit-identical to
    nvf_silu_and_mul's, the scale and int8 rows bit-exact against the oracle's
    quantizer on that output, and the output within the SwiGLU tolerance."""
    o = H.oracle()
    r = H.rng(rows * inter + dt)
    gu = H.gen_act(r, (rows, 2 * inter), dt, 0.0, 2.0)
    gu[1] = H.to_storage(np.zeros(2 * inter, np.float32), dt)  # an all-zero SwiGLU row: scale 0
    d_gu = H.to_dev(gu, gpu, dt)
    case(f"silu_and_mul_q8 rows={rows} inter={inter} dt={dt}")
    out, scale, q = ops.silu_and_mul_q8(d_gu, want_out=True)
    plain = ops.silu_and_mul(d_gu)
    got_out = H.to_host(out)
    H.assert_bitexact(got_out, H.to_host(plain), "fused fp output vs nvf_silu_and_mul")
    ref = np.empty((rows, inter), H.NP_STORAGE[dt])
    o.orc_silu_and_mul(H.ptr(gu), H.ptr(ref), rows, inter, dt)
    H.assert_close(got_out, ref, dt, what="fused silu")
    exp_scale = np.empty(rows, np.float32)
    o.orc_q8_row_scale(H.ptr(got_out), H.ptr(exp_scale), rows, inter, dt)
    H.assert_bitexact(scale.cpu().numpy(), exp_scale, "row scale")
    exp_q = np.empty((rows, inter), np.int8)
    o.orc_q8_quantize(H.ptr(got_out), H.ptr(exp_scale), exp_q.ctypes.data, rows, inter, dt)
    H.assert_bitexact(q.cpu().numpy(), exp_q, "int8 rows")
    assert scale[1].item() == 0.0
    # without the fp output: the same scale and int8 rows
    none, scale2, q2 = ops.silu_and_mul_q8(d_gu)
    assert none is None
    H.assert_bitexact(scale2.cpu().numpy(), exp_scale, "row scale (no out)")
    H.assert_bitexact(q2.cpu().numpy(), exp_q, "int8 rows (no out)")


@pytest.mark.parametrize("dt", [H.F16, H.BF16], ids=["f16", "bf16"])
def test_fused_quantizers_feed_the_gemm(gpu, dt):
    """The norm and the SwiGLU hand the GEMM exactly what quantizing their stored
    output would: the products are bit-identical to quantize-then-GEMM."""
    r = H.rng(91 + dt)
    rows, hidden, inter, n = 40, 1024, 2048, 384
    x, res = H.gen_act(r, (rows, hidden), dt), H.gen_act(r, (rows, hidden), dt)
    w = H.gen_act(r, (hidden,), dt, 1.0, 0.1)
    w8a, wsa = H.gen_q8_0(r, n, hidden)
    w8b, wsb = H.gen_q8_0(r, n, inter)
    gu = H.gen_act(r, (rows, 2 * inter), dt)
    case(f"norm -> gemm, swiglu -> gemm dt={dt}")
    d_res = H.to_dev(res, gpu, dt)
    out, sc, q = ops.rms_norm_q8(H.to_dev(x, gpu, dt), H.to_dev(w, gpu, dt), 1e-6, d_res)
    fused = ops.matmul_q8_0(q, sc, H.to_dev(w8a, gpu), H.to_dev(wsa, gpu), n, torch.float32)
    plain = ops.matmul_q8(out, H.to_dev(w8a, gpu), H.to_dev(wsa, gpu), n, torch.float32)
    H.assert_bitexact(fused.cpu().numpy(), plain.cpu().numpy(), "norm -> gemm")
    sout, ssc, sq = ops.silu_and_mul_q8(H.to_dev(gu, gpu, dt), want_out=True)
    fused = ops.matmul_q8_0(sq, ssc, H.to_dev(w8b, gpu), H.to_dev(wsb, gpu), n, torch.float32)
    plain = ops.matmul_q8(sout, H.to_dev(w8b, gpu), H.to_dev(wsb, gpu), n, torch.float32)
    H.assert_bitexact(fused.cpu().numpy(), plain.cpu().numpy(), "swiglu -> gemm")


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("m,k,n,swiglu", [
    (1, 3584, 3584, False),    # batch-1 o projection (W8 S8 workgroups)
    (1, 3584, 37888, False),   # batch-1 gate_up (W4 S1)
    (1, 18944, 3584, True),    # batch-1 down over the SwiGLU of gate | up
    (3, 18944, 3584, True),
    (16, 3584, 4608, False),   # 16 rows: the GEMV's most
    (5, 1024, 520, True),      # ragged column count
])
def test_gemv_with_fused_quantizer(gpu, dt, m, k, n, swiglu):
    """nvf_matmul_q8_0_act (the decode GEMV quantizing fp rows in its prologue) is
    bit-identical to the separate quantizer (nvf_q8_quantize_rows, or nvf_silu_and_mul_q8
    over [gate | up]) followed by nvf_matmul_q8_0; rows may be strided."""
    r = H.rng(m * 7 + k + n + dt + 3 * swiglu)
    w8, ws = H.gen_q8_0(r, n, k)
    d_w8, d_ws = H.to_dev(w8, gpu), H.to_dev(ws, gpu)
    width = 2 * k if swiglu else k
    x_full = H.to_dev(H.gen_act(r, (m, width + 64), dt), gpu, dt)
    x = x_full[:, :width]  # strided rows
    case(f"gemv act m={m} k={k} n={n} swiglu={swiglu} dt={dt}")
    got = ops.matmul_q8_0_act(x, d_w8, d_ws, n, swiglu=swiglu)
    if swiglu:
        _, sc, q = ops.silu_and_mul_q8(x.contiguous())
    else:
        sc, q = ops.q8_quantize_rows(x.contiguous())
    want = ops.matmul_q8_0(q, sc, d_w8, d_ws, n, x.dtype)
    torch.cuda.synchronize()
    H.assert_bitexact(H.to_host(got), H.to_host(want), "fused quantizer vs separate pass")
    # the product against the oracle's bound (fp32 summation of exact block dots)
    o = H.oracle()
    exact = np.empty((m, n), np.float64)
    err = np.empty((m, n), np.float64)
    q_h, sc_h = np.ascontiguousarray(q.cpu().numpy()), sc.cpu().numpy()  # kept alive across the call
    o.orc_matmul_q8_i8(H.ptr(q_h), H.ptr(sc_h), H.ptr(w8), H.ptr(ws), m, n, k, H.ptr(exact), H.ptr(err))
    g = H.from_storage(H.to_host(got), dt)
    assert (np.abs(g - exact) <= err + (0.0 if dt == H.F32 else 0.5 * H.ulp(exact, dt))).all()


def test_gemv_with_fused_quantizer_rejects(gpu):
    x = torch.zeros(17, 1024, dtype=torch.float16, device=gpu)
    w8 = torch.zeros(64 * 1024, dtype=torch.int8, device=gpu)
    ws = torch.zeros(64 * 32, dtype=torch.int16, device=gpu)
    with pytest.raises(RuntimeError, match="m=17"):
        ops.matmul_q8_0_act(x, w8, ws, 64)
    with pytest.raises(RuntimeError, match="do not fit"):  # 8 rows of 18944 bytes: past the staged-row LDS
        ops.matmul_q8_0_act(torch.zeros(8, 2 * 18944, dtype=torch.float16, device=gpu),
                            torch.zeros(64 * 18944, dtype=torch.int8, device=gpu),
                            torch.zeros(64 * 592, dtype=torch.int16, device=gpu), 64, swiglu=True)


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("m,k,n,add", [
    (1, 3584, 4608, True),     # batch-1 qkv after the input norm (W8 S8 workgroups)
    (1, 3584, 37888, True),    # batch-1 gate_up after the post-attention norm (W4 S1)
    (1, 4096, 6144, False),    # first layer: no residual yet
    (3, 3584, 4608, True),
    (16, 2048, 1040, True),    # 16 rows, ragged column count
    (2, 1024, 520, False),     # a 2-wave norm row for fp16/bf16 (128 vectors)
    (1, 512, 256, True),       # a 1-wave norm row
    (1, 8192, 1024, True),     # fp32: a norm row past the preloaded 4 vectors per lane
])
def test_gemv_with_fused_rms_norm(gpu, dt, m, k, n, add):
    """nvf_matmul_q8_0_rms (residual-add + RMSNorm + quantizer in the decode GEMV's
    prologue) is bit-identical to nvf_rms_norm_q8 followed by nvf_matmul_q8_0, the
    residual it writes to the residual of the separate norm, and residual and x are
    left unchanged."""
    r = H.rng(m * 11 + k + n + dt + 5 * add)
    w8, ws = H.gen_q8_0(r, n, k)
    d_w8, d_ws = H.to_dev(w8, gpu), H.to_dev(ws, gpu)
    x_full = H.to_dev(H.gen_act(r, (m, k + 64), dt), gpu, dt)
    x = x_full[:, :k]  # strided rows
    g = H.to_dev(H.gen_act(r, (k,), dt), gpu, dt)
    res = H.to_dev(H.gen_act(r, (m, k), dt), gpu, dt) if add else None
    res_before = res.clone() if add else None
    x_before = x.clone()
    res_out = torch.full_like(res, float("nan")) if add else None
    case(f"gemv rms m={m} k={k} n={n} add={add} dt={dt}")
    got = ops.matmul_q8_0_rms(x, g, 1e-6, d_w8, d_ws, n, residual=res, residual_out=res_out)
    res_sep = res.clone() if add else None
    _, sc, q = ops.rms_norm_q8(x.contiguous(), g, 1e-6, residual=res_sep, want_out=False)
    want = ops.matmul_q8_0(q, sc, d_w8, d_ws, n, x.dtype)
    torch.cuda.synchronize()
    H.assert_bitexact(H.to_host(got), H.to_host(want), "fused norm vs separate norm + GEMV")
    H.assert_bitexact(H.to_host(x), H.to_host(x_before), "x unchanged")
    if add:
        H.assert_bitexact(H.to_host(res_out), H.to_host(res_sep), "residual_out vs the norm's residual")
        H.assert_bitexact(H.to_host(res), H.to_host(res_before), "residual unchanged")


def test_gemv_with_fused_rms_norm_rejects(gpu):
    x = torch.zeros(1, 1024, dtype=torch.float16, device=gpu)
    g = torch.ones(1024, dtype=torch.float16, device=gpu)
    w8 = torch.zeros(64 * 1024, dtype=torch.int8, device=gpu)
    ws = torch.zeros(64 * 32, dtype=torch.int16, device=gpu)
    res = torch.zeros_like(x)
    with pytest.raises(RuntimeError, match="overlap"):
        ops.matmul_q8_0_rms(x, g, 1e-6, w8, ws, 64, residual=res, residual_out=res)
    with pytest.raises(RuntimeError, match="m=17"):
        ops.matmul_q8_0_rms(torch.zeros(17, 1024, dtype=torch.float16, device=gpu), g, 1e-6, w8, ws, 64)


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("tokens,qh,kvh,hd,norm", [
    (37, 28, 4, 128, False),   # Qwen2.5-7B heads, packed [q | k | v] rows
    (5, 32, 8, 128, True),     # Qwen3-8B: QK-norm fused as well
    (7, 40, 8, 128, True),     # 40 + 8 heads (Qwen3-14B): a token's heads in two passes
    (9, 14, 2, 64, False),     # Qwen2.5-0.5B heads
    (3, 4, 1, 256, True),
    (6, 4, 2, 80, False),      # head_dim 80: the two-launch fallback
    (4, 8, 40, 128, False),    # kv row of 5120 elements: past the fused kernel's v row, the fallback
])
def test_qk_norm_rope_store_kv(gpu, dt, tokens, qh, kvh, hd, norm):
    """The fused RoPE + KV store equals nvf_qk_norm_rope followed by nvf_store_kv bit for
    bit: q and k in place, both caches (slot -1 rows untouched, including their prior
    contents)."""
    r = H.rng(tokens * 131 + qh * 7 + kvh + hd + dt)
    tdt = H.torch_dtype(dt)
    width = (qh + 2 * kvh) * hd
    qkv = H.to_dev(H.gen_act(r, (tokens, width), dt, 0.0, 1.0), gpu, dt)
    pos = torch.from_numpy(r.integers(0, 8192, tokens).astype(np.int64)).to(gpu)
    inv = ops.rope_inv_freq(1e6, hd, gpu)
    qw = torch.randn(hd, device=gpu).mul(0.1).add(1.0).to(tdt) if norm else None
    kw = torch.randn(hd, device=gpu).mul(0.1).add(1.0).to(tdt) if norm else None
    rows = 2 * tokens + 3
    slots = r.permutation(rows)[:tokens].astype(np.int32)
    slots[1 % tokens] = -1
    d_slots = torch.from_numpy(slots).to(gpu)
    kc0 = torch.randn(rows, kvh, hd, device=gpu).to(tdt)
    vc0 = torch.randn(rows, kvh, hd, device=gpu).to(tdt)
    qs, ks = qh * hd, kvh * hd

    case(f"qk_norm_rope_store_kv tokens={tokens} heads={qh}/{kvh} hd={hd} norm={norm} dt={dt}")
    a = qkv.clone()
    kc_a, vc_a = kc0.clone(), vc0.clone()
    ops.qk_norm_rope(a[:, :qs], a[:, qs:qs + ks], pos, qw, kw, inv, qh, kvh, hd, 1e-6)
    kv3 = (tokens, kvh, hd)
    ops.store_kv(a[:, qs:qs + ks].view(kv3), a[:, qs + ks:].view(kv3), kc_a, vc_a, d_slots)

    b = qkv.clone()
    kc_b, vc_b = kc0.clone(), vc0.clone()
    ops.qk_norm_rope_store_kv(b[:, :qs], b[:, qs:qs + ks], b[:, qs + ks:], pos, qw, kw, inv, qh, kvh, hd,
                              kc_b, vc_b, d_slots, 1e-6)
    torch.cuda.synchronize()
    H.assert_bitexact(H.to_host(b), H.to_host(a), "q, k in place (and v untouched)")
    H.assert_bitexact(H.to_host(kc_b), H.to_host(kc_a), "k cache")
    H.assert_bitexact(H.to_host(vc_b), H.to_host(vc_a), "v cache")
    untouched = np.setdiff1d(np.arange(rows), slots[slots >= 0])
    H.assert_bitexact(H.to_host(kc_b[untouched]), H.to_host(kc0[untouched]), "rows without a slot")


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("tokens,qh,kvh,hd,norm", [
    (37, 28, 4, 128, False),   # Qwen2.5-7B heads, packed [q | k | v] rows: the bias is Qwen2.5's
    (5, 32, 8, 128, True),     # Qwen3-8B heads with QK-norm (bias and norm together)
    (7, 40, 8, 128, True),     # 40 + 8 heads (Qwen3-14B): a token's heads in two passes
    (9, 14, 2, 64, False),     # Qwen2.5-0.5B heads
    (3, 4, 1, 256, True),
    (6, 4, 2, 80, False),      # head_dim 80: the separate-op fallback (add bias, RoPE, store)
    (4, 8, 40, 128, False),    # kv row of 5120 elements: the fallback
])
def test_qkv_bias_qk_norm_rope_store_kv(gpu, dt, tokens, qh, kvh, hd, norm):
    """nvf_qkv_bias_qk_norm_rope_store_kv against the oracle (model.cpp:768-781 with the
    biased head kept in fp32): q, k within the RoPE tolerance, the v cache bit-exact
    (v + b, one rounding), the k cache equal to the stored k, the v tensor unchanged and
    rows without a slot untouched."""
    o = H.oracle()
    r = H.rng(tokens * 173 + qh * 5 + kvh + hd + dt + 11 * norm)
    tdt = H.torch_dtype(dt)
    qs, ks = qh * hd, kvh * hd
    width = qs + 2 * ks
    qkv_h = H.gen_act(r, (tokens, width), dt, 0.0, 1.0)
    bias = r.normal(0, 0.5, width).astype(np.float32)
    pos = r.integers(0, 8192, tokens).astype(np.int64)
    inv = ops.rope_inv_freq(1e6, hd)
    qw_h = H.gen_act(r, (hd,), dt, 1.0, 0.1) if norm else None
    kw_h = H.gen_act(r, (hd,), dt, 1.0, 0.1) if norm else None
    rows = 2 * tokens + 3
    slots = r.permutation(rows)[:tokens].astype(np.int32)
    slots[1 % tokens] = -1
    kc0 = H.gen_act(r, (rows, ks), dt)
    vc0 = H.gen_act(r, (rows, ks), dt)

    # oracle on separate q, k, v copies
    rq = np.ascontiguousarray(qkv_h[:, :qs])
    rk = np.ascontiguousarray(qkv_h[:, qs:qs + ks])
    rv = np.ascontiguousarray(qkv_h[:, qs + ks:])
    rkc, rvc = kc0.copy(), vc0.copy()
    o.orc_qkv_bias_qk_norm_rope_store_kv(H.ptr(rq), H.ptr(rk), H.ptr(rv), H.ptr(bias), H.ptr(pos), H.ptr(qw_h),
                                         H.ptr(kw_h), H.ptr(inv.numpy()), tokens, qh, kvh, hd, qs, ks, ks, 1e-6,
                                         H.ptr(rkc), H.ptr(rvc), H.ptr(slots), dt)

    case(f"qkv_bias_qk_norm_rope_store_kv tokens={tokens} heads={qh}/{kvh} hd={hd} norm={norm} dt={dt}")
    qkv = H.to_dev(qkv_h, gpu, dt)
    kc, vc = H.to_dev(kc0, gpu, dt).view(rows, kvh, hd), H.to_dev(vc0, gpu, dt).view(rows, kvh, hd)
    ops.qk_norm_rope_store_kv(qkv[:, :qs], qkv[:, qs:qs + ks], qkv[:, qs + ks:], torch.from_numpy(pos).to(gpu),
                              H.to_dev(qw_h, gpu, dt) if norm else None, H.to_dev(kw_h, gpu, dt) if norm else None,
                              inv.to(gpu), qh, kvh, hd, kc, vc, torch.from_numpy(slots).to(gpu), 1e-6,
                              qkv_bias=torch.from_numpy(bias).to(gpu))
    torch.cuda.synchronize()
    got = H.to_host(qkv)
    H.assert_close(np.ascontiguousarray(got[:, :qs]), rq, dt, floor=1e-6, what="q")
    H.assert_close(np.ascontiguousarray(got[:, qs:qs + ks]), rk, dt, floor=1e-6, what="k")
    H.assert_bitexact(np.ascontiguousarray(got[:, qs + ks:]), rv, "v tensor unchanged")
    gkc, gvc = H.to_host(kc).reshape(rows, ks), H.to_host(vc).reshape(rows, ks)
    live = slots[slots >= 0]
    H.assert_bitexact(gvc, rvc, "v cache (v + b)")
    H.assert_bitexact(gkc[live], np.ascontiguousarray(got[:, qs:qs + ks])[slots >= 0], "k cache == stored k")
    untouched = np.setdiff1d(np.arange(rows), live)
    H.assert_bitexact(gkc[untouched], kc0[untouched], "k rows without a slot")


def test_add_bias_vs_reference_kernel(gpu):
    """hip_add_bias_inplace (drop-in) bit-exact against the reference's own add_bias_kernel
    (src/hip_ops.hip:366-371) and the oracle; the typed nvf_add_bias on strided 16-bit rows
    bit-exact against the oracle."""
    ref = H.ref_hip()
    r = H.rng(21)
    rows, cols = 37, 4608
    x = r.normal(0, 1, (rows, cols)).astype(np.float32)
    b = r.normal(0, 1, cols).astype(np.float32)
    want = x.copy()
    H.oracle().orc_add_bias(H.ptr(want), H.ptr(b), rows, cols, cols, H.F32)
    db = torch.from_numpy(b).to(gpu)
    mine = torch.from_numpy(x).to(gpu)
    case("hip_add_bias_inplace")
    ops.lib().hip_add_bias_inplace(mine.data_ptr(), db.data_ptr(), rows, cols)
    torch.cuda.synchronize()
    H.assert_bitexact(mine.cpu().numpy(), want, "drop-in vs oracle")
    if ref is not None:
        theirs = torch.from_numpy(x).to(gpu)
        case("reference add_bias kernel")
        ref.ref_hip_add_bias_inplace(theirs.data_ptr(), db.data_ptr(), rows, cols)
        H.assert_bitexact(mine.cpu().numpy(), theirs.cpu().numpy(), "drop-in vs reference kernel")
    for dt in (H.F16, H.BF16):
        xs = H.gen_act(r, (rows, cols + 64), dt)
        want = xs.copy()
        H.oracle().orc_add_bias(H.ptr(want), H.ptr(b), rows, cols, cols + 64, dt)
        d = H.to_dev(xs, gpu, dt)
        case(f"nvf_add_bias dt={dt}")
        ops.add_bias(d[:, :cols], db)
        torch.cuda.synchronize()
        H.assert_bitexact(H.to_host(d), want, f"nvf_add_bias dt={dt}")


def test_qk_norm_rope_store_kv_bad_args(gpu):
    q = torch.zeros(2, 256, dtype=torch.float16, device=gpu)
    k = torch.zeros(2, 128, dtype=torch.float16, device=gpu)
    pos = torch.zeros(2, dtype=torch.int64, device=gpu)
    inv = ops.rope_inv_freq(1e6, 128, gpu)
    kc = torch.zeros(4, 1, 128, dtype=torch.float16, device=gpu)
    slots = torch.zeros(2, dtype=torch.int32, device=gpu)
    v_narrow = torch.zeros(2, 64, dtype=torch.float16, device=gpu)  # row stride 64 < kv_heads * head_dim
    with pytest.raises(ValueError):  # the Python front end checks v's shape
        ops.qk_norm_rope_store_kv(q, k, v_narrow, pos, None, None, inv, 2, 1, 128, kc, kc.clone(), slots)
    with pytest.raises(ValueError):  # an int64 slot mapping
        ops.qk_norm_rope_store_kv(q, k, k, pos, None, None, inv, 2, 1, 128, kc, kc.clone(), slots.long())
    with pytest.raises(ValueError):  # a cache of another dtype
        ops.qk_norm_rope_store_kv(q, k, k, pos, None, None, inv, 2, 1, 128, kc.float(), kc.clone(), slots)
    with pytest.raises(RuntimeError):  # and so does the C ABI (v row stride 64 < kv_heads * head_dim)
        ops._check(ops.lib().nvf_qk_norm_rope_store_kv(q.data_ptr(), k.data_ptr(), v_narrow.data_ptr(),
                                                       pos.data_ptr(), None, None, inv.data_ptr(), 2, 2, 1, 128, 256,
                                                       128, 64, 1e-6, kc.data_ptr(), kc.data_ptr(), slots.data_ptr(),
                                                       1, None), "qk_norm_rope_store_kv")
    with pytest.raises(RuntimeError):  # no slot mapping
        lib_rc = ops.lib().nvf_qk_norm_rope_store_kv(q.data_ptr(), k.data_ptr(), k.data_ptr(), pos.data_ptr(), None,
                                                     None, inv.data_ptr(), 2, 2, 1, 128, 256, 128, 128, 1e-6,
                                                     kc.data_ptr(), kc.data_ptr(), None, 1, None)
        ops._check(lib_rc, "qk_norm_rope_store_kv")
