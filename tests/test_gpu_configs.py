"""The BASELINE configs at full size on the GPU.

Every op of each config runs at its real shape and dtype.  Rows are independent
in every op, so the oracle checks a seeded sample of rows (all rows where the C
oracle finishes in seconds) and size-independent properties cover the rest:
finite outputs, residual_out == x + residual_in rounded once (checked on the
GPU for every element), and RoPE's per-pair norm preservation.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_vllm_cpp_amd import ops
from tests import harness as H

pytestmark = pytest.mark.gpu


def case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def gen(shape, dt, g, mean=0.0, std=1.0, device="cuda:0"):
    return (torch.randn(shape, generator=g, device=device) * std + mean).to(H.torch_dtype(dt))


def sample_rows(n: int, k: int, seed: int) -> np.ndarray:
    if n <= k:
        return np.arange(n)
    return np.sort(np.random.default_rng(seed).choice(n, k, replace=False))


@pytest.mark.parametrize("ci", [1, 2, 3, 4])
def test_config_full_size(gpu, ci):
    cfg = H.CONFIGS[ci]
    o = H.oracle()
    g = torch.Generator(device=gpu).manual_seed(cfg.seed)
    T, Hd, I, V, dt = cfg.tokens, cfg.hidden, cfg.inter, cfg.vocab, cfg.dtype
    tdt = H.torch_dtype(dt)
    rows = sample_rows(T, 2048 if T <= 16384 else 1024, cfg.seed)
    np_rows = np.ascontiguousarray(rows)

    # --- embedding gather ---------------------------------------------------
    ids = torch.randint(0, V, (T,), generator=g, device=gpu, dtype=torch.int64)
    ids_h = ids.cpu().numpy()
    sub_ids = np.ascontiguousarray(ids_h[rows])
    if cfg.emb == "q8_0":
        w8 = torch.randint(-127, 128, (V * Hd,), generator=g, device=gpu, dtype=torch.int8)
        ws = torch.empty(V * Hd // 32, device=gpu).uniform_(1e-3, 1e-2, generator=g).half().view(torch.int16)
        case(f"c{ci} embedding_q8_0 T={T} H={Hd}")
        emb = ops.embedding_q8_0(ids, w8, ws, Hd, V, out_dtype=tdt)
        ref = np.empty((rows.size, Hd), H.NP_STORAGE[dt])
        w8h, wsh = w8.cpu().numpy(), ws.cpu().numpy().view(np.uint16)
        o.orc_embedding_q8_split(H.ptr(sub_ids), H.ptr(w8h), H.ptr(wsh), rows.size, Hd, H.ptr(ref), dt)
        H.assert_bitexact(H.to_host(emb)[rows], ref, f"c{ci} embedding_q8_0")
        blocks = torch.from_numpy(H.q8_split_to_blocks(w8h, wsh)).to(gpu)
        del w8, ws
        case(f"c{ci} embedding_q8_0_blocks")
        emb2 = ops.embedding_q8_0_blocks(ids, blocks, Hd, V, out_dtype=tdt)
        assert torch.equal(emb.view(torch.int16), emb2.view(torch.int16))
        del blocks, emb2
    else:
        nb = V * Hd // 256
        blocks_h = H.gen_q4_k(np.random.default_rng(cfg.seed), nb)
        case(f"c{ci} embedding_q4_k T={T} H={Hd}")
        emb = ops.embedding_qk(ids, torch.from_numpy(blocks_h).to(gpu), Hd, ops.Q4_K, V, out_dtype=tdt)
        ref = np.empty((rows.size, Hd), H.NP_STORAGE[dt])
        o.orc_embedding_qk(H.ptr(sub_ids), H.ptr(blocks_h), rows.size, Hd, 12, H.GGML, H.ptr(ref), dt)
        H.assert_bitexact(H.to_host(emb)[rows], ref, f"c{ci} embedding_q4_k")
    del emb

    # --- residual-add + RMSNorm ---------------------------------------------
    x, res = gen((T, Hd), dt, g), gen((T, Hd), dt, g)
    w = gen((Hd,), dt, g, 1.0, 0.1)
    x_h, res_h, w_h = H.to_host(x), H.to_host(res), H.to_host(w)
    expect_res = (x.float() + res.float()).to(tdt)
    case(f"c{ci} rms_norm_add [{T},{Hd}]")
    out = ops.rms_norm_add(x, res, w, cfg.eps)
    assert torch.equal(res.view(torch.int16), expect_res.view(torch.int16)), "residual != x + residual"
    assert torch.isfinite(out).all()
    sr = np.ascontiguousarray(res_h[rows])
    ref = np.empty_like(sr)
    sx = np.ascontiguousarray(x_h[rows])  # keep every array the oracle reads alive across the call
    o.orc_rms_norm_add(H.ptr(sx), H.ptr(sr), H.ptr(w_h), H.ptr(ref), rows.size, Hd, cfg.eps, dt)
    H.assert_close(H.to_host(out)[rows], ref, dt, what=f"c{ci} rms_norm_add")
    del x, res, out, expect_res

    # --- (QK-norm +) RoPE ----------------------------------------------------
    qs, ks = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    q, k = gen((T, qs), dt, g), gen((T, ks), dt, g)
    q_h, k_h = H.to_host(q), H.to_host(k)
    pos = cfg.positions()
    inv = ops.rope_inv_freq(cfg.theta, cfg.head_dim)
    qw = gen((cfg.head_dim,), dt, g, 1.0, 0.1) if cfg.qk_norm else None
    kw = gen((cfg.head_dim,), dt, g, 1.0, 0.1) if cfg.qk_norm else None
    case(f"c{ci} qk_norm_rope T={T} norm={cfg.qk_norm}")
    ops.qk_norm_rope(q, k, torch.from_numpy(pos).to(gpu), qw, kw, inv.to(gpu), cfg.q_heads, cfg.kv_heads,
                     cfg.head_dim, cfg.eps)
    rq, rk = np.ascontiguousarray(q_h[rows]), np.ascontiguousarray(k_h[rows])
    rpos = np.ascontiguousarray(pos[rows])
    qw_h = H.to_host(qw) if qw is not None else None
    kw_h = H.to_host(kw) if kw is not None else None
    inv_h = inv.numpy()
    o.orc_qk_norm_rope(H.ptr(rq), H.ptr(rk), H.ptr(rpos), H.ptr(qw_h), H.ptr(kw_h), H.ptr(inv_h), rows.size,
                       cfg.q_heads, cfg.kv_heads, cfg.head_dim, qs, ks, cfg.eps, dt)
    H.assert_close(H.to_host(q)[rows], rq, dt, floor=1e-6, what=f"c{ci} rope q")
    H.assert_close(H.to_host(k)[rows], rk, dt, floor=1e-6, what=f"c{ci} rope k")
    if not cfg.qk_norm:  # rotation preserves each pair's norm (all rows, on the GPU)
        a = torch.from_numpy(q_h.view(np.int16)).to(gpu).view(tdt).float().view(T, cfg.q_heads, 2, -1)
        b = q.float().view(T, cfg.q_heads, 2, -1)
        na, nb_ = (a * a).sum(2), (b * b).sum(2)
        assert torch.allclose(na, nb_, rtol=2e-2 if dt != H.F32 else 1e-5, atol=1e-2)
    del q, k

    # --- SwiGLU ----------------------------------------------------------------
    gu = gen((T, 2 * I), dt, g, 0.0, 1.0)
    case(f"c{ci} silu_and_mul [{T},{I}]")
    out = ops.silu_and_mul(gu)
    assert not torch.isnan(out).any()
    sub = np.ascontiguousarray(H.to_host(gu[torch.from_numpy(rows).to(gpu)]))
    ref = np.empty((rows.size, I), H.NP_STORAGE[dt])
    o.orc_silu_and_mul(H.ptr(sub), H.ptr(ref), rows.size, I, dt)
    H.assert_close(H.to_host(out)[rows], ref, dt, what=f"c{ci} silu_and_mul")
    torch.cuda.synchronize()
