"""GPU parity: every HIP path of libnvf_ops.so against the C oracle on the same
seeded inputs (oracle-speed sizes), through the C ABI.

Bars: embedding gathers and the stored residual bit-exact; RMSNorm, SwiGLU,
RoPE and QK-norm within max(1e-5 * |ref|, 1 ulp of the output dtype), with an
absolute floor of 1e-6 (inputs have rms ~1) for RoPE outputs that come from
cancellation (x1 c - x2 s near zero).
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


def o():
    return H.oracle()


# ---------------------------------------------------------------------------
# embeddings
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("hidden", [896, 3584, 4096, 96, 160])
def test_embedding_q8_0_split_and_blocks(gpu, dt, hidden):
    r = H.rng(hidden + dt)
    V, T = 1000, 77
    w8, ws = H.gen_q8_0(r, V, hidden)
    ws[:8] = [0x0001, 0x03FF, 0x8001, 0x0400, 0x7BFF, 0x0000, 0x8000, 0x3C00]  # subnormal/normal edges
    blocks = H.q8_split_to_blocks(w8, ws)
    ids = r.integers(0, V, T).astype(np.int64)
    ids[:3] = [0, V - 1, 0]
    ref = np.empty((T, hidden), H.NP_STORAGE[dt])
    o().orc_embedding_q8_split(H.ptr(ids), H.ptr(w8), H.ptr(ws), T, hidden, H.ptr(ref), dt)
    case(f"embedding_q8_0 split hidden={hidden} dt={dt}")
    d_ids = H.to_dev(ids, gpu)
    got = ops.embedding_q8_0(d_ids, H.to_dev(w8, gpu), H.to_dev(ws, gpu), hidden, V, out_dtype=H.torch_dtype(dt))
    H.assert_bitexact(H.to_host(got), ref, "q8_0 split")
    case(f"embedding_q8_0 blocks hidden={hidden} dt={dt}")
    got = ops.embedding_q8_0_blocks(d_ids, H.to_dev(blocks, gpu), hidden, V, out_dtype=H.torch_dtype(dt))
    H.assert_bitexact(H.to_host(got), ref, "q8_0 blocks")


def test_embedding_q8_0_blocks_odd_offsets(gpu):
    """Tables whose block starts are 2 mod 4 (hidden 896 -> 952 B rows; a 2-byte table offset)."""
    r = H.rng(31)
    V, T, hidden = 300, 64, 896
    w8, ws = H.gen_q8_0(r, V, hidden)
    blocks = H.q8_split_to_blocks(w8, ws)
    ids = r.integers(0, V, T).astype(np.int64)
    ref = np.empty((T, hidden), np.uint16)
    o().orc_embedding_q8_split(H.ptr(ids), H.ptr(w8), H.ptr(ws), T, hidden, H.ptr(ref), H.F16)
    padded = np.zeros(blocks.size + 4, np.uint8)
    padded[2:2 + blocks.size] = blocks
    dev = H.to_dev(padded, gpu)
    case("embedding_q8_0 blocks at a 2-byte table offset")
    got = ops.embedding_q8_0_blocks(H.to_dev(ids, gpu), dev[2:2 + blocks.size], hidden, V, out_dtype=torch.float16)
    H.assert_bitexact(H.to_host(got), ref, "q8_0 blocks, 2-byte offset")


@pytest.mark.parametrize("layout", [H.GGML, H.HIP_LEGACY], ids=["ggml", "hip_legacy"])
@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("hidden", [3584, 256, 896])
def test_embedding_q4_k(gpu, layout, dt, hidden):
    r = H.rng(hidden * 3 + dt + 10 * layout)
    V, T = 256, 70
    blocks = H.gen_q4_k(r, V * hidden // 256)
    blocks[0:2] = np.array([np.float16(6e-8)], np.float16).view(np.uint8)  # subnormal d
    ids = r.integers(0, V, T).astype(np.int64)
    ids[0] = 0
    ref = np.empty((T, hidden), H.NP_STORAGE[dt])
    o().orc_embedding_qk(H.ptr(ids), H.ptr(blocks), T, hidden, 12, layout, H.ptr(ref), dt)
    case(f"embedding_q4_k hidden={hidden} dt={dt} layout={layout}")
    got = ops.embedding_qk(H.to_dev(ids, gpu), H.to_dev(blocks, gpu), hidden, ops.Q4_K, V, layout,
                           out_dtype=H.torch_dtype(dt))
    H.assert_bitexact(H.to_host(got), ref, "q4_k")


@pytest.mark.parametrize("kind,bb,fp16_off", [(13, 176, (0, 2)), (14, 210, (208,))], ids=["q5_k", "q6_k"])
@pytest.mark.parametrize("hidden", [512, 896, 3584])
def test_embedding_q5_q6_k(gpu, kind, bb, fp16_off, hidden):
    r = H.rng(kind * 7 + hidden)
    V, T = 64, 33
    blocks = H.gen_raw_blocks(r, V * hidden // 256, bb, fp16_off)
    ids = r.integers(0, V, T).astype(np.int64)
    ids[:2] = [V - 1, 0]  # the table's last superblock (Q6_K: 2-byte aligned end) and its first
    for dt in DTYPES:
        ref = np.empty((T, hidden), H.NP_STORAGE[dt])
        o().orc_embedding_qk(H.ptr(ids), H.ptr(blocks), T, hidden, kind, H.GGML, H.ptr(ref), dt)
        case(f"embedding kind={kind} hidden={hidden} dt={dt}")
        got = ops.embedding_qk(H.to_dev(ids, gpu), H.to_dev(blocks, gpu), hidden, kind, V,
                               out_dtype=H.torch_dtype(dt))
        H.assert_bitexact(H.to_host(got), ref, f"kind {kind}")


@pytest.mark.parametrize("fmt,hidden", [("q8_0_blocks", 15424), ("q4_k", 29440), ("q5_k", 24064),
                                        ("q6_k", 20480)])
def test_embedding_rows_beyond_the_lds_stage(gpu, fmt, hidden):
    """Rows longer than the 16 KiB per-wave LDS stage take the direct-load path."""
    r = H.rng(hidden)
    V, T = 8, 12
    ids = r.integers(0, V, T).astype(np.int64)
    ids[0] = V - 1
    if fmt == "q8_0_blocks":
        w8, ws = H.gen_q8_0(r, V, hidden)
        blocks = H.q8_split_to_blocks(w8, ws)
        ref = np.empty((T, hidden), np.uint16)
        o().orc_embedding_q8_split(H.ptr(ids), H.ptr(w8), H.ptr(ws), T, hidden, H.ptr(ref), H.F16)
        case(f"q8_0 blocks direct path hidden={hidden}")
        got = ops.embedding_q8_0_blocks(H.to_dev(ids, gpu), H.to_dev(blocks, gpu), hidden, V, out_dtype=torch.float16)
    else:
        kind, bb, offs = {"q4_k": (12, 144, (0, 2)), "q5_k": (13, 176, (0, 2)), "q6_k": (14, 210, (208,))}[fmt]
        blocks = H.gen_raw_blocks(r, V * hidden // 256, bb, offs)
        ref = np.empty((T, hidden), np.uint16)
        o().orc_embedding_qk(H.ptr(ids), H.ptr(blocks), T, hidden, kind, H.GGML, H.ptr(ref), H.F16)
        case(f"{fmt} direct path hidden={hidden}")
        got = ops.embedding_qk(H.to_dev(ids, gpu), H.to_dev(blocks, gpu), hidden, kind, V, out_dtype=torch.float16)
    H.assert_bitexact(H.to_host(got), ref, f"{fmt} direct path")


@pytest.mark.parametrize("tdt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("hidden", [896, 100])
def test_embedding_table(gpu, tdt, hidden):
    r = H.rng(tdt + hidden)
    V, T = 500, 40
    table = H.gen_act(r, (V, hidden), tdt)
    ids = r.integers(0, V, T).astype(np.int64)
    vals = H.from_storage(table, tdt)[ids]
    for odt in DTYPES:
        case(f"embedding table tdt={tdt} out={odt} hidden={hidden}")
        got = ops.embedding(H.to_dev(ids, gpu), H.to_dev(table, gpu, tdt), V, out_dtype=H.torch_dtype(odt))
        H.assert_bitexact(H.to_host(got), H.to_storage(vals, odt), "table gather")


def test_embedding_out_of_range_ids_give_nan_rows(gpu):
    r = H.rng(41)
    V, hidden = 100, 512
    w8, ws = H.gen_q8_0(r, V, hidden)
    ids = np.array([5, -1, V, 7, 1 << 40], np.int64)
    case("embedding out-of-range ids")
    got = ops.embedding_q8_0(H.to_dev(ids, gpu), H.to_dev(w8, gpu), H.to_dev(ws, gpu), hidden, V,
                             out_dtype=torch.float32).cpu().numpy()
    assert np.isnan(got[[1, 2, 4]]).all() and np.isfinite(got[[0, 3]]).all()
    blocks = H.gen_q4_k(r, V * hidden // 256)
    got = ops.embedding_qk(H.to_dev(ids, gpu), H.to_dev(blocks, gpu), hidden, ops.Q4_K, V,
                           out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.isnan(got[[1, 2, 4]]).all() and np.isfinite(got[[0, 3]]).all()
    # the staged gathers with two waves per row (8 blocks of 256), Q6_K's four-slot decode among them
    wide = 2048
    for kind in (ops.Q5_K, ops.Q6_K):
        bb, offs = H.KQ_BLOCK[kind]
        blocks = H.gen_raw_blocks(r, V * wide // 256, bb, offs)
        case(f"embedding out-of-range ids kind={kind}")
        got = ops.embedding_qk(H.to_dev(ids, gpu), H.to_dev(blocks, gpu), wide, kind, V,
                               out_dtype=torch.float16).float().cpu().numpy()
        assert np.isnan(got[[1, 2, 4]]).all() and np.isfinite(got[[0, 3]]).all()


# ---------------------------------------------------------------------------
# residual-add + RMSNorm
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("rows,hidden", [(64, 896), (37, 3584), (16, 4096), (5, 1000), (3, 999), (2, 20000),
                                         (1, 8)])
def test_rms_norm_add(gpu, dt, rows, hidden):
    r = H.rng(rows * hidden + dt)
    x, res = H.gen_act(r, (rows, hidden), dt), H.gen_act(r, (rows, hidden), dt)
    w = H.gen_act(r, (hidden,), dt, 1.0, 0.1)
    ref_res, ref_out = res.copy(), np.empty_like(x)
    o().orc_rms_norm_add(H.ptr(x), H.ptr(ref_res), H.ptr(w), H.ptr(ref_out), rows, hidden, 1e-6, dt)
    case(f"rms_norm_add rows={rows} hidden={hidden} dt={dt}")
    d_res = H.to_dev(res, gpu, dt)
    out = ops.rms_norm_add(H.to_dev(x, gpu, dt), d_res, H.to_dev(w, gpu, dt), 1e-6)
    H.assert_bitexact(H.to_host(d_res), ref_res, "residual")
    H.assert_close(H.to_host(out), ref_out, dt, what="rms_norm_add out")


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("rows,hidden", [(100, 128), (7, 3584), (4, 333)])
def test_rms_norm_inplace(gpu, dt, rows, hidden):
    r = H.rng(rows + hidden + dt)
    x = H.gen_act(r, (rows, hidden), dt)
    w = H.gen_act(r, (hidden,), dt, 1.0, 0.1)
    ref = np.empty_like(x)
    o().orc_rms_norm(H.ptr(x), H.ptr(w), H.ptr(ref), rows, hidden, 1e-6, dt)
    case(f"rms_norm in place rows={rows} hidden={hidden} dt={dt}")
    dx = H.to_dev(x, gpu, dt)
    ops.rms_norm(dx, H.to_dev(w, gpu, dt), 1e-6, out=dx)
    H.assert_close(H.to_host(dx), ref, dt, what="rms_norm")


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("rows,inter", [(64, 4864), (3, 18944), (17, 12288), (5, 999), (1, 8)])
def test_silu_and_mul(gpu, dt, rows, inter):
    r = H.rng(rows * inter + dt)
    gu = H.gen_act(r, (rows, 2 * inter), dt, 0.0, 2.0)
    ref = np.empty((rows, inter), H.NP_STORAGE[dt])
    o().orc_silu_and_mul(H.ptr(gu), H.ptr(ref), rows, inter, dt)
    case(f"silu_and_mul rows={rows} inter={inter} dt={dt}")
    got = ops.silu_and_mul(H.to_dev(gu, gpu, dt))
    H.assert_close(H.to_host(got), ref, dt, what="silu_and_mul")


def test_silu_extremes(gpu):
    g = np.array([0, 1e-30, -1e-30, 88, -88, 100, -100, 1e4, -1e4, np.inf, -np.inf, 3.5], np.float32)
    for dt in DTYPES:
        gu = H.to_storage(np.concatenate([g, np.full_like(g, 1.5)]).reshape(1, -1), dt)
        ref = np.empty((1, g.size), H.NP_STORAGE[dt])
        o().orc_silu_and_mul(H.ptr(gu), H.ptr(ref), 1, g.size, dt)
        case(f"silu extremes dt={dt}")
        got = H.to_host(ops.silu_and_mul(H.to_dev(gu, gpu, dt)))
        # both NaN for -inf (-inf * 0), otherwise within tolerance; the 1e-35 floor covers
        # g < -87 where 1/(1 + e^-g) is an fp32 subnormal (bf16 keeps fp32's range)
        H.assert_close(got, ref, dt, floor=1e-35, what=f"silu extremes dt={dt}")


# ---------------------------------------------------------------------------
# QK-norm + RoPE
# ---------------------------------------------------------------------------
def _rope_case(gpu, dt, T, hq, hk, hd, norm, packed, seed, positions=None):
    r = H.rng(seed)
    qs, ks = hq * hd, hk * hd
    inv = np.empty(hd // 2, np.float32)
    o().orc_inv_freq(1e6, hd, H.ptr(inv))
    pos = positions if positions is not None else r.integers(0, 4096, T).astype(np.int64)
    qw = H.gen_act(r, (hd,), dt, 1.0, 0.1) if norm else None
    kw = H.gen_act(r, (hd,), dt, 1.0, 0.1) if norm else None
    if packed:  # one [T, q | k | v] buffer, as the fused qkv projection writes it
        qkv = H.gen_act(r, (T, qs + 2 * ks), dt)
        ref = qkv.copy()
        stride = qs + 2 * ks
        # oracle on views with the same strides: work on copies of q and k columns
        q, k = np.ascontiguousarray(ref[:, :qs]), np.ascontiguousarray(ref[:, qs:qs + ks])
        o().orc_qk_norm_rope(H.ptr(q), H.ptr(k), H.ptr(pos), H.ptr(qw), H.ptr(kw), H.ptr(inv), T, hq, hk, hd, qs, ks,
                             1e-6, dt)
        ref[:, :qs], ref[:, qs:qs + ks] = q, k
        d = H.to_dev(qkv, gpu, dt)
        flat = d.view(-1)
        case(f"qk_norm_rope packed T={T} hq={hq} hk={hk} hd={hd} norm={norm} dt={dt}")
        # hold every device tensor in a name: a temporary's memory can be reused before the kernel runs
        d_pos, d_inv = H.to_dev(pos, gpu), H.to_dev(inv, gpu)
        d_qw = H.to_dev(qw, gpu, dt) if norm else None
        d_kw = H.to_dev(kw, gpu, dt) if norm else None
        rc = ops.lib().nvf_qk_norm_rope(flat.data_ptr(), flat[qs:].data_ptr(), d_pos.data_ptr(),
                                        d_qw.data_ptr() if norm else None, d_kw.data_ptr() if norm else None,
                                        d_inv.data_ptr(), T, hq, hk, hd, stride, stride, 1e-6, dt,
                                        torch.cuda.current_stream().cuda_stream)
        assert rc == 0, ops.lib().nvf_last_error()
        got = H.to_host(d)
        H.assert_close(got, ref, dt, floor=1e-6, what="qk_norm_rope packed")
        # the same through the Python front end, on views of the packed row (v untouched)
        d2 = H.to_dev(qkv, gpu, dt)
        ops.qk_norm_rope(d2[:, :qs], d2[:, qs:qs + ks], d_pos, d_qw, d_kw, d_inv, hq, hk, hd)
        H.assert_close(H.to_host(d2), ref, dt, floor=1e-6, what="qk_norm_rope packed views")
        return
    q, k = H.gen_act(r, (T, qs), dt), H.gen_act(r, (T, ks), dt)
    rq, rk = q.copy(), k.copy()
    o().orc_qk_norm_rope(H.ptr(rq), H.ptr(rk), H.ptr(pos), H.ptr(qw), H.ptr(kw), H.ptr(inv), T, hq, hk, hd, qs, ks,
                         1e-6, dt)
    dq, dk = H.to_dev(q, gpu, dt), H.to_dev(k, gpu, dt)
    case(f"qk_norm_rope T={T} hq={hq} hk={hk} hd={hd} norm={norm} dt={dt}")
    ops.qk_norm_rope(dq, dk, H.to_dev(pos, gpu), H.to_dev(qw, gpu, dt) if norm else None,
                     H.to_dev(kw, gpu, dt) if norm else None, H.to_dev(inv, gpu), hq, hk, hd)
    H.assert_close(H.to_host(dq), rq, dt, floor=1e-6, what="q")
    H.assert_close(H.to_host(dk), rk, dt, floor=1e-6, what="k")


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("norm", [False, True], ids=["rope", "qknorm_rope"])
@pytest.mark.parametrize("hq,hk,hd", [(14, 2, 64), (28, 4, 128), (32, 8, 128), (40, 8, 128), (64, 8, 128), (4, 1, 256), (3, 1, 80)])
def test_qk_norm_rope(gpu, dt, norm, hq, hk, hd):
    _rope_case(gpu, dt, 61, hq, hk, hd, norm, False, seed=hq * hd + dt + norm)


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
def test_qk_norm_rope_packed_qkv(gpu, dt):
    _rope_case(gpu, dt, 40, 32, 8, 128, True, True, seed=99 + dt)
    _rope_case(gpu, dt, 40, 28, 4, 128, False, True, seed=98 + dt)


def test_rope_large_positions(gpu):
    pos = np.array([0, 1, 4095, 8191, 65535, 1 << 20, 12345, 3], np.int64)
    _rope_case(gpu, H.F32, pos.size, 4, 2, 128, False, False, seed=5, positions=pos)


# ---------------------------------------------------------------------------
# streams
# ---------------------------------------------------------------------------
def test_ops_follow_the_current_stream(gpu):
    r = H.rng(77)
    rows, inter = 256, 4096
    gu = H.gen_act(r, (rows, 2 * inter), H.F16)
    ref = np.empty((rows, inter), np.uint16)
    o().orc_silu_and_mul(H.ptr(gu), H.ptr(ref), rows, inter, H.F16)
    d = H.to_dev(gu, gpu, H.F16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    case("silu on a side stream")
    with torch.cuda.stream(s):
        out = ops.silu_and_mul(d)
    s.synchronize()
    H.assert_close(H.to_host(out), ref, H.F16, what="side stream")


def test_stream_copy(gpu):
    src = torch.arange(1 << 20, dtype=torch.int32, device=gpu)
    dst = torch.zeros_like(src)
    case("stream_copy 4 MiB")
    ops.stream_copy(dst, src)
    assert torch.equal(dst, src)


def test_stream_expand(gpu):
    src = torch.arange(1 << 18, dtype=torch.int32, device=gpu)
    dst = torch.zeros(1 << 19, dtype=torch.int32, device=gpu)
    case("stream_expand 1 MiB -> 2 MiB")
    ops.stream_expand(dst, src)
    # each 8 bytes (two int32) written twice into 16 bytes
    assert torch.equal(dst.view(-1, 4), src.view(-1, 2).repeat(1, 2))
