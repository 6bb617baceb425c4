"""Pins the C oracle (oracle/nvf_oracle.c) before it is trusted as the checker.

Each function is checked against the reference's own outputs (golden vectors
written by the reference's gguf.cpp / common.hpp, and the live reference build
in oracle/_ref when present), hand vectors from the reference's tests, or what
the mathematics fixes (closed forms, invariants, exhaustive codec checks).
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from tests import harness as H

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "reference_vectors.npz")


@pytest.fixture(scope="module")
def o():
    return H.oracle()


# ---------------------------------------------------------------------------
# storage codecs
# ---------------------------------------------------------------------------
def test_fp16_decode_exhaustive(o):
    codes = np.arange(65536, dtype=np.uint16)
    got = np.array([o.orc_fp16_to_f32(int(c)) for c in codes], np.float32)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp16_codecs_match_reference_vectors(o):
    got = np.array([o.orc_fp16_to_f32(int(c)) for c in GOLD["fp16_codes"]], np.float32)
    ref = GOLD["fp16_decoded"]
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    enc = np.array([o.orc_f32_to_fp16(float(v)) for v in GOLD["f32_values"]], np.uint16)
    assert np.array_equal(enc, GOLD["fp16_encoded"])


def test_fp16_encode_matches_numpy_rne(o):
    r = np.random.default_rng(1)
    f = np.concatenate([r.normal(0, 1, 4000), r.normal(0, 1e-6, 2000), r.uniform(-7e4, 7e4, 2000),
                        (np.arange(1, 3000) + 0.5) * 2.0 ** -24, [0.0, -0.0, np.inf, -np.inf]]).astype(np.float32)
    got = np.array([o.orc_f32_to_fp16(float(v)) for v in f], np.uint16)
    with np.errstate(over="ignore"):
        assert np.array_equal(got, f.astype(np.float16).view(np.uint16))


def test_bf16_codecs_match_torch(o):
    r = np.random.default_rng(2)
    f = np.concatenate([r.normal(0, 1, 4000), r.normal(0, 1e30, 500), r.normal(0, 1e-30, 500),
                        [0.0, -0.0, np.inf, -np.inf]]).astype(np.float32)
    # exact ties: low 16 bits == 0x8000 with even and odd kept mantissa
    ties = (r.integers(0x3F000000 >> 16, 0x43000000 >> 16, 200).astype(np.uint32) << 16) | 0x8000
    f = np.concatenate([f, ties.view(np.float32)])
    got = np.array([o.orc_f32_to_bf16(float(v)) for v in f], np.uint16)
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    back = np.array([o.orc_bf16_to_f32(int(c)) for c in got], np.float32)
    assert np.array_equal(back.view(np.uint32), got.astype(np.uint32) << 16)
    assert np.array_equal(H.to_storage(f, H.BF16), ref)


# ---------------------------------------------------------------------------
# Q8_0
# ---------------------------------------------------------------------------
def test_q8_0_hand_vector(o):
    """vulkanised/test_gguf2vk.py:77-83: scale 2.0 x [0,1,-1,127,-127] -> [0,2,-2,254,-254]."""
    q = np.array([0, 1, -1, 127, -127] + [0] * 27, np.int8)
    ws = np.array([np.float16(2.0)], np.float16).view(np.uint16)
    blocks = H.q8_split_to_blocks(q, ws)
    ids = np.zeros(1, np.int64)
    for dt in (H.F32, H.F16, H.BF16):
        a = np.empty(32, H.NP_STORAGE[dt])
        b = np.empty(32, H.NP_STORAGE[dt])
        o.orc_embedding_q8_split(H.ptr(ids), H.ptr(q), H.ptr(ws), 1, 32, H.ptr(a), dt)
        o.orc_embedding_q8_blocks(H.ptr(ids), H.ptr(blocks), 1, 32, H.ptr(b), dt)
        assert list(H.from_storage(a, dt)[:5]) == [0, 2, -2, 254, -254]
        assert np.array_equal(a, b)


def test_q8_0_gather_exact_product(o):
    """Split planes == 34 B blocks == fp16(scale) * int8 computed in float64 (exact)."""
    r = H.rng(3)
    V, Hd, T = 37, 96, 50
    w8, ws = H.gen_q8_0(r, V, Hd)
    ws[0] = 0x0001  # a subnormal scale: exact decode required
    blocks = H.q8_split_to_blocks(w8, ws)
    ids = r.integers(0, V, T).astype(np.int64)
    ids[0] = 0
    a = np.empty((T, Hd), np.float32)
    b = np.empty((T, Hd), np.float32)
    o.orc_embedding_q8_split(H.ptr(ids), H.ptr(w8), H.ptr(ws), T, Hd, H.ptr(a), H.F32)
    o.orc_embedding_q8_blocks(H.ptr(ids), H.ptr(blocks), T, Hd, H.ptr(b), H.F32)
    scale = ws.view(np.float16).astype(np.float64).reshape(V, Hd // 32).repeat(32, axis=1)
    exact = (scale * w8.reshape(V, Hd).astype(np.float64))[ids]
    assert np.array_equal(a.astype(np.float64), exact)
    assert np.array_equal(a, b)


def test_q8_0_split_blocks_hand_block(o):
    """A hand-built 34-byte block (fp16 2.0 = 0x4000 little-endian, then the
    values of vulkanised/test_gguf2vk.py:77-83) splits into scale 0x4000 and
    those int8 values; the split planes gather what the blocks gather."""
    blk = np.zeros(2 * 34, np.uint8)
    blk[0:2] = [0x00, 0x40]
    blk[2:7] = [0, 1, 0xFF, 127, 0x81]
    blk[34:36] = [0x01, 0x80]              # -2^-24: a subnormal scale, bits kept as they are
    blk[36:68] = np.arange(32, dtype=np.uint8) * 7
    w8 = np.empty(64, np.int8)
    ws = np.empty(2, np.uint16)
    o.orc_q8_0_split_blocks(H.ptr(blk), 2, H.ptr(w8), H.ptr(ws))
    assert list(ws) == [0x4000, 0x8001]
    assert list(w8[:5]) == [0, 1, -1, 127, -127] and not w8[5:32].any()
    assert list(w8[32:].view(np.uint8)) == [(7 * i) & 0xFF for i in range(32)]
    ids = np.array([0, 1], np.int64)
    a = np.empty((2, 32), np.float32)
    b = np.empty((2, 32), np.float32)
    o.orc_embedding_q8_split(H.ptr(ids), H.ptr(w8), H.ptr(ws), 2, 32, H.ptr(a), H.F32)
    o.orc_embedding_q8_blocks(H.ptr(ids), H.ptr(blk), 2, 32, H.ptr(b), H.F32)
    assert list(a[0, :5]) == [0, 2, -2, 254, -254]
    assert np.array_equal(a, b)


def test_q8_0_split_blocks_round_trip(o):
    """split(join(w8, ws)) == (w8, ws) for random planes, and join(split(bytes))
    == bytes for random bytes."""
    r = H.rng(34)
    w8, ws = H.gen_q8_0(r, 13, 96)
    blk = H.q8_split_to_blocks(w8, ws)
    nb = ws.size
    g8 = np.empty(nb * 32, np.int8)
    gs = np.empty(nb, np.uint16)
    o.orc_q8_0_split_blocks(H.ptr(blk), nb, H.ptr(g8), H.ptr(gs))
    assert np.array_equal(g8, w8) and np.array_equal(gs, ws)
    raw = r.integers(0, 256, 34 * 9, dtype=np.uint8)
    g8 = np.empty(9 * 32, np.int8)
    gs = np.empty(9, np.uint16)
    o.orc_q8_0_split_blocks(H.ptr(raw), 9, H.ptr(g8), H.ptr(gs))
    assert np.array_equal(H.q8_split_to_blocks(g8, gs), raw)


# ---------------------------------------------------------------------------
# K-quants
# ---------------------------------------------------------------------------
def _deq(o, fn, blocks, bb, *extra):
    n = blocks.size // bb
    y = np.empty(n * 256, np.float32)
    for i in range(n):
        blk = np.ascontiguousarray(blocks[i * bb:(i + 1) * bb])
        fn(H.ptr(blk), y[i * 256:].ctypes.data, *extra)
    return y


def test_q4k_matches_reference_gguf_cpp(o):
    y = _deq(o, o.orc_dequant_q4k_block, GOLD["q4k_blocks"], 144, H.GGML)
    assert np.array_equal(y.view(np.uint32), GOLD["q4k_expected"].view(np.uint32))


def test_q6k_matches_reference_gguf_cpp(o):
    y = _deq(o, o.orc_dequant_q6k_block, GOLD["q6k_blocks"], 210)
    assert np.array_equal(y.view(np.uint32), GOLD["q6k_expected"].view(np.uint32))


def test_kquant_vs_live_reference_build(o):
    ref = H.ref_host()
    if ref is None:
        pytest.skip("oracle/_ref not built here")
    r = H.rng(4)
    for kind, bb, fn, extra in (("Q4_K", 144, o.orc_dequant_q4k_block, (H.GGML,)),
                                ("Q6_K", 210, o.orc_dequant_q6k_block, ())):
        blocks = H.gen_raw_blocks(r, 64, bb, (0, 2) if kind == "Q4_K" else (208,))
        mine = _deq(o, fn, blocks, bb, *extra)
        theirs = np.empty_like(mine)
        for i in range(64):
            blk = np.ascontiguousarray(blocks[i * bb:(i + 1) * bb])
            assert ref.ref_dequant_block_f32(kind.encode(), H.ptr(blk), theirs[i * 256:].ctypes.data)
        assert np.array_equal(mine.view(np.uint32), theirs.view(np.uint32)), kind


def _unit_block_q4k(sc, mn):
    b = np.zeros(144, np.uint8)
    b[0:4] = np.array([1.0, 1.0], np.float16).view(np.uint8)
    b[4:16] = H.pack_q4k_scales(np.array(sc), np.array(mn))
    return b


def test_q4k_legacy_layout_closed_form(o):
    """src/hip_ops.hip:130-140: element 32j+e reads byte 16 + 16j + (e & 15), low nibble for e < 16."""
    b = _unit_block_q4k([1] * 8, [0] * 8)
    b[16:] = (np.arange(128) * 37 % 256).astype(np.uint8)
    y = np.empty(256, np.float32)
    o.orc_dequant_q4k_block(H.ptr(b), y.ctypes.data, H.HIP_LEGACY)
    qs = b[16:].astype(int)
    for i in range(256):
        j, e = divmod(i, 32)
        byte = qs[16 * j + (e & 15)]
        assert y[i] == (byte & 15 if e < 16 else byte >> 4), i
    # and the GGML layout differs on the same bytes
    g = np.empty(256, np.float32)
    o.orc_dequant_q4k_block(H.ptr(b), g.ctypes.data, H.GGML)
    assert not np.array_equal(g, y)


def test_q5k_closed_form(o):
    """Q5_K (src/hip_ops.hip:142-155): with d = 1, dmin = 0, unit scales the
    element equals its 5-bit code: low nibble from ql, bit 4 from qh."""
    r = H.rng(5)
    codes = r.integers(0, 32, 256)
    b = np.zeros(176, np.uint8)
    b[0:4] = np.array([1.0, 0.0], np.float16).view(np.uint8)
    b[4:16] = H.pack_q4k_scales(np.ones(8, int), np.zeros(8, int))
    qh = np.zeros(32, np.uint8)
    ql = np.zeros(128, np.uint8)
    for i, v in enumerate(codes):
        group, slot, l = i // 64, (i % 64) // 32, i % 32
        ql[group * 32 + l] |= (v & 15) << (4 * slot)
        qh[l] |= (v >> 4) << (2 * group + slot)
    b[16:48] = qh
    b[48:] = ql
    y = np.empty(256, np.float32)
    o.orc_dequant_q5k_block(H.ptr(b), y.ctypes.data)
    assert np.array_equal(y, codes.astype(np.float32))
    # scale/min path: group j scaled by (j+1), offset by -j*dmin
    b[0:4] = np.array([1.0, 0.5], np.float16).view(np.uint8)
    b[4:16] = H.pack_q4k_scales(np.arange(1, 9), np.arange(8))
    o.orc_dequant_q5k_block(H.ptr(b), y.ctypes.data)
    j = np.arange(256) // 32
    assert np.array_equal(y, ((j + 1) * codes - 0.5 * j).astype(np.float32))


def test_q4k_scale_min_unpack_closed_form(o):
    """All 64 x 64 (scale, min) values survive the 12-byte packing for every group."""
    for s in range(0, 64, 7):
        for m in range(0, 64, 5):
            sc = (np.arange(8) * 9 + s) % 64
            mn = (np.arange(8) * 13 + m) % 64
            b = _unit_block_q4k(sc, mn)
            b[16:] = 0x11  # every nibble = 1
            y = np.empty(256, np.float32)
            o.orc_dequant_q4k_block(H.ptr(b), y.ctypes.data, H.GGML)
            assert np.array_equal(y, np.repeat(sc - mn, 32).astype(np.float32))


def test_embedding_qk_matches_block_decode(o):
    """Gather = block decode at element id*H + c, including rows that straddle superblocks."""
    r = H.rng(6)
    V, Hd, T = 24, 320, 20  # 320 is not a multiple of 256: rows straddle superblocks
    for kind, bb in ((12, 144), (13, 176), (14, 210)):
        nb = V * Hd // 256
        blocks = H.gen_raw_blocks(r, nb, bb, (0, 2) if kind != 14 else (208,))
        full = np.empty(nb * 256, np.float32)
        for i in range(nb):
            blk = np.ascontiguousarray(blocks[i * bb:(i + 1) * bb])
            if kind == 12:
                o.orc_dequant_q4k_block(H.ptr(blk), full[i * 256:].ctypes.data, H.GGML)
            elif kind == 13:
                o.orc_dequant_q5k_block(H.ptr(blk), full[i * 256:].ctypes.data)
            else:
                o.orc_dequant_q6k_block(H.ptr(blk), full[i * 256:].ctypes.data)
        ids = r.integers(0, V, T).astype(np.int64)
        out = np.empty((T, Hd), np.float32)
        o.orc_embedding_qk(H.ptr(ids), H.ptr(blocks), T, Hd, kind, H.GGML, H.ptr(out), H.F32)
        assert np.array_equal(out, full.reshape(V, Hd)[ids])


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
def test_rms_norm_closed_form(o):
    """test/test_basic.cpp:23-31: [1,2,3,4], w = 1, eps = 1e-6."""
    x = np.array([1, 2, 3, 4], np.float32)
    w = np.ones(4, np.float32)
    out = np.empty(4, np.float32)
    o.orc_rms_norm(H.ptr(x), H.ptr(w), H.ptr(out), 1, 4, 1e-6, H.F32)
    expected0 = 1.0 / math.sqrt(30.0 / 4.0 + 1e-6)
    assert abs(out[0] - expected0) < 1e-4 and out[3] > out[0]
    assert np.allclose(out, x / math.sqrt(7.5 + 1e-6), rtol=1e-6, atol=0)


def test_rms_norm_invariants(o):
    r = H.rng(7)
    x = r.normal(0, 1, (8, 96)).astype(np.float32)
    w = r.normal(1, 0.1, 96).astype(np.float32)
    a = np.empty_like(x)
    b = np.empty_like(x)
    o.orc_rms_norm(H.ptr(x), H.ptr(w), H.ptr(a), 8, 96, 0.0, H.F32)
    x2 = (x * 4.0).astype(np.float32)  # power-of-two scaling is exact
    o.orc_rms_norm(H.ptr(x2), H.ptr(w), H.ptr(b), 8, 96, 0.0, H.F32)
    assert np.allclose(a, b, rtol=2e-6, atol=0)
    w2 = (w * 2.0).astype(np.float32)  # linear in the gamma
    o.orc_rms_norm(H.ptr(x), H.ptr(w2), H.ptr(b), 8, 96, 0.0, H.F32)
    assert np.array_equal(b, a * 2)
    # mean of the squares of the normalised row (w = 1) is 1
    ones = np.ones(96, np.float32)
    o.orc_rms_norm(H.ptr(x), H.ptr(ones), H.ptr(b), 8, 96, 0.0, H.F32)
    assert np.allclose((b.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-6)


def test_rms_norm_add_residual_and_norm(o):
    r = H.rng(8)
    for dt in (H.F32, H.F16, H.BF16):
        x, res = H.gen_act(r, (5, 64), dt), H.gen_act(r, (5, 64), dt)
        w = H.gen_act(r, (64,), dt, 1.0, 0.1)
        res_out = res.copy()
        out = np.empty_like(x)
        o.orc_rms_norm_add(H.ptr(x), H.ptr(res_out), H.ptr(w), H.ptr(out), 5, 64, 1e-6, dt)
        # residual = one RNE rounding of the fp32 sum
        s = (H.from_storage(x, dt).astype(np.float32) + H.from_storage(res, dt).astype(np.float32))
        assert np.array_equal(res_out, H.to_storage(s, dt))
        # out = rms_norm of the stored residual
        out2 = np.empty_like(x)
        o.orc_rms_norm(H.ptr(res_out), H.ptr(w), H.ptr(out2), 5, 64, 1e-6, dt)
        assert np.array_equal(out, out2)


# ---------------------------------------------------------------------------
# SiLU * up
# ---------------------------------------------------------------------------
def test_silu_closed_forms(o):
    g = np.array([0.0, 1.0, -1.0, 20.0, -20.0, 100.0, -100.0, 3.5, -3.5], np.float32)
    gu = np.concatenate([g, np.ones_like(g)]).reshape(1, -1).astype(np.float32)
    out = np.empty((1, g.size), np.float32)
    o.orc_silu_and_mul(H.ptr(gu), H.ptr(out), 1, g.size, H.F32)
    s = out[0].astype(np.float64)
    assert s[0] == 0.0
    assert s[5] == 100.0 and s[6] == 0.0 or abs(s[6]) < 1e-40
    for i, j in ((1, 2), (3, 4), (7, 8)):  # silu(g) - silu(-g) = g
        assert abs((s[i] - s[j]) - g[i]) <= 2e-7 * abs(g[i])
    exact = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    assert np.allclose(s, exact, rtol=1e-6, atol=1e-30)


def test_silu_brute_force(o):
    r = H.rng(9)
    R, I = 4, 1000
    gu = r.normal(0, 3, (R, 2 * I)).astype(np.float32)
    out = np.empty((R, I), np.float32)
    o.orc_silu_and_mul(H.ptr(gu), H.ptr(out), R, I, H.F32)
    g, u = gu[:, :I].astype(np.float64), gu[:, I:].astype(np.float64)
    assert np.allclose(out, g / (1 + np.exp(-g)) * u, rtol=1e-6, atol=1e-12)


# ---------------------------------------------------------------------------
# RoPE / QK-norm
# ---------------------------------------------------------------------------
def _inv(o, theta, hd):
    inv = np.empty(hd // 2, np.float32)
    o.orc_inv_freq(theta, hd, H.ptr(inv))
    return inv


def test_inv_freq_closed_form(o):
    inv = _inv(o, 1e6, 128)
    assert inv[0] == 1.0
    assert inv[32] == np.float32(1e-3)  # theta^(-64/128) = 1e-3
    assert inv[16] == np.float32(10 ** -1.5)


def test_rope_identity_at_zero_and_unit_vector(o):
    r = H.rng(10)
    T, heads, hd = 6, 3, 64
    inv = _inv(o, 1e6, hd)
    x = r.normal(0, 1, (T, heads * hd)).astype(np.float32)
    y = x.copy()
    pos = np.zeros(T, np.int64)
    o.orc_rope(H.ptr(y), H.ptr(pos), T, heads, hd, heads * hd, H.ptr(inv), H.F32)
    assert np.array_equal(x, y)  # cos 0 = 1, sin 0 = 0 exactly
    # e_0 rotates to (cos p, sin p) with angle p * inv_freq[0] = p
    e = np.zeros((T, hd), np.float32)
    e[:, 0] = 1.0
    pos = np.array([1, 2, 100, 4095, 8191, 3], np.int64)
    o.orc_rope(H.ptr(e), H.ptr(pos), T, 1, hd, hd, H.ptr(inv), H.F32)
    assert np.allclose(e[:, 0], np.cos(pos.astype(np.float64)), rtol=0, atol=2e-7)
    assert np.allclose(e[:, hd // 2], np.sin(pos.astype(np.float64)), rtol=0, atol=2e-7)


def test_rope_norm_preserving_and_inverse(o):
    r = H.rng(11)
    T, heads, hd = 16, 4, 128
    inv = _inv(o, 1e6, hd)
    x = r.normal(0, 1, (T, heads, hd)).astype(np.float32)
    y = x.copy()
    pos = r.integers(0, 4096, T).astype(np.int64)
    o.orc_rope(H.ptr(y), H.ptr(pos), T, heads, hd, heads * hd, H.ptr(inv), H.F32)
    n0 = x[..., :64].astype(np.float64) ** 2 + x[..., 64:].astype(np.float64) ** 2
    n1 = y[..., :64].astype(np.float64) ** 2 + y[..., 64:].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)
    neg = -pos
    o.orc_rope(H.ptr(y), H.ptr(neg), T, heads, hd, heads * hd, H.ptr(inv), H.F32)
    assert np.allclose(y, x, rtol=0, atol=5e-5)


def test_qk_norm_rope_is_the_composition(o):
    """fp32: fused oracle == rms_norm (rows = T*heads, hidden = hd) then rope, bit for bit."""
    r = H.rng(12)
    T, hq, hk, hd = 9, 4, 2, 128
    inv = _inv(o, 1e6, hd)
    q = r.normal(0, 1, (T, hq * hd)).astype(np.float32)
    k = r.normal(0, 1, (T, hk * hd)).astype(np.float32)
    qw = r.normal(1, 0.1, hd).astype(np.float32)
    kw = r.normal(1, 0.1, hd).astype(np.float32)
    pos = r.integers(0, 4096, T).astype(np.int64)
    fq, fk = q.copy(), k.copy()
    o.orc_qk_norm_rope(H.ptr(fq), H.ptr(fk), H.ptr(pos), H.ptr(qw), H.ptr(kw), H.ptr(inv), T, hq, hk, hd,
                       hq * hd, hk * hd, 1e-6, H.F32)
    uq, uk = np.empty_like(q), np.empty_like(k)
    o.orc_rms_norm(H.ptr(q), H.ptr(qw), H.ptr(uq), T * hq, hd, 1e-6, H.F32)
    o.orc_rms_norm(H.ptr(k), H.ptr(kw), H.ptr(uk), T * hk, hd, 1e-6, H.F32)
    o.orc_rope(H.ptr(uq), H.ptr(pos), T, hq, hd, hq * hd, H.ptr(inv), H.F32)
    o.orc_rope(H.ptr(uk), H.ptr(pos), T, hk, hd, hk * hd, H.ptr(inv), H.F32)
    assert np.array_equal(fq, uq) and np.array_equal(fk, uk)


@pytest.mark.parametrize("dt", [H.F32, H.F16, H.BF16])
def test_add_bias_closed_form(o, dt):
    """x + b in fp32, one rounding to the storage type; rows with a stride (the columns
    past cols untouched)."""
    r = H.rng(13)
    rows, cols, stride = 7, 96, 100
    x = H.gen_act(r, (rows, stride), dt)
    b = r.normal(0, 1, cols).astype(np.float32)
    y = x.copy()
    o.orc_add_bias(H.ptr(y), H.ptr(b), rows, cols, stride, dt)
    want = H.to_storage(H.from_storage(x[:, :cols], dt).astype(np.float32) + b[None, :], dt)
    assert np.array_equal(y[:, :cols], want) and np.array_equal(y[:, cols:], x[:, cols:])
    # hand values: 1.5 + 0.25 = 1.75 exactly; 1 + 2^-11 rounds to 1 in fp16 (a tie, to even)
    if dt == H.F16:
        hx = H.to_storage(np.array([[1.5, 1.0]], np.float32), dt)
        hb = np.array([0.25, 2.0 ** -11], np.float32)
        o.orc_add_bias(H.ptr(hx), H.ptr(hb), 1, 2, 2, dt)
        assert np.array_equal(H.from_storage(hx, dt).astype(np.float32), np.array([[1.75, 1.0]], np.float32))


def _qkv_case(r, dt, T=9, hq=4, hk=2, hd=128, norm=True):
    q = H.gen_act(r, (T, hq * hd), dt)
    k = H.gen_act(r, (T, hk * hd), dt)
    v = H.gen_act(r, (T, hk * hd), dt)
    bias = r.normal(0, 0.5, (hq + 2 * hk) * hd).astype(np.float32)
    qw = H.gen_act(r, (hd,), dt, 1.0, 0.1) if norm else None
    kw = H.gen_act(r, (hd,), dt, 1.0, 0.1) if norm else None
    pos = r.integers(0, 4096, T).astype(np.int64)
    slots = r.permutation(2 * T)[:T].astype(np.int32)
    slots[1] = -1  # a skipped token
    return q, k, v, bias, qw, kw, pos, slots


def _fused_qkv(o, q, k, v, bias, qw, kw, pos, slots, inv, hq, hk, hd, dt):
    T = q.shape[0]
    fq, fk = q.copy(), k.copy()
    kc = np.zeros((2 * T, hk * hd), q.dtype)
    vc = np.zeros((2 * T, hk * hd), q.dtype)
    v0 = v.copy()
    o.orc_qkv_bias_qk_norm_rope_store_kv(H.ptr(fq), H.ptr(fk), H.ptr(v), H.ptr(bias), H.ptr(pos), H.ptr(qw),
                                         H.ptr(kw), H.ptr(inv), T, hq, hk, hd, hq * hd, hk * hd, hk * hd, 1e-6,
                                         H.ptr(kc), H.ptr(vc), H.ptr(slots), dt)
    assert np.array_equal(v, v0)  # v is read, not written
    return fq, fk, kc, vc


@pytest.mark.parametrize("norm", [True, False])
def test_qkv_bias_fused_is_the_composition_fp32(o, norm):
    """fp32: bias + QK-norm + RoPE + store == add_bias (q, k, v) -> qk_norm_rope -> store_kv
    (model.cpp:768-781 as separate passes), bit for bit."""
    r = H.rng(14)
    hq, hk, hd = 4, 2, 128
    inv = _inv(o, 1e6, hd)
    q, k, v, bias, qw, kw, pos, slots = _qkv_case(r, H.F32, hq=hq, hk=hk, hd=hd, norm=norm)
    T = q.shape[0]
    fq, fk, kc, vc = _fused_qkv(o, q, k, v, bias, qw, kw, pos, slots, inv, hq, hk, hd, H.F32)
    uq, uk, uv = q.copy(), k.copy(), v.copy()
    o.orc_add_bias(H.ptr(uq), H.ptr(bias), T, hq * hd, hq * hd, H.F32)
    o.orc_add_bias(H.ptr(uk), H.ptr(bias[hq * hd:]), T, hk * hd, hk * hd, H.F32)
    o.orc_add_bias(H.ptr(uv), H.ptr(bias[(hq + hk) * hd:]), T, hk * hd, hk * hd, H.F32)
    o.orc_qk_norm_rope(H.ptr(uq), H.ptr(uk), H.ptr(pos), H.ptr(qw), H.ptr(kw), H.ptr(inv), T, hq, hk, hd,
                       hq * hd, hk * hd, 1e-6, H.F32)
    ukc, uvc = np.zeros_like(kc), np.zeros_like(vc)
    o.orc_store_kv(H.ptr(uk), H.ptr(uv), H.ptr(ukc), H.ptr(uvc), H.ptr(slots), T, hk, hd, H.F32)
    assert np.array_equal(fq, uq) and np.array_equal(fk, uk)
    assert np.array_equal(kc, ukc) and np.array_equal(vc, uvc)


@pytest.mark.parametrize("dt", [H.F16, H.BF16])
def test_qkv_bias_fused_zero_bias_and_identity(o, dt):
    """16-bit storage: a zero bias gives the unbiased qk_norm_rope + store_kv exactly; at
    position 0 without norm the op is x + b rounded once (RoPE is the identity there)."""
    r = H.rng(15)
    hq, hk, hd = 4, 2, 128
    inv = _inv(o, 1e6, hd)
    q, k, v, bias, qw, kw, pos, slots = _qkv_case(r, dt, hq=hq, hk=hk, hd=hd)
    T = q.shape[0]
    fq, fk, kc, vc = _fused_qkv(o, q, k, v, np.zeros_like(bias), qw, kw, pos, slots, inv, hq, hk, hd, dt)
    uq, uk = q.copy(), k.copy()
    o.orc_qk_norm_rope(H.ptr(uq), H.ptr(uk), H.ptr(pos), H.ptr(qw), H.ptr(kw), H.ptr(inv), T, hq, hk, hd,
                       hq * hd, hk * hd, 1e-6, dt)
    ukc, uvc = np.zeros_like(kc), np.zeros_like(vc)
    o.orc_store_kv(H.ptr(uk), H.ptr(v), H.ptr(ukc), H.ptr(uvc), H.ptr(slots), T, hk, hd, dt)
    assert np.array_equal(fq, uq) and np.array_equal(fk, uk) and np.array_equal(kc, ukc) and np.array_equal(vc, uvc)
    pos0 = np.zeros(T, np.int64)
    fq, fk, kc, vc = _fused_qkv(o, q, k, v, bias, None, None, pos0, slots, inv, hq, hk, hd, dt)
    assert np.array_equal(fq, H.to_storage(H.from_storage(q, dt).astype(np.float32) + bias[None, :hq * hd], dt))
    assert np.array_equal(fk, H.to_storage(H.from_storage(k, dt).astype(np.float32) + bias[None, hq * hd:(hq + hk) * hd], dt))
    live = slots >= 0
    assert np.array_equal(vc[slots[live]], H.to_storage(H.from_storage(v[live], dt).astype(np.float32) + bias[None, (hq + hk) * hd:], dt))
    assert np.array_equal(kc[slots[live]], fk[live])


# ---------------------------------------------------------------------------
# Q8 activation row scale / quantize, fused layer-0 embedding + norm
# ---------------------------------------------------------------------------
def test_q8_row_scale_closed_form(o):
    x = np.array([[1.0, -4.0, 2.0, 0.5], [0, 0, 0, 0], [1e-9, -1e-9, 0, 0], [3.0, 3.0, -3.0, 1.5]], np.float32)
    sc = np.empty(4, np.float32)
    o.orc_q8_row_scale(H.ptr(x), H.ptr(sc), 4, 4, H.F32)
    assert sc[0] == np.float32(127.0) / np.float32(4.0) and sc[1] == 0 and sc[2] == 0
    assert sc[3] == np.float32(127.0) / np.float32(3.0)
    q = np.empty((4, 4), np.int8)
    o.orc_q8_quantize(H.ptr(x), H.ptr(sc), q.ctypes.data, 4, 4, H.F32)
    assert list(q[0]) == [31, -127, 63, 15]          # 31.75 -> 31, 63.5 -> 63, 15.875 -> 15 (truncation)
    assert list(q[1]) == [0, 0, 0, 0]
    assert abs(int(q[3, 0])) == 127 and q[3, 2] == -127  # the row maximum maps to +-127


def test_q8_quantize_bounds_and_truncation(o):
    r = H.rng(20)
    x = r.normal(0, 1, (16, 256)).astype(np.float32)
    sc = np.empty(16, np.float32)
    q = np.empty((16, 256), np.int8)
    o.orc_q8_row_scale(H.ptr(x), H.ptr(sc), 16, 256, H.F32)
    o.orc_q8_quantize(H.ptr(x), H.ptr(sc), q.ctypes.data, 16, 256, H.F32)
    v = x.astype(np.float32) * sc[:, None]
    assert np.array_equal(q, np.trunc(np.clip(v, -127, 127)).astype(np.int8))
    # the row maximum lands on 127, or on 126 when max * (127 / max) rounds just below 127
    assert np.isin(np.abs(q.astype(np.int32)).max(axis=1), (126, 127)).all()


def test_embedding_rms_norm_is_the_composition(o):
    r = H.rng(21)
    V, Hd, T = 50, 256, 9
    w8, ws = H.gen_q8_0(r, V, Hd)
    ids = r.integers(0, V, T).astype(np.int64)
    for dt in (H.F32, H.F16, H.BF16):
        w = H.gen_act(r, (Hd,), dt, 1.0, 0.1)
        res, out = np.empty((T, Hd), H.NP_STORAGE[dt]), np.empty((T, Hd), H.NP_STORAGE[dt])
        o.orc_embedding_rms_norm(H.ptr(ids), 0, H.ptr(w8), H.ptr(ws), T, Hd, H.ptr(w), H.ptr(res), H.ptr(out), 1e-6, dt)
        emb = np.empty((T, Hd), H.NP_STORAGE[dt])
        o.orc_embedding_q8_split(H.ptr(ids), H.ptr(w8), H.ptr(ws), T, Hd, H.ptr(emb), dt)
        zero = H.to_storage(np.zeros((T, Hd), np.float32), dt)
        out2 = np.empty_like(out)
        o.orc_rms_norm_add(H.ptr(emb), H.ptr(zero), H.ptr(w), H.ptr(out2), T, Hd, 1e-6, dt)
        assert np.array_equal(res, zero) and np.array_equal(out, out2)
        # residual = emb + 0: identical to the gather except -0 becomes +0
        assert np.array_equal(H.from_storage(res, dt), H.from_storage(emb, dt) + 0.0)


# ---------------------------------------------------------------------------
# tolerance helpers themselves
# ---------------------------------------------------------------------------
def test_tolerance_rule_rejects_two_ulp():
    ref = H.to_storage(np.array([1.0, 3.0, -0.125], np.float32), H.F16)
    one = ref + np.uint16(1)
    H.assert_close(one, ref, H.F16)
    with pytest.raises(AssertionError):
        H.assert_close(ref + np.uint16(2), ref, H.F16)
    refb = H.to_storage(np.array([1.0, 3.0], np.float32), H.BF16)
    H.assert_close(refb + np.uint16(1), refb, H.BF16)
    with pytest.raises(AssertionError):
        H.assert_close(refb + np.uint16(2), refb, H.BF16)


# ---------------------------------------------------------------------------
# Q8_0 GEMM (src/hip_ops.hip:639-686)
# ---------------------------------------------------------------------------
def _gemm(o, x, dt, w8, ws, m, n, k):
    out = np.empty((m, n), np.float64)
    err = np.empty((m, n), np.float64)
    sc = np.empty(m, np.float32)
    xq = np.empty((m, k), np.int8)
    o.orc_matmul_q8(H.ptr(x), dt, H.ptr(w8), H.ptr(ws), m, n, k, H.ptr(out), H.ptr(err), H.ptr(sc), H.ptr(xq))
    return out, err, sc, xq


@pytest.mark.parametrize("dt", [H.F32, H.F16, H.BF16])
def test_matmul_q8_exact_against_dequantized_matmul(o, dt):
    """Rows whose maximum is 127 quantize with scale 1 (xq == x) and power-of-two
    block scales keep every product exact, so the oracle must equal a textbook
    float64 matmul of the activations with the dequantized weight matrix
    W[c,i] = ws[c, i // 32] * w8[c,i] -- a different route through the same
    arithmetic (dequantize first, contract second).  A zero row gives scale 0."""
    r = H.rng(11 + dt)
    m, n, k = 6, 9, 160
    x = r.integers(-127, 128, (m, k)).astype(np.float32)
    x[:, 7] = 127.0
    x[3] = 0.0
    w8 = r.integers(-127, 128, n * k, dtype=np.int8)
    exps = (np.arange(n)[:, None] + 3 * np.arange(k // 32)[None, :]) % 7 + 3
    ws = np.ldexp(1.0, -exps).astype(np.float16).view(np.uint16).reshape(-1)
    out, err, sc, xq = _gemm(o, H.to_storage(x, dt), dt, w8, ws, m, n, k)
    W = ws.view(np.float16).astype(np.float64).reshape(n, k // 32).repeat(32, axis=1) * w8.reshape(n, k)
    expect = x.astype(np.float64) @ W.T
    expect[3] = 0.0
    assert np.array_equal(sc, np.where(np.arange(m) == 3, 0.0, 1.0).astype(np.float32))
    assert np.array_equal(xq, x.astype(np.int8))
    assert np.array_equal(out, expect)
    assert (err >= 0).all() and (err[3] == 0).all()


def test_matmul_q8_bound_covers_fp32_summation_orders(o):
    """The stated tolerance holds for fp32 sums of the block terms in the
    reference's order (16-element halves, src/hip_ops.hip:297-302), in whole
    blocks, and reversed -- each computed here in numpy float32."""
    r = H.rng(12)
    m, n, k = 5, 7, 512
    x = r.standard_normal((m, k)).astype(np.float32)
    w8, ws = H.gen_q8_0(r, n, k)
    out, err, sc, xq = _gemm(o, x, H.F32, w8, ws, m, n, k)
    s = ws.view(np.float16).astype(np.float32).reshape(n, k // 32)
    q = xq.astype(np.int64).reshape(m, 1, k // 16, 16)
    w = w8.astype(np.int64).reshape(1, n, k // 16, 16)
    halves = (q * w).sum(-1)                                         # [m, n, k/16] exact
    blocks = halves.reshape(m, n, k // 32, 2).sum(-1)
    adq = np.where(sc > 0, np.float32(1) / sc, np.float32(0)).astype(np.float32)
    for terms, sidx in ((halves, np.arange(k // 16) // 2), (blocks, np.arange(k // 32)),
                        (blocks[..., ::-1], np.arange(k // 32)[::-1])):
        acc = np.zeros((m, n), np.float32)
        for j in range(terms.shape[-1]):
            acc = (acc + s[:, sidx[j]][None, :] * terms[..., j].astype(np.float32)).astype(np.float32)
        got = (acc * adq[:, None]).astype(np.float64)
        assert (np.abs(got - out) <= err).all()
    assert (np.abs(out) > 0).any()


# ---------------------------------------------------------------------------
# KV store and paged attention (src/hip_ops.hip:452-550)
# ---------------------------------------------------------------------------
def _dense_reference(b, q_heads, kv_heads, hd, bs, scale):
    """A textbook route: gather each sequence's keys densely, softmax(q K^T) V in numpy."""
    qf = b.q.astype(np.float64)
    kf = b.k_cache.astype(np.float64)
    vf = b.v_cache.astype(np.float64)
    out = np.zeros(qf.shape)
    g = q_heads // kv_heads
    for t in range(b.tokens):
        L = int(b.query_key_len[t])
        if L <= 0:
            continue
        s_ = int(b.query_seq[t])
        rows = np.array([b.block_tables[s_, j // bs] * bs + j % bs for j in range(L)])
        for h in range(q_heads):
            K = kf[rows, h // g]
            V = vf[rows, h // g]
            sc = K @ qf[t, h] * scale
            p = np.exp(sc - sc.max())
            out[t, h] = p @ V / p.sum()
    return out


def test_paged_attention_matches_dense_softmax(o):
    r = H.rng(40)
    b = H.make_paged(r, [5, 17, 33], [5, 3, 1], 6, 2, 16, 8, H.F32)
    out, exact, vmax = H.oracle_attention(b, 6, 2, 16, 8, 0.25, H.F32)
    dense = _dense_reference(b, 6, 2, 16, 8, 0.25)
    assert np.allclose(exact, dense, rtol=1e-12, atol=1e-12)
    assert np.array_equal(out, exact.astype(np.float32))
    assert (vmax > 0).all()


def test_paged_attention_closed_forms(o):
    """One key -> that V row exactly; q = 0 -> the mean of the attended V rows;
    key_len 0 -> zeros."""
    r = H.rng(41)
    b = H.make_paged(r, [1, 9], [1, 1], 4, 4, 8, 4, H.F32)
    b.q[1] = 0.0
    b.query_key_len[:] = [1, 9]
    out, exact, _ = H.oracle_attention(b, 4, 4, 8, 4, 0.3, H.F32)
    row0 = b.block_tables[0, 0] * 4
    assert np.array_equal(out[0], b.v_cache[row0])
    rows = [b.block_tables[1, j // 4] * 4 + j % 4 for j in range(9)]
    assert np.allclose(exact[1], b.v_cache[rows].astype(np.float64).mean(axis=0), rtol=1e-12, atol=1e-13)
    b.query_key_len[:] = [0, 0]
    out, _, _ = H.oracle_attention(b, 4, 4, 8, 4, 0.3, H.F32)
    assert not out.any()


def test_paged_attention_block_permutation_invariance(o):
    """Relocating the physical blocks (and the table with them) changes nothing."""
    r = H.rng(42)
    b = H.make_paged(r, [24, 10], [4, 10], 4, 2, 8, 4, H.BF16)
    out1, _, _ = H.oracle_attention(b, 4, 2, 8, 4, 0.35, H.BF16)
    perm = r.permutation(b.num_blocks)
    inv = np.argsort(perm)
    kc = b.k_cache.reshape(b.num_blocks, 4, 2, 8)[perm].reshape(b.k_cache.shape)
    vc = b.v_cache.reshape(b.num_blocks, 4, 2, 8)[perm].reshape(b.v_cache.shape)
    tables = np.where(b.block_tables >= 0, inv[np.maximum(b.block_tables, 0)], -1).astype(np.int32)
    b2 = H.PagedBatch(b.q, np.ascontiguousarray(kc), np.ascontiguousarray(vc), b.query_seq, b.query_key_len, tables,
                      b.tokens, b.max_blocks, b.num_blocks)
    out2, _, _ = H.oracle_attention(b2, 4, 2, 8, 4, 0.35, H.BF16)
    assert np.array_equal(out1, out2)


@pytest.mark.parametrize("dt", [H.F32, H.BF16])
def test_store_kv_is_a_slot_copy(o, dt):
    r = H.rng(43)
    T, kvh, hd, rows = 6, 2, 8, 20
    key, val = H.gen_act(r, (T, kvh, hd), dt), H.gen_act(r, (T, kvh, hd), dt)
    kc, vc = np.zeros((rows, kvh, hd), H.NP_STORAGE[dt]), np.zeros((rows, kvh, hd), H.NP_STORAGE[dt])
    slots = np.array([3, 0, -1, 19, 7, 8], np.int32)
    o.orc_store_kv(H.ptr(key), H.ptr(val), H.ptr(kc), H.ptr(vc), H.ptr(slots), T, kvh, hd, dt)
    for t, sl in enumerate(slots):
        if sl >= 0:
            assert np.array_equal(kc[sl], key[t]) and np.array_equal(vc[sl], val[t])
    untouched = np.setdiff1d(np.arange(rows), slots[slots >= 0])
    assert not kc[untouched].any() and not vc[untouched].any()


# ---------------------------------------------------------------------------
# dense / K-quant weight GEMM (src/hip_ops.hip:43-64, :577-598) and row gather (:611-619)
# ---------------------------------------------------------------------------
def _dequant_matrix(o, w, w_format, n, k, layout=H.GGML):
    """W [n, k] as float64, dense formats by numpy, K-quants block by block through the
    pinned orc_dequant_*_block functions (a route independent of orc_matmul_w's)."""
    if w_format == H.F32:
        return w.reshape(n, k).astype(np.float64)
    if w_format in (H.F16, H.BF16):
        return H.from_storage(w.reshape(n, k), w_format).astype(np.float64)
    bb = H.KQ_BLOCK[w_format][0]
    flat = np.empty(n * k, np.float32)
    for b in range(n * k // 256):
        blk = np.ascontiguousarray(w[b * bb:(b + 1) * bb])
        y = flat[b * 256:(b + 1) * 256]
        if w_format == 12:
            o.orc_dequant_q4k_block(H.ptr(blk), y.ctypes.data, layout)
        elif w_format == 13:
            o.orc_dequant_q5k_block(H.ptr(blk), y.ctypes.data)
        else:
            o.orc_dequant_q6k_block(H.ptr(blk), y.ctypes.data)
    return flat.reshape(n, k).astype(np.float64)


def _matmul_w(o, x, x_dt, w, w_format, m, n, k, layout=H.GGML):
    out = np.empty((m, n), np.float64)
    err = np.empty((m, n), np.float64)
    o.orc_matmul_w(H.ptr(x), x_dt, H.ptr(w), w_format, layout, m, n, k, H.ptr(out), H.ptr(err))
    return out, err


@pytest.mark.parametrize("w_format", [H.F32, H.F16, H.BF16, 12, 13, 14], ids=["f32", "f16", "bf16", "q4k", "q5k", "q6k"])
def test_matmul_w_equals_dequantized_matmul(o, w_format):
    """Against a textbook float64 matmul of the dequantized weight matrix.  Exact when
    every product and partial sum is exact in fp32 (small integer activations and
    dense weights that are small multiples of a power of two); within the bound in
    general (K-quant weights are products of fp16 scales and small integers)."""
    r = H.rng(40 + w_format)
    m, n, k = 5, 6, 512
    x = r.integers(-8, 9, (m, k)).astype(np.float32)
    if w_format in (H.F32, H.F16, H.BF16):
        w = H.to_storage((r.integers(-16, 17, (n, k)) * 0.125).astype(np.float32), w_format)
    else:
        w = H.gen_weights(r, n, k, w_format)
    out, err = _matmul_w(o, x, H.F32, w, w_format, m, n, k)
    expect = x.astype(np.float64) @ _dequant_matrix(o, w, w_format, n, k).T
    if w_format in (H.F32, H.F16, H.BF16):
        assert np.array_equal(out, expect)
    else:
        assert (np.abs(out - expect) <= 1e-12 * np.abs(expect).max()).all()
    assert (err >= 0).all()


def test_matmul_w_q4k_layout_reaches_the_decoder(o):
    """The layout argument selects the Q4_K nibble order: the two orders give the
    products of their own dequantized matrices, and differ."""
    r = H.rng(47)
    m, n, k = 3, 4, 256
    x = r.standard_normal((m, k)).astype(np.float32)
    w = H.gen_weights(r, n, k, 12)
    for layout in (H.GGML, H.HIP_LEGACY):
        out, _ = _matmul_w(o, x, H.F32, w, 12, m, n, k, layout)
        expect = x.astype(np.float64) @ _dequant_matrix(o, w, 12, n, k, layout).T
        assert np.allclose(out, expect, rtol=1e-12, atol=1e-12)
    a, _ = _matmul_w(o, x, H.F32, w, 12, m, n, k, H.GGML)
    b, _ = _matmul_w(o, x, H.F32, w, 12, m, n, k, H.HIP_LEGACY)
    assert not np.allclose(a, b)


def test_matmul_w_bound_covers_fp32_summation_orders(o):
    """The stated tolerance holds for fp32 sums of the products in the reference's
    order (k ascending, fp32 products), reversed, and pairwise, computed in numpy."""
    r = H.rng(48)
    m, n, k = 4, 5, 1024                     # a power of two for the pairwise tree
    x = H.to_storage(r.standard_normal((m, k)).astype(np.float32), H.BF16)
    w = H.gen_weights(r, n, k, 14)
    out, err = _matmul_w(o, x, H.BF16, w, 14, m, n, k)
    xf = H.from_storage(x, H.BF16).astype(np.float32)
    W = _dequant_matrix(o, w, 14, n, k).astype(np.float32)
    prods = (xf[:, None, :] * W[None, :, :]).astype(np.float32)       # [m, n, k], fp32 products
    for order in (np.arange(k), np.arange(k)[::-1]):
        acc = np.zeros((m, n), np.float32)
        for i in order:
            acc = (acc + prods[..., i]).astype(np.float32)
        assert (np.abs(acc.astype(np.float64) - out) <= err).all()
    pw = prods.copy()
    while pw.shape[-1] > 1:
        pw = (pw[..., 0::2] + pw[..., 1::2]).astype(np.float32)
    assert (np.abs(pw[..., 0].astype(np.float64) - out) <= err).all()


@pytest.mark.parametrize("dt", [H.F32, H.F16, H.BF16], ids=["f32", "f16", "bf16"])
def test_gather_rows_is_indexing(o, dt):
    r = H.rng(49 + dt)
    rows = H.gen_act(r, (11, 40), dt)
    idx = np.array([3, 0, 10, 3, 7], np.int32)
    out = np.empty((5, 40), rows.dtype)
    o.orc_gather_rows(H.ptr(rows), H.ptr(idx), 40, 5, H.ptr(out), dt)
    assert np.array_equal(out, rows[idx])


# ---------------------------------------------------------------------------
# MoE routing (src/hip_ops.hip:813-844) and expert FFN (:861-893)
# ---------------------------------------------------------------------------
def _route(o, logits, k, norm):
    rows, e = logits.shape
    idx = np.empty((rows, k), np.int32)
    sc = np.empty((rows, k), np.float32)
    o.orc_moe_route(H.ptr(np.ascontiguousarray(logits, np.float32)), rows, e, k, int(norm), H.ptr(idx), H.ptr(sc))
    return idx, sc


@pytest.mark.parametrize("norm", [False, True])
def test_moe_route_is_sorted_softmax(o, norm):
    """Distinct logits: the experts are the K largest in descending order and the scores the
    softmax probabilities (renormalised over the K with norm), from numpy's own routes."""
    r = H.rng(60 + norm)
    logits = (r.permutation(64 * 40).reshape(40, 64) * 0.01 - 12.0).astype(np.float32)  # distinct values
    idx, sc = _route(o, logits, 6, norm)
    l64 = logits.astype(np.float64)
    p = np.exp(l64 - l64.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    want = np.argsort(-l64, axis=1, kind="stable")[:, :6]
    assert np.array_equal(idx, want)
    top = np.take_along_axis(p, want, 1)
    if norm:
        top = top / top.sum(1, keepdims=True)
    assert np.allclose(sc, top.astype(np.float32), rtol=2 ** -23, atol=0)


@pytest.mark.parametrize("logits,k,want", [
    ([1.0, 1.0, 1.0, 1.0], 4, [0, 1, 2, 3]),
    ([1.0, 3.0, 1.0, 1.0], 3, [1, 0, 2]),
    # the first selection pass swaps expert 0 to position 2, behind expert 1: ties follow positions, not ids
    ([1.0, 1.0, 3.0, 1.0], 3, [2, 1, 0]),
    # the second selection pass swaps expert 0 (value 2) forward past experts 1 and 2, which end up reversed
    ([2.0, 1.0, 1.0, 5.0, 1.0], 4, [3, 0, 2, 1]),
])
def test_moe_route_tie_order_is_the_selection_sorts(o, logits, k, want):
    """Hand-worked selection sorts: each round takes the first position holding the maximum
    among positions >= i, then swaps it with position i."""
    idx, sc = _route(o, np.array([logits], np.float32), k, False)
    assert idx[0].tolist() == want
    assert np.all(np.diff(sc[0]) <= 0)


def _moe_case(r, rows, hid, inter, k, n_exp, slots, w_bf16):
    x = r.standard_normal((rows, hid)).astype(np.float32)
    gu = H.to_storage((r.standard_normal((slots, 2 * inter, hid)) * 0.05).astype(np.float32), H.BF16 if w_bf16 else H.F16)
    dn = H.to_storage((r.standard_normal((slots, hid, inter)) * 0.05).astype(np.float32), H.BF16 if w_bf16 else H.F16)
    idx = np.stack([r.permutation(n_exp)[:k] for _ in range(rows)]).astype(np.int32)
    score = r.uniform(0.05, 0.5, (rows, k)).astype(np.float32)
    slot_of = r.permutation(slots)[:n_exp].astype(np.int32)
    return x, gu, dn, idx, score, slot_of


def _moe_oracle(o, x, x_dt, gu, dn, w_bf16, idx, score, slot_of, slots, out_in):
    rows, hid = out_in.shape
    inter = dn.shape[-1]
    k = idx.shape[1]
    out = np.empty((rows, hid), np.float64)
    err = np.empty((rows, hid), np.float64)
    o.orc_moe_ffn(H.ptr(x), x_dt, H.ptr(idx), H.ptr(score), H.ptr(gu), H.ptr(dn), int(w_bf16), H.ptr(slot_of), rows,
                  hid, inter, k, slots, H.ptr(np.ascontiguousarray(out_in, np.float64)), H.ptr(out), H.ptr(err))
    return out, err


def test_moe_ffn_equals_numpy(o):
    """Against numpy's float64 matrix products of the same experts; a pair with score 0 and
    a pair whose expert has no slot (-1) add nothing."""
    r = H.rng(61)
    rows, hid, inter, k, n_exp, slots = 5, 48, 40, 3, 6, 8
    x, gu, dn, idx, score, slot_of = _moe_case(r, rows, hid, inter, k, n_exp, slots, False)
    score[1, 2] = 0.0
    slot_of[idx[3, 0]] = -1
    out_in = r.standard_normal((rows, hid))
    out, err = _moe_oracle(o, x, H.F32, gu, dn, False, idx, score, slot_of, slots, out_in)
    G = H.from_storage(gu, H.F16)
    D = H.from_storage(dn, H.F16)
    want = out_in.copy()
    for t in range(rows):
        for j in range(k):
            s = slot_of[idx[t, j]]
            if score[t, j] == 0 or s < 0:
                continue
            g, u = G[s, :inter] @ x[t].astype(np.float64), G[s, inter:] @ x[t].astype(np.float64)
            want[t] += float(score[t, j]) * (D[s] @ (g / (1 + np.exp(-g)) * u))
    assert np.allclose(out, want, rtol=1e-12, atol=1e-12)
    assert (err > 0).all()


def _ref_block_dot(a, b):
    """The reference's block_dot (src/hip_ops.hip:846-859) in fp32: 256 strided partial
    sums (fused multiply-adds), then one thread sums the partials in order."""
    n = a.shape[-1]
    part = np.zeros(256, np.float32)
    for i in range(n):
        part[i % 256] = np.float32(np.float64(part[i % 256]) + np.float64(a[i]) * np.float64(b[i]))
    s = np.float32(0)
    for v in part:
        s = np.float32(s + v)
    return s


def test_moe_ffn_bound_covers_the_references_fp32_order(o):
    """The reference kernel's own fp32 evaluation order (block_dot, expf, res += w * v as a
    fused multiply-add, out += res) lies within the oracle's bound."""
    r = H.rng(62)
    rows, hid, inter, k, n_exp, slots = 3, 300, 260, 2, 4, 4
    x, gu, dn, idx, score, slot_of = _moe_case(r, rows, hid, inter, k, n_exp, slots, True)
    out_in = r.standard_normal((rows, hid)).astype(np.float32)
    out, err = _moe_oracle(o, x, H.F32, gu, dn, True, idx, score, slot_of, slots, out_in.astype(np.float64))
    G = H.from_storage(gu, H.BF16).astype(np.float32)
    D = H.from_storage(dn, H.BF16).astype(np.float32)
    for t in range(rows):
        res = np.zeros(hid, np.float32)
        for j in range(k):
            s = slot_of[idx[t, j]]
            ys = np.empty(inter, np.float32)
            for c in range(inter):
                gg = _ref_block_dot(x[t], G[s, c])
                uu = _ref_block_dot(x[t], G[s, inter + c])
                ys[c] = np.float32(np.float32(gg / np.float32(np.float32(1) + np.exp(-gg))) * uu)
            for c in range(hid):
                v = _ref_block_dot(ys, D[s, c])
                res[c] = np.float32(np.float64(res[c]) + np.float64(score[t, j]) * np.float64(v))
        got = (out_in[t] + res).astype(np.float64)
        assert (np.abs(got - out[t]) <= err[t]).all()
