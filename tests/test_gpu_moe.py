"""GPU parity of the MoE ops: routing (the reference's hip_moe_route,
src/hip_ops.hip:813-844), the expert FFN (hip_moe_ffn, :861-912) and the shared-expert
helpers hip_add_inplace / hip_scale_rows_sigmoid (:914-939).

Bars:
* routing: expert ids bit-exact against the oracle and the reference's kernel (ties
  included); scores bit-exact against the reference's kernel (the same device exp), and
  within one fp32 ulp of the oracle (host libm exp);
* FFN: every output within twice the oracle's first-order fp32 bound `err` (plus half an
  ulp for 16-bit outputs) around its float64 value -- six times for bf16 experts and
  twelve for fp16 ones, whose split products sum three (six) exact bf16 piece products
  per term; the reference's own kernel is held to the same bar on the same inputs;
* add_inplace bit-exact; scale_rows_sigmoid bit-exact against the reference's kernel.
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


def dptr(t: torch.Tensor) -> int:
    return t.data_ptr()


@pytest.fixture(scope="module")
def ref():
    r = H.ref_hip()
    if r is None:
        pytest.skip("oracle/_ref/libref_hip_ops.so not present")
    return r


def oracle_route(logits: np.ndarray, k: int, norm: bool):
    rows, e = logits.shape
    idx = np.empty((rows, k), np.int32)
    sc = np.empty((rows, k), np.float32)
    H.oracle().orc_moe_route(H.ptr(logits), rows, e, k, int(norm), H.ptr(idx), H.ptr(sc))
    return idx, sc


def route_logits(r, rows: int, e: int) -> np.ndarray:
    lg = r.standard_normal((rows, e)).astype(np.float32)
    lg[::3] = np.round(lg[::3] * 2) / 2  # every third row: many ties
    lg[1] = 0.0                          # one row entirely tied
    return lg


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("e,k", [(8, 2), (60, 4), (128, 8), (200, 1), (64, 64)])
def test_moe_route_vs_oracle(gpu, e, k, norm):
    r = H.rng(e * 10 + k + norm)
    lg = route_logits(r, 300, e)
    want_idx, want_sc = oracle_route(lg, k, norm)
    case(f"nvf_moe_route E={e} K={k} norm={norm}")
    idx, sc = ops.moe_route(torch.from_numpy(lg).to(gpu), k, norm)
    H.assert_bitexact(idx.cpu().numpy(), want_idx, "expert ids")
    got = sc.cpu().numpy()
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want_sc.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1, f"scores differ by {ulps.max()} ulp"


def test_moe_route_vs_reference_kernel(gpu, ref):
    r = H.rng(7)
    for e, k, norm in ((60, 4, True), (128, 8, False), (16, 16, True)):
        lg = route_logits(r, 257, e)
        d_lg = torch.from_numpy(lg).to(gpu)
        idx = torch.empty((257, k), dtype=torch.int32, device=gpu)
        sc = torch.empty((257, k), dtype=torch.float32, device=gpu)
        idx2, sc2 = torch.empty_like(idx), torch.empty_like(sc)
        torch.cuda.synchronize()
        case(f"reference moe_route E={e} K={k} norm={norm}")
        ref.ref_hip_moe_route(dptr(d_lg), 257, e, k, norm, dptr(idx), dptr(sc))
        case(f"hip_moe_route E={e} K={k} norm={norm}")
        ops.lib().hip_moe_route(dptr(d_lg), 257, e, k, norm, dptr(idx2), dptr(sc2))
        torch.cuda.synchronize()
        H.assert_bitexact(idx2.cpu().numpy(), idx.cpu().numpy(), "ids vs reference kernel")
        H.assert_bitexact(sc2.cpu().numpy(), sc.cpu().numpy(), "scores vs reference kernel")


@pytest.mark.parametrize("e,k", [(60, 4), (128, 8), (16, 16)])
def test_moe_route_nan_rows(gpu, ref, e, k):
    """A row with one NaN logit and an all-NaN row: every probability is NaN, and the
    reference's scan (best = i, strict >) keeps ids 0..K-1 in order; no id leaves [0, E)."""
    lg = H.rng(e + k).standard_normal((4, e)).astype(np.float32)
    lg[1, e // 2] = np.nan
    lg[2, :] = np.nan
    want_idx, want_sc = oracle_route(lg, k, True)
    d_lg = torch.from_numpy(lg).to(gpu)
    case(f"nvf_moe_route NaN rows E={e} K={k}")
    idx, sc = ops.moe_route(d_lg, k, True)
    got_idx, got_sc = idx.cpu().numpy(), sc.cpu().numpy()
    assert ((got_idx >= 0) & (got_idx < e)).all(), "expert id out of range"
    H.assert_bitexact(got_idx, want_idx, "expert ids (NaN rows) vs oracle")
    np.testing.assert_array_equal(np.isnan(got_sc), np.isnan(want_sc))
    np.testing.assert_array_equal(got_idx[1:3], np.tile(np.arange(k, dtype=np.int32), (2, 1)))
    ok = ~np.isnan(want_sc)
    H.assert_bitexact(got_sc[ok], want_sc[ok], "finite scores (NaN rows) vs oracle")
    ridx = torch.empty((4, k), dtype=torch.int32, device=gpu)
    rsc = torch.empty((4, k), dtype=torch.float32, device=gpu)
    torch.cuda.synchronize()
    case(f"reference moe_route NaN rows E={e} K={k}")
    ref.ref_hip_moe_route(dptr(d_lg), 4, e, k, True, dptr(ridx), dptr(rsc))
    torch.cuda.synchronize()
    H.assert_bitexact(got_idx, ridx.cpu().numpy(), "expert ids (NaN rows) vs reference kernel")


def moe_case(r, rows, hid, inter, k, n_exp, slots, w_bf16, x_dt=H.F32):
    x = H.gen_act(r, (rows, hid), x_dt)
    wdt = H.BF16 if w_bf16 else H.F16
    gu = H.to_storage((r.standard_normal((slots, 2 * inter, hid)) * 0.05).astype(np.float32), wdt)
    dn = H.to_storage((r.standard_normal((slots, hid, inter)) * 0.05).astype(np.float32), wdt)
    if not w_bf16:  # normal fp16 values (the reference's device fp16 decoder mishandles subnormals)
        for a in (gu, dn):
            sub = (a & 0x7C00) == 0
            a[sub] = (a[sub] & 0x8000) | 0x0400
    idx = np.stack([r.permutation(n_exp)[:k] for _ in range(rows)]).astype(np.int32)
    score = r.uniform(0.05, 0.5, (rows, k)).astype(np.float32)
    slot_of = r.permutation(slots)[:n_exp].astype(np.int32)
    return x, gu, dn, idx, score, slot_of


def oracle_ffn(x, x_dt, gu, dn, w_bf16, idx, score, slot_of, slots, out_in):
    rows, hid = out_in.shape
    inter = dn.shape[-1]
    out = np.empty((rows, hid), np.float64)
    err = np.empty((rows, hid), np.float64)
    H.oracle().orc_moe_ffn(H.ptr(x), x_dt, H.ptr(idx), H.ptr(score), H.ptr(gu), H.ptr(dn), int(w_bf16),
                           H.ptr(slot_of), rows, hid, inter, idx.shape[1], slots,
                           H.ptr(np.ascontiguousarray(out_in, np.float64)), H.ptr(out), H.ptr(err))
    return out, err


def assert_within(got, ideal, err, out_dt, what, w_bf16=False):
    g = H.from_storage(got, out_dt)
    tol = (6.0 if w_bf16 else 12.0) * err + (0.0 if out_dt == H.F32 else 0.5 * H.ulp(ideal, out_dt))
    bad = ~(np.abs(g - ideal) <= tol)
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside the bound; first at {i}: "
                             f"got {g[i]!r} ideal {ideal[i]!r} tol {tol[i]!r}")


@pytest.mark.parametrize("x_dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("w_bf16", [False, True], ids=["w_f16", "w_bf16"])
@pytest.mark.parametrize("rows,hid,inter,k,n_exp,slots", [
    (1, 256, 128, 2, 8, 8),          # decode: one token
    (37, 512, 320, 4, 16, 20),       # 32-row tiles, ragged 2I / H against the 128-column tile
    (600, 256, 96, 8, 32, 32),       # 4800 pairs: 128-row tiles
    (9, 200, 72, 3, 6, 6),           # H and I not multiples of 16
    (300, 256, 128, 8, 16, 16),      # 2400 pairs, 150 per slot
    (5, 100, 44, 2, 4, 4),           # H not a multiple of 8: the tile kernel, element-wise staging
    (300, 64, 32, 1, 1, 1),          # every pair in one slot: one long run of tiles
])
def test_moe_ffn_vs_oracle(gpu, x_dt, w_bf16, rows, hid, inter, k, n_exp, slots):
    r = H.rng(rows * 7 + hid + x_dt + 2 * w_bf16)
    x, gu, dn, idx, score, slot_of = moe_case(r, rows, hid, inter, k, n_exp, slots, w_bf16, x_dt)
    score[0, -1] = 0.0                       # skipped: weight 0
    if rows > 2:
        slot_of[idx[2, 0]] = -1              # skipped: the expert has no slot
    for out_dt in (H.F32, x_dt) if x_dt != H.F32 else (H.F32,):
        out_in = H.gen_act(r, (rows, hid), out_dt)
        ideal, err = oracle_ffn(x, x_dt, gu, dn, w_bf16, idx, score, slot_of, slots, H.from_storage(out_in, out_dt))
        out = H.to_dev(out_in, gpu, out_dt)
        wdt = torch.bfloat16 if w_bf16 else torch.float16
        case(f"nvf_moe_ffn_ws rows={rows} H={hid} I={inter} K={k} x={x_dt} out={out_dt} bf16={w_bf16}")
        ops.moe_ffn(H.to_dev(x, gpu, x_dt), torch.from_numpy(idx).to(gpu), torch.from_numpy(score).to(gpu),
                    H.to_dev(gu, gpu, H.BF16 if w_bf16 else H.F16).view(wdt),
                    H.to_dev(dn, gpu, H.BF16 if w_bf16 else H.F16).view(wdt), torch.from_numpy(slot_of).to(gpu),
                    inter, slots, out)
        assert_within(H.to_host(out), ideal, err, out_dt, f"moe ffn x={x_dt} out={out_dt}", w_bf16)


@pytest.mark.parametrize("w_bf16", [False, True], ids=["w_f16", "w_bf16"])
def test_dropin_moe_ffn_vs_reference_kernel(gpu, ref, w_bf16):
    r = H.rng(90 + w_bf16)
    rows, hid, inter, k, n_exp, slots = 24, 384, 192, 4, 12, 12
    x, gu, dn, idx, score, slot_of = moe_case(r, rows, hid, inter, k, n_exp, slots, w_bf16)
    out_in = r.standard_normal((rows, hid)).astype(np.float32)
    ideal, err = oracle_ffn(x, H.F32, gu, dn, w_bf16, idx, score, slot_of, slots, out_in.astype(np.float64))
    d = [torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in (x, idx, score, gu, dn, slot_of)]
    mine, theirs = torch.from_numpy(out_in).to(gpu), torch.from_numpy(out_in).to(gpu)
    torch.cuda.synchronize()
    case(f"reference moe_ffn bf16={w_bf16}")
    ref.ref_hip_moe_ffn(*[dptr(t) for t in d], rows, hid, inter, k, w_bf16, dptr(theirs))
    case(f"hip_moe_ffn bf16={w_bf16}")
    ops.lib().hip_moe_ffn(*[dptr(t) for t in d], rows, hid, inter, k, w_bf16, dptr(mine))
    torch.cuda.synchronize()
    assert_within(theirs.cpu().numpy(), ideal, err, H.F32, "reference kernel")
    assert_within(mine.cpu().numpy(), ideal, err, H.F32, "drop-in", w_bf16)


def test_dropin_moe_ffn_runs_in_chunks(gpu):
    """More rows than the 64 MiB scratch takes at once (3 chunks): each token's result is
    independent of the chunking."""
    r = H.rng(95)
    rows, hid, inter, k, n_exp, slots = 7000, 256, 128, 8, 32, 32
    x, gu, dn, idx, score, slot_of = moe_case(r, rows, hid, inter, k, n_exp, slots, True)
    per_chunk_bytes = ops.lib().nvf_moe_ffn_workspace_size(rows, hid, inter, k, 65536)
    assert per_chunk_bytes > 64 << 20  # the drop-in must split this call
    out_in = np.zeros((rows, hid), np.float32)
    ideal, err = oracle_ffn(x, H.F32, gu, dn, True, idx, score, slot_of, slots, out_in.astype(np.float64))
    d = [torch.from_numpy(np.ascontiguousarray(a)).to(gpu) for a in (x, idx, score, gu, dn, slot_of)]
    out = torch.zeros((rows, hid), device=gpu)
    torch.cuda.synchronize()
    case("hip_moe_ffn 7000 rows (chunked)")
    ops.lib().hip_moe_ffn(*[dptr(t) for t in d], rows, hid, inter, k, True, dptr(out))
    torch.cuda.synchronize()
    assert_within(out.cpu().numpy(), ideal, err, H.F32, "chunked drop-in", True)


def test_add_inplace_and_scale_rows_sigmoid(gpu, ref):
    r = H.rng(96)
    for n in (1, 7, 4096, 100003):
        a = r.standard_normal(n).astype(np.float32)
        b = r.standard_normal(n).astype(np.float32)
        d_a, d_b = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
        case(f"hip_add_inplace n={n}")
        ops.lib().hip_add_inplace(dptr(d_a), dptr(d_b), n)
        torch.cuda.synchronize()
        H.assert_bitexact(d_a.cpu().numpy(), a + b, "add_inplace")
    for rows, cols in ((1, 5), (33, 2048), (300, 1000)):
        dst = r.standard_normal((rows, cols)).astype(np.float32)
        s = (r.standard_normal(rows) * 4).astype(np.float32)
        d_s = torch.from_numpy(s).to(gpu)
        mine, theirs = torch.from_numpy(dst).to(gpu), torch.from_numpy(dst).to(gpu)
        torch.cuda.synchronize()
        case(f"scale_rows_sigmoid {rows}x{cols}")
        ref.ref_hip_scale_rows_sigmoid(dptr(theirs), dptr(d_s), rows, cols)
        ops.lib().hip_scale_rows_sigmoid(dptr(mine), dptr(d_s), rows, cols)
        torch.cuda.synchronize()
        H.assert_bitexact(mine.cpu().numpy(), theirs.cpu().numpy(), "scale_rows_sigmoid vs reference kernel")
        want = dst * (1.0 / (1.0 + np.exp(-s.astype(np.float64))))[:, None]
        assert np.allclose(mine.cpu().numpy(), want, rtol=4 * 2 ** -24, atol=0)
