"""GPU parity of the Q8_0 GEMM (the reference's hip_matmul_q8, src/hip_ops.hip:639-686)
and its row quantizer (q8_row_scale_kernel :205-217, quantizer :244-245).

Bars:
* row scales and int8 rows bit-exact against the oracle;
* GEMM outputs within the oracle's fp32 summation bound `err` (each output is
  sum_b ws*I_b / scale with exact integer block dots I_b, summed in fp32 in some
  order), plus half an ulp of the output dtype for fp16/bf16 outputs;
* bit-exact on inputs where every fp32 partial sum is exact (power-of-two block
  scales, small integers);
* the drop-in hip_matmul_q8 within the bound of the oracle, and within twice the
  bound of the reference's own hip_matmul_q8 (tile path for m > 8, GEMV path for
  m <= 8 with k % 128 == 0) where oracle/_ref was built.
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


def oracle_gemm(x: np.ndarray, dt: int, w8: np.ndarray, ws: np.ndarray, m: int, n: int, k: int):
    o = H.oracle()
    out = np.empty((m, n), np.float64)
    err = np.empty((m, n), np.float64)
    sc = np.empty(m, np.float32)
    xq = np.empty((m, k), np.int8)
    o.orc_matmul_q8(H.ptr(x), dt, H.ptr(w8), H.ptr(ws), m, n, k, H.ptr(out), H.ptr(err), H.ptr(sc), H.ptr(xq))
    return out, err, sc, xq


def assert_within(got: np.ndarray, ideal: np.ndarray, err: np.ndarray, out_dt: int, what: str,
                  factor: float = 1.0) -> None:
    g = H.from_storage(got, out_dt)
    tol = factor * err + (0.0 if out_dt == H.F32 else 0.5 * H.ulp(ideal, out_dt))
    bad = ~(np.abs(g - ideal) <= tol)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside the bound; first at {tuple(i)}: "
                             f"got {g[tuple(i)]!r} ideal {ideal[tuple(i)]!r} tol {tol[tuple(i)]!r}")


def make(seed: int, m: int, n: int, k: int, dt: int):
    r = H.rng(seed)
    x = H.gen_act(r, (m, k), dt)
    w8, ws = H.gen_q8_0(r, n, k)
    return x, w8, ws


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("m,k", [(7, 3584), (33, 96), (5, 100), (300, 18944)])
def test_quantize_rows_bitexact(gpu, dt, m, k):
    r = H.rng(m * k + dt)
    x = H.gen_act(r, (m, k), dt)
    x[1] = H.to_storage(np.zeros(k, np.float32), dt)
    o = H.oracle()
    sc = np.empty(m, np.float32)
    q = np.empty((m, k), np.int8)
    o.orc_q8_row_scale(H.ptr(x), H.ptr(sc), m, k, dt)
    o.orc_q8_quantize(H.ptr(x), H.ptr(sc), q.ctypes.data, m, k, dt)
    case(f"q8_quantize_rows m={m} k={k} dt={dt}")
    gs, gq = ops.q8_quantize_rows(H.to_dev(x, gpu, dt))
    H.assert_bitexact(gs.cpu().numpy(), sc, "row scale")
    H.assert_bitexact(gq.cpu().numpy(), q, "int8 rows")
    assert gs[1].item() == 0.0


@pytest.mark.parametrize("out_dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("m,n,k", [(1, 32, 32), (5, 7, 96), (130, 250, 320), (257, 129, 1056), (64, 4608, 3584),
                                   (8, 1000, 4864), (16, 500, 352), (17, 64, 128), (3, 3584, 18944), (12, 37, 160),
                                   # decode GEMV: batch-1 qkv (activation rows staged in LDS) and a wide output
                                   # whose staged rows would cost resident workgroups (register activations)
                                   (1, 4608, 3584), (8, 20000, 3584),
                                   # fewer column groups than CUs, long K
                                   (12, 1000, 9216),
                                   # at least 2048 column groups: waves of two 16-column groups
                                   # (the last one partial)
                                   (3, 33000, 512), (12, 32784, 256)])
def test_matmul_q8_0_vs_oracle(gpu, out_dt, m, n, k):
    x, w8, ws = make(m + 3 * n + k + out_dt, m, n, k, H.F32)
    zero_row = 2 if m > 2 else None
    if zero_row is not None:
        x[zero_row] = 0.0  # a zero row: scale 0, output 0
    ideal, err, sc, xq = oracle_gemm(x, H.F32, w8, ws, m, n, k)
    case(f"matmul_q8_0 m={m} n={n} k={k} out_dt={out_dt}")
    out = ops.matmul_q8_0(H.to_dev(xq, gpu), H.to_dev(sc, gpu), H.to_dev(w8, gpu), H.to_dev(ws, gpu), n,
                          H.torch_dtype(out_dt))
    got = H.to_host(out)
    assert_within(got, ideal, err, out_dt, "gemm")
    if zero_row is not None:
        assert (H.from_storage(got, out_dt)[zero_row] == 0).all()


@pytest.mark.parametrize("out_dt", DTYPES, ids=DT_IDS)
def test_matmul_q8_0_exact_inputs_bitexact(gpu, out_dt):
    """Small integers with one 127 per row (scale 1, xq == x) and power-of-two
    block scales: every fp32 partial sum is exact, so the GEMM is bit-exact."""
    r = H.rng(77)
    m, n, k = 150, 140, 160
    x = r.integers(-8, 9, (m, k)).astype(np.float32)
    x[:, 5] = 127.0
    w8 = r.integers(-127, 128, n * k, dtype=np.int8)
    exps = (np.arange(n)[:, None] + np.arange(k // 32)[None, :]) % 3 + 4
    ws = np.ldexp(1.0, -exps).astype(np.float16).view(np.uint16).reshape(-1)
    ideal, err, sc, xq = oracle_gemm(x, H.F32, w8, ws, m, n, k)
    case(f"matmul_q8_0 exact inputs out_dt={out_dt}")
    out = ops.matmul_q8_0(H.to_dev(xq, gpu), H.to_dev(sc, gpu), H.to_dev(w8, gpu), H.to_dev(ws, gpu), n,
                          H.torch_dtype(out_dt))
    H.assert_bitexact(H.to_host(out), H.to_storage(ideal.astype(np.float32), out_dt), "exact gemm")


@pytest.mark.parametrize("dt", [H.F16, H.BF16], ids=["f16", "bf16"])
def test_matmul_q8_typed_activations(gpu, dt):
    """Quantize fp16/bf16 activations then the GEMM: the oracle quantizes the same
    storage values (upcast exactly), so scales and int8 rows agree bit for bit."""
    m, n, k = 97, 300, 1024
    x, w8, ws = make(5 + dt, m, n, k, dt)
    ideal, err, sc, xq = oracle_gemm(x, dt, w8, ws, m, n, k)
    case(f"matmul_q8 typed dt={dt}")
    out = ops.matmul_q8(H.to_dev(x, gpu, dt), H.to_dev(w8, gpu), H.to_dev(ws, gpu), n)
    assert_within(H.to_host(out), ideal, err, dt, "typed gemm")


def test_matmul_q8_large_grid_sampled_rows(gpu):
    """The gate_up projection shape of BASELINE config 2 (n = 2 x 18944, k = 3584)
    at 2048 tokens: every output column of 12 sampled rows against the oracle."""
    m, n, k = 2048, 37888, 3584
    r = H.rng(2024)
    x = r.standard_normal((m, k)).astype(np.float32)
    w8, ws = H.gen_q8_0(r, n, k)
    case("matmul_q8 gate_up shape, sampled rows")
    xd = H.to_dev(x, gpu)
    out = ops.matmul_q8(xd, H.to_dev(w8, gpu), H.to_dev(ws, gpu), n)
    got = out.cpu().numpy()
    rows = np.array([0, 1, 127, 128, 129, 511, 1000, 1023, 1024, 1500, 2046, 2047])
    ideal, err, _, _ = oracle_gemm(np.ascontiguousarray(x[rows]), H.F32, w8, ws, rows.size, n, k)
    assert_within(got[rows], ideal, err, H.F32, "gate_up rows")


@pytest.mark.parametrize("m,n,k", [(4, 256, 1024), (8, 96, 3584), (37, 200, 320), (130, 64, 896)])
def test_dropin_matmul_q8_vs_oracle_and_reference(gpu, m, n, k):
    x, w8, ws = make(m * 7 + n + k, m, n, k, H.F32)
    ideal, err, _, _ = oracle_gemm(x, H.F32, w8, ws, m, n, k)
    xd, w8d, wsd = H.to_dev(x, gpu), H.to_dev(w8, gpu), H.to_dev(ws, gpu)
    out = torch.empty((m, n), dtype=torch.float32, device=gpu)
    case(f"hip_matmul_q8 drop-in m={m} n={n} k={k}")
    ops.lib().hip_matmul_q8(xd.data_ptr(), w8d.data_ptr(), wsd.data_ptr(), m, n, k, out.data_ptr())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_within(got, ideal, err, H.F32, "drop-in vs oracle")
    r = H.ref_hip()
    if r is None:
        return
    ref_out = torch.empty((m, n), dtype=torch.float32, device=gpu)
    case(f"reference hip_matmul_q8 m={m} n={n} k={k}")
    r.ref_hip_matmul_q8(xd.data_ptr(), w8d.data_ptr(), wsd.data_ptr(), m, n, k, ref_out.data_ptr())
    rg = ref_out.cpu().numpy()
    assert_within(rg, ideal, err, H.F32, "reference vs oracle")
    assert (np.abs(got.astype(np.float64) - rg) <= 2 * err).all()


def test_dropin_matmul_q8_grows_scratch(gpu):
    """Two drop-in calls in a row, the second larger: the grow-only scratch is
    re-allocated and both results are right."""
    for m, n, k in ((3, 64, 256), (200, 96, 512)):
        x, w8, ws = make(m + n, m, n, k, H.F32)
        ideal, err, _, _ = oracle_gemm(x, H.F32, w8, ws, m, n, k)
        xd, w8d, wsd = H.to_dev(x, gpu), H.to_dev(w8, gpu), H.to_dev(ws, gpu)
        out = torch.empty((m, n), dtype=torch.float32, device=gpu)
        case(f"hip_matmul_q8 scratch m={m}")
        ops.lib().hip_matmul_q8(xd.data_ptr(), w8d.data_ptr(), wsd.data_ptr(), m, n, k, out.data_ptr())
        torch.cuda.synchronize()
        assert_within(out.cpu().numpy(), ideal, err, H.F32, "drop-in")


SPLITK = [(130, 300, 2048), (40, 1000, 4096), (300, 257, 1024), (256, 3584, 3584)]


@pytest.mark.parametrize("out_dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("m,n,k", SPLITK)
def test_matmul_q8_0_split_k(gpu, out_dt, m, n, k):
    """Outputs with too few 128 x 128 tiles to fill the GPU split K (fp32 partial
    sums, then an in-order reduction): within the oracle's summation bound, like
    the unsplit kernel; odd n exercises the reduction's column tail."""
    assert ops.lib().nvf_matmul_q8_0_workspace_size(m, n, k) > 0
    x, w8, ws = make(m * 5 + n + k + out_dt, m, n, k, H.F32)
    x[1] = 0.0
    rows = np.arange(m) if m * n * k <= 1 << 30 else np.array([0, 1, 2, 63, 64, 127, 128, 200, m - 1])
    ideal, err, sc, xq = oracle_gemm(np.ascontiguousarray(x[rows]), H.F32, w8, ws, rows.size, n, k)
    _, _, sc_all, xq_all = oracle_gemm(x, H.F32, w8, ws[: (k // 32)], m, 1, k)  # all rows' scale and int8 row
    args = (H.to_dev(xq_all, gpu), H.to_dev(sc_all, gpu), H.to_dev(w8, gpu), H.to_dev(ws, gpu), n,
            H.torch_dtype(out_dt))
    case(f"matmul_q8_0 split-K m={m} n={n} k={k} out_dt={out_dt}")
    got = H.to_host(ops.matmul_q8_0(*args))
    assert_within(got[rows], ideal, err, out_dt, "split-K gemm")
    assert (H.from_storage(got, out_dt)[1] == 0).all()
    case(f"matmul_q8_0 unsplit m={m} n={n} k={k} out_dt={out_dt}")
    got = H.to_host(ops.matmul_q8_0(*args, split=False))
    assert_within(got[rows], ideal, err, out_dt, "unsplit gemm")


def test_matmul_q8_config2_full_vs_torch(gpu):
    """BASELINE config 2's gate_up GEMM at full size (16384 x 37888 x 3584, every
    tile of the XCD-aware order) against a torch fp32 matmul of the exactly
    dequantized weights (x int8 and ws * w8 are exact in fp32).  Every element is
    within both sides' summation bounds: this kernel's (nblk + 2) u S, torch's
    (k + 1) u S, with S = (|x| |w|^T) / row_scale and u = 2^-24."""
    m, n, k = 16384, 37888, 3584
    g = torch.Generator(device=gpu)
    g.manual_seed(11)
    xq = torch.randint(-127, 128, (m, k), device=gpu, dtype=torch.int8, generator=g)
    sc = torch.rand(m, device=gpu, generator=g) * 10.0 + 1.0
    w8 = torch.randint(-127, 128, (n, k), device=gpu, dtype=torch.int8, generator=g)
    ws = (torch.rand(n, k // 32, device=gpu, generator=g) * 9e-3 + 1e-3).half()
    case("matmul_q8_0 config 2 gate_up, full size, vs torch fp32")
    out = ops.matmul_q8_0(xq, sc, w8.view(-1), ws.view(-1), n, torch.float32)
    torch.backends.cuda.matmul.allow_tf32 = False
    w = (w8.float().view(n, k // 32, 32) * ws.float().view(n, k // 32, 1)).view(n, k)
    x = xq.float()
    ideal = (x @ w.t()) / sc[:, None]
    bound = (x.abs() @ w.abs().t()) / sc[:, None]
    del x, w
    tol = (k + k // 32 + 3) * 2.0 ** -24 * bound + 1e-30
    bad = ((out - ideal).abs() > tol).sum().item()
    assert bad == 0, f"{bad} of {m * n} outputs outside the summation bounds"
