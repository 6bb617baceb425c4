"""GPU parity of the dense / K-quant weight GEMM (the reference's hip_matmul,
hip_matmul_u16 and hip_matmul_qk: src/hip_ops.hip:43-64, :577-598, :746-777) and of
the row gather (hip_gather_rows, :611-619, :788-795).

Bars:
* GEMM outputs within the oracle's bound `err` = (k + 2) 2^-24 sum_i |x_i w_i|
  around the exact (float64) product of the exactly decoded weights, which covers
  fp32 sums in any order (tests/test_oracle.py pins it against three orders), plus
  half an ulp of the output dtype for fp16/bf16 outputs.  bf16 weights: three times
  that bound, fp16 weights six times -- the split products take each activation as three
  exact bf16 pieces (and an fp16 weight as two) and sum the exact piece products in
  fp32, 3k (6k) terms instead of k;
* bit-exact where every fp32 partial sum is exact (small integer activations,
  weights that are small multiples of 1/8);
* the reference's own kernels (oracle/_ref, where built) held to the same bound on
  the same inputs, so both sides agree with each other within twice of it;
* gather bit-exact, with a NaN row for an index outside the table when checked.
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
FORMATS = [H.F32, H.F16, H.BF16, 12, 13, 14]
FMT_IDS = ["f32", "f16", "bf16", "q4k", "q5k", "q6k"]


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


def oracle_matmul(x, x_dt, w, w_format, m, n, k, layout=H.GGML):
    out = np.empty((m, n), np.float64)
    err = np.empty((m, n), np.float64)
    H.oracle().orc_matmul_w(H.ptr(x), x_dt, H.ptr(w), w_format, layout, m, n, k, H.ptr(out), H.ptr(err))
    return out, err


def assert_within(got: np.ndarray, ideal: np.ndarray, err: np.ndarray, out_dt: int, what: str,
                  w_format: int | None = None) -> None:
    g = H.from_storage(got, out_dt)
    tol = {H.BF16: 3.0, H.F16: 6.0}.get(w_format, 1.0) * err + (0.0 if out_dt == H.F32 else 0.5 * H.ulp(ideal, out_dt))
    bad = ~(np.abs(g - ideal) <= tol)
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside the bound; first at {i}: "
                             f"got {g[i]!r} ideal {ideal[i]!r} tol {tol[i]!r}")


def w_dev(w: np.ndarray, w_format: int, gpu):
    return H.to_dev(w, gpu, w_format if w_format in (H.F16, H.BF16) else None)


@pytest.mark.parametrize("w_format", FORMATS, ids=FMT_IDS)
@pytest.mark.parametrize("x_dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("m,n,k", [(1, 200, 512), (29, 131, 768), (300, 260, 1024)])
def test_matmul_within_bound(gpu, w_format, x_dt, m, n, k):
    r = H.rng(1000 * w_format + 10 * x_dt + m)
    x = H.gen_act(r, (m, k), x_dt)
    w = H.gen_weights(r, n, k, w_format)
    ideal, err = oracle_matmul(x, x_dt, w, w_format, m, n, k)
    for out_dt in DTYPES:
        case(f"nvf_matmul fmt={w_format} x={x_dt} out={out_dt} m={m} n={n} k={k}")
        got = ops.matmul(H.to_dev(x, gpu, x_dt), w_dev(w, w_format, gpu), n, w_format,
                         out_dtype=H.torch_dtype(out_dt))
        assert_within(H.to_host(got), ideal, err, out_dt, f"fmt {w_format} x {x_dt} out {out_dt}", w_format)


@pytest.mark.parametrize("w_format", [H.F16, H.BF16], ids=["f16", "bf16"])
def test_matmul_tile_near_flt_max(gpu, w_format):
    """fp32 activations above the largest bf16 (~3.39e38) on the 16-bit matrix-core tile
    path (m > 16): the exact three-piece split must not turn them into inf - inf = NaN."""
    r = H.rng(4242 + w_format)
    m, n, k = 64, 128, 256
    x = H.gen_act(r, (m, k), H.F32)
    x[::2, 7] = np.float32(3.4e38)    # above the largest bf16, below FLT_MAX
    x[1::2, 9] = np.float32(-3.39e38)
    w = H.to_storage((r.standard_normal((n, k)) * 1e-3).astype(np.float32), w_format)
    ideal, err = oracle_matmul(x, H.F32, w, w_format, m, n, k)
    assert np.isfinite(ideal).all()
    case(f"nvf_matmul near FLT_MAX fmt={w_format} m={m} n={n} k={k}")
    got = ops.matmul(H.to_dev(x, gpu), w_dev(w, w_format, gpu), n, w_format)
    g = H.to_host(got)
    assert np.isfinite(g).all(), "non-finite output for finite inputs"
    assert_within(g, ideal, err, H.F32, f"near FLT_MAX fmt {w_format}", w_format)


@pytest.mark.parametrize("w_format", FORMATS, ids=FMT_IDS)
@pytest.mark.parametrize("m,n,k", [(3, 256, 100), (70, 128, 200), (33, 512, 4)])
def test_matmul_ragged_k(gpu, w_format, m, n, k):
    """k not a multiple of the 16-element stage (the reference takes any k)."""
    r = H.rng(77 + w_format + k)
    x = H.gen_act(r, (m, k), H.F32)
    w = H.gen_weights(r, n, k, w_format)
    ideal, err = oracle_matmul(x, H.F32, w, w_format, m, n, k)
    case(f"nvf_matmul ragged fmt={w_format} m={m} n={n} k={k}")
    got = ops.matmul(H.to_dev(x, gpu), w_dev(w, w_format, gpu), n, w_format)
    assert_within(H.to_host(got), ideal, err, H.F32, f"ragged fmt {w_format}", w_format)


@pytest.mark.parametrize("w_format", FORMATS, ids=FMT_IDS)
@pytest.mark.parametrize("m,n,k", [(1, 1000, 3584), (2, 37, 264), (4, 4100, 256), (5, 513, 1032), (8, 9000, 512),
                                   (12, 20000, 256), (16, 64, 8), (3, 256, 40), (2, 66000, 256),
                                   (1, 65601, 512), (1, 20000, 1000), (2, 40001, 3584)])
def test_matmul_decode_rows(gpu, w_format, m, n, k):
    """m <= 16 with k % 8 == 0: the weight-streaming decode product (every row-group
    size, column-quad count, a k that is not a multiple of the 128- or 512-element step;
    wide and mid-width dense outputs take 64 lanes per weight row)."""
    if w_format >= 12 and (n * k) % 256:
        pytest.skip("K-quant weights cover whole 256-element superblocks")
    r = H.rng(700 + w_format + m + k)
    x = H.gen_act(r, (m, k), H.BF16)
    w = H.gen_weights(r, n, k, w_format)
    ideal, err = oracle_matmul(x, H.BF16, w, w_format, m, n, k)
    case(f"nvf_matmul decode fmt={w_format} m={m} n={n} k={k}")
    got = ops.matmul(H.to_dev(x, gpu, H.BF16), w_dev(w, w_format, gpu), n, w_format, out_dtype=torch.float32)
    assert_within(H.to_host(got), ideal, err, H.F32, f"decode fmt {w_format}", w_format)


@pytest.mark.parametrize("w_format", [H.F32, H.BF16, 14], ids=["f32", "bf16", "q6k"])
@pytest.mark.parametrize("m", [3, 40])
def test_matmul_unaligned_operands(gpu, w_format, m):
    """x (and dense weights) 16-byte misaligned: every value read on its own."""
    r = H.rng(800 + w_format + m)
    n, k = 96, 512
    x = H.gen_act(r, (m, k), H.F32)
    w = H.gen_weights(r, n, k, w_format)
    ideal, err = oracle_matmul(x, H.F32, w, w_format, m, n, k)
    xb = torch.zeros(m * k + 1, device=gpu)
    xb[1:] = torch.from_numpy(x.reshape(-1)).to(gpu)
    xv = xb[1:].view(m, k)
    if w_format < 12:
        wt = w_dev(w, w_format, gpu).reshape(-1)
        wb = torch.zeros(wt.numel() + 1, dtype=wt.dtype, device=gpu)
        wb[1:] = wt
        wv = wb[1:]
    else:
        wb = torch.zeros(w.size + 2, dtype=torch.uint8, device=gpu)  # Q6_K blocks need 2-byte alignment only
        wb[2:] = H.to_dev(w, gpu)
        wv = wb[2:]
    case(f"nvf_matmul unaligned fmt={w_format} m={m}")
    got = ops.matmul(xv, wv, n, w_format)
    assert_within(H.to_host(got), ideal, err, H.F32, f"unaligned fmt {w_format}", w_format)


@pytest.mark.parametrize("w_format", [H.F32, H.F16, H.BF16], ids=DT_IDS)
def test_matmul_exact_inputs_bitexact(gpu, w_format):
    r = H.rng(90 + w_format)
    m, n, k = 150, 140, 512
    x = r.integers(-8, 9, (m, k)).astype(np.float32)
    w = H.to_storage((r.integers(-16, 17, (n, k)) * 0.125).astype(np.float32), w_format)
    ideal, _ = oracle_matmul(x, H.F32, w, w_format, m, n, k)
    case(f"nvf_matmul exact fmt={w_format}")
    got = ops.matmul(H.to_dev(x, gpu), w_dev(w, w_format, gpu), n, w_format)
    H.assert_bitexact(H.to_host(got).astype(np.float64), ideal, "exact inputs")


def test_matmul_q4k_layouts(gpu):
    r = H.rng(95)
    m, n, k = 40, 96, 512
    x = H.gen_act(r, (m, k), H.BF16)
    w = H.gen_weights(r, n, k, 12)
    d_x, d_w = H.to_dev(x, gpu, H.BF16), H.to_dev(w, gpu)
    for layout in (H.GGML, H.HIP_LEGACY):
        ideal, err = oracle_matmul(x, H.BF16, w, 12, m, n, k, layout)
        case(f"nvf_matmul q4k layout={layout}")
        got = ops.matmul(d_x, d_w, n, 12, out_dtype=torch.float32, qk_layout=layout)
        assert_within(H.to_host(got), ideal, err, H.F32, f"q4k layout {layout}")


def test_matmul_rejects_bad_arguments(gpu):
    x = torch.zeros((4, 256), device=gpu)
    w = torch.zeros(3 * 144, dtype=torch.uint8, device=gpu)
    case("nvf_matmul bad arguments")
    with pytest.raises(ops.NvfError, match="superblocks"):
        ops.matmul(torch.zeros((4, 100), device=gpu), w, 1, 12)  # n*k = 100: not whole superblocks
    with pytest.raises(ops.NvfError, match="format"):
        ops.matmul(x, w, 3, 7)
    torch.cuda.synchronize()


def dropin(lib, w_format: int, d_x, d_w, m, n, k, out) -> None:
    if w_format == H.F32:
        lib.hip_matmul(dptr(d_x), dptr(d_w), m, n, k, dptr(out))
    elif w_format in (H.F16, H.BF16):
        lib.hip_matmul_u16(dptr(d_x), dptr(d_w), m, n, k, dptr(out), w_format == H.BF16)
    else:
        lib.hip_matmul_qk(dptr(d_x), dptr(d_w), m, n, k, dptr(out), w_format)


@pytest.mark.parametrize("w_format", FORMATS, ids=FMT_IDS)
@pytest.mark.parametrize("m,n,k", [(5, 300, 512), (200, 136, 1024), (17, 256, 50)])
def test_dropin_matmul_vs_oracle(gpu, w_format, m, n, k):
    """hip_matmul / hip_matmul_u16 / hip_matmul_qk: fp32 activations and outputs; the
    Q4_K drop-in decodes the process-wide drop-in nibble order (GGML by default)."""
    r = H.rng(300 + w_format + m)
    x = H.gen_act(r, (m, k), H.F32)
    w = H.gen_weights(r, n, k, w_format)
    if w_format == H.F16:
        assert (((w & 0x7C00) == 0) & ((w & 0x03FF) != 0)).any()  # subnormals are in the draw
    ideal, err = oracle_matmul(x, H.F32, w, w_format, m, n, k)
    d_x, d_w = H.to_dev(x, gpu), H.to_dev(w, gpu)
    out = torch.empty((m, n), device=gpu)
    torch.cuda.synchronize()
    case(f"drop-in matmul fmt={w_format} m={m} n={n} k={k}")
    dropin(ops.lib(), w_format, d_x, d_w, m, n, k, out)
    torch.cuda.synchronize()
    assert_within(out.cpu().numpy(), ideal, err, H.F32, f"drop-in fmt {w_format}", w_format)


@pytest.mark.parametrize("w_format", FORMATS, ids=FMT_IDS)
@pytest.mark.parametrize("m,n,k", [(5, 300, 512), (130, 72, 768), (9, 256, 100)])
def test_dropin_matmul_vs_reference_kernels(gpu, ref, w_format, m, n, k):
    """The reference's own kernels and the drop-ins on the same inputs: both within the
    oracle's bound (the reference's device Q4_K decoder reads the HIP_LEGACY nibble
    order, so the drop-in is switched to it for that comparison).  fp16 weights are kept
    normal here: the reference's device fp16 decoder (fp16_to_float_u,
    src/hip_ops.hip:15-32) gives every subnormal one constant magnitude; the drop-in
    decodes them exactly (test_dropin_matmul_vs_oracle covers subnormals)."""
    r = H.rng(500 + w_format + m)
    x = H.gen_act(r, (m, k), H.F32)
    w = H.gen_weights(r, n, k, w_format)
    if w_format == H.F16:
        sub = (w & 0x7C00) == 0
        w[sub] = (w[sub] & 0x8000) | 0x0400  # +-2^-14, the smallest normal
    layout = H.HIP_LEGACY if w_format == 12 else H.GGML
    ideal, err = oracle_matmul(x, H.F32, w, w_format, m, n, k, layout)
    d_x, d_w = H.to_dev(x, gpu), H.to_dev(w, gpu)
    mine, theirs = torch.empty((m, n), device=gpu), torch.empty((m, n), device=gpu)
    torch.cuda.synchronize()
    case(f"reference matmul fmt={w_format} m={m} n={n} k={k}")
    if w_format == H.F32:
        ref.ref_hip_matmul(dptr(d_x), dptr(d_w), m, n, k, dptr(theirs))
    elif w_format in (H.F16, H.BF16):
        ref.ref_hip_matmul_u16(dptr(d_x), dptr(d_w), m, n, k, dptr(theirs), w_format == H.BF16)
    else:
        ref.ref_hip_matmul_qk(dptr(d_x), dptr(d_w), m, n, k, dptr(theirs), w_format)
    if w_format == 12:
        ops._check(ops.lib().nvf_set_dropin_q4k_layout(H.HIP_LEGACY), "set layout")
    try:
        case(f"drop-in matmul fmt={w_format} layout={layout}")
        dropin(ops.lib(), w_format, d_x, d_w, m, n, k, mine)
        torch.cuda.synchronize()
    finally:
        if w_format == 12:
            ops._check(ops.lib().nvf_set_dropin_q4k_layout(H.GGML), "set layout")
    assert_within(theirs.cpu().numpy(), ideal, err, H.F32, f"reference kernel fmt {w_format}")
    assert_within(mine.cpu().numpy(), ideal, err, H.F32, f"drop-in fmt {w_format}", w_format)


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("rows,cols,out_rows", [(1000, 3584, 257), (50, 33, 64), (7, 1, 5)])
def test_gather_rows_bitexact(gpu, dt, rows, cols, out_rows):
    r = H.rng(rows + cols + dt)
    table = H.gen_act(r, (rows, cols), dt)
    idx = r.integers(0, rows, out_rows).astype(np.int32)
    expect = np.empty((out_rows, cols), table.dtype)
    H.oracle().orc_gather_rows(H.ptr(table), H.ptr(idx), cols, out_rows, H.ptr(expect), dt)
    assert np.array_equal(expect, table[idx])
    case(f"nvf_gather_rows dt={dt} rows={rows} cols={cols} out_rows={out_rows}")
    got = ops.gather_rows(H.to_dev(table, gpu, dt), torch.from_numpy(idx).to(gpu))
    H.assert_bitexact(H.to_host(got), expect, "gather")


def test_gather_rows_bad_index_gives_nan_row(gpu):
    r = H.rng(8)
    table = r.standard_normal((10, 70)).astype(np.float32)
    idx = np.array([2, -1, 10, 9, 1 << 30], np.int32)
    case("nvf_gather_rows out-of-range indices")
    got = ops.gather_rows(torch.from_numpy(table).to(gpu), torch.from_numpy(idx).to(gpu)).cpu().numpy()
    assert np.array_equal(got[[0, 3]], table[[2, 9]])
    assert np.isnan(got[[1, 2, 4]]).all()
    case("hip_gather_rows out-of-range indices")
    d_t, d_i = torch.from_numpy(table).to(gpu), torch.from_numpy(idx).to(gpu)
    out = torch.empty((5, 70), device=gpu)
    torch.cuda.synchronize()
    ops.lib().hip_gather_rows(dptr(d_t), dptr(d_i), 10, 70, 5, dptr(out))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got[[0, 3]], table[[2, 9]])
    assert np.isnan(got[[1, 2, 4]]).all()


def test_dropin_gather_rows_vs_reference_kernel(gpu, ref):
    r = H.rng(9)
    rows, cols, out_rows = 300, 896, 100
    table = r.standard_normal((rows, cols)).astype(np.float32)
    idx = r.integers(0, rows, out_rows).astype(np.int32)
    d_t, d_i = torch.from_numpy(table).to(gpu), torch.from_numpy(idx).to(gpu)
    mine, theirs = torch.empty((out_rows, cols), device=gpu), torch.empty((out_rows, cols), device=gpu)
    torch.cuda.synchronize()
    case("reference gather_rows")
    ref.ref_hip_gather_rows(dptr(d_t), dptr(d_i), rows, cols, out_rows, dptr(theirs))
    case("hip_gather_rows")
    ops.lib().hip_gather_rows(dptr(d_t), dptr(d_i), rows, cols, out_rows, dptr(mine))
    torch.cuda.synchronize()
    H.assert_bitexact(mine.cpu().numpy(), theirs.cpu().numpy(), "gather vs reference kernel")
    H.assert_bitexact(mine.cpu().numpy(), table[idx], "gather vs indexing")


@pytest.mark.parametrize("w_format", [H.F16, H.BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("m", [5, 16, 200])
def test_split_products_keep_every_activation_bit(gpu, w_format, m):
    """One-hot weight columns holding powers of two: out[r, c] = x[r, perm(c)] * 2^e exactly.
    Full 24-bit activations therefore come back bit for bit only if the split into bf16
    pieces (decode product for m <= 16, tile kernel beyond) loses nothing."""
    r = H.rng(900 + m + w_format)
    n, k = 96, 256
    x = (r.uniform(0.5, 1.0, (m, k)) * (2.0 ** r.integers(-20, 20, (m, k)))).astype(np.float32)
    x *= np.where(r.random((m, k)) < 0.5, -1, 1).astype(np.float32)
    perm = r.integers(0, k, n)
    scale = 2.0 ** (np.arange(n) % 5 - 2)
    wf = np.zeros((n, k), np.float32)
    wf[np.arange(n), perm] = scale
    w = H.to_storage(wf, w_format)
    case(f"nvf_matmul split exactness fmt={w_format} m={m}")
    got = ops.matmul(H.to_dev(x, gpu), w_dev(w, w_format, gpu), n, w_format)
    want = (x[:, perm] * scale[None, :].astype(np.float32)).astype(np.float32)
    H.assert_bitexact(np.ascontiguousarray(H.to_host(got)), np.ascontiguousarray(want), "one-hot products")
