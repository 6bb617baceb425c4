"""The drop-in entry points (reference names and fp32 signatures) against the
C oracle and, where oracle/_ref was built, against the reference's own
src/hip_ops.hip kernels compiled for gfx950 and run on the same inputs."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from nano_vllm_cpp_amd import ops
from tests import harness as H

pytestmark = pytest.mark.gpu


def case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def dptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def f32(gpu, a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(gpu)


@pytest.fixture(scope="module")
def ref():
    r = H.ref_hip()
    if r is None:
        pytest.skip("oracle/_ref/libref_hip_ops.so not present")
    return r


def bit_fraction(a: np.ndarray, b: np.ndarray) -> float:
    return float((a.view(np.uint32) == b.view(np.uint32)).mean())


def test_test_basic_closed_form(gpu):
    """test/test_basic.cpp:23-31 through the drop-in hip_rms_norm."""
    x, w, out = f32(gpu, [1, 2, 3, 4]), f32(gpu, [1, 1, 1, 1]), torch.zeros(4, device=gpu)
    case("hip_rms_norm [1,2,3,4]")
    ops.lib().hip_rms_norm(dptr(x), dptr(w), dptr(out), 1, 4, 1e-6)
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert o[0] > 0 and o[3] > o[0] and abs(o[0] - 1 / math.sqrt(7.5 + 1e-6)) < 1e-4


def test_dropin_rms_norm_add_and_rms_norm(gpu):
    r = H.rng(1)
    rows, hidden = 48, 3584
    x = r.normal(0, 1, (rows, hidden)).astype(np.float32)
    res = r.normal(0, 1, (rows, hidden)).astype(np.float32)
    w = r.normal(1, 0.1, hidden).astype(np.float32)
    ref_res, ref_out = res.copy(), np.empty_like(x)
    H.oracle().orc_rms_norm_add(H.ptr(x), H.ptr(ref_res), H.ptr(w), H.ptr(ref_out), rows, hidden, 1e-6, H.F32)
    dres, out = f32(gpu, res), torch.empty(rows, hidden, device=gpu)
    case("hip_rms_norm_add")
    dx, dw = f32(gpu, x), f32(gpu, w)  # named: a temporary's memory could be reused before the launch
    ops.lib().hip_rms_norm_add(dptr(dx), dptr(dres), dptr(dw), dptr(out), rows, hidden, 1e-6)
    torch.cuda.synchronize()
    H.assert_bitexact(dres.cpu().numpy(), ref_res, "residual")
    H.assert_close(out.cpu().numpy(), ref_out, H.F32, what="hip_rms_norm_add")
    # QK-norm use: rows = T*heads, hidden = head_dim, in place
    q = r.normal(0, 1, (64 * 28, 128)).astype(np.float32)
    qw = r.normal(1, 0.1, 128).astype(np.float32)
    refq = np.empty_like(q)
    H.oracle().orc_rms_norm(H.ptr(q), H.ptr(qw), H.ptr(refq), q.shape[0], 128, 1e-6, H.F32)
    dq = f32(gpu, q)
    case("hip_rms_norm in place, head_dim rows")
    dqw = f32(gpu, qw)
    ops.lib().hip_rms_norm(dptr(dq), dptr(dqw), dptr(dq), q.shape[0], 128, 1e-6)
    torch.cuda.synchronize()
    H.assert_close(dq.cpu().numpy(), refq, H.F32, what="hip_rms_norm")


def test_dropin_vs_reference_kernels_norms(gpu, ref):
    r = H.rng(2)
    rows, hidden = 40, 896
    x = r.normal(0, 1, (rows, hidden)).astype(np.float32)
    res = r.normal(0, 1, (rows, hidden)).astype(np.float32)
    w = r.normal(1, 0.1, hidden).astype(np.float32)
    mine_res, theirs_res = f32(gpu, res), f32(gpu, res)
    mine, theirs = torch.empty(rows, hidden, device=gpu), torch.empty(rows, hidden, device=gpu)
    dx, dw = f32(gpu, x), f32(gpu, w)
    torch.cuda.synchronize()
    case("reference rms_norm_add kernel")
    ref.ref_hip_rms_norm_add(dptr(dx), dptr(theirs_res), dptr(dw), dptr(theirs), rows, hidden, 1e-6)
    case("hip_rms_norm_add")
    ops.lib().hip_rms_norm_add(dptr(dx), dptr(mine_res), dptr(dw), dptr(mine), rows, hidden, 1e-6)
    torch.cuda.synchronize()
    H.assert_bitexact(mine_res.cpu().numpy(), theirs_res.cpu().numpy(), "residual vs reference kernel")
    H.assert_close(mine.cpu().numpy(), theirs.cpu().numpy(), H.F32, what="rms_norm_add vs reference kernel")


def test_dropin_vs_reference_kernels_silu(gpu, ref):
    r = H.rng(3)
    rows, inter = 64, 4864
    gu = r.normal(0, 2, (rows, 2 * inter)).astype(np.float32)
    dgu = f32(gpu, gu)
    mine, theirs = torch.empty(rows, inter, device=gpu), torch.empty(rows, inter, device=gpu)
    torch.cuda.synchronize()
    case("reference silu kernel")
    ref.ref_hip_silu_and_mul(dptr(dgu), dptr(theirs), rows, inter)
    case("hip_silu_and_mul")
    ops.lib().hip_silu_and_mul(dptr(dgu), dptr(mine), rows, inter)
    torch.cuda.synchronize()
    a, b = mine.cpu().numpy(), theirs.cpu().numpy()
    print(f"silu bit-identical fraction vs reference kernel: {bit_fraction(a, b):.6f}")
    H.assert_close(a, b, H.F32, what="silu vs reference kernel")
    oref = np.empty((rows, inter), np.float32)
    H.oracle().orc_silu_and_mul(H.ptr(gu), H.ptr(oref), rows, inter, H.F32)
    H.assert_close(a, oref, H.F32, what="silu vs oracle")


def test_dropin_vs_reference_kernels_rope(gpu, ref):
    r = H.rng(4)
    T, heads, hd = 64, 14, 64
    stride = heads * hd
    inv = ops.rope_inv_freq(1e6, hd)
    data = r.normal(0, 1, (T, stride)).astype(np.float32)
    pos = r.integers(0, 4096, T).astype(np.int64)
    mine, theirs = f32(gpu, data), f32(gpu, data)
    dpos, dinv = torch.from_numpy(pos).to(gpu), inv.to(gpu)
    torch.cuda.synchronize()
    case("reference rope kernel")
    ref.ref_hip_rope_inplace(dptr(theirs), dptr(dpos), T, heads, hd, stride, dptr(dinv))
    case("hip_rope_inplace")
    ops.lib().hip_rope_inplace(dptr(mine), dptr(dpos), T, heads, hd, stride, dptr(dinv))
    torch.cuda.synchronize()
    a, b = mine.cpu().numpy(), theirs.cpu().numpy()
    print(f"rope bit-identical fraction vs reference kernel: {bit_fraction(a, b):.6f}")
    H.assert_close(a, b, H.F32, floor=1e-6, what="rope vs reference kernel")
    oref = data.copy()
    H.oracle().orc_rope(H.ptr(oref), H.ptr(pos), T, heads, hd, stride, H.ptr(inv.numpy()), H.F32)
    H.assert_close(a, oref, H.F32, floor=1e-6, what="rope vs oracle")


def test_dropin_vs_reference_kernels_embeddings(gpu, ref):
    r = H.rng(5)
    V, hidden, T = 2000, 896, 64
    w8, ws = H.gen_q8_0(r, V, hidden)  # normal fp16 scales: the reference's device decode is exact there
    ids = r.integers(0, V, T).astype(np.int64)
    d_ids, d_w8, d_ws = torch.from_numpy(ids).to(gpu), H.to_dev(w8, gpu), H.to_dev(ws, gpu)
    mine, theirs = torch.empty(T, hidden, device=gpu), torch.empty(T, hidden, device=gpu)
    torch.cuda.synchronize()
    case("reference embedding_q8 kernel")
    ref.ref_hip_embedding_q8(dptr(d_ids), dptr(d_w8), dptr(d_ws), T, hidden, dptr(theirs))
    case("hip_embedding_q8")
    ops.lib().hip_embedding_q8(dptr(d_ids), dptr(d_w8), dptr(d_ws), T, hidden, dptr(mine))
    torch.cuda.synchronize()
    H.assert_bitexact(mine.cpu().numpy(), theirs.cpu().numpy(), "q8 vs reference kernel")

    hidden = 512
    for kind, bb, offs in ((12, 144, (0, 2)), (13, 176, (0, 2)), (14, 210, (208,))):
        blocks = H.gen_raw_blocks(r, V * hidden // 256, bb, offs)
        d_b = H.to_dev(blocks, gpu)
        mine, theirs = torch.empty(T, hidden, device=gpu), torch.empty(T, hidden, device=gpu)
        torch.cuda.synchronize()
        case(f"reference embedding_qk kernel kind={kind}")
        ref.ref_hip_embedding_qk(dptr(d_ids), dptr(d_b), T, hidden, dptr(theirs), kind)
        torch.cuda.synchronize()
        # the reference's device Q4_K decoder uses the HIP_LEGACY nibble order
        layout = H.HIP_LEGACY if kind == 12 else H.GGML
        case(f"nvf_embedding_qk kind={kind} layout={layout}")
        ops.embedding_qk(d_ids, d_b, hidden, kind, V, layout, out_dtype=torch.float32, out=mine)
        torch.cuda.synchronize()
        H.assert_bitexact(mine.cpu().numpy(), theirs.cpu().numpy(), f"kind {kind} vs reference kernel")
        # drop-in hip_embedding_qk decodes GGUF (GGML) order, as the reference's host code does
        oref = np.empty((T, hidden), np.float32)
        H.oracle().orc_embedding_qk(H.ptr(ids), H.ptr(blocks), T, hidden, kind, H.GGML, H.ptr(oref), H.F32)
        case(f"hip_embedding_qk kind={kind}")
        ops.lib().hip_embedding_qk(dptr(d_ids), dptr(d_b), T, hidden, dptr(mine), kind)
        torch.cuda.synchronize()
        H.assert_bitexact(mine.cpu().numpy(), oref, f"hip_embedding_qk kind {kind} vs oracle")
        if kind == 12:  # switched to the reference's nibble order, the drop-in matches its kernel too
            ops._check(ops.lib().nvf_set_dropin_q4k_layout(H.HIP_LEGACY), "set layout")
            try:
                case("hip_embedding_qk kind=12 in the reference's nibble order")
                ops.lib().hip_embedding_qk(dptr(d_ids), dptr(d_b), T, hidden, dptr(mine), kind)
                torch.cuda.synchronize()
            finally:
                ops._check(ops.lib().nvf_set_dropin_q4k_layout(H.GGML), "set layout")
            H.assert_bitexact(mine.cpu().numpy(), theirs.cpu().numpy(), "hip_embedding_qk legacy vs reference kernel")

    for bf16 in (0, 1):
        table = H.gen_act(r, (V, hidden), H.BF16 if bf16 else H.F16)
        d_t = H.to_dev(table, gpu)
        mine, theirs = torch.empty(T, hidden, device=gpu), torch.empty(T, hidden, device=gpu)
        torch.cuda.synchronize()
        case(f"reference embedding_u16 bf16={bf16}")
        ref.ref_hip_embedding_u16(dptr(d_ids), dptr(d_t), T, hidden, dptr(theirs), bf16)
        case(f"hip_embedding_u16 bf16={bf16}")
        ops.lib().hip_embedding_u16(dptr(d_ids), dptr(d_t), T, hidden, dptr(mine), bool(bf16))
        torch.cuda.synchronize()
        H.assert_bitexact(mine.cpu().numpy(), theirs.cpu().numpy(), "u16 table vs reference kernel")


def test_dropin_empty_sizes_do_nothing(gpu):
    lib = ops.lib()
    case("drop-in zero sizes")
    lib.hip_rms_norm_add(None, None, None, None, 0, 3584, 1e-6)
    lib.hip_silu_and_mul(None, None, 0, 10)
    lib.hip_rope_inplace(None, None, 0, 4, 128, 512, None)
    lib.hip_embedding_q8(None, None, None, 0, 896, None)
    lib.hip_embedding_qk(None, None, 0, 896, None, 12)
    torch.cuda.synchronize()
