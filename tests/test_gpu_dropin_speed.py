"""The fp32 drop-in entry points against the reference's own kernels
(src/hip_ops.hip built for gfx950 into oracle/_ref), timed on the same inputs
in the same process at BASELINE config 2's shapes (Q4_K at config 4's), plus the decode
products of the other weight formats (bf16 LM head, Q4_K gate_up) and the MoE ops at
Qwen3-30B-A3B's expert shape.

Each pair is timed with HIP events, median of 20 launches after 3 warm-ups (3 for the
MoE FFN, whose reference kernel takes about 0.3 s a call),
inputs resident in HBM.  The test asserts only that the drop-in is faster (the
measured margins are 1.4x and up) and prints the table; run it with -s to see
it.  Skipped when oracle/_ref was not built."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_vllm_cpp_amd import ops
from tests import harness as H

pytestmark = pytest.mark.gpu

T, HID, INTER, VOCAB = 16384, 3584, 18944, 152064  # Qwen2.5-7B, config 2 (4 x 4096 tokens)


@pytest.fixture(scope="module")
def ref():
    r = H.ref_hip()
    if r is None:
        pytest.skip("oracle/_ref/libref_hip_ops.so not present")
    return r


def median_us(f, it: int = 20) -> float:
    for _ in range(3):
        f()
    torch.cuda.synchronize()
    ts = []
    for _ in range(it):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        f()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) * 1000.0)
    return float(np.median(ts))


def compare(name: str, nbytes: float, ours, theirs, it: int = 20) -> None:
    print(f"[case] drop-in speed: {name}", flush=True)
    to, tr = median_us(ours, it), median_us(theirs, it)
    print(f"| {name} | {to:.1f} | {nbytes / to / 1e3:.0f} | {tr:.1f} | {nbytes / tr / 1e3:.0f} | {tr / to:.1f}x |",
          flush=True)
    assert to < tr, f"{name}: drop-in {to:.1f} us, reference {tr:.1f} us"


def p(t: torch.Tensor) -> int:
    return t.data_ptr()


def test_dropins_faster_than_reference_kernels(gpu, ref):
    lib = ops.lib()
    print("\n| op (fp32, drop-in entry point) | this build us | GB/s | reference us | GB/s | speedup |")
    print("|---|---|---|---|---|---|")
    g = torch.Generator(device=gpu)
    g.manual_seed(7)

    x = torch.randn(T, HID, device=gpu, generator=g)
    res = torch.randn(T, HID, device=gpu, generator=g)
    w = torch.rand(HID, device=gpu, generator=g) + 0.5
    out = torch.empty_like(x)
    compare("residual-add + RMSNorm [16384, 3584]", 4.0 * T * HID * 4 + HID * 4,
            lambda: lib.hip_rms_norm_add(p(x), p(res), p(w), p(out), T, HID, 1e-6),
            lambda: ref.ref_hip_rms_norm_add(p(x), p(res), p(w), p(out), T, HID, 1e-6))
    del x, res, out

    gu = torch.randn(T, 2 * INTER, device=gpu, generator=g)
    so = torch.empty(T, INTER, device=gpu)
    compare("SiLU·up [16384, 18944]", 3.0 * T * INTER * 4,
            lambda: lib.hip_silu_and_mul(p(gu), p(so), T, INTER),
            lambda: ref.ref_hip_silu_and_mul(p(gu), p(so), T, INTER))
    del gu, so

    # q and k inside the packed qkv row (model.cpp:777-778: one call each, stride 4608)
    qkv = torch.randn(T, 4608, device=gpu, generator=g)
    pos = (torch.arange(T, device=gpu) % 4096).long()
    inv = torch.tensor([1.0 / (1e6 ** (2 * i / 128)) for i in range(64)], device=gpu, dtype=torch.float32)
    kptr = p(qkv) + 3584 * 4

    def rope(fn):
        def run():
            fn(p(qkv), p(pos), T, 28, 128, 4608, p(inv))
            fn(kptr, p(pos), T, 4, 128, 4608, p(inv))
        return run

    compare("NeoX RoPE q [16384, 28, 128] + k [16384, 4, 128], two calls", 2.0 * T * 32 * 128 * 4 + 8.0 * T,
            rope(lib.hip_rope_inplace), rope(ref.ref_hip_rope_inplace))
    del qkv

    ids = torch.randint(0, VOCAB, (T,), device=gpu, generator=g)
    w8 = torch.randint(-127, 128, (VOCAB * HID,), device=gpu, dtype=torch.int8, generator=g)
    ws = (torch.rand(VOCAB * HID // 32, device=gpu, generator=g) * 1e-2 + 1e-3).half()
    eo = torch.empty(T, HID, device=gpu)
    compare("Q8_0 embedding gather [16384 x 3584]", T * HID * (1 + 2 / 32) + 8.0 * T + T * HID * 4,
            lambda: lib.hip_embedding_q8(p(ids), p(w8), p(ws), T, HID, p(eo)),
            lambda: ref.ref_hip_embedding_q8(p(ids), p(w8), p(ws), T, HID, p(eo)))
    del w8, ws, eo

    t4 = 2 * T  # config 4: 8 x 4096 tokens, Q4_K table
    ids4 = torch.randint(0, VOCAB, (t4,), device=gpu, generator=g)
    wq = torch.randint(0, 256, (VOCAB * HID // 256 * 144,), device=gpu, dtype=torch.uint8, generator=g)
    wq.view(-1, 144)[:, 0:4] = torch.tensor([0x00, 0x1C, 0x00, 0x18], dtype=torch.uint8, device=gpu)  # d, dmin
    eo4 = torch.empty(t4, HID, device=gpu)
    compare("Q4_K embedding gather [32768 x 3584], config 4", t4 * HID * 144 / 256 + 8.0 * t4 + t4 * HID * 4,
            lambda: lib.hip_embedding_qk(p(ids4), p(wq), t4, HID, p(eo4), 12),
            lambda: ref.ref_hip_embedding_qk(p(ids4), p(wq), t4, HID, p(eo4), 12))
    del ids4, wq, eo4

    # the other weight formats at decode: the LM head in bf16, gate_up in Q4_K (m = 1, fp32 logits)
    xl = torch.randn(1, HID, device=gpu, generator=g)
    wl = (torch.randn(VOCAB, HID, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    ol = torch.empty(1, VOCAB, device=gpu)
    compare("bf16 LM head at decode, m = 1 [152064, 3584]", VOCAB * HID * 2 + HID * 4 + VOCAB * 4,
            lambda: lib.hip_matmul_u16(p(xl), p(wl), 1, VOCAB, HID, p(ol), True),
            lambda: ref.ref_hip_matmul_u16(p(xl), p(wl), 1, VOCAB, HID, p(ol), True))
    del wl, ol
    wg = torch.randint(0, 256, (2 * INTER * HID // 256, 144), device=gpu, dtype=torch.uint8, generator=g)
    wg[:, 0:4] = torch.tensor([0x1E, 0x1C, 0x1E, 0x1C], dtype=torch.uint8, device=gpu)  # d, dmin ~ 4e-3
    og = torch.empty(1, 2 * INTER, device=gpu)
    compare("Q4_K gate_up at decode, m = 1 [37888, 3584]", 2 * INTER * HID // 256 * 144 + HID * 4 + 2 * INTER * 4,
            lambda: lib.hip_matmul_qk(p(xl), p(wg), 1, 2 * INTER, HID, p(og), 12),
            lambda: ref.ref_hip_matmul_qk(p(xl), p(wg), 1, 2 * INTER, HID, p(og), 12))
    del wg, og

    # MoE at Qwen3-30B-A3B's expert shape: routing 256 rows; the FFN for one decode token
    mH, mI, mE, mK = 2048, 768, 128, 8
    lg = torch.randn(256, mE, device=gpu, generator=g)
    idx = torch.empty(256, mK, dtype=torch.int32, device=gpu)
    sc = torch.empty(256, mK, device=gpu)
    compare("MoE routing, 256 rows x 128 experts, top 8", 256 * mE * 4 + 256 * mK * 8,
            lambda: lib.hip_moe_route(p(lg), 256, mE, mK, True, p(idx), p(sc)),
            lambda: ref.ref_hip_moe_route(p(lg), 256, mE, mK, True, p(idx), p(sc)))
    mgu = (torch.randn(mE, 2 * mI, mH, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    mdn = (torch.randn(mE, mH, mI, device=gpu, generator=g) * 0.05).to(torch.bfloat16)
    slot_of = torch.arange(mE, dtype=torch.int32, device=gpu)
    mx = torch.randn(1, mH, device=gpu, generator=g)
    mo = torch.zeros(1, mH, device=gpu)
    compare("MoE expert FFN, 1 token, top 8 of 128 (bf16 experts)", mK * 3 * mH * mI * 2,
            lambda: lib.hip_moe_ffn(p(mx), p(idx), p(sc), p(mgu), p(mdn), p(slot_of), 1, mH, mI, mK, True, p(mo)),
            lambda: ref.ref_hip_moe_ffn(p(mx), p(idx), p(sc), p(mgu), p(mdn), p(slot_of), 1, mH, mI, mK, True, p(mo)),
            it=3)
