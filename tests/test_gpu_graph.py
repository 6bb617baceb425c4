"""A decode-step layer captured into a HIP graph (torch.cuda.CUDAGraph) and
replayed: every replay is bit-identical to the eager run of the same layer (the
kernels are deterministic and record no memset), with the program's own eager
work (restoring the residual) and synchronizations between the replays.

The layer is model.cpp:758-833's sequence on this library's ops: input RMSNorm
writing int8 rows, qkv GEMM (the decode GEMV at these row counts), RoPE on views
of the packed row, KV store, paged attention (split across key ranges at this
batch size), row quantizer + o GEMM, residual-add RMSNorm, gate_up, SwiGLU writing
int8 rows, down.  The fused form runs the input norm in the qkv GEMV's prologue (the
summed residual to a second buffer) and quantizes the o and down GEMVs' rows in
theirs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_vllm_cpp_amd import ops

pytestmark = pytest.mark.gpu

HID, QH, KVH, HD, INTER, BS = 512, 4, 1, 128, 1024, 64


def case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def _q8w(g, n, k, dev):
    return (torch.randint(-127, 128, (n * k,), generator=g, device=dev, dtype=torch.int8),
            torch.empty(n * k // 32, device=dev).uniform_(1e-3, 1e-2, generator=g).half().view(torch.int16))


def _build(dev, batch, ctx):
    g = torch.Generator(device=dev).manual_seed(11)
    qs, ks = QH * HD, KVH * HD
    nb = -(-ctx // BS)
    tab = torch.arange(batch * nb, dtype=torch.int32, device=dev).view(batch, nb)
    rows = batch * nb * BS
    pos = torch.full((batch,), ctx - 1, dtype=torch.int64, device=dev)
    slots = (tab[:, (ctx - 1) // BS].to(torch.int64) * BS + (ctx - 1) % BS).to(torch.int32)
    L = dict(h=torch.randn(batch, HID, generator=g, device=dev).half(),
             r=torch.randn(batch, HID, generator=g, device=dev).half(),
             r2=torch.empty(batch, HID, dtype=torch.float16, device=dev),
             w_in=(1 + 0.1 * torch.randn(HID, generator=g, device=dev)).half(),
             w_post=(1 + 0.1 * torch.randn(HID, generator=g, device=dev)).half(),
             qkv=_q8w(g, qs + 2 * ks, HID, dev), o=_q8w(g, HID, qs, dev), gu=_q8w(g, 2 * INTER, HID, dev),
             down=_q8w(g, HID, INTER, dev),
             kc=torch.randn(rows, KVH, HD, generator=g, device=dev).half(),
             vc=torch.randn(rows, KVH, HD, generator=g, device=dev).half(),
             pos=pos, qseq=torch.arange(batch, dtype=torch.int32, device=dev),
             qlen=torch.full((batch,), ctx, dtype=torch.int32, device=dev), tab=tab, slots=slots,
             inv=ops.rope_inv_freq(1e6, HD, dev), out=torch.empty(batch, HID, dtype=torch.float16, device=dev))
    return L


def _layer(L, noalloc=False, fused=False):
    qs, ks = QH * HD, KVH * HD
    n = L["h"].shape[0]
    if fused:
        qkv = ops.matmul_q8_0_rms(L["h"], L["w_in"], 1e-6, *L["qkv"], qs + 2 * ks, residual=L["r"],
                                  residual_out=L["r2"])
    else:
        _, sc, xq = ops.rms_norm_q8(L["h"], L["w_in"], 1e-6, residual=L["r"], want_out=False)
        qkv = ops.matmul_q8_0(xq, sc, *L["qkv"], qs + 2 * ks, torch.float16)
    ops.qk_norm_rope(qkv[:, :qs], qkv[:, qs:qs + ks], L["pos"], None, None, L["inv"], QH, KVH, HD)
    ops.store_kv(qkv[:, qs:qs + ks].view(n, KVH, HD), qkv[:, qs + ks:].view(n, KVH, HD), L["kc"], L["vc"],
                 L["slots"])
    att = ops.paged_attention(qkv[:, :qs].view(n, QH, HD), L["kc"], L["vc"], L["qseq"], L["qlen"], L["tab"], BS,
                              HD ** -0.5, max_query_len=1, noalloc=noalloc)
    if fused:
        o = ops.matmul_q8_0_act(att.view(n, qs), *L["o"], HID)
    else:
        sc2, xq2 = ops.q8_quantize_rows(att.view(n, qs))
        o = ops.matmul_q8_0(xq2, sc2, *L["o"], HID, torch.float16)
    _, sc3, xq3 = ops.rms_norm_q8(o, L["w_post"], 1e-6, residual=L["r2"] if fused else L["r"], want_out=False)
    gu = ops.matmul_q8_0(xq3, sc3, *L["gu"], 2 * INTER, torch.float16)
    if fused:
        ops.matmul_q8_0_act(gu, *L["down"], HID, swiglu=True, out=L["out"])
    else:
        _, sc4, xq4 = ops.silu_and_mul_q8(gu)
        ops.matmul_q8_0(xq4, sc4, *L["down"], HID, torch.float16, out=L["out"])


@pytest.mark.parametrize("fused", [False, True], ids=["plain", "fused"])
@pytest.mark.parametrize("noalloc", [False, True], ids=["ws", "noalloc"])
@pytest.mark.parametrize("batch,ctx", [(1, 4096), (3, 1500)])
def test_decode_layer_graph_replays_match_eager(gpu, batch, ctx, noalloc, fused):
    """noalloc: the attention through nvf_paged_attention_noalloc, its split partials
    in the library's static device scratch rather than a pool allocation made during
    the capture."""
    L = _build(gpu, batch, ctx)
    assert ops.lib().nvf_paged_attention_workspace_size(batch, QH, KVH, HD, BS, L["tab"].shape[1], 1) > 0
    r0 = L["r"].clone()
    case(f"decode layer eager batch={batch} ctx={ctx} noalloc={noalloc} fused={fused}")
    _layer(L, noalloc, fused)
    torch.cuda.synchronize()
    rk = "r2" if fused else "r"  # where the layer leaves the residual
    want_out, want_r, want_kc = L["out"].clone(), L[rk].clone(), L["kc"].clone()
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):  # warm the side stream the capture uses
        for _ in range(2):
            L["r"].copy_(r0)
            _layer(L, noalloc, fused)
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    case(f"decode layer capture batch={batch} ctx={ctx} noalloc={noalloc}")
    with torch.cuda.graph(graph):
        _layer(L, noalloc, fused)
    torch.cuda.synchronize()
    for rep in range(4):
        L["r"].copy_(r0)           # eager work between the replays
        L["out"].fill_(float("nan"))
        L["r2"].fill_(float("nan"))
        torch.cuda.synchronize()
        case(f"decode layer replay {rep} batch={batch} ctx={ctx}")
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(L["out"].view(torch.int16), want_out.view(torch.int16)), f"replay {rep}: output"
        assert torch.equal(L[rk].view(torch.int16), want_r.view(torch.int16)), f"replay {rep}: residual"
        assert torch.equal(L["kc"].view(torch.int16), want_kc.view(torch.int16)), f"replay {rep}: k cache"
        assert not torch.isnan(L["out"]).any()


@pytest.mark.parametrize("batch,ctx", [(1, 4096), (3, 1500)])
def test_decode_layer_fused_matches_plain(gpu, batch, ctx):
    """The fused decode layer (norm and quantizers inside the GEMVs) gives the plain
    layer's output, residual and KV cache bit for bit."""
    case(f"decode layer fused vs plain batch={batch} ctx={ctx}")
    A, B = _build(gpu, batch, ctx), _build(gpu, batch, ctx)
    _layer(A, fused=False)
    _layer(B, fused=True)
    torch.cuda.synchronize()
    assert torch.equal(A["out"].view(torch.int16), B["out"].view(torch.int16)), "output"
    assert torch.equal(A["r"].view(torch.int16), B["r2"].view(torch.int16)), "residual"
    assert torch.equal(A["kc"].view(torch.int16), B["kc"].view(torch.int16)), "k cache"
    assert torch.equal(A["vc"].view(torch.int16), B["vc"].view(torch.int16)), "v cache"
