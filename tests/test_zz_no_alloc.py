"""nvf_paged_attention_noalloc: the split attention with its workspace in the
library's static device scratch instead of a caller buffer.

Called through the C ABI and compared with nvf_paged_attention_ws (same kernels,
same split plan, a caller workspace) bit for bit -- and with the oracle, within
the attention tolerance of the other attention tests -- on two calls in a row,
the second smaller than the first, so it runs over the first call's leftovers in
the shared scratch.  A call whose split needs more scratch than the static size
is rejected without launching.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_vllm_cpp_amd import ops
from tests import harness as H

pytestmark = pytest.mark.gpu

BS = 256  # KV block size (the reference's)
# the attention tests' bar: |got - exact| <= REL * max|V| (+ one ulp of a 16-bit output)
REL = {H.F32: 1e-4, H.F16: 2.0 ** -10}


def case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def _dev(b: H.PagedBatch, gpu, dt):
    return (H.to_dev(b.q, gpu, dt), H.to_dev(b.k_cache, gpu, dt), H.to_dev(b.v_cache, gpu, dt),
            torch.from_numpy(b.query_seq).to(gpu), torch.from_numpy(b.query_key_len).to(gpu),
            torch.from_numpy(b.block_tables).to(gpu))


def _run(fn_name, d, b, qh, kvh, mql, dt, gpu, ws=None):
    q, kc, vc, qs, ql, tb = d
    out = torch.full_like(q, float("nan"))
    lib = ops.lib()
    args = [q.data_ptr(), out.data_ptr(), kc.data_ptr(), vc.data_ptr(), qs.data_ptr(), ql.data_ptr(), tb.data_ptr(),
            b.tokens, qh, kvh, 128, BS, b.max_blocks, 128 ** -0.5, qh * 128, mql]
    if fn_name == "ws":
        rc = lib.nvf_paged_attention_ws(*args, ws.data_ptr() if ws is not None else None,
                                        ws.numel() * 4 if ws is not None else 0, dt, ops._stream())
    else:
        rc = lib.nvf_paged_attention_noalloc(*args, dt, ops._stream())
    ops._check(rc, f"paged_attention_{fn_name}")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dt", [H.F16, H.F32], ids=["f16", "f32"])
def test_noalloc_matches_workspace_entry(gpu, dt):
    r = H.rng(4242 + dt)
    lib = ops.lib()
    assert lib.nvf_paged_attention_noalloc_max_bytes() == 32 << 20
    qh, kvh = 28, 4
    cases = [
        ("decode 8 x 8192", [8192] * 8, [1] * 8, 1),
        ("decode 2 x 3000 (smaller, after the larger)", [3000, 2100], [1, 1], 1),
        ("prefill chunk 256 after 4096", [4352], [256], 0),
        ("prefill chunk 130 after 2000 (smaller again)", [2130], [130], 0),
        ("decode 1 x 500 (no split: no scratch)", [500], [1], 1),
    ]
    for name, ctx, ql, mql in cases:
        b = H.make_paged(r, ctx, ql, qh, kvh, 128, BS, dt)
        need = lib.nvf_paged_attention_workspace_size(b.tokens, qh, kvh, 128, BS, b.max_blocks, mql)
        case(f"noalloc {name} dt={dt} need={need}")
        assert need <= lib.nvf_paged_attention_noalloc_max_bytes()
        d = _dev(b, gpu, dt)
        ws = torch.empty((need + 15) // 16 * 4, dtype=torch.float32, device=gpu) if need > 0 else None
        want = _run("ws", d, b, qh, kvh, mql, dt, gpu, ws)
        got = _run("noalloc", d, b, qh, kvh, mql, dt, gpu)
        H.assert_bitexact(H.to_host(got), H.to_host(want), f"{name}: noalloc vs ws")
        if mql == 1:  # decode: the oracle as well, with the attention tests' bar
            _, exact, vmax = H.oracle_attention(b, qh, kvh, 128, BS, 128 ** -0.5, dt)
            g = H.from_storage(H.to_host(got), dt)
            tol = REL[dt] * vmax[..., None] + 1e-7 + (H.ulp(exact, dt) if dt != H.F32 else 0.0)
            assert (np.abs(g - exact) <= tol).all(), f"{name}: outside the attention tolerance of the oracle"


def test_noalloc_rejects_a_split_beyond_the_scratch(gpu):
    """A 128-token chunk after a 64K-token prefix over 28 heads wants 37 splits of
    (128 x 28) partial rows: ~69 MB, past the 32 MiB scratch.  The call fails with
    NVF_ERR_INVALID and names the limit; nothing is launched, out stays untouched."""
    lib = ops.lib()
    qh, kvh, tokens, max_blocks = 28, 4, 128, 65536 // BS + 1
    need = lib.nvf_paged_attention_workspace_size(tokens, qh, kvh, 128, BS, max_blocks, 0)
    assert need > lib.nvf_paged_attention_noalloc_max_bytes()
    q = torch.zeros(tokens, qh, 128, dtype=torch.float16, device=gpu)
    out = torch.full_like(q, 3.0)
    kc = torch.zeros(8, kvh, 128, dtype=torch.float16, device=gpu)
    meta = torch.zeros(tokens, dtype=torch.int32, device=gpu)
    tab = torch.zeros(1, max_blocks, dtype=torch.int32, device=gpu)
    case("noalloc beyond the scratch")
    rc = lib.nvf_paged_attention_noalloc(q.data_ptr(), out.data_ptr(), kc.data_ptr(), kc.data_ptr(), meta.data_ptr(),
                                         meta.data_ptr(), tab.data_ptr(), tokens, qh, kvh, 128, BS, max_blocks,
                                         0.088, qh * 128, 0, ops.F16, None)
    assert rc == -1
    assert "static scratch" in lib.nvf_last_error().decode()
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
