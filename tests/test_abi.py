"""The C-ABI library: loads, exports every symbol include/nvf_ops.h declares, and
rejects bad arguments on the host (no GPU work is issued by these tests)."""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

from nano_vllm_cpp_amd import ops
from tests import harness as H

HEADER = Path(__file__).resolve().parents[1] / "include" / "nvf_ops.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*([a-z_0-9]+)\s*\(", text, flags=re.M)


def test_header_declares_expected_surface():
    names = set(declared_functions())
    dropins = {"hip_rms_norm", "hip_rms_norm_add", "hip_silu_and_mul", "hip_rope_inplace", "hip_embedding",
               "hip_embedding_u16", "hip_embedding_q8", "hip_embedding_qk"}
    assert dropins <= names
    assert {"nvf_rms_norm_add", "nvf_qk_norm_rope", "nvf_silu_and_mul", "nvf_embedding_q8_0",
            "nvf_embedding_q8_0_blocks", "nvf_embedding_qk"} <= names


def test_library_exports_every_declared_symbol():
    lib = ops.lib()
    names = declared_functions()
    assert names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in nvf_ops.h but not exported"
        assert n in ops.SIGNATURES, f"{n} has no ctypes signature in ops.py"
    assert set(ops.SIGNATURES) == set(names)
    assert lib.nvf_abi_version() == 1


def _status(rc: int) -> tuple[int, str]:
    return rc, ops.lib().nvf_last_error().decode()


def test_host_argument_checks():
    lib = ops.lib()
    p = 0x1000  # never dereferenced: every call below fails or returns before a launch
    rc, msg = _status(lib.nvf_rms_norm_add(p, p, p, p, 4, 64, 1e-6, 7, None))
    assert rc == -1 and "dtype" in msg
    rc, msg = _status(lib.nvf_rms_norm_add(p, p, p, p, -1, 64, 1e-6, 1, None))
    assert rc == -1 and "shape" in msg
    assert lib.nvf_rms_norm_add(p, p, p, p, 0, 64, 1e-6, 1, None) == 0       # empty: no launch
    rc, msg = _status(lib.nvf_rms_norm_add(None, p, p, p, 4, 64, 1e-6, 1, None))
    assert rc == -1 and "NULL" in msg
    rc, msg = _status(lib.nvf_silu_and_mul(p, p, 3, -2, 1, None))
    assert rc == -1
    assert lib.nvf_silu_and_mul(p, p, 0, 10, 1, None) == 0
    rc, msg = _status(lib.nvf_embedding_qk(p, p, 4, 256, 0, 11, 0, p, 1, None))
    assert rc == -1 and "kind" in msg
    rc, msg = _status(lib.nvf_embedding_qk(p, p, 4, 256, 0, 12, 5, p, 1, None))
    assert rc == -1 and "layout" in msg
    assert lib.nvf_matmul_q8_0_workspace_size(256, 3584, 3584) > 0      # 56 output tiles: split-K
    assert lib.nvf_matmul_q8_0_workspace_size(16384, 37888, 3584) == 0  # enough tiles
    assert lib.nvf_matmul_q8_0_workspace_size(8, 3584, 3584) == 0       # the GEMV's rows
    rc, msg = _status(lib.nvf_matmul_q8_0_ws(p, p, p, p, 256, 3584, 3584, p, 1, p + 8, 1 << 26, None))
    assert rc == -1 and "workspace" in msg
    assert lib.nvf_paged_attention_workspace_size(1, 28, 4, 128, 256, 16, 1) > 0     # one long-context decode: split
    assert lib.nvf_paged_attention_workspace_size(256, 28, 4, 128, 256, 16, 1) == 0  # enough (token, kv head) pairs
    assert lib.nvf_paged_attention_workspace_size(1, 28, 4, 64, 256, 16, 1) == 0     # not a matrix-core shape
    assert lib.nvf_paged_attention_workspace_size(1, 28, 3, 128, 256, 16, 1) == 0    # bad heads: 0, no error
    rc, msg = _status(lib.nvf_paged_attention_ws(p, p, p, p, p, p, p, 1, 28, 4, 128, 256, 16, 0.1, 3584, 1,
                                                 p + 4, 1 << 20, 1, None))
    assert rc == -1 and "workspace" in msg
    rc, msg = _status(lib.nvf_q8_0_split_blocks(p, 3, p, p + 2, None))
    assert rc == -1 and "aligned" in msg
    rc, msg = _status(lib.nvf_q8_0_split_blocks(p, -1, p, p, None))
    assert rc == -1
    assert lib.nvf_q8_0_split_blocks(None, 0, None, None, None) == 0      # empty: no launch
    rc, msg = _status(lib.nvf_embedding_q8_0_blocks(p, p, 4, 48, 0, p, 1, None))
    assert rc == -1 and "multiple of 32" in msg
    rc, msg = _status(lib.nvf_embedding_q8_0(p, p, None, 4, 64, 0, p, 1, None))
    assert rc == -1 and "scale" in msg
    assert lib.nvf_embedding_q8_0(p, p, p, 0, 64, 0, p, 1, None) == 0
    rc, msg = _status(lib.nvf_qk_norm_rope(p, p, p, p, None, p, 4, 2, 1, 128, 256, 128, 1e-6, 1, None))
    assert rc == -1 and "q_w and k_w" in msg
    rc, msg = _status(lib.nvf_qk_norm_rope(p, p, p, None, None, p, 4, 2, 1, 128, 200, 128, 1e-6, 1, None))
    assert rc == -1 and "stride" in msg
    assert lib.nvf_qk_norm_rope(p, p, p, None, None, p, 0, 2, 1, 128, 256, 128, 1e-6, 1, None) == 0
    rc, msg = _status(lib.nvf_stream_copy(p, p, 24, None))
    assert rc == -1 and "multiple of 16" in msg
    rc, msg = _status(lib.nvf_stream_copy(p + 8, p, 32, None))
    assert rc == -1 and "unaligned" in msg
    assert lib.nvf_stream_copy(p, p, 0, None) == 0
    # Q8_0 GEMM and its quantizer
    rc, msg = _status(lib.nvf_matmul_q8_0(p, p, p, p, 4, 8, 48, p, 0, None))
    assert rc == -1 and "multiple" in msg
    rc, msg = _status(lib.nvf_matmul_q8_0(p, p, p, p, 4, 8, 64, p, 9, None))
    assert rc == -1 and "dtype" in msg
    rc, msg = _status(lib.nvf_matmul_q8_0(p, None, p, p, 4, 8, 64, p, 0, None))
    assert rc == -1 and "null" in msg
    rc, msg = _status(lib.nvf_matmul_q8_0(p + 4, p, p, p, 4, 8, 64, p, 0, None))
    assert rc == -1 and "aligned" in msg
    rc, msg = _status(lib.nvf_matmul_q8_0(p, p, p, p + 1, 4, 8, 64, p, 0, None))
    assert rc == -1 and "aligned" in msg
    rc, msg = _status(lib.nvf_matmul_q8_0(p, p, p, p, -4, 8, 64, p, 0, None))
    assert rc == -1 and "negative" in msg
    assert lib.nvf_matmul_q8_0(p, p, p, p, 0, 8, 64, p, 0, None) == 0
    assert lib.nvf_matmul_q8_0(p, p, p, p, 4, 0, 64, p, 0, None) == 0
    rc, msg = _status(lib.nvf_q8_quantize_rows(p, None, p, 4, 64, 0, None))
    assert rc == -1 and "null" in msg
    rc, msg = _status(lib.nvf_q8_quantize_rows(p, p, p, 4, 64, 5, None))
    assert rc == -1 and "dtype" in msg
    assert lib.nvf_q8_quantize_rows(p, p, p, 0, 64, 0, None) == 0
    lib.hip_matmul_q8(p, p, p, 0, 8, 64, p)  # empty: returns before any HIP call
    rc, msg = _status(lib.nvf_silu_and_mul_q8(p, None, None, p, 4, 64, 1, None))
    assert rc == -1 and "NULL" in msg
    rc, msg = _status(lib.nvf_silu_and_mul_q8(p, None, p, p, 4, 64, 3, None))
    assert rc == -1 and "dtype" in msg
    assert lib.nvf_silu_and_mul_q8(p, None, p, p, 0, 64, 1, None) == 0
    # KV store and paged attention
    rc, msg = _status(lib.nvf_paged_attention(p, p, p, p, p, p, p, 4, 6, 4, 128, 64, 4, 0.1, 768, 0, 1, None))
    assert rc == -1 and "multiple" in msg
    rc, msg = _status(lib.nvf_paged_attention(p, p, p, p, p, p, p, 4, 8, 4, 512, 64, 4, 0.1, 4096, 0, 1, None))
    assert rc == -1 and "256" in msg
    rc, msg = _status(lib.nvf_paged_attention(p, p, p, p, p, p, p, 4, 8, 4, 128, 64, 4, 0.1, 100, 0, 1, None))
    assert rc == -1 and "q_stride" in msg
    rc, msg = _status(lib.nvf_paged_attention(p, None, p, p, p, p, p, 4, 8, 4, 128, 64, 4, 0.1, 1024, 0, 1, None))
    assert rc == -1 and "NULL" in msg
    assert lib.nvf_paged_attention(p, p, p, p, p, p, p, 0, 8, 4, 128, 64, 4, 0.1, 1024, 0, 1, None) == 0
    rc, msg = _status(lib.nvf_store_kv(p, p, p, p, p, 4, 4, 128, 100, 512, 1, None))
    assert rc == -1 and "stride" in msg
    assert lib.nvf_store_kv(p, p, p, p, p, 0, 4, 128, 512, 512, 1, None) == 0


def test_inv_freq_host_helper_matches_oracle():
    for theta, hd in ((1e6, 128), (1e6, 64), (10000.0, 256), (5e5, 80)):
        mine = ops.rope_inv_freq(theta, hd).numpy()
        ref = np.empty(hd // 2, np.float32)
        H.oracle().orc_inv_freq(theta, hd, H.ptr(ref))
        assert np.array_equal(mine, ref)
    with pytest.raises(ops.NvfError):
        ops.rope_inv_freq(1e6, 0)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(ops, "LIB_PATH", tmp_path / "nope.so")
    monkeypatch.setattr(ops, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        ops.lib()


@pytest.mark.parametrize("n", [0, 1, 5, 8, 13, 200, 256, 1000])
def test_decode_token_order(n):
    """nvf_decode_token_order (host only): a permutation of the tokens with every id
    below n, the 8 longest contexts first (one per XCD), and each XCD's (workgroup id
    mod 8) sum of key counts within one maximal context of every other's."""
    r = np.random.default_rng(n)
    kl = r.integers(0, 4097, n).astype(np.int32)
    if n == 0:
        assert ops.lib().nvf_decode_token_order(None, 0, None) == 0
        return
    order = ops.decode_token_order(kl)
    assert sorted(order.tolist()) == list(range(n))
    k = min(n, 8)
    assert sorted(kl[order[:k]].tolist(), reverse=True) == sorted(kl.tolist(), reverse=True)[:k]
    if n >= 16:
        full = n // 8 * 8
        sums = [int(kl[order[x:full:8]].sum()) for x in range(8)]
        assert max(sums) - min(sums) <= int(kl.max())
    with pytest.raises(RuntimeError):
        ops._check(ops.lib().nvf_decode_token_order(kl.ctypes.data, -1, order.ctypes.data), "decode_token_order")
