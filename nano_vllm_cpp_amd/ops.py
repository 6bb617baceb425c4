"""Python front end of libnvf_ops.so (the gfx950 fused per-layer ops).

`lib()` returns the ctypes handle with every C-ABI symbol of include/nvf_ops.h
typed.  The torch-facing wrappers below only validate shapes, pick the stream
(torch's current stream) and call the C ABI; all compute is in the HIP
library.  There is no fallback: a missing library raises immediately.

Names and argument meaning follow the reference op interface
(include/nanovllm/hip_ops.hpp:14-33 in Nano_vLLM_cpp).
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import numpy as np
import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libnvf_ops.so"

F32, F16, BF16 = 0, 1, 2
EMB_Q8_0, EMB_Q8_0_BLOCKS, EMB_Q4_K, EMB_Q5_K, EMB_Q6_K = 0, 1, 12, 13, 14
QK_LAYOUT_GGML, QK_LAYOUT_HIP_LEGACY = 0, 1
Q4_K, Q5_K, Q6_K = 12, 13, 14
W_F32, W_F16, W_BF16 = 0, 1, 2

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_vp, _i64, _i32, _f32, _f64 = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_double

# symbol -> (restype, argtypes); mirrors include/nvf_ops.h
SIGNATURES: dict[str, tuple] = {
    "hip_rms_norm": (None, [_vp, _vp, _vp, _i32, _i32, _f32]),
    "hip_rms_norm_add": (None, [_vp, _vp, _vp, _vp, _i32, _i32, _f32]),
    "hip_silu_and_mul": (None, [_vp, _vp, _i32, _i32]),
    "hip_rope_inplace": (None, [_vp, _vp, _i32, _i32, _i32, _i64, _vp]),
    "hip_add_bias_inplace": (None, [_vp, _vp, _i32, _i32]),
    "hip_embedding": (None, [_vp, _vp, _i32, _i32, _vp]),
    "hip_embedding_u16": (None, [_vp, _vp, _i32, _i32, _vp, C.c_bool]),
    "hip_embedding_q8": (None, [_vp, _vp, _vp, _i32, _i32, _vp]),
    "hip_embedding_qk": (None, [_vp, _vp, _i32, _i32, _vp, _i32]),
    "hip_gather_rows": (None, [_vp, _vp, _i32, _i32, _i32, _vp]),
    "hip_moe_route": (None, [_vp, _i32, _i32, _i32, C.c_bool, _vp, _vp]),
    "hip_moe_ffn": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, C.c_bool, _vp]),
    "hip_add_inplace": (None, [_vp, _vp, C.c_size_t]),
    "hip_scale_rows_sigmoid": (None, [_vp, _vp, _i32, _i32]),
    "nvf_moe_route": (_i32, [_vp, _i64, _i64, _i64, _i32, _vp, _vp, _vp]),
    "nvf_moe_ffn_workspace_size": (_i64, [_i64, _i64, _i64, _i64, _i64]),
    "nvf_moe_ffn_ws": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _i32, _vp,
                              _i64, _vp]),
    "nvf_add_inplace": (_i32, [_vp, _vp, _i64, _vp]),
    "nvf_scale_rows_sigmoid": (_i32, [_vp, _vp, _i64, _i64, _vp]),
    "hip_matmul": (None, [_vp, _vp, _i32, _i32, _i32, _vp]),
    "hip_matmul_u16": (None, [_vp, _vp, _i32, _i32, _i32, _vp, C.c_bool]),
    "hip_matmul_qk": (None, [_vp, _vp, _i32, _i32, _i32, _vp, _i32]),
    "nvf_matmul": (_i32, [_vp, _i32, _vp, _i32, _i32, _i64, _i64, _i64, _vp, _i32, _vp]),
    "nvf_gather_rows": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp]),
    "hip_matmul_q8": (None, [_vp, _vp, _vp, _i32, _i32, _i32, _vp]),
    "hip_store_kv": (None, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32]),
    "hip_paged_attention": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _f32]),
    "nvf_store_kv": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i64, _i64, _i32, _vp]),
    "nvf_paged_attention": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _i64,
                                   _i64, _i32, _vp]),
    "nvf_paged_attention_ws": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _f32,
                                      _i64, _i64, _vp, _i64, _i32, _vp]),
    "nvf_paged_attention_seqs_ws": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _i32, _i32, _i32,
                                           _i32, _i32, _f32, _i64, _i64, _vp, _i64, _i32, _vp]),
    "nvf_paged_attention_order_ws": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32,
                                            _i32, _f32, _i64, _i64, _vp, _i64, _i32, _vp]),
    "nvf_decode_token_order": (_i32, [_vp, _i64, _vp]),
    "nvf_paged_attention_noalloc": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32,
                                           _f32, _i64, _i64, _i32, _vp]),
    "nvf_paged_attention_noalloc_max_bytes": (_i64, []),
    "nvf_paged_attention_workspace_size": (_i64, [_i64, _i32, _i32, _i32, _i32, _i32, _i64]),
    "nvf_q8_quantize_rows": (_i32, [_vp, _vp, _vp, _i64, _i64, _i32, _vp]),
    "nvf_matmul_q8_0": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp]),
    "nvf_matmul_q8_0_ws": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp, _i64, _vp]),
    "nvf_matmul_q8_0_workspace_size": (_i64, [_i64, _i64, _i64]),
    "nvf_matmul_q8_0_act": (_i32, [_vp, _i64, _i32, _vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp]),
    "nvf_matmul_q8_0_rms": (_i32, [_vp, _i64, _vp, _vp, _vp, C.c_float, _vp, _vp, _i64, _i64, _i64, _vp, _i32,
                                   _vp]),
    "nvf_rms_norm_add": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32, _vp]),
    "nvf_rms_norm": (_i32, [_vp, _vp, _vp, _i64, _i64, _f32, _i32, _vp]),
    "nvf_rms_norm_q8": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32, _vp]),
    "nvf_silu_and_mul": (_i32, [_vp, _vp, _i64, _i64, _i32, _vp]),
    "nvf_silu_and_mul_q8": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp]),
    "nvf_qk_norm_rope": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64, _i64, _f32, _i32, _vp]),
    "nvf_qk_norm_rope_store_kv": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64, _i64, _i64,
                                         _f32, _vp, _vp, _vp, _i32, _vp]),
    "nvf_qkv_bias_qk_norm_rope_store_kv": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32,
                                                  _i64, _i64, _i64, _f32, _vp, _vp, _vp, _i32, _vp]),
    "nvf_add_bias": (_i32, [_vp, _vp, _i64, _i64, _i64, _i32, _vp]),
    "nvf_embedding_q8_0": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp]),
    "nvf_embedding_q8_0_blocks": (_i32, [_vp, _vp, _i64, _i64, _i64, _vp, _i32, _vp]),
    "nvf_embedding_qk": (_i32, [_vp, _vp, _i64, _i64, _i64, _i32, _i32, _vp, _i32, _vp]),
    "nvf_embedding": (_i32, [_vp, _vp, _i64, _i64, _i64, _i32, _vp, _i32, _vp]),
    "nvf_embedding_rms_norm": (_i32, [_vp, _i32, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _f32, _i32, _vp]),
    "nvf_rope_inv_freq": (_i32, [_f64, _i32, _vp]),
    "nvf_stream_copy": (_i32, [_vp, _vp, _i64, _vp]),
    "nvf_stream_expand": (_i32, [_vp, _vp, _i64, _vp]),
    "nvf_q8_0_split_blocks": (_i32, [_vp, _i64, _vp, _vp, _vp]),
    "nvf_set_dropin_q4k_layout": (_i32, [_i32]),
    "nvf_last_error": (C.c_char_p, []),
    "nvf_abi_version": (_i32, []),
}

_lock = threading.Lock()
_lib: C.CDLL | None = None


class NvfError(RuntimeError):
    """A nonzero status from the C ABI."""


def lib() -> C.CDLL:
    """Loads libnvf_ops.so once; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m nano_vllm_cpp_amd.build` "
                    "(there is no CPU fallback)")
            h = C.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(h, name)
                fn.restype = res
                fn.argtypes = args
            _lib = h
        return _lib


def _check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().nvf_last_error().decode(errors="replace")
        raise NvfError(f"{what} failed ({status}): {msg}")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, name: str) -> int:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def _dev_rows(t: torch.Tensor, name: str) -> int:
    """Device pointer of a tensor whose rows (dim 0) may be strided but whose
    remaining dimensions are contiguous within a row."""
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not t[0:1].reshape(-1).is_contiguous() or t.stride(-1) != 1 or \
            (t.dim() > 2 and t.stride(-2) != t.shape[-1]):
        raise ValueError(f"{name} must have contiguous rows")
    return t.data_ptr()


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


# ---------------------------------------------------------------------------
# norms
# ---------------------------------------------------------------------------
def rms_norm_add(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """residual <- x + residual (in place); returns RMSNorm(residual) * weight."""
    rows, hidden = x.shape
    if residual.shape != x.shape or weight.shape != (hidden,):
        raise ValueError("shape mismatch")
    if not (x.dtype == residual.dtype == weight.dtype):
        raise ValueError("x, residual and weight must share a dtype")
    out = torch.empty_like(x) if out is None else out
    _check(lib().nvf_rms_norm_add(_dev(x, "x"), _dev(residual, "residual"), _dev(weight, "weight"),
                                  _dev(out, "out"), rows, hidden, eps, _dt(x), _stream()), "rms_norm_add")
    return out


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    rows, hidden = x.shape
    if weight.shape != (hidden,) or weight.dtype != x.dtype:
        raise ValueError("weight must be [hidden] in x's dtype")
    out = torch.empty_like(x) if out is None else out
    _check(lib().nvf_rms_norm(_dev(x, "x"), _dev(weight, "weight"), _dev(out, "out"), rows, hidden, eps, _dt(x),
                              _stream()), "rms_norm")
    return out


def rms_norm_q8(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None,
                want_out: bool = True, want_q: bool = True):
    """(Residual-add +) RMSNorm that also emits the Q8_0 GEMM's per-row scale
    127/max|out| and, optionally, the int8 row.  Returns (out | None, row_scale, q | None)."""
    rows, hidden = x.shape
    out = torch.empty_like(x) if want_out else None
    scale = torch.empty(rows, dtype=torch.float32, device=x.device)
    q = torch.empty((rows, hidden), dtype=torch.int8, device=x.device) if want_q else None
    _check(lib().nvf_rms_norm_q8(_dev(x, "x"), _dev(residual, "residual") if residual is not None else None,
                                 _dev(weight, "weight"), _dev(out, "out") if out is not None else None,
                                 _dev(scale, "row_scale"), _dev(q, "q_out") if q is not None else None, rows, hidden,
                                 eps, _dt(x), _stream()), "rms_norm_q8")
    return out, scale, q


# ---------------------------------------------------------------------------
# Q8_0 GEMM
# ---------------------------------------------------------------------------
def q8_0_split_blocks(blocks: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Splits interleaved 34-byte GGUF Q8_0 blocks (uint8 [nblocks*34], on the
    device) into the planes the GEMM and the split-plane gather read: (w8 int8
    [nblocks*32], ws int16 holding the fp16 bits [nblocks]).  The device form of the
    reference's host-side upload_q8_split (src/model.cpp:396-405)."""
    nbytes = blocks.numel()
    if blocks.dtype != torch.uint8 or nbytes % 34:
        raise ValueError("q8_0_split_blocks: blocks must be uint8 with a multiple of 34 bytes")
    nblk = nbytes // 34
    w8 = torch.empty(nblk * 32, dtype=torch.int8, device=blocks.device)
    ws = torch.empty(nblk, dtype=torch.int16, device=blocks.device)
    _check(lib().nvf_q8_0_split_blocks(_dev(blocks, "blocks"), nblk, _dev(w8, "w8"), _dev(ws, "ws"), _stream()),
           "q8_0_split_blocks")
    return w8, ws


def q8_quantize_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row int8 quantization for the Q8_0 GEMM: (row_scale [rows] fp32, xq [rows, k] int8)."""
    rows, k = x.shape
    scale = torch.empty(rows, dtype=torch.float32, device=x.device)
    xq = torch.empty((rows, k), dtype=torch.int8, device=x.device)
    _check(lib().nvf_q8_quantize_rows(_dev(x, "x"), _dev(scale, "row_scale"), _dev(xq, "xq"), rows, k, _dt(x),
                                      _stream()), "q8_quantize_rows")
    return scale, xq


def matmul_q8_0(xq: torch.Tensor, row_scale: torch.Tensor, w8: torch.Tensor, ws: torch.Tensor, n: int,
                out_dtype: torch.dtype = torch.float32, out: torch.Tensor | None = None,
                split: bool = True) -> torch.Tensor:
    """out [m, n] = dequantized Q8_0 product of pre-quantized activations xq [m, k]
    (int8, with row_scale) and split-plane weights w8 [n*k] int8, ws [n*k/32] fp16 bits.
    split: give the library a workspace for split-K when the output is too small to
    fill the GPU; False runs unsplit."""
    m, k = xq.shape
    out = torch.empty((m, n), dtype=out_dtype, device=xq.device) if out is None else out
    wb = lib().nvf_matmul_q8_0_workspace_size(m, n, k) if split else 0
    work = torch.empty((wb + 15) // 16 * 4, dtype=torch.float32, device=xq.device) if wb > 0 else None
    _check(lib().nvf_matmul_q8_0_ws(_dev(xq, "xq"), _dev(row_scale, "row_scale"), _dev(w8, "w8"), _dev(ws, "ws"), m,
                                    n, k, _dev(out, "out"), _dt(out), work.data_ptr() if work is not None else None,
                                    wb, _stream()), "matmul_q8_0")
    return out


def matmul_q8_0_act(x: torch.Tensor, w8: torch.Tensor, ws: torch.Tensor, n: int, swiglu: bool = False,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode GEMV (x.shape[0] <= 16 rows) on fp activations quantized inside the kernel:
    x [m, k] (or [gate | up] rows [m, 2k] with swiglu) in fp32/fp16/bf16; out [m, n] in x's
    dtype, bit-identical to quantize-then-matmul_q8_0.  Rows may be strided."""
    m, width = x.shape
    k = width // 2 if swiglu else width
    out = torch.empty((m, n), dtype=x.dtype, device=x.device) if out is None else out
    if out.dtype != x.dtype or out.shape != (m, n):
        raise ValueError("out must be [m, n] in x's dtype")
    _check(lib().nvf_matmul_q8_0_act(_dev_rows(x, "x"), x.stride(0), 1 if swiglu else 0, _dev(w8, "w8"),
                                     _dev(ws, "ws"), m, n, k, _dev(out, "out"), _dt(x), _stream()), "matmul_q8_0_act")
    return out


def matmul_q8_0_rms(x: torch.Tensor, weight: torch.Tensor, eps: float, w8: torch.Tensor, ws: torch.Tensor, n: int,
                    residual: torch.Tensor | None = None, residual_out: torch.Tensor | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Decode GEMV (x.shape[0] <= 16 rows) with (residual-add +) RMSNorm and the quantizer
    in its prologue: out [m, n] is bit-identical to rms_norm_q8 then matmul_q8_0.  With a
    residual [m, k] the summed rows go to residual_out (a second [m, k] buffer; required
    with residual, and it must not overlap x or residual)."""
    m, k = x.shape
    if weight.dtype != x.dtype or weight.numel() != k:
        raise ValueError("weight must be [k] in x's dtype")
    if (residual is None) != (residual_out is None):
        raise ValueError("residual and residual_out go together")
    for name, t in (("residual", residual), ("residual_out", residual_out)):
        if t is not None and (t.dtype != x.dtype or t.shape != (m, k) or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous [m, k] tensor in x's dtype")
    out = torch.empty((m, n), dtype=x.dtype, device=x.device) if out is None else out
    if out.dtype != x.dtype or out.shape != (m, n):
        raise ValueError("out must be [m, n] in x's dtype")
    _check(lib().nvf_matmul_q8_0_rms(
        _dev_rows(x, "x"), x.stride(0), _dev(residual, "residual") if residual is not None else None,
        _dev(residual_out, "residual_out") if residual_out is not None else None, _dev(weight, "weight"), eps,
        _dev(w8, "w8"), _dev(ws, "ws"), m, n, k, _dev(out, "out"), _dt(x), _stream()), "matmul_q8_0_rms")
    return out


def matmul_q8(x: torch.Tensor, w8: torch.Tensor, ws: torch.Tensor, n: int,
              out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """The reference's hip_matmul_q8 on activations x [m, k] (fp32/fp16/bf16):
    quantize the rows, then the int8 GEMM.  Output in out_dtype (default x's)."""
    scale, xq = q8_quantize_rows(x)
    return matmul_q8_0(xq, scale, w8, ws, n, out_dtype or x.dtype)


# ---------------------------------------------------------------------------
# KV cache and paged attention
# ---------------------------------------------------------------------------
def store_kv(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
             slot_mapping: torch.Tensor) -> None:
    """k_cache[slot, ...] = key[t] (and values) for slot = slot_mapping[t] >= 0.
    key/value [tokens, kv_heads, head_dim] (row stride from the tensor), caches
    [rows, kv_heads, head_dim] contiguous."""
    tokens, kv_heads, head_dim = key.shape
    if value.shape != key.shape:
        raise ValueError("value must have key's shape [tokens, kv_heads, head_dim]")
    for name, x in (("value", value), ("k_cache", k_cache), ("v_cache", v_cache)):
        if x.dtype != key.dtype:
            raise ValueError(f"{name} must have key's dtype {key.dtype}")
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        if c.dim() != 3 or tuple(c.shape[1:]) != (kv_heads, head_dim):
            raise ValueError(f"{name} must be [rows, kv_heads, head_dim]")
    if slot_mapping.dtype != torch.int32 or slot_mapping.shape != (tokens,):
        raise ValueError("slot_mapping must be int32 [tokens]")
    _check(lib().nvf_store_kv(_dev_rows(key, "key"), _dev_rows(value, "value"), _dev(k_cache, "k_cache"),
                              _dev(v_cache, "v_cache"), _dev(slot_mapping, "slot_mapping"), tokens, kv_heads, head_dim,
                              key.stride(0), value.stride(0), _dt(key), _stream()), "store_kv")


def decode_token_order(key_len) -> np.ndarray:
    """Host-side schedule for a decode batch (nvf_decode_token_order): the tokens
    longest-first, dealt over the GPU's 8 XCDs in snake order.  key_len: the tokens' key
    counts on the host.  Returns int32 [tokens] to upload as paged_attention's token_order."""
    kl = np.ascontiguousarray(np.asarray(key_len, dtype=np.int32))
    order = np.empty(len(kl), dtype=np.int32)
    _check(lib().nvf_decode_token_order(kl.ctypes.data, len(kl), order.ctypes.data), "decode_token_order")
    return order


def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, query_seq: torch.Tensor,
                    query_key_len: torch.Tensor, block_tables: torch.Tensor, block_size: int, scale: float,
                    out: torch.Tensor | None = None, max_query_len: int = 0, split: bool = True,
                    cu_seqlens=None, noalloc: bool = False, token_order: torch.Tensor | None = None) -> torch.Tensor:
    """q [tokens, q_heads, head_dim] (row stride from the tensor); caches
    [rows, kv_heads, head_dim]; block_tables [seqs, max_blocks] int32.
    max_query_len = 1 promises a decode batch (one query per sequence).  split:
    give the library the workspace for split attention when the shape calls for
    it (little work over long contexts); False runs unsplit.  cu_seqlens: the
    batch's packing on the host ([seqs + 1] ints, 0 .. tokens), if the caller has it
    (nvf_paged_attention_seqs_ws: no launch for mixed tiles when every sequence
    starts at a multiple of 128 tokens).  noalloc: nvf_paged_attention_noalloc (the
    split's partials in the library's static device scratch, no workspace
    allocated).  token_order: a device int32 [tokens] permutation of the tokens over the
    decode kernel's workgroups (decode_token_order; nvf_paged_attention_order_ws), results
    unchanged.
    Returns out [tokens, q_heads, head_dim] in q's dtype."""
    tokens, q_heads, head_dim = q.shape
    kv_heads = k_cache.shape[1]
    max_blocks = block_tables.shape[1]
    out = torch.empty((tokens, q_heads, head_dim), dtype=q.dtype, device=q.device) if out is None else out
    if noalloc:
        if cu_seqlens is not None or not split or token_order is not None:
            raise ValueError("noalloc takes neither cu_seqlens, token_order nor split=False")
        _check(lib().nvf_paged_attention_noalloc(
            _dev_rows(q, "q"), _dev(out, "out"), _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"),
            _dev(query_seq, "query_seq"), _dev(query_key_len, "query_key_len"), _dev(block_tables, "block_tables"),
            tokens, q_heads, kv_heads, head_dim, block_size, max_blocks, scale, q.stride(0), max_query_len, _dt(q),
            _stream()), "paged_attention_noalloc")
        return out
    ws_bytes = lib().nvf_paged_attention_workspace_size(tokens, q_heads, kv_heads, head_dim, block_size,
                                                       max_blocks, max_query_len) if split else 0
    ws = torch.empty((ws_bytes + 15) // 16 * 4, dtype=torch.float32, device=q.device) if ws_bytes > 0 else None
    if token_order is not None:
        if cu_seqlens is not None:
            raise ValueError("token_order takes no cu_seqlens")
        if token_order.dtype != torch.int32 or token_order.shape != (tokens,):
            raise ValueError("token_order must be int32 [tokens]")
        _check(lib().nvf_paged_attention_order_ws(
            _dev_rows(q, "q"), _dev(out, "out"), _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"),
            _dev(query_seq, "query_seq"), _dev(query_key_len, "query_key_len"), _dev(block_tables, "block_tables"),
            _dev(token_order, "token_order"), tokens, q_heads, kv_heads, head_dim, block_size, max_blocks, scale,
            q.stride(0), max_query_len, ws.data_ptr() if ws is not None else None, ws_bytes, _dt(q), _stream()),
            "paged_attention")
        return out
    if cu_seqlens is not None:
        cu = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))
        _check(lib().nvf_paged_attention_seqs_ws(
            _dev_rows(q, "q"), _dev(out, "out"), _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"),
            _dev(query_seq, "query_seq"), _dev(query_key_len, "query_key_len"), _dev(block_tables, "block_tables"),
            cu.ctypes.data, len(cu) - 1, tokens, q_heads, kv_heads, head_dim, block_size, max_blocks, scale,
            q.stride(0), max_query_len, ws.data_ptr() if ws is not None else None, ws_bytes, _dt(q), _stream()),
            "paged_attention")
        return out
    _check(lib().nvf_paged_attention_ws(_dev_rows(q, "q"), _dev(out, "out"), _dev(k_cache, "k_cache"),
                                        _dev(v_cache, "v_cache"), _dev(query_seq, "query_seq"),
                                        _dev(query_key_len, "query_key_len"), _dev(block_tables, "block_tables"),
                                        tokens, q_heads, kv_heads, head_dim, block_size, max_blocks, scale,
                                        q.stride(0), max_query_len, ws.data_ptr() if ws is not None else None,
                                        ws_bytes, _dt(q), _stream()), "paged_attention")
    return out


# ---------------------------------------------------------------------------
# SwiGLU
# ---------------------------------------------------------------------------
def silu_and_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    rows, two_i = gate_up.shape
    if two_i % 2:
        raise ValueError("gate_up width must be even")
    inter = two_i // 2
    out = torch.empty((rows, inter), dtype=gate_up.dtype, device=gate_up.device) if out is None else out
    _check(lib().nvf_silu_and_mul(_dev(gate_up, "gate_up"), _dev(out, "out"), rows, inter, _dt(gate_up), _stream()),
           "silu_and_mul")
    return out


def silu_and_mul_q8(gate_up: torch.Tensor, want_out: bool = False):
    """SwiGLU that also emits the Q8_0 GEMM's row scale and int8 rows.
    Returns (out | None, row_scale, q)."""
    rows, two_i = gate_up.shape
    if two_i % 2:
        raise ValueError("gate_up width must be even")
    inter = two_i // 2
    out = torch.empty((rows, inter), dtype=gate_up.dtype, device=gate_up.device) if want_out else None
    scale = torch.empty(rows, dtype=torch.float32, device=gate_up.device)
    q = torch.empty((rows, inter), dtype=torch.int8, device=gate_up.device)
    _check(lib().nvf_silu_and_mul_q8(_dev(gate_up, "gate_up"), _dev(out, "out") if out is not None else None,
                                     _dev(scale, "row_scale"), _dev(q, "q_out"), rows, inter, _dt(gate_up),
                                     _stream()), "silu_and_mul_q8")
    return out, scale, q


# ---------------------------------------------------------------------------
# QK-norm + RoPE
# ---------------------------------------------------------------------------
def rope_inv_freq(theta: float, head_dim: int, device: str | torch.device = "cpu") -> torch.Tensor:
    """inv_freq[i] = float(1 / theta^(2i/head_dim)) computed in double (model.cpp:416-420)."""
    out = torch.empty(head_dim // 2, dtype=torch.float32)
    _check(lib().nvf_rope_inv_freq(theta, head_dim, out.data_ptr()), "rope_inv_freq")
    return out.to(device)


def qk_norm_rope(q: torch.Tensor, k: torch.Tensor | None, positions: torch.Tensor, q_w: torch.Tensor | None,
                 k_w: torch.Tensor | None, inv_freq: torch.Tensor, q_heads: int, kv_heads: int, head_dim: int,
                 eps: float = 1e-6) -> None:
    """In place on q [T, q_heads * head_dim] and k [T, kv_heads * head_dim] (row strides
    from the tensors, so views into a packed qkv row work).

    q_w / k_w None -> plain NeoX RoPE.  positions: int64 [T] on the GPU."""
    tokens = q.shape[0]
    if positions.dtype != torch.int64 or positions.shape != (tokens,):
        raise ValueError("positions must be int64 [tokens]")
    if inv_freq.dtype != torch.float32 or inv_freq.numel() != head_dim // 2:
        raise ValueError("inv_freq must be float32 [head_dim/2]")
    # rows may be strided (e.g. the q and k columns of a packed [q | k | v] row); the
    # heads within a row are contiguous
    _check(lib().nvf_qk_norm_rope(
        _dev_rows(q, "q"), _dev_rows(k, "k") if k is not None else None, _dev(positions, "positions"),
        _dev(q_w, "q_w") if q_w is not None else None, _dev(k_w, "k_w") if k_w is not None else None,
        _dev(inv_freq, "inv_freq"), tokens, q_heads, kv_heads, head_dim, q.stride(0),
        k.stride(0) if k is not None else 0, eps, _dt(q), _stream()), "qk_norm_rope")


def qk_norm_rope_store_kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
                          q_w: torch.Tensor | None, k_w: torch.Tensor | None, inv_freq: torch.Tensor, q_heads: int,
                          kv_heads: int, head_dim: int, k_cache: torch.Tensor, v_cache: torch.Tensor,
                          slot_mapping: torch.Tensor, eps: float = 1e-6, qkv_bias: torch.Tensor | None = None) -> None:
    """(qkv bias +) qk_norm_rope(q, k, ...) then store_kv(k, v, k_cache, v_cache, slot_mapping),
    in one launch where the shape allows.  q [T, q_heads * head_dim], k and v [T, kv_heads *
    head_dim] (row strides from the tensors); caches [rows, kv_heads, head_dim] contiguous;
    slot_mapping int32 [T].  qkv_bias: fp32 [(q_heads + 2 * kv_heads) * head_dim] (Qwen2.5),
    added to q, k and the stored v before the norm and rotation; v itself is left unchanged."""
    tokens = q.shape[0]
    if positions.dtype != torch.int64 or positions.shape != (tokens,):
        raise ValueError("positions must be int64 [tokens]")
    if inv_freq.dtype != torch.float32 or inv_freq.numel() != head_dim // 2:
        raise ValueError("inv_freq must be float32 [head_dim/2]")
    kn = kv_heads * head_dim
    if q.dim() != 2 or q.shape[1] != q_heads * head_dim:
        raise ValueError("q must be [tokens, q_heads * head_dim]")
    for name, x in (("k", k), ("v", v)):
        if x.dim() != 2 or x.shape != (tokens, kn):
            raise ValueError(f"{name} must be [tokens, kv_heads * head_dim] = [{tokens}, {kn}]")
    for name, x in (("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache)):
        if x.dtype != q.dtype:
            raise ValueError(f"{name} must have q's dtype {q.dtype}")
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        if c.dim() != 3 or tuple(c.shape[1:]) != (kv_heads, head_dim):
            raise ValueError(f"{name} must be [rows, kv_heads, head_dim]")
    if slot_mapping.dtype != torch.int32 or slot_mapping.shape != (tokens,):
        raise ValueError("slot_mapping must be int32 [tokens]")
    if qkv_bias is not None and (qkv_bias.dtype != torch.float32 or
                                 qkv_bias.numel() != (q_heads + 2 * kv_heads) * head_dim):
        raise ValueError("qkv_bias must be float32 [(q_heads + 2 * kv_heads) * head_dim]")
    _check(lib().nvf_qkv_bias_qk_norm_rope_store_kv(
        _dev_rows(q, "q"), _dev_rows(k, "k"), _dev_rows(v, "v"),
        _dev(qkv_bias, "qkv_bias") if qkv_bias is not None else None, _dev(positions, "positions"),
        _dev(q_w, "q_w") if q_w is not None else None, _dev(k_w, "k_w") if k_w is not None else None,
        _dev(inv_freq, "inv_freq"), tokens, q_heads, kv_heads, head_dim, q.stride(0), k.stride(0), v.stride(0), eps,
        _dev(k_cache, "k_cache"), _dev(v_cache, "v_cache"), _dev(slot_mapping, "slot_mapping"), _dt(q), _stream()),
        "qk_norm_rope_store_kv")


def add_bias(x: torch.Tensor, bias: torch.Tensor) -> None:
    """x[r, :] += bias in place (x [rows, cols] with a row stride; bias fp32 [cols])."""
    rows, cols = x.shape
    if bias.dtype != torch.float32 or bias.shape != (cols,):
        raise ValueError("bias must be float32 [cols]")
    _check(lib().nvf_add_bias(_dev_rows(x, "x"), _dev(bias, "bias"), rows, cols, x.stride(0), _dt(x), _stream()),
           "add_bias")


# ---------------------------------------------------------------------------
# embeddings
# ---------------------------------------------------------------------------
def _out(tokens: int, hidden: int, dtype: torch.dtype, device) -> torch.Tensor:
    return torch.empty((tokens, hidden), dtype=dtype, device=device)


def embedding_q8_0(ids: torch.Tensor, w8: torch.Tensor, ws: torch.Tensor, hidden: int, vocab: int = 0,
                   out_dtype: torch.dtype = torch.float16, out: torch.Tensor | None = None) -> torch.Tensor:
    """Q8_0 gather from split planes: w8 int8/uint8 [V*H], ws fp16-bits [V*H/32]."""
    tokens = ids.numel()
    out = _out(tokens, hidden, out_dtype, ids.device) if out is None else out
    _check(lib().nvf_embedding_q8_0(_dev(ids, "ids"), _dev(w8, "w8"), _dev(ws, "ws"), tokens, hidden, vocab,
                                    _dev(out, "out"), _dt(out), _stream()), "embedding_q8_0")
    return out


def embedding_q8_0_blocks(ids: torch.Tensor, blocks: torch.Tensor, hidden: int, vocab: int = 0,
                          out_dtype: torch.dtype = torch.float16, out: torch.Tensor | None = None) -> torch.Tensor:
    """Q8_0 gather from interleaved 34-byte GGUF blocks (uint8 [V*H/32*34])."""
    tokens = ids.numel()
    out = _out(tokens, hidden, out_dtype, ids.device) if out is None else out
    _check(lib().nvf_embedding_q8_0_blocks(_dev(ids, "ids"), _dev(blocks, "blocks"), tokens, hidden, vocab,
                                           _dev(out, "out"), _dt(out), _stream()), "embedding_q8_0_blocks")
    return out


def embedding_qk(ids: torch.Tensor, wq: torch.Tensor, hidden: int, kind: int = Q4_K, vocab: int = 0,
                 layout: int = QK_LAYOUT_GGML, out_dtype: torch.dtype = torch.float16,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    tokens = ids.numel()
    out = _out(tokens, hidden, out_dtype, ids.device) if out is None else out
    _check(lib().nvf_embedding_qk(_dev(ids, "ids"), _dev(wq, "wq"), tokens, hidden, vocab, kind, layout,
                                  _dev(out, "out"), _dt(out), _stream()), "embedding_qk")
    return out


def embedding_rms_norm(ids: torch.Tensor, fmt: int, table: torch.Tensor, scales: torch.Tensor | None, hidden: int,
                       weight: torch.Tensor, eps: float, vocab: int = 0):
    """Layer-0 embedding + residual-add (onto zeros) + RMSNorm; returns (residual, out) in weight's dtype."""
    tokens = ids.numel()
    residual = _out(tokens, hidden, weight.dtype, ids.device)
    out = torch.empty_like(residual)
    _check(lib().nvf_embedding_rms_norm(_dev(ids, "ids"), fmt, _dev(table, "table"),
                                        _dev(scales, "scales") if scales is not None else None, tokens, hidden, vocab,
                                        _dev(weight, "weight"), _dev(residual, "residual"), _dev(out, "out"), eps,
                                        _dt(weight), _stream()), "embedding_rms_norm")
    return residual, out


def embedding(ids: torch.Tensor, table: torch.Tensor, vocab: int = 0, out_dtype: torch.dtype | None = None,
              out: torch.Tensor | None = None) -> torch.Tensor:
    tokens, hidden = ids.numel(), table.shape[-1]
    out = _out(tokens, hidden, out_dtype or table.dtype, ids.device) if out is None else out
    _check(lib().nvf_embedding(_dev(ids, "ids"), _dev(table, "table"), tokens, hidden, vocab, _dt(table),
                               _dev(out, "out"), _dt(out), _stream()), "embedding")
    return out


def stream_copy(dst: torch.Tensor, src: torch.Tensor) -> None:
    """Bandwidth reference copy (16-byte non-temporal loads/stores)."""
    n = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != n:
        raise ValueError("size mismatch")
    _check(lib().nvf_stream_copy(_dev(dst, "dst"), _dev(src, "src"), n, _stream()), "stream_copy")


def stream_expand(dst: torch.Tensor, src: torch.Tensor) -> None:
    """dst (2x src's bytes) <- each 8 bytes of src written as 16 (the gather's 1:2 mix)."""
    if dst.numel() * dst.element_size() != 2 * src.numel() * src.element_size():
        raise ValueError("dst must hold twice src's bytes")
    _check(lib().nvf_stream_expand(_dev(dst, "dst"), _dev(src, "src"), src.numel() * src.element_size(), _stream()),
           "stream_expand")


def gather_rows(rows: torch.Tensor, indices: torch.Tensor, out: torch.Tensor | None = None,
                check: bool = True) -> torch.Tensor:
    """out[r] = rows[indices[r]] (rows [n, cols]; indices int32 [out_rows]).  check: an
    index outside [0, n) gives a NaN row (otherwise indices are trusted)."""
    n, cols = rows.shape
    if indices.dtype != torch.int32 or indices.dim() != 1:
        raise ValueError("indices must be int32 [out_rows]")
    out_rows = indices.numel()
    out = torch.empty((out_rows, cols), dtype=rows.dtype, device=rows.device) if out is None else out
    if out.shape != (out_rows, cols) or out.dtype != rows.dtype:
        raise ValueError("out must be [out_rows, cols] in rows' dtype")
    _check(lib().nvf_gather_rows(_dev(rows, "rows"), _dev(indices, "indices"), n if check else 0, cols, out_rows,
                                 _dev(out, "out"), _dt(rows), _stream()), "gather_rows")
    return out


def matmul(x: torch.Tensor, w: torch.Tensor, n: int, w_format: int, out_dtype=None, qk_layout: int = QK_LAYOUT_GGML,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """out [m, n] = x [m, k] . W^T, W [n, k] in `w_format` (W_F32/W_F16/W_BF16 as a tensor of that
    dtype, or Q4_K/Q5_K/Q6_K as a uint8 tensor of superblocks) decoded exactly to fp32."""
    m, k = x.shape
    out_dtype = out_dtype or x.dtype
    out = torch.empty((m, n), dtype=out_dtype, device=x.device) if out is None else out
    if out.shape != (m, n) or out.dtype != out_dtype:
        raise ValueError("out must be [m, n] in out_dtype")
    _check(lib().nvf_matmul(_dev(x, "x"), _dt(x), _dev(w, "w"), w_format, qk_layout, m, n, k, _dev(out, "out"),
                            _DT[out_dtype], _stream()), "matmul")
    return out


# ---------------------------------------------------------------------------
# mixture of experts
# ---------------------------------------------------------------------------
def moe_route(logits: torch.Tensor, k: int, norm: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k experts of each fp32 logits row [rows, E] (the reference's hip_moe_route):
    (idx int32 [rows, k], score fp32 [rows, k])."""
    if logits.dtype != torch.float32 or logits.dim() != 2:
        raise ValueError("logits must be float32 [rows, E]")
    rows, e = logits.shape
    idx = torch.empty((rows, k), dtype=torch.int32, device=logits.device)
    score = torch.empty((rows, k), dtype=torch.float32, device=logits.device)
    _check(lib().nvf_moe_route(_dev(logits, "logits"), rows, e, k, 1 if norm else 0, _dev(idx, "idx"),
                               _dev(score, "score"), _stream()), "moe_route")
    return idx, score


def moe_ffn(x: torch.Tensor, idx: torch.Tensor, score: torch.Tensor, gu: torch.Tensor, dn: torch.Tensor,
            slot_of: torch.Tensor, inter: int, slots: int, out: torch.Tensor) -> torch.Tensor:
    """out[t] += sum_k score[t,k] * down(silu(gate(x[t])) * up(x[t])) for expert slot
    slot_of[idx[t,k]] (the reference's hip_moe_ffn): x [rows, H] and out [rows, H] fp32 /
    fp16 / bf16, gu [slots, 2*inter, H] and dn [slots, H, inter] fp16 or bf16."""
    rows, hidden = x.shape
    k = idx.shape[1]
    if idx.dtype != torch.int32 or score.dtype != torch.float32 or idx.shape != (rows, k) or score.shape != (rows, k):
        raise ValueError("idx must be int32 and score float32, both [rows, K]")
    if gu.dtype != dn.dtype or gu.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("gu and dn must both be float16 or bfloat16")
    if gu.numel() < slots * 2 * inter * hidden or dn.numel() < slots * hidden * inter:
        raise ValueError("gu / dn hold fewer than `slots` experts")
    if slot_of.dtype != torch.int32 or out.shape != (rows, hidden):
        raise ValueError("slot_of must be int32 and out [rows, H]")
    wb = lib().nvf_moe_ffn_workspace_size(rows, hidden, inter, k, slots)
    work = torch.empty(max(wb, 16), dtype=torch.uint8, device=x.device)
    _check(lib().nvf_moe_ffn_ws(_dev(x, "x"), _dt(x), _dev(idx, "idx"), _dev(score, "score"), _dev(gu, "gu"),
                                _dev(dn, "dn"), 1 if gu.dtype == torch.bfloat16 else 0, _dev(slot_of, "slot_of"),
                                rows, hidden, inter, k, slots, _dev(out, "out"), _dt(out), work.data_ptr(), wb,
                                _stream()), "moe_ffn")
    return out
