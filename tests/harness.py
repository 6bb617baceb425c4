"""Shared test infrastructure: C-oracle bindings, seeded synthetic inputs for the
BASELINE configs, and the tolerance rules.

The oracle (oracle/_build/libnvf_oracle.so) and the reference builds
(oracle/_ref/*.so) are checkers only; this module is imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_LIB = ROOT / "oracle" / "_build" / "libnvf_oracle.so"
REF_HOST_LIB = ROOT / "oracle" / "_ref" / "libref_host.so"
REF_HIP_LIB = ROOT / "oracle" / "_ref" / "libref_hip_ops.so"

F32, F16, BF16 = 0, 1, 2
GGML, HIP_LEGACY = 0, 1

_vp, _i64, _i32, _f32, _f64 = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_double

_ORACLE_SIGS = {
    "orc_fp16_to_f32": (_f32, [C.c_uint16]),
    "orc_f32_to_fp16": (C.c_uint16, [_f32]),
    "orc_bf16_to_f32": (_f32, [C.c_uint16]),
    "orc_f32_to_bf16": (C.c_uint16, [_f32]),
    "orc_inv_freq": (None, [_f64, _i32, _vp]),
    "orc_dequant_q4k_block": (None, [_vp, _vp, _i32]),
    "orc_dequant_q5k_block": (None, [_vp, _vp]),
    "orc_dequant_q6k_block": (None, [_vp, _vp]),
    "orc_embedding_q8_split": (None, [_vp, _vp, _vp, _i64, _i64, _vp, _i32]),
    "orc_embedding_q8_blocks": (None, [_vp, _vp, _i64, _i64, _vp, _i32]),
    "orc_q8_0_split_blocks": (None, [_vp, _i64, _vp, _vp]),
    "orc_embedding_qk": (None, [_vp, _vp, _i64, _i64, _i32, _i32, _vp, _i32]),
    "orc_embedding_u16": (None, [_vp, _vp, _i64, _i64, _i32, _vp, _i32]),
    "orc_rms_norm": (None, [_vp, _vp, _vp, _i64, _i64, _f32, _i32]),
    "orc_rms_norm_add": (None, [_vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32]),
    "orc_silu_and_mul": (None, [_vp, _vp, _i64, _i64, _i32]),
    "orc_rope": (None, [_vp, _vp, _i64, _i32, _i32, _i64, _vp, _i32]),
    "orc_qk_norm_rope": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64, _i64, _f32, _i32]),
    "orc_q8_row_scale": (None, [_vp, _vp, _i64, _i64, _i32]),
    "orc_q8_quantize": (None, [_vp, _vp, _vp, _i64, _i64, _i32]),
    "orc_embedding_rms_norm": (None, [_vp, _i32, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _f32, _i32]),
    "orc_matmul_q8_i8": (None, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "orc_store_kv": (None, [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32]),
    "orc_add_bias": (None, [_vp, _vp, _i64, _i64, _i64, _i32]),
    "orc_qkv_bias_qk_norm_rope_store_kv": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32,
                                                  _i64, _i64, _i64, _f32, _vp, _vp, _vp, _i32]),
    "orc_paged_attention": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _f32,
                                   _i32, _vp, _vp]),
    "orc_matmul_q8": (None, [_vp, _i32, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "orc_matmul_w": (None, [_vp, _i32, _vp, _i32, _i32, _i64, _i64, _i64, _vp, _vp]),
    "orc_gather_rows": (None, [_vp, _vp, _i64, _i64, _vp, _i32]),
    "orc_moe_route": (None, [_vp, _i64, _i32, _i32, _i32, _vp, _vp]),
    "orc_moe_ffn": (None, [_vp, _i32, _vp, _vp, _vp, _vp, _i32, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
}

_cache: dict[str, C.CDLL] = {}


def _load(path: Path, sigs: dict | None = None) -> C.CDLL:
    key = str(path)
    if key not in _cache:
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (run __graft_entry__.build() or make -C oracle)")
        h = C.CDLL(key)
        for name, (res, args) in (sigs or {}).items():
            fn = getattr(h, name)
            fn.restype, fn.argtypes = res, args
        _cache[key] = h
    return _cache[key]


def oracle() -> C.CDLL:
    return _load(ORACLE_LIB, _ORACLE_SIGS)


def ref_host() -> C.CDLL | None:
    """The reference's own gguf.cpp dequant + common.hpp codecs, if built."""
    if not REF_HOST_LIB.exists():
        return None
    h = _load(REF_HOST_LIB)
    h.ref_dequant_block_f32.restype = _i32
    h.ref_dequant_block_f32.argtypes = [C.c_char_p, _vp, _vp]
    h.ref_fp16_to_float.restype = _f32
    h.ref_fp16_to_float.argtypes = [C.c_uint16]
    h.ref_float_to_fp16.restype = C.c_uint16
    h.ref_float_to_fp16.argtypes = [_f32]
    return h


def ref_hip() -> C.CDLL | None:
    """The reference's own src/hip_ops.hip compiled for gfx950, if built."""
    if not REF_HIP_LIB.exists():
        return None
    h = _load(REF_HIP_LIB)
    h.ref_hip_rms_norm.argtypes = [_vp, _vp, _vp, _i32, _i32, _f32]
    h.ref_hip_rms_norm_add.argtypes = [_vp, _vp, _vp, _vp, _i32, _i32, _f32]
    h.ref_hip_silu_and_mul.argtypes = [_vp, _vp, _i32, _i32]
    h.ref_hip_rope_inplace.argtypes = [_vp, _vp, _i32, _i32, _i32, _i64, _vp]
    h.ref_hip_embedding_q8.argtypes = [_vp, _vp, _vp, _i32, _i32, _vp]
    h.ref_hip_embedding_qk.argtypes = [_vp, _vp, _i32, _i32, _vp, _i32]
    h.ref_hip_embedding_u16.argtypes = [_vp, _vp, _i32, _i32, _vp, _i32]
    h.ref_hip_matmul_q8.argtypes = [_vp, _vp, _vp, _i32, _i32, _i32, _vp]
    h.ref_hip_store_kv.argtypes = [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32]
    h.ref_hip_add_bias_inplace.argtypes = [_vp, _vp, _i32, _i32]
    h.ref_hip_paged_attention.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _f32]
    h.ref_hip_matmul.argtypes = [_vp, _vp, _i32, _i32, _i32, _vp]
    h.ref_hip_matmul_u16.argtypes = [_vp, _vp, _i32, _i32, _i32, _vp, C.c_bool]
    h.ref_hip_matmul_qk.argtypes = [_vp, _vp, _i32, _i32, _i32, _vp, _i32]
    h.ref_hip_matmul_any_async.argtypes = [_i32, _vp, _vp, _i32, _i32, _i32, _vp]
    h.ref_hip_gather_rows.argtypes = [_vp, _vp, _i32, _i32, _i32, _vp]
    h.ref_hip_moe_route.argtypes = [_vp, _i32, _i32, _i32, C.c_bool, _vp, _vp]
    h.ref_hip_moe_ffn.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, C.c_bool, _vp]
    h.ref_hip_add_inplace.argtypes = [_vp, _vp, C.c_size_t]
    h.ref_hip_scale_rows_sigmoid.argtypes = [_vp, _vp, _i32, _i32]
    return h


def ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------------------------------------------------------------------
# storage helpers (numpy has no bf16: 16-bit storage is kept as uint16 bits)
# ---------------------------------------------------------------------------
NP_STORAGE = {F32: np.float32, F16: np.uint16, BF16: np.uint16}


def to_storage(x: np.ndarray, dt: int) -> np.ndarray:
    """fp32/float64 values -> storage array of dtype `dt` (RNE)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dt == F32:
        return x.copy()
    if dt == F16:
        return x.astype(np.float16).view(np.uint16)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = ((x.view(np.uint32)[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def from_storage(a: np.ndarray, dt: int) -> np.ndarray:
    """storage array -> float64 values."""
    if dt == F32:
        return a.astype(np.float64)
    if dt == F16:
        return a.view(np.float16).astype(np.float64)
    return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def ulp(ref: np.ndarray, dt: int) -> np.ndarray:
    """Spacing of the storage format at |ref| (float64)."""
    a = np.abs(ref).astype(np.float64)
    if dt == F32:
        return np.spacing(a.astype(np.float32)).astype(np.float64)
    if dt == F16:
        return np.spacing(a.astype(np.float16)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (np.maximum(e, -126) - 7)


def assert_close(got: np.ndarray, ref: np.ndarray, dt: int, *, rel: float = 1e-5, floor: float = 0.0,
                 what: str = "") -> None:
    """|got - ref| <= max(rel*|ref|, 1 ulp_dtype(ref), floor), elementwise.

    `floor` is the absolute allowance for values produced by cancellation
    (1e-6 x the input rms in the tests that need one)."""
    g = from_storage(np.asarray(got), dt)
    r = from_storage(np.asarray(ref), dt)
    both_nan = np.isnan(g) & np.isnan(r)
    with np.errstate(invalid="ignore", over="ignore"):
        tol = np.maximum(np.maximum(rel * np.abs(r), ulp(r, dt)), floor)
        bad = ~both_nan & (g != r) & ~(np.abs(g - r) <= tol)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        rows = ", ".join(f"{tuple(i)}: got {g[tuple(i)]!r} ref {r[tuple(i)]!r}" for i in idx)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside tolerance; {rows}")


def assert_bitexact(got: np.ndarray, ref: np.ndarray, what: str = "") -> None:
    g, r = np.asarray(got), np.asarray(ref)
    assert g.shape == r.shape and g.dtype == r.dtype, (g.shape, r.shape, g.dtype, r.dtype)
    gb = g.view(np.uint8).reshape(g.shape + (-1,))
    rb = r.view(np.uint8).reshape(r.shape + (-1,))
    bad = (gb != rb).any(axis=-1)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        rows = ", ".join(f"{tuple(i)}: got {g[tuple(i)]!r} ref {r[tuple(i)]!r}" for i in idx)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} elements differ; {rows}")


# ---------------------------------------------------------------------------
# the BASELINE configs
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class Config:
    name: str
    tokens: int
    vocab: int
    hidden: int
    inter: int
    q_heads: int
    kv_heads: int
    head_dim: int
    dtype: int
    seqs: int = 1
    random_positions: bool = False
    qk_norm: bool = False
    emb: str = "q8_0"
    theta: float = 1e6
    eps: float = 1e-6
    seed: int = 0
    extra: dict = field(default_factory=dict)

    def positions(self) -> np.ndarray:
        if self.random_positions:
            return np.random.default_rng(self.seed + 7).integers(0, 4096, self.tokens, dtype=np.int64)
        per = self.tokens // self.seqs
        return np.tile(np.arange(per, dtype=np.int64), self.seqs)

    def cu_seqlens(self) -> np.ndarray:
        if self.random_positions:  # decode: one token per sequence
            return np.arange(self.tokens + 1, dtype=np.int32)
        return np.arange(0, self.tokens + 1, self.tokens // self.seqs, dtype=np.int32)


CONFIGS = {
    0: Config("qwen2.5-0.5b chain, 64 tokens", 64, 151936, 896, 4864, 14, 2, 64, F16, seed=100),
    1: Config("qwen2.5-7b decode, 256 seqs x 1 token", 256, 152064, 3584, 18944, 28, 4, 128, F16,
              seqs=256, random_positions=True, seed=101),
    2: Config("qwen2.5-7b chunked prefill, 4 x 4096 tokens", 16384, 152064, 3584, 18944, 28, 4, 128, F16,
              seqs=4, seed=102),
    3: Config("qwen3-8b prefill, 8192 tokens, QK-norm", 8192, 151936, 4096, 12288, 32, 8, 128, BF16,
              qk_norm=True, seed=103),
    4: Config("qwen2.5-7b Q4_K stress, 8 x 4096 tokens", 32768, 152064, 3584, 18944, 28, 4, 128, BF16,
              seqs=8, emb="q4_k", seed=104),
}


def scaled(cfg: Config, tokens: int, vocab: int | None = None) -> Config:
    """The same config at fewer tokens (and optionally a smaller vocab) for oracle-speed tests."""
    seqs = max(1, min(cfg.seqs, tokens))
    return Config(**{**cfg.__dict__, "tokens": tokens, "vocab": vocab or cfg.vocab, "seqs": seqs,
                     "name": cfg.name + f" @ {tokens} tokens"})


# ---------------------------------------------------------------------------
# numpy generators (seeded; used by the oracle-speed parity tests)
# ---------------------------------------------------------------------------
def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def gen_q8_0(r: np.random.Generator, vocab: int, hidden: int) -> tuple[np.ndarray, np.ndarray]:
    """Split planes: int8 plane [V*H] (U{-127..127}) and fp16 scale bits [V*H/32] (U[1e-3, 1e-2])."""
    n = vocab * hidden
    w8 = r.integers(-127, 128, n, dtype=np.int8)
    ws = r.uniform(1e-3, 1e-2, n // 32).astype(np.float16).view(np.uint16)
    return w8, ws


def q8_split_to_blocks(w8: np.ndarray, ws: np.ndarray) -> np.ndarray:
    """Interleave split planes into 34-byte GGUF blocks (inverse of model.cpp:394-404)."""
    nb = ws.size
    blk = np.empty((nb, 34), dtype=np.uint8)
    blk[:, :2] = ws.view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = w8.view(np.uint8).reshape(nb, 32)
    return blk.reshape(-1)


def gen_q4_k(r: np.random.Generator, nblocks: int) -> np.ndarray:
    """Q4_K superblocks: d, dmin U[1e-3,1e-2] fp16; 6-bit scales/mins U{0..63}; nibbles U{0..15}."""
    blk = np.empty((nblocks, 144), dtype=np.uint8)
    blk[:, 0:2] = r.uniform(1e-3, 1e-2, nblocks).astype(np.float16).view(np.uint8).reshape(nblocks, 2)
    blk[:, 2:4] = r.uniform(1e-3, 1e-2, nblocks).astype(np.float16).view(np.uint8).reshape(nblocks, 2)
    blk[:, 4:16] = pack_q4k_scales(r.integers(0, 64, (nblocks, 8)), r.integers(0, 64, (nblocks, 8)))
    blk[:, 16:] = r.integers(0, 256, (nblocks, 128), dtype=np.uint8)
    return blk.reshape(-1)


def pack_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Packs 8 six-bit scales and mins per block into the 12-byte table (ggml get_scale_min_k4 inverse)."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.zeros(sc.shape[:-1] + (12,), dtype=np.uint8)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (mn[..., 0:4] & 63) | ((mn[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 0xF) | ((mn[..., 4:8] & 0xF) << 4)
    return out


def gen_raw_blocks(r: np.random.Generator, nblocks: int, block_bytes: int, fp16_offsets: tuple[int, ...]) -> np.ndarray:
    """Random K-quant blocks whose fp16 fields hold U[1e-3, 1e-2]."""
    blk = r.integers(0, 256, (nblocks, block_bytes), dtype=np.uint8)
    for off in fp16_offsets:
        blk[:, off:off + 2] = r.uniform(1e-3, 1e-2, nblocks).astype(np.float16).view(np.uint8).reshape(nblocks, 2)
    return blk.reshape(-1)


KQ_BLOCK = {12: (144, (0, 2)), 13: (176, (0, 2)), 14: (210, (208,))}  # bytes, fp16 field offsets


def gen_weights(r: np.random.Generator, n: int, k: int, w_format: int) -> np.ndarray:
    """A weight matrix [n, k] in nvf_matmul's format: fp32 N(0, 0.05), fp16/bf16 bits of the
    same, or K-quant superblocks (fp16 fields U[1e-3, 1e-2], other bytes uniform)."""
    if w_format in (F32, F16, BF16):
        return to_storage(r.normal(0.0, 0.05, (n, k)).astype(np.float32), w_format)
    bb, offs = KQ_BLOCK[w_format]
    return gen_q4_k(r, n * k // 256) if w_format == 12 else gen_raw_blocks(r, n * k // 256, bb, offs)


def gen_act(r: np.random.Generator, shape, dt: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    return to_storage(r.normal(mean, std, shape).astype(np.float32), dt)


# ---------------------------------------------------------------------------
# numpy <-> torch (device memory is torch's; compute is the HIP library's)
# ---------------------------------------------------------------------------
def torch_dtype(dt: int):
    import torch

    return {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}[dt]


def to_dev(a: np.ndarray, device, dt: int | None = None):
    """numpy -> GPU tensor; uint16 arrays become fp16/bf16 tensors of dtype `dt`."""
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).to(device)
        return t.view(torch_dtype(dt)) if dt in (F16, BF16) else t
    return torch.from_numpy(a).to(device)


def to_host(t) -> np.ndarray:
    """GPU tensor -> numpy; 16-bit floats come back as uint16 bit patterns."""
    import torch

    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16, torch.int16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


# ---------------------------------------------------------------------------
# the smoke chain (config 0 on the GPU vs the oracle)
# ---------------------------------------------------------------------------
def smoke_chain(device: str = "cuda:0") -> None:
    """Config-0 layer-op chain through the C ABI on `device`, each op checked against the oracle."""
    import torch

    from nano_vllm_cpp_amd import ops

    cfg = CONFIGS[0]
    o = oracle()
    r = rng(cfg.seed)
    T, H, I, V, dt = cfg.tokens, cfg.hidden, cfg.inter, 4096, cfg.dtype
    tdt = torch_dtype(dt)

    def dev(a):
        return to_dev(a, device, dt)

    host = to_host

    ids = r.integers(0, V, T, dtype=np.int64)
    w8, ws = gen_q8_0(r, V, H)
    emb = ops.embedding_q8_0(dev(ids), dev(w8), to_dev(ws, device), H, V, out_dtype=tdt)
    ref = np.empty((T, H), np.uint16)
    o.orc_embedding_q8_split(ptr(ids), ptr(w8), ptr(ws), T, H, ptr(ref), dt)
    assert_bitexact(host(emb), ref, "smoke embedding_q8_0")

    x, res, g = gen_act(r, (T, H), dt), gen_act(r, (T, H), dt), gen_act(r, (H,), dt, 1.0, 0.1)
    dres = dev(res)
    out = ops.rms_norm_add(dev(x), dres, dev(g), cfg.eps)
    ref_res, ref_out = res.copy(), np.empty_like(x)
    o.orc_rms_norm_add(ptr(x), ptr(ref_res), ptr(g), ptr(ref_out), T, H, cfg.eps, dt)
    assert_bitexact(host(dres), ref_res, "smoke residual")
    assert_close(host(out), ref_out, dt, what="smoke rms_norm_add")

    qs, ks = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    q, k = gen_act(r, (T, qs), dt), gen_act(r, (T, ks), dt)
    pos = cfg.positions()
    inv = np.empty(cfg.head_dim // 2, np.float32)
    o.orc_inv_freq(cfg.theta, cfg.head_dim, ptr(inv))
    dq, dk = dev(q), dev(k)
    ops.qk_norm_rope(dq, dk, dev(pos), None, None, dev(inv), cfg.q_heads, cfg.kv_heads, cfg.head_dim)
    o.orc_qk_norm_rope(ptr(q), ptr(k), ptr(pos), None, None, ptr(inv), T, cfg.q_heads, cfg.kv_heads,
                       cfg.head_dim, qs, ks, cfg.eps, dt)
    assert_close(host(dq), q, dt, floor=1e-6, what="smoke rope q")
    assert_close(host(dk), k, dt, floor=1e-6, what="smoke rope k")

    gu = gen_act(r, (T, 2 * I), dt)
    out = ops.silu_and_mul(dev(gu))
    ref = np.empty((T, I), NP_STORAGE[dt])
    o.orc_silu_and_mul(ptr(gu), ptr(ref), T, I, dt)
    assert_close(host(out), ref, dt, what="smoke silu_and_mul")
    torch.cuda.synchronize(device)



# ---------------------------------------------------------------------------
# paged KV batches (src/model_runner.cpp:43-128 semantics)
# ---------------------------------------------------------------------------
@dataclass
class PagedBatch:
    """A batch of sequences over a paged KV cache: per-token (query_seq,
    query_key_len), block tables of randomly permuted physical blocks, and caches
    [num_blocks * block_size, kv_heads, head_dim] filled with N(0, 1) values
    (the rows the queries attend hold the sequences' keys/values)."""
    q: np.ndarray
    k_cache: np.ndarray
    v_cache: np.ndarray
    query_seq: np.ndarray
    query_key_len: np.ndarray
    block_tables: np.ndarray
    tokens: int
    max_blocks: int
    num_blocks: int


def make_paged(r: np.random.Generator, ctx_lens: list[int], q_lens: list[int], q_heads: int, kv_heads: int,
               head_dim: int, block_size: int, dt: int, spare_blocks: int = 3) -> PagedBatch:
    """Sequence s has ctx_lens[s] keys in the cache and q_lens[s] query tokens at
    its last positions (prefill: q_len = ctx_len; decode: q_len = 1), each
    query's key_len = its position + 1, as prepare_prefill/prepare_decode build them."""
    need = [-(-c // block_size) for c in ctx_lens]
    max_blocks = max(max(need), 1)
    num_blocks = sum(need) + spare_blocks
    perm = r.permutation(num_blocks).astype(np.int32)
    tables = np.full((len(ctx_lens), max_blocks), -1, np.int32)
    o = 0
    for s_, nb in enumerate(need):
        tables[s_, :nb] = perm[o:o + nb]
        o += nb
    qs, ql = [], []
    for s_, (c, n) in enumerate(zip(ctx_lens, q_lens)):
        for i in range(n):
            qs.append(s_)
            ql.append(c - n + i + 1)
    tokens = len(qs)
    rows = num_blocks * block_size
    k_cache = gen_act(r, (rows, kv_heads, head_dim), dt)
    v_cache = gen_act(r, (rows, kv_heads, head_dim), dt)
    q = gen_act(r, (tokens, q_heads, head_dim), dt)
    return PagedBatch(q, k_cache, v_cache, np.array(qs, np.int32), np.array(ql, np.int32), tables, tokens,
                      max_blocks, num_blocks)


def oracle_attention(b: PagedBatch, q_heads: int, kv_heads: int, head_dim: int, block_size: int, scale: float,
                     dt: int):
    """(out in storage dtype, exact double values, vmax per (token, head))."""
    o = oracle()
    out = np.empty_like(b.q)
    exact = np.empty(b.q.shape, np.float64)
    vmax = np.empty((b.tokens, q_heads), np.float32)
    o.orc_paged_attention(ptr(b.q), ptr(out), ptr(b.k_cache), ptr(b.v_cache), ptr(b.query_seq), ptr(b.query_key_len),
                          ptr(b.block_tables), b.tokens, q_heads, kv_heads, head_dim, block_size, b.max_blocks, scale,
                          dt, ptr(exact), ptr(vmax))
    return out, exact, vmax
