"""GPU parity of the KV-cache store and paged attention (the reference's
hip_store_kv / hip_paged_attention, src/hip_ops.hip:452-550, 724-744).

Bars:
* store: bit-exact (a copy), slot -1 skipped, strided key/value rows;
* attention: |got - exact| <= tol with `exact` the oracle's double value and
  tol = rel * max|V| over the attended keys plus one ulp of a 16-bit output.
  rel = 1e-4 for fp32 (online-softmax rounding over up to a few thousand keys;
  a typical error is two orders smaller); for 16-bit caches the matrix-core path
  rounds the softmax weights P to the cache dtype before P . V, an error of at
  most 2^-8 (bf16) / 2^-11 (fp16) of max|V|, so rel = 2^-7 / 2^-10; 0 rows for
  key_len 0, the V row itself for one key; a key just past a query's range
  that would dominate its softmax must not reach it (masking);
* against the reference's own hip_paged_attention (fp32, same inputs): within
  twice that tolerance.
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


REL = {H.F32: 1e-4, H.F16: 2.0 ** -10, H.BF16: 2.0 ** -7}


def tol_for(exact: np.ndarray, vmax: np.ndarray, dt: int) -> np.ndarray:
    t = REL[dt] * vmax[..., None] * np.ones_like(exact) + 1e-7
    if dt != H.F32:
        t = t + H.ulp(exact, dt)
    return t


def assert_attn(got: np.ndarray, exact: np.ndarray, vmax: np.ndarray, dt: int, what: str, factor: float = 1.0):
    g = H.from_storage(got, dt)
    tol = factor * tol_for(exact, vmax, dt)
    bad = ~(np.abs(g - exact) <= tol)
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside tolerance; first {i}: got {g[i]!r} "
                             f"exact {exact[i]!r} tol {tol[i]!r}")


def run_attention(gpu, b: H.PagedBatch, q_heads, kv_heads, hd, bs, scale, dt, max_query_len=0):
    return ops.paged_attention(H.to_dev(b.q, gpu, dt), H.to_dev(b.k_cache, gpu, dt), H.to_dev(b.v_cache, gpu, dt),
                               H.to_dev(b.query_seq, gpu), H.to_dev(b.query_key_len, gpu),
                               H.to_dev(b.block_tables, gpu), bs, scale, max_query_len=max_query_len)


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
def test_store_kv(gpu, dt):
    r = H.rng(7 + dt)
    T, kvh, hd, rows = 37, 4, 128, 64
    qkv = H.gen_act(r, (T, (8 + 2 * kvh) * hd), dt)  # packed [q | k | v] rows: strided views
    kc0 = H.gen_act(r, (rows, kvh, hd), dt)
    vc0 = H.gen_act(r, (rows, kvh, hd), dt)
    slots = r.permutation(rows)[:T].astype(np.int32)
    slots[[3, 10]] = -1
    o = H.oracle()
    key = np.ascontiguousarray(qkv[:, 8 * hd:(8 + kvh) * hd])
    val = np.ascontiguousarray(qkv[:, (8 + kvh) * hd:])
    kc_ref, vc_ref = kc0.copy(), vc0.copy()
    o.orc_store_kv(H.ptr(key), H.ptr(val), H.ptr(kc_ref), H.ptr(vc_ref), H.ptr(slots), T, kvh, hd, dt)
    d_qkv = H.to_dev(qkv, gpu, dt)
    kc, vc = H.to_dev(kc0, gpu, dt), H.to_dev(vc0, gpu, dt)
    case(f"store_kv dt={dt}")
    k_view = d_qkv[:, 8 * hd:(8 + kvh) * hd].view(T, kvh, hd)
    v_view = d_qkv[:, (8 + kvh) * hd:].view(T, kvh, hd)
    ops.store_kv(k_view, v_view, kc, vc, H.to_dev(slots, gpu))
    H.assert_bitexact(H.to_host(kc), kc_ref, "k cache")
    H.assert_bitexact(H.to_host(vc), vc_ref, "v cache")


CASES = [
    # (ctx_lens, q_lens, q_heads, kv_heads, head_dim, block_size)
    ([17, 64, 130], [17, 64, 130], 8, 2, 128, 16),       # prefill, several blocks per sequence
    ([300, 1, 77, 513], [1, 1, 1, 1], 28, 4, 128, 256),  # decode, Qwen2.5-7B heads
    ([40, 200], [5, 200], 4, 4, 64, 32),                  # chunked prefill with a cached prefix
    ([9, 33], [9, 2], 6, 3, 80, 8),                       # odd head_dim
    # matrix-core tiles (16-bit, head_dim 128, block_size % 64 == 0): sequence
    # switches mid-tile go to the wave kernel, the rest to the tiles
    ([300, 130, 64], [300, 130, 64], 8, 2, 128, 64),
    ([700, 90], [200, 90], 28, 4, 128, 256),              # chunked prefill after a 500-token prefix
    ([256], [256], 4, 1, 128, 128),                       # exact tiles
    ([33, 64, 1], [2, 1, 1], 32, 1, 128, 64),             # 32 heads per kv head: beyond the 16-column tiles
    ([150, 70], [150, 70], 21, 3, 128, 64),               # 3 kv heads; a tile spans the sequence switch
    ([385, 200], [385, 200], 32, 2, 128, 64),             # 16 query heads per kv head; tails ending mid-chunk
    ([1100], [1100], 8, 1, 128, 512),                     # 512-key blocks: chunks of a block's interior
]


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("heads", [(28, 4), (32, 8), (16, 1), (21, 3), (8, 8)],
                         ids=["qwen25", "qwen3", "g16", "kv3", "mha"])
def test_paged_attention_decode_batch(gpu, dt, heads):
    """A decode batch (one query per sequence) through the decode-only route
    (max_query_len = 1) and through the automatic one."""
    qh, kvh = heads
    r = H.rng(300 + qh + dt)
    ctx = [int(x) for x in r.integers(1, 1500, 24)] + [1, 64, 65, 2048]
    b = H.make_paged(r, ctx, [1] * len(ctx), qh, kvh, 128, 256, dt)
    scale = 128 ** -0.5
    _, exact, vmax = H.oracle_attention(b, qh, kvh, 128, 256, scale, dt)
    for mql in (1, 0):
        case(f"paged_attention decode heads={heads} dt={dt} max_query_len={mql}")
        got = H.to_host(run_attention(gpu, b, qh, kvh, 128, 256, scale, dt, max_query_len=mql))
        assert_attn(got, exact, vmax, dt, f"decode (max_query_len={mql})")


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("ci", range(len(CASES)))
def test_paged_attention_vs_oracle(gpu, dt, ci):
    ctx, ql, qh, kvh, hd, bs = CASES[ci]
    r = H.rng(100 + ci * 3 + dt)
    b = H.make_paged(r, ctx, ql, qh, kvh, hd, bs, dt)
    scale = float(hd) ** -0.5
    _, exact, vmax = H.oracle_attention(b, qh, kvh, hd, bs, scale, dt)
    case(f"paged_attention case={ci} dt={dt}")
    got = H.to_host(run_attention(gpu, b, qh, kvh, hd, bs, scale, dt))
    assert_attn(got, exact, vmax, dt, "attention")


def test_paged_attention_closed_forms(gpu):
    """key_len 0 -> zeros; one key -> exactly that V row."""
    r = H.rng(5)
    b = H.make_paged(r, [1, 20], [1, 1], 4, 2, 128, 16, H.F32)
    b.query_key_len[:] = [1, 0]
    case("paged_attention closed forms")
    got = run_attention(gpu, b, 4, 2, 128, 16, 0.1, H.F32).cpu().numpy()
    row0 = b.block_tables[0, 0] * 16
    for h in range(4):
        assert np.array_equal(got[0, h], b.v_cache[row0, h // 2])
    assert not got[1].any()


def test_dropins_vs_oracle_and_reference(gpu):
    ctx, ql, qh, kvh, hd, bs = [57, 130, 5], [57, 2, 5], 8, 2, 128, 32
    r = H.rng(9)
    b = H.make_paged(r, ctx, ql, qh, kvh, hd, bs, H.F32)
    scale = float(hd) ** -0.5
    _, exact, vmax = H.oracle_attention(b, qh, kvh, hd, bs, scale, H.F32)
    dq, dk, dv = H.to_dev(b.q, gpu), H.to_dev(b.k_cache, gpu), H.to_dev(b.v_cache, gpu)
    dqs, dql, dtab = H.to_dev(b.query_seq, gpu), H.to_dev(b.query_key_len, gpu), H.to_dev(b.block_tables, gpu)
    out = torch.empty_like(dq)
    case("hip_paged_attention drop-in")
    ops.lib().hip_paged_attention(dq.data_ptr(), out.data_ptr(), dk.data_ptr(), dv.data_ptr(), dqs.data_ptr(),
                                  dql.data_ptr(), dtab.data_ptr(), b.tokens, qh, kvh, hd, bs, b.max_blocks, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert_attn(got, exact, vmax, H.F32, "drop-in")
    # store: the new tokens' keys and values into fresh slots, drop-in vs oracle
    T = 6
    key, val = H.gen_act(r, (T, kvh, hd), H.F32), H.gen_act(r, (T, kvh, hd), H.F32)
    slots = np.array([0, 5, -1, 40, 41, 90], np.int32)
    kc_ref, vc_ref = b.k_cache.copy(), b.v_cache.copy()
    H.oracle().orc_store_kv(H.ptr(key), H.ptr(val), H.ptr(kc_ref), H.ptr(vc_ref), H.ptr(slots), T, kvh, hd, H.F32)
    dkey, dval, dsl = H.to_dev(key, gpu), H.to_dev(val, gpu), H.to_dev(slots, gpu)
    case("hip_store_kv drop-in")
    ops.lib().hip_store_kv(dkey.data_ptr(), dval.data_ptr(), dk.data_ptr(), dv.data_ptr(), dsl.data_ptr(), T, kvh, hd)
    torch.cuda.synchronize()
    H.assert_bitexact(dk.cpu().numpy(), kc_ref, "k cache")
    H.assert_bitexact(dv.cpu().numpy(), vc_ref, "v cache")
    ref = H.ref_hip()
    if ref is None:
        return
    # the reference's own kernels on the same (pre-store) inputs
    rk, rv = H.to_dev(b.k_cache, gpu), H.to_dev(b.v_cache, gpu)
    rout = torch.empty_like(dq)
    case("reference hip_paged_attention")
    ref.ref_hip_paged_attention(dq.data_ptr(), rout.data_ptr(), rk.data_ptr(), rv.data_ptr(), dqs.data_ptr(),
                                dql.data_ptr(), dtab.data_ptr(), b.tokens, qh, kvh, hd, bs, b.max_blocks, scale)
    rg = rout.cpu().numpy()
    assert_attn(rg, exact, vmax, H.F32, "reference vs oracle")
    assert (np.abs(got.astype(np.float64) - rg) <= 2 * tol_for(exact, vmax, H.F32)).all()
    ref.ref_hip_store_kv(dkey.data_ptr(), dval.data_ptr(), rk.data_ptr(), rv.data_ptr(), dsl.data_ptr(), T, kvh, hd)
    H.assert_bitexact(rk.cpu().numpy(), kc_ref, "reference k cache")


@pytest.mark.parametrize("dt", [H.F16, H.BF16], ids=["f16", "bf16"])
def test_paged_attention_masks_keys_past_the_range(gpu, dt):
    """Key 200 of a 256-token prefill carries a score that would dominate any
    softmax it enters: queries at positions < 200 must not see it, later ones
    must be pulled to its V row."""
    r = H.rng(31 + dt)
    b = H.make_paged(r, [256], [256], 4, 1, 128, 64, dt)
    qf = np.full((256, 4, 128), 0.25, np.float32)
    b.q[:] = H.to_storage(qf, dt)
    kf = H.from_storage(b.k_cache, dt).astype(np.float32) * 0.1
    row = b.block_tables[0, 200 // 64] * 64 + 200 % 64
    kf[row] = 6.0
    b.k_cache[:] = H.to_storage(kf, dt)
    scale = 128 ** -0.5
    _, exact, vmax = H.oracle_attention(b, 4, 1, 128, 64, scale, dt)
    case(f"paged_attention masking spike dt={dt}")
    got = H.to_host(run_attention(gpu, b, 4, 1, 128, 64, scale, dt))
    assert_attn(got, exact, vmax, dt, "masking")
    g = H.from_storage(got, dt)
    spike_v = H.from_storage(b.v_cache[row, 0], dt)
    assert np.abs(g[220:, 0] - spike_v).max() < 0.05 * np.abs(spike_v).max()  # pulled to the spike
    assert np.abs(g[:199, 0] - spike_v).max() > 0.5                          # never saw it


@pytest.mark.parametrize("dt", [H.F32, H.F16], ids=["f32", "f16"])
@pytest.mark.parametrize("scale", [-0.09, 0.0], ids=["negative", "zero"])
def test_paged_attention_nonpositive_scale(gpu, scale, dt):
    """A scale <= 0 at a matrix-core-eligible shape (those kernels keep the
    running max on unscaled scores, valid for scale > 0) is still right: it takes
    the wave kernel."""
    r = H.rng(61)
    b = H.make_paged(r, [300, 130], [300, 130], 8, 2, 128, 64, dt)
    _, exact, vmax = H.oracle_attention(b, 8, 2, 128, 64, scale, dt)
    case(f"paged_attention scale={scale} dt={dt}")
    got = H.to_host(run_attention(gpu, b, 8, 2, 128, 64, scale, dt))
    assert_attn(got, exact, vmax, dt, f"scale {scale}")


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
def test_paged_attention_late_rising_max(gpu, dt):
    """Keys in a late block score far higher than the earlier ones, so each
    query's running max rises after many chunks (the rescale of the partial sums
    runs late) while other waves' maxima stay put."""
    r = H.rng(62 + dt)
    bs = 64
    b = H.make_paged(r, [900], [900], 4, 1, 128, bs, dt)
    kc = H.from_storage(b.k_cache, dt).astype(np.float32)
    for lb in (9, 12):  # keys 576..639 and 768..831
        blk = int(b.block_tables[0, lb])
        kc[blk * bs:(blk + 1) * bs] *= 4.0
    b.k_cache = H.to_storage(kc, dt)
    scale = 128 ** -0.5
    _, exact, vmax = H.oracle_attention(b, 4, 1, 128, bs, scale, dt)
    case(f"paged_attention late rising max dt={dt}")
    got = H.to_host(run_attention(gpu, b, 4, 1, 128, bs, scale, dt))
    assert_attn(got, exact, vmax, dt, "late max")


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
def test_paged_attention_many_short_sequences(gpu, dt):
    """700 five-token prefills: 3500 tokens, every 128-token tile spans several
    sequences, so the tile launch does nothing and the decode kernel that follows
    it takes every token."""
    r = H.rng(70 + dt)
    ctx = [5] * 700
    b = H.make_paged(r, ctx, ctx, 8, 2, 128, 64, dt)
    scale = 128 ** -0.5
    _, exact, vmax = H.oracle_attention(b, 8, 2, 128, 64, scale, dt)
    case(f"paged_attention 700 short sequences dt={dt}")
    got = H.to_host(run_attention(gpu, b, 8, 2, 128, 64, scale, dt))
    assert_attn(got, exact, vmax, dt, "many short sequences")


SPLIT_CASES = [
    # (context lengths of a decode batch, (q_heads, kv_heads)): few (token, kv head) pairs
    ([4096], (28, 4)),
    ([5000, 77, 1, 2049, 300], (28, 4)),   # ragged; one query also gets key_len 0 below
    ([8192, 1024], (32, 8)),
    ([640], (16, 1)),
    ([3000, 40], (8, 8)),                  # one query head per kv head
]


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("ci", range(len(SPLIT_CASES)))
def test_paged_attention_split_decode(gpu, dt, ci):
    """Small decode batches over long contexts take the split path (partial
    softmax per key range, then a merge): within the same tolerance of the
    oracle as the unsplit kernel, for a promised decode batch and an unhinted one."""
    ctx, (qh, kvh) = SPLIT_CASES[ci]
    r = H.rng(400 + ci * 3 + dt)
    b = H.make_paged(r, ctx, [1] * len(ctx), qh, kvh, 128, 256, dt)
    if len(ctx) > 2:
        b.query_key_len[1] = 0
    assert ops.lib().nvf_paged_attention_workspace_size(b.tokens, qh, kvh, 128, 256, b.max_blocks, 1) > 0
    scale = 128 ** -0.5
    _, exact, vmax = H.oracle_attention(b, qh, kvh, 128, 256, scale, dt)
    args = (H.to_dev(b.q, gpu, dt), H.to_dev(b.k_cache, gpu, dt), H.to_dev(b.v_cache, gpu, dt),
            H.to_dev(b.query_seq, gpu), H.to_dev(b.query_key_len, gpu), H.to_dev(b.block_tables, gpu), 256, scale)
    for mql in (1, 0):
        case(f"paged_attention split decode case={ci} dt={dt} max_query_len={mql}")
        got = H.to_host(ops.paged_attention(*args, max_query_len=mql))
        assert_attn(got, exact, vmax, dt, f"split (max_query_len={mql})")
        if len(ctx) > 2:
            assert not H.from_storage(got, dt)[1].any()  # key_len 0: zeros
    case(f"paged_attention unsplit case={ci} dt={dt}")
    got = H.to_host(ops.paged_attention(*args, max_query_len=1, split=False))
    assert_attn(got, exact, vmax, dt, "unsplit")


def test_dropin_split_decode_uses_the_static_scratch(gpu):
    """The fp32 drop-in splits small decode batches through the library's static
    scratch (it allocates nothing): a short-context call, then a longer one needing
    more of it."""
    for ctx, seed in (([700, 33], 1), ([6000, 4096, 17], 2)):
        r = H.rng(500 + seed)
        b = H.make_paged(r, ctx, [1] * len(ctx), 28, 4, 128, 256, H.F32)
        scale = 128 ** -0.5
        _, exact, vmax = H.oracle_attention(b, 28, 4, 128, 256, scale, H.F32)
        dq, dk, dv = H.to_dev(b.q, gpu), H.to_dev(b.k_cache, gpu), H.to_dev(b.v_cache, gpu)
        dqs, dql, dtab = H.to_dev(b.query_seq, gpu), H.to_dev(b.query_key_len, gpu), H.to_dev(b.block_tables, gpu)
        out = torch.empty_like(dq)
        case(f"hip_paged_attention split drop-in ctx={ctx}")
        ops.lib().hip_paged_attention(dq.data_ptr(), out.data_ptr(), dk.data_ptr(), dv.data_ptr(), dqs.data_ptr(),
                                      dql.data_ptr(), dtab.data_ptr(), b.tokens, 28, 4, 128, 256, b.max_blocks, scale)
        torch.cuda.synchronize()
        assert_attn(out.cpu().numpy(), exact, vmax, H.F32, "split drop-in")


TILE_SPLIT_CASES = [
    # (context lengths, query counts): few 128-token tiles over long contexts
    ([8192], [256]),                 # a 256-token chunk after a 7936-token prefix
    ([4000, 3000], [200, 60]),       # uniform tiles (split tiles) and a mixed tile (split decode) together
    ([2048, 5], [300, 5]),
]


@pytest.mark.parametrize("dt", DTYPES, ids=DT_IDS)
@pytest.mark.parametrize("ci", range(len(TILE_SPLIT_CASES)))
def test_paged_attention_split_tiles(gpu, dt, ci):
    """Chunked prefill with few tiles over long contexts takes the split path for
    the tiles (and for the decode kernel's mixed-tile tokens), merged once."""
    ctx, ql = TILE_SPLIT_CASES[ci]
    r = H.rng(600 + ci * 3 + dt)
    b = H.make_paged(r, ctx, ql, 8, 2, 128, 256, dt)
    assert ops.lib().nvf_paged_attention_workspace_size(b.tokens, 8, 2, 128, 256, b.max_blocks, 0) > 0
    scale = 128 ** -0.5
    _, exact, vmax = H.oracle_attention(b, 8, 2, 128, 256, scale, dt)
    args = (H.to_dev(b.q, gpu, dt), H.to_dev(b.k_cache, gpu, dt), H.to_dev(b.v_cache, gpu, dt),
            H.to_dev(b.query_seq, gpu), H.to_dev(b.query_key_len, gpu), H.to_dev(b.block_tables, gpu), 256, scale)
    case(f"paged_attention split tiles case={ci} dt={dt}")
    assert_attn(H.to_host(ops.paged_attention(*args)), exact, vmax, dt, "split tiles")
    case(f"paged_attention unsplit tiles case={ci} dt={dt}")
    assert_attn(H.to_host(ops.paged_attention(*args, split=False)), exact, vmax, dt, "unsplit tiles")


def test_paged_attention_ws_too_small_runs_unsplit(gpu):
    """nvf_paged_attention_ws with a workspace one byte short of the size query's
    answer takes the unsplit path: the same results, no out-of-bounds writes."""
    r = H.rng(77)
    b = H.make_paged(r, [4096, 300], [1, 1], 28, 4, 128, 256, H.F16)
    need = ops.lib().nvf_paged_attention_workspace_size(b.tokens, 28, 4, 128, 256, b.max_blocks, 1)
    assert need > 0
    scale = 128 ** -0.5
    _, exact, vmax = H.oracle_attention(b, 28, 4, 128, 256, scale, H.F16)
    dq, dk, dv = H.to_dev(b.q, gpu, H.F16), H.to_dev(b.k_cache, gpu, H.F16), H.to_dev(b.v_cache, gpu, H.F16)
    dqs, dql, dtab = H.to_dev(b.query_seq, gpu), H.to_dev(b.query_key_len, gpu), H.to_dev(b.block_tables, gpu)
    guard = torch.full(((need + 15) // 16 * 4 + 64,), 7.0, dtype=torch.float32, device=gpu)
    out = torch.empty_like(dq)
    case("paged_attention_ws one byte short")
    rc = ops.lib().nvf_paged_attention_ws(dq.data_ptr(), out.data_ptr(), dk.data_ptr(), dv.data_ptr(), dqs.data_ptr(),
                                          dql.data_ptr(), dtab.data_ptr(), b.tokens, 28, 4, 128, 256, b.max_blocks,
                                          scale, 28 * 128, 1, guard.data_ptr(), need - 1, H.F16, None)
    assert rc == 0
    torch.cuda.synchronize()
    assert_attn(H.to_host(out), exact, vmax, H.F16, "unsplit fallback")
    assert (guard == 7.0).all()  # the workspace was not touched


@pytest.mark.parametrize("dt", [H.F16, H.F32], ids=["f16", "f32"])
def test_paged_attention_config2_full_vs_torch(gpu, dt):
    """BASELINE config 2's causal prefill at full size (4 x 4096 tokens, 28 / 4
    heads x 128, KV blocks of 256 in a permuted cache) against torch's fp32
    scaled_dot_product_attention of the gathered keys.  Tolerance as the other
    attention tests, with vmax the largest |V| of the sequence's kv head (at least
    the largest |V| a query attends)."""
    S, L, qh, kvh, hd, bs = 4, 4096, 28, 4, 128, 256
    g = torch.Generator(device=gpu)
    g.manual_seed(12)
    tdt = H.torch_dtype(dt)
    nb = L // bs
    q = torch.randn(S * L, qh, hd, device=gpu, generator=g).to(tdt)
    kc = torch.randn(S * nb * bs, kvh, hd, device=gpu, generator=g).to(tdt)
    vc = torch.randn(S * nb * bs, kvh, hd, device=gpu, generator=g).to(tdt)
    tab = torch.randperm(S * nb, device=gpu, generator=g).to(torch.int32).view(S, nb)
    qs = torch.arange(S, device=gpu, dtype=torch.int32).repeat_interleave(L)
    ql = (torch.arange(L, device=gpu, dtype=torch.int32) + 1).repeat(S)
    scale = hd ** -0.5
    case(f"paged_attention config 2 full size dt={dt}")
    out = ops.paged_attention(q, kc, vc, qs, ql, tab, bs, scale).float()
    rel = REL[dt]
    for s_ in range(S):
        rows = (tab[s_].long()[:, None] * bs + torch.arange(bs, device=gpu)[None, :]).reshape(-1)  # key order
        k_ = kc[rows].float().permute(1, 0, 2).repeat_interleave(qh // kvh, dim=0)[None]
        v_ = vc[rows].float().permute(1, 0, 2).repeat_interleave(qh // kvh, dim=0)[None]
        q_ = q[s_ * L:(s_ + 1) * L].float().permute(1, 0, 2)[None]
        ref = torch.nn.functional.scaled_dot_product_attention(q_, k_, v_, is_causal=True, scale=scale)[0]
        ref = ref.permute(1, 0, 2)  # [L, qh, hd]
        vmax = v_[0].abs().amax(dim=(1, 2))  # per q head
        got = out[s_ * L:(s_ + 1) * L]
        tol = rel * vmax[None, :, None] + 1e-6
        if dt != H.F32:
            tol = tol + ref.abs() * 2.0 ** -10  # one ulp of the fp16 output
        bad = ((got - ref).abs() > tol).sum().item()
        assert bad == 0, f"sequence {s_}: {bad} of {got.numel()} outputs outside tolerance"


@pytest.mark.parametrize("shape", ["config1", "long"], ids=["config1_decode", "split_4x32768"])
def test_paged_attention_decode_full_vs_torch(gpu, shape):
    """Decode batches at full size against torch's fp32 attention of each
    sequence's gathered keys: config 1 (256 sequences, context U[1, 4096], 28 / 4
    heads) and a split long-context batch (4 x 32768 keys), fp16 caches."""
    qh, kvh, hd, bs = 28, 4, 128, 256
    g = torch.Generator(device=gpu)
    g.manual_seed(13)
    if shape == "config1":
        ctx = (torch.randint(1, 4097, (256,), generator=g, device=gpu)).tolist()
    else:
        ctx = [32768] * 4
    nbk = [-(-c // bs) for c in ctx]
    mb = max(nbk)
    total = sum(nbk)
    perm = torch.randperm(total, device=gpu, generator=g).to(torch.int32)
    tab = torch.full((len(ctx), mb), -1, dtype=torch.int32, device=gpu)
    o = 0
    for s_, n_ in enumerate(nbk):
        tab[s_, :n_] = perm[o:o + n_]
        o += n_
    kc = torch.randn(total * bs, kvh, hd, device=gpu, generator=g).half()
    vc = torch.randn(total * bs, kvh, hd, device=gpu, generator=g).half()
    B = len(ctx)
    q = torch.randn(B, qh, hd, device=gpu, generator=g).half()
    qs = torch.arange(B, dtype=torch.int32, device=gpu)
    ql = torch.tensor(ctx, dtype=torch.int32, device=gpu)
    scale = hd ** -0.5
    case(f"paged_attention decode full size {shape}")
    out = ops.paged_attention(q, kc, vc, qs, ql, tab, bs, scale, max_query_len=1).float()
    for s_, c in enumerate(ctx):
        rows = (tab[s_, :nbk[s_]].long()[:, None] * bs + torch.arange(bs, device=gpu)[None, :]).reshape(-1)[:c]
        k_ = kc[rows].float().permute(1, 0, 2).repeat_interleave(qh // kvh, dim=0)  # [qh, c, hd]
        v_ = vc[rows].float().permute(1, 0, 2).repeat_interleave(qh // kvh, dim=0)
        p = torch.softmax((k_ @ q[s_].float()[:, :, None])[..., 0] * scale, dim=-1)  # [qh, c]
        ref = (p[:, None, :] @ v_)[:, 0, :]  # [qh, hd]
        vmax = v_.abs().amax(dim=(1, 2))
        tol = REL[H.F16] * vmax[:, None] + ref.abs() * 2.0 ** -10 + 1e-6
        bad = ((out[s_] - ref).abs() > tol).sum().item()
        assert bad == 0, f"sequence {s_} (context {c}): {bad} outputs outside tolerance"


@pytest.mark.parametrize("dt", [H.F16, H.BF16, H.F32], ids=["f16", "bf16", "f32"])
@pytest.mark.parametrize("lens,prefix", [([256, 384, 128], 0),      # every start a multiple of 128
                                         ([200, 312, 100], 0),      # mixed tiles: the second launch runs
                                         ([256], 8192),             # a chunk after a long prefix: split tiles
                                         ([384, 130], 64)])         # a partial last tile
def test_paged_attention_host_cu_seqlens(gpu, dt, lens, prefix):
    """nvf_paged_attention_seqs_ws (host cu_seqlens) gives the bit-identical output of
    nvf_paged_attention_ws: with 128-aligned sequence starts it only leaves out the
    launch whose workgroups would all exit."""
    g = torch.Generator(device=gpu)
    g.manual_seed(sum(lens) + prefix + dt)
    tdt = H.torch_dtype(dt)
    qh, kvh, hd, bs = 28, 4, 128, 256
    ctx = [prefix + n for n in lens]
    nbs = [-(-c // bs) for c in ctx]
    rows = sum(nbs) * bs
    kc = torch.randn(rows, kvh, hd, device=gpu, generator=g).to(tdt)
    vc = torch.randn(rows, kvh, hd, device=gpu, generator=g).to(tdt)
    tab = torch.full((len(lens), max(nbs)), -1, dtype=torch.int32)
    perm = torch.randperm(sum(nbs), generator=torch.Generator().manual_seed(3)).to(torch.int32)
    o = 0
    for s_, nb in enumerate(nbs):
        tab[s_, :nb] = perm[o:o + nb]
        o += nb
    tab = tab.to(gpu)
    T = sum(lens)
    qs = torch.cat([torch.full((n,), s_, dtype=torch.int32) for s_, n in enumerate(lens)]).to(gpu)
    ql = torch.cat([torch.arange(prefix + 1, prefix + n + 1, dtype=torch.int32) for n in lens]).to(gpu)
    q = torch.randn(T, qh, hd, device=gpu, generator=g).to(tdt)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    case(f"paged_attention host cu_seqlens lens={lens} prefix={prefix} dt={dt}")
    ref = ops.paged_attention(q, kc, vc, qs, ql, tab, bs, hd ** -0.5)
    got = ops.paged_attention(q, kc, vc, qs, ql, tab, bs, hd ** -0.5, cu_seqlens=cu)
    torch.cuda.synchronize()
    H.assert_bitexact(H.to_host(got), H.to_host(ref), "host cu_seqlens vs device-only metadata")
    with pytest.raises(RuntimeError):  # the last entry must be the token count
        ops.paged_attention(q, kc, vc, qs, ql, tab, bs, hd ** -0.5, cu_seqlens=cu[:-1])


@pytest.mark.parametrize("n,lens", [(300, (64, 128)), (512, (5,)), (77, (1, 300, 300, 2048)), (513, (64, 700))],
                         ids=["ties", "all-equal", "mixed", "past-self-order"])
def test_paged_attention_decode_self_order(gpu, n, lens):
    """Decode batches of at most 512 tokens without a token order rank their tokens
    inside the kernel (longest first, ties by token): every token is computed exactly
    once -- an output pre-filled with NaN keeps none -- and the result is bit-identical
    to the host-ordered launch's; 513 tokens take the unranked path."""
    g = torch.Generator(device=gpu)
    g.manual_seed(n)
    qh, kvh, hd, bs = 28, 4, 128, 256
    r = np.random.default_rng(n + len(lens))
    kl = np.array([lens[i % len(lens)] for i in range(n)], np.int32)
    r.shuffle(kl)
    kl[n // 3] = 0  # a query with no keys: a zero row
    nbs = [max(1, -(-int(c) // bs)) for c in kl]
    rows = sum(nbs) * bs
    kc = torch.randn(rows, kvh, hd, device=gpu, generator=g).half()
    vc = torch.randn(rows, kvh, hd, device=gpu, generator=g).half()
    tab = np.full((n, max(nbs)), -1, np.int32)
    perm = r.permutation(sum(nbs)).astype(np.int32)
    o = 0
    for s_, nb in enumerate(nbs):
        tab[s_, :nb] = perm[o:o + nb]
        o += nb
    q = torch.randn(n, qh, hd, device=gpu, generator=g).half()
    args = (q, kc, vc, torch.arange(n, dtype=torch.int32, device=gpu), torch.from_numpy(kl).to(gpu),
            torch.from_numpy(tab).to(gpu), bs, hd ** -0.5)
    case(f"paged_attention decode self-order n={n} lens={lens}")
    out = torch.full((n, qh, hd), float("nan"), dtype=torch.float16, device=gpu)
    ops.paged_attention(*args, max_query_len=1, split=False, out=out)
    ref = ops.paged_attention(*args, max_query_len=1, split=False,
                              token_order=torch.from_numpy(ops.decode_token_order(kl)).to(gpu))
    torch.cuda.synchronize()
    assert not torch.isnan(out).any().item(), "a token was not computed"
    H.assert_bitexact(H.to_host(out), H.to_host(ref), "self-ordered vs host-ordered")
    assert not out[n // 3].float().abs().sum().item()


@pytest.mark.parametrize("dt", [H.F16, H.BF16, H.F32], ids=["f16", "bf16", "f32"])
@pytest.mark.parametrize("n,ctx_max,order_kind,heads", [(256, 4096, "schedule", (28, 4)),  # config 1's batch
                                                        (256, 4096, "schedule", (32, 8)),  # Qwen3-8B's heads
                                                        (13, 2048, "schedule", (28, 4)),   # not a multiple of 8
                                                        (200, 1024, "random", (28, 4)),    # any permutation
                                                        (3, 20000, "schedule", (28, 4))])  # the split path
def test_paged_attention_token_order(gpu, dt, n, ctx_max, order_kind, heads):
    """nvf_paged_attention_order_ws (the caller's token order for the decode kernel's
    workgroups) gives the bit-identical output of nvf_paged_attention_ws, for the
    nvf_decode_token_order schedule and for any permutation; key_len 0 included."""
    g = torch.Generator(device=gpu)
    g.manual_seed(n + ctx_max + dt)
    tdt = H.torch_dtype(dt)
    (qh, kvh), hd, bs = heads, 128, 256
    r = np.random.default_rng(n * 7 + dt + qh)
    ctx = r.integers(1, ctx_max + 1, n).astype(np.int32)
    nbs = [-(-int(c) // bs) for c in ctx]
    rows = sum(nbs) * bs
    kc = torch.randn(rows, kvh, hd, device=gpu, generator=g).to(tdt)
    vc = torch.randn(rows, kvh, hd, device=gpu, generator=g).to(tdt)
    tab = np.full((n, max(nbs)), -1, np.int32)
    perm = r.permutation(sum(nbs)).astype(np.int32)
    o = 0
    for s_, nb in enumerate(nbs):
        tab[s_, :nb] = perm[o:o + nb]
        o += nb
    kl = ctx.copy()
    kl[n // 2] = 0  # a query with no keys: a zero row
    q = torch.randn(n, qh, hd, device=gpu, generator=g).to(tdt)
    args = (q, kc, vc, torch.arange(n, dtype=torch.int32, device=gpu), torch.from_numpy(kl).to(gpu),
            torch.from_numpy(tab).to(gpu), bs, hd ** -0.5)
    order = ops.decode_token_order(kl) if order_kind == "schedule" else r.permutation(n).astype(np.int32)
    case(f"paged_attention token order n={n} ctx_max={ctx_max} {order_kind} heads={heads} dt={dt}")
    ref = ops.paged_attention(*args, max_query_len=1)
    got = ops.paged_attention(*args, max_query_len=1, token_order=torch.from_numpy(order).to(gpu))
    torch.cuda.synchronize()
    H.assert_bitexact(H.to_host(got), H.to_host(ref), "token order vs none")
    assert not got[n // 2].float().abs().sum().item()


def test_paged_attention_token_order_out_of_range_entry(gpu):
    """An order entry outside 0 .. tokens-1 computes nothing and touches no memory (the
    call completes); every token the order names equals the unordered result (this batch
    takes the split path, whose merge also covers the unnamed token: its row is
    unspecified)."""
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    n, qh, kvh, hd, bs = 24, 28, 4, 128, 256
    ctx = np.random.default_rng(5).integers(1, 1500, n).astype(np.int32)
    nbs = [-(-int(c) // bs) for c in ctx]
    tab = np.full((n, max(nbs)), -1, np.int32)
    o = 0
    for s_, nb in enumerate(nbs):
        tab[s_, :nb] = np.arange(o, o + nb)
        o += nb
    kc = torch.randn(o * bs, kvh, hd, device=gpu, generator=g).half()
    vc = torch.randn(o * bs, kvh, hd, device=gpu, generator=g).half()
    q = torch.randn(n, qh, hd, device=gpu, generator=g).half()
    args = (q, kc, vc, torch.arange(n, dtype=torch.int32, device=gpu), torch.from_numpy(ctx).to(gpu),
            torch.from_numpy(tab).to(gpu), bs, hd ** -0.5)
    order = np.arange(n, dtype=np.int32)
    order[3] = 10 ** 6  # token 3 is not named
    case("paged_attention token order with an out-of-range entry")
    ref = ops.paged_attention(*args, max_query_len=1)
    out = torch.full_like(q, 7.0)
    ops.paged_attention(*args, max_query_len=1, out=out, token_order=torch.from_numpy(order).to(gpu))
    torch.cuda.synchronize()
    keep = [i for i in range(n) if i != 3]
    H.assert_bitexact(H.to_host(out[keep]), H.to_host(ref[keep]), "the named tokens")
