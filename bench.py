"""Layer-op benchmark of the MI355X fused per-layer ops (one GPU).

One step = one pass of the hot path over one batch of the workload (BASELINE
config 2 by default: Qwen2.5-7B chunked prefill, 4 x 4096 = 16384 packed
tokens, fp16 activations):

  Q8_0 embedding gather (152064 x 3584 table, split planes) -> fp16 [T, 3584]
  residual-add + RMSNorm [T, 3584]
  NeoX RoPE on q [T, 28, 128] and k [T, 4, 128] (one fused launch)
  SiLU(gate) * up [T, 18944]

Every op reads synthetic inputs already resident in HBM.  Each op rotates over
enough independent buffer sets (>= 1 GiB per op) that its inputs were last
touched long before the launch, so the 256 MB MALL cannot serve them: the
figures are HBM figures.  Per-op times come from HIP events on the stream the
kernels run on; the dominant kernel (SwiGLU) gives the roofline object.

Beside the chain, `q8_gemm` times the Q8_0 GEMM (the reference's hip_matmul_q8) at
the gate_up projection shape [T, H] x [2I, H]^T on pre-quantized activations, in
TOP/s against the dense int8 MFMA peak; it does not enter `value`.

The CPU baseline is the C oracle (single thread, -O2) timed on a bounded
sample of the same workload on this host.

Prints ONE JSON line.  `python bench.py --gpus N` with N > 1 exits: this build
measures one GPU only.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_OPS = 5.0e15  # MI355X dense int8 MFMA
FP32_PEAK_FLOPS = 157.3e12  # MI355X dense fp32 matrix rate
METRIC = "fused-op HBM GB/s (% of peak) + layer-op tokens/s at Qwen2.5-7B shapes"
POOL_BYTES = 1 << 30
GEMV_M = 8  # decode rows for the GEMV line


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", type=int, default=2, help="BASELINE config index (1-4)")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU-baseline budget (0 = skip)")
    p.add_argument("--configs", default="0,1,3,4",
                   help="after the headline config, the chain (gather, norm, RoPE, SwiGLU) of each of these BASELINE "
                        "configs, GPU and CPU, under \"configs\" ('' = none; the headline config is skipped here)")
    p.add_argument("--emb", default="", choices=["", "q8_0", "q8_0_blocks", "q4_k", "q5_k", "q6_k", "f16"],
                   help="embedding table format (default: the config's)")
    p.add_argument("--write-traffic", default="", metavar="DIR",
                   help="no benchmark: build profiles/traffic.json from rocprofv3 FETCH_SIZE / WRITE_SIZE runs under DIR")
    p.add_argument("--source-commit", default="",
                   help="with --write-traffic: the commit the profiled tree was built from (run where .git is; "
                        "the stamp then also records whether the kernel sources differ from it)")
    p.add_argument("--only", default="",
                   help="comma list of ops (default emb,rms,rope,silu,copy,gemm,gemv,gemv_down,gemv_qkv,gemv_o,split,attn,attn_decode,attn_f32,"
                        "attn_decode_ordered,attn_decode_f32,attn_decode_small,layer,layer_decode,layer_b1,layer_b1_graph); "
                        "also emb_rms, rms_q8, silu_q8 (fusions)")
    return p.parse_args()


TABLE_BYTES_PER_ELEM = {"q8_0": 34 / 32, "q8_0_blocks": 34 / 32, "q4_k": 144 / 256, "q5_k": 176 / 256,
                        "q6_k": 210 / 256, "f16": 2.0}


def op_bytes(cfg, e: int, emb_fmt: str) -> dict[str, int]:
    """Algorithmic HBM bytes per launch (each input read once, each output written once)."""
    T, Hd, I = cfg.tokens, cfg.hidden, cfg.inter
    heads = cfg.q_heads + cfg.kv_heads
    emb = int(T * Hd * TABLE_BYTES_PER_ELEM[emb_fmt]) + 8 * T + T * Hd * e
    rope = 2 * T * heads * cfg.head_dim * e + 8 * T + (2 * cfg.head_dim * e if cfg.qk_norm else 0)
    return {"emb": emb, "rms": 4 * T * Hd * e + Hd * e, "rope": rope, "silu": 3 * T * I * e,
            # fusions with the neighbours (not in the default chain):
            # layer-0 gather + norm: table rows + ids + residual and out writes
            "emb_rms": int(T * Hd * TABLE_BYTES_PER_ELEM[emb_fmt]) + 8 * T + 2 * T * Hd * e + Hd * e,
            # residual-add + RMSNorm + Q8 row scale + int8 row
            "rms_q8": 4 * T * Hd * e + Hd * e + T * Hd + 4 * T,
            # SwiGLU writing only the down projection's int8 rows and row scales
            "silu_q8": 2 * T * I * e + T * I + 4 * T,
            # decode GEMV (m = GEMV_M) at the gate_up shape: the weights once, plus activations and output
            "gemv": int(2 * I * Hd * 34 / 32) + GEMV_M * Hd + 4 * GEMV_M + GEMV_M * 2 * I * e,
            # the layer's other decode GEMVs (m = GEMV_M): down [H, I], qkv [q + 2 kv, H], o [H, q]
            **{k_: n_ * k2 // 32 * 34 + GEMV_M * k2 + 4 * GEMV_M + GEMV_M * n_ * e
               for k_, (n_, k2, _) in gemv_shapes(cfg).items() if k_ != "gemv"},
            # on-device Q8_0 block split of the gate_up weights: 34 bytes in and 34 out per block
            "split": 2 * I * Hd // 32 * 68,
            # LM head at decode (m = 1): the [vocab, hidden] weights once (bf16 or Q4_K superblocks), x, fp32 logits
            "lm_head": cfg.vocab * Hd * 2 + Hd * e + 4 * cfg.vocab,
            "lm_head_q4k": cfg.vocab * Hd // 256 * 144 + Hd * e + 4 * cfg.vocab}


def gemv_shapes(cfg) -> dict[str, tuple[int, int, str]]:
    """Decode Q8_0 GEMV lines: name -> (n, k, projection)."""
    qs, ks = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    return {"gemv": (2 * cfg.inter, cfg.hidden, "gate_up"), "gemv_down": (cfg.hidden, cfg.inter, "down"),
            "gemv_qkv": (qs + 2 * ks, cfg.hidden, "qkv"), "gemv_o": (cfg.hidden, qs, "o")}


def main() -> int:
    args = parse()
    if args.write_traffic:
        print(json.dumps(write_traffic(args.write_traffic, args.config, args.source_commit)[f"c{args.config}"],
                         indent=1))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1",
                          "n_gpus_requested": args.gpus}))
        return 2

    import torch

    from nano_vllm_cpp_amd import ops
    from tests import harness as H

    cfg = H.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    dt = cfg.dtype
    tdt = H.torch_dtype(dt)
    e = 2 if dt != H.F32 else 4
    T, Hd, I, V = cfg.tokens, cfg.hidden, cfg.inter, cfg.vocab
    qs, ks = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    g = torch.Generator(device=dev).manual_seed(cfg.seed)
    emb_fmt = args.emb or cfg.emb
    nbytes = op_bytes(cfg, e, emb_fmt)
    only = set(filter(None, args.only.split(","))) or {"emb", "rms", "rope", "silu", "copy", "copy12", "copy12_emb",
                                                       "gemm", "gemv", "gemv_down", "gemv_qkv", "gemv_o", "split", "lm_head", "lm_head_q4k", "moe",
                                                       "attn", "attn_decode", "attn_decode_ordered", "attn_f32", "attn_decode_f32", "attn_decode_small", "layer", "layer_decode", "layer_b1", "layer_b1_graph"}

    def nsets(b: int) -> int:
        return max(2, -(-POOL_BYTES // b))

    def randn(shape, mean=0.0, std=1.0):
        return (torch.randn(shape, generator=g, device=dev) * std + mean).to(tdt)

    # ---- inputs (resident in HBM before timing) ------------------------------
    if emb_fmt in ("q8_0", "q8_0_blocks"):
        w8 = torch.randint(-127, 128, (V * Hd,), generator=g, device=dev, dtype=torch.int8)
        ws = torch.empty(V * Hd // 32, device=dev).uniform_(1e-3, 1e-2, generator=g).half().view(torch.int16)
        if emb_fmt == "q8_0_blocks":
            blocks = torch.cat([ws.view(torch.uint8).view(-1, 2), w8.view(torch.uint8).view(-1, 32)], 1).reshape(-1)
            del w8, ws
    elif emb_fmt == "q4_k":
        blocks = torch.from_numpy(H.gen_q4_k(np.random.default_rng(cfg.seed), V * Hd // 256)).to(dev)
    elif emb_fmt in ("q5_k", "q6_k"):
        bb, offs = (176, (0, 2)) if emb_fmt == "q5_k" else (210, (208,))
        blocks = torch.from_numpy(H.gen_raw_blocks(np.random.default_rng(cfg.seed), V * Hd // 256, bb, offs)).to(dev)
    else:
        f16_table = randn((V, Hd)).half()
    n_emb = nsets(nbytes["emb"])
    emb_sets = [(torch.randint(0, V, (T,), generator=g, device=dev), torch.empty(T, Hd, dtype=tdt, device=dev))
                for _ in range(n_emb)] if "emb" in only else []
    rms_sets = [(randn((T, Hd)), randn((T, Hd)), torch.empty(T, Hd, dtype=tdt, device=dev))
                for _ in range(nsets(nbytes["rms"]))] if "rms" in only else []
    gamma = randn((Hd,), 1.0, 0.1)
    rope_sets = [(randn((T, qs)), randn((T, ks))) for _ in range(nsets(nbytes["rope"]))] if "rope" in only else []
    pos = torch.from_numpy(cfg.positions()).to(dev)
    inv = ops.rope_inv_freq(cfg.theta, cfg.head_dim, dev)
    qw = randn((cfg.head_dim,), 1.0, 0.1) if cfg.qk_norm else None
    kw = randn((cfg.head_dim,), 1.0, 0.1) if cfg.qk_norm else None
    silu_sets = [(randn((T, 2 * I)), torch.empty(T, I, dtype=tdt, device=dev))
                 for _ in range(nsets(nbytes["silu"]))] if "silu" in only else []
    q8_sets = [(randn((T, Hd)), randn((T, Hd)), torch.empty(T, Hd, dtype=tdt, device=dev),
                torch.empty(T, dtype=torch.float32, device=dev), torch.empty(T, Hd, dtype=torch.int8, device=dev))
               for _ in range(nsets(nbytes["rms_q8"]))] if "rms_q8" in only else []
    er_sets = [(torch.randint(0, V, (T,), generator=g, device=dev), torch.empty(T, Hd, dtype=tdt, device=dev),
                torch.empty(T, Hd, dtype=tdt, device=dev)) for _ in range(nsets(nbytes["emb_rms"]))] \
        if "emb_rms" in only else []
    gemm_in = None
    if "gemm" in only:  # Q8_0 GEMM at the gate_up projection shape: [T, H] x [2I, H]^T
        gw8 = torch.randint(-127, 128, (2 * I * Hd,), generator=g, device=dev, dtype=torch.int8)
        gws = torch.empty(2 * I * Hd // 32, device=dev).uniform_(1e-3, 1e-2, generator=g).half().view(torch.int16)
        gsc, gxq = ops.q8_quantize_rows(randn((T, Hd)))
        gemm_in = (gxq, gsc, gw8, gws, torch.empty(T, 2 * I, dtype=tdt, device=dev))
    sq_sets = [(randn((T, 2 * I)), torch.empty(T, dtype=torch.float32, device=dev),
                torch.empty(T, I, dtype=torch.int8, device=dev)) for _ in range(nsets(nbytes["silu_q8"]))] \
        if "silu_q8" in only else []
    gemv_in = {}
    for gn_, (gnn, gk, _) in gemv_shapes(cfg).items():
        if gn_ in only:  # weights rotated over >= 1 GiB so every launch streams them from HBM
            gsc1, gxq1 = ops.q8_quantize_rows(randn((GEMV_M, gk)))
            gsets = [(torch.randint(-127, 128, (gnn * gk,), generator=g, device=dev, dtype=torch.int8),
                      torch.empty(gnn * gk // 32, device=dev).uniform_(1e-3, 1e-2, generator=g).half().view(torch.int16))
                     for _ in range(nsets(nbytes[gn_]))]
            gemv_in[gn_] = (gxq1, gsc1, gsets, gnn, torch.empty(GEMV_M, gnn, dtype=tdt, device=dev))
    split_sets = []
    lm_sets = {}
    for n_, wf_ in (("lm_head", ops.W_BF16), ("lm_head_q4k", 12)):
        if n_ in only:  # one [vocab, hidden] matrix (>= 0.3 GB, beyond the caches), m = 1, fp32 logits
            if wf_ == 12:
                blk = torch.randint(0, 256, (V * Hd // 256, 144), generator=g, device=dev, dtype=torch.uint8)
                blk[:, :4] = torch.tensor([0x1e, 0x1c, 0x1e, 0x1c], dtype=torch.uint8, device=dev)  # d, dmin ~ 4e-3
                lm_w = blk.reshape(-1)
            else:
                lm_w = (torch.randn(V, Hd, generator=g, device=dev) * 0.05).to(torch.bfloat16)
            lm_sets[n_] = (lm_w, wf_, randn((1, Hd)), torch.empty(1, V, dtype=torch.float32, device=dev))
    moe_in = None
    if "moe" in only:  # Qwen3-30B-A3B's experts (H 2048, expert intermediate 768, 128 experts, top 8), bf16,
        # 256 rows (config 1's decode batch) routed from random logits; workspace allocated once
        mH, mI, mE, mK, mrows = 2048, 768, 128, 8, 256
        m_gu = (torch.randn(mE, 2 * mI, mH, generator=g, device=dev) * 0.05).to(torch.bfloat16)
        m_dn = (torch.randn(mE, mH, mI, generator=g, device=dev) * 0.05).to(torch.bfloat16)
        m_x = torch.randn(mrows, mH, generator=g, device=dev)
        m_idx, m_sc = ops.moe_route(torch.randn(mrows, mE, generator=g, device=dev), mK, True)
        m_slot = torch.arange(mE, dtype=torch.int32, device=dev)
        m_wb = ops.lib().nvf_moe_ffn_workspace_size(mrows, mH, mI, mK, mE)
        moe_in = dict(H=mH, I=mI, E=mE, K=mK, rows=mrows, gu=m_gu, dn=m_dn, x=m_x, idx=m_idx, sc=m_sc, slot=m_slot,
                      out=torch.zeros(mrows, mH, device=dev), work=torch.empty(m_wb, dtype=torch.uint8, device=dev),
                      wb=m_wb, experts=int(torch.unique(m_idx).numel()))
    if "split" in only:  # gate_up weights as GGUF blocks, rotated like the GEMV's
        nb_split = 2 * I * Hd // 32
        for _ in range(nsets(nbytes["split"])):
            split_sets.append((torch.randint(0, 256, (nb_split * 34,), generator=g, device=dev, dtype=torch.uint8),
                               torch.empty(nb_split * 32, dtype=torch.int8, device=dev),
                               torch.empty(nb_split, dtype=torch.int16, device=dev)))
    attn_in = attn_dec = None
    bs_kv = 256  # the reference's KV block size (a multiple of 256, config.hpp:254)
    if {"attn", "attn_f32"} & only:  # causal prefill over the config's sequences, KV already in the paged cache
        apos = cfg.positions()
        cu = cfg.cu_seqlens()
        lens = [int(n) for n in np.diff(cu)]
        # a sequence's cache holds every key its queries attend: max position + 1 (config 1's
        # one-token sequences sit at random positions, so this is not the sequence's length)
        sctx = [int(apos[cu[s_]:cu[s_ + 1]].max()) + 1 for s_ in range(len(lens))]
        nblk = [-(-n // bs_kv) for n in sctx]
        tables = torch.full((len(lens), max(nblk)), -1, dtype=torch.int32)
        perm = torch.randperm(sum(nblk), generator=torch.Generator().manual_seed(cfg.seed))
        o_ = 0
        for s_, nb in enumerate(nblk):
            tables[s_, :nb] = perm[o_:o_ + nb]
            o_ += nb
        rows = sum(nblk) * bs_kv
        attn_in = (randn((T, cfg.q_heads, cfg.head_dim)), randn((rows, cfg.kv_heads, cfg.head_dim)),
                   randn((rows, cfg.kv_heads, cfg.head_dim)),
                   torch.from_numpy(np.repeat(np.arange(len(lens), dtype=np.int32), lens)).to(dev),
                   torch.from_numpy((apos + 1).astype(np.int32)).to(dev), tables.to(dev))
        attn_flops = 4.0 * cfg.q_heads * cfg.head_dim * float((apos + 1).sum())
        # host-side guard before any kernel runs: every key a query attends has a block
        aseq = np.repeat(np.arange(len(lens)), lens)
        assert ((apos + 1) <= np.array(nblk)[aseq] * bs_kv).all(), "attention inputs: keys past the block tables"
    if {"attn_decode", "attn_decode_ordered", "attn_decode_f32"} & only:  # one token per sequence, 256 sequences, context uniform in 1..4096
        ctx = np.random.default_rng(cfg.seed + 11).integers(1, 4097, 256)
        nblk = [-(-int(n) // bs_kv) for n in ctx]
        tables = torch.full((256, max(nblk)), -1, dtype=torch.int32)
        perm = torch.randperm(sum(nblk), generator=torch.Generator().manual_seed(cfg.seed + 1))
        o_ = 0
        for s_, nb in enumerate(nblk):
            tables[s_, :nb] = perm[o_:o_ + nb]
            o_ += nb
        rows = sum(nblk) * bs_kv
        attn_dec = (randn((256, cfg.q_heads, cfg.head_dim)), randn((rows, cfg.kv_heads, cfg.head_dim)),
                    randn((rows, cfg.kv_heads, cfg.head_dim)), torch.arange(256, dtype=torch.int32, device=dev),
                    torch.from_numpy(ctx.astype(np.int32)).to(dev), tables.to(dev))
        dec_bytes = float(ctx.sum()) * cfg.kv_heads * cfg.head_dim * 2 * e + 2 * 256 * cfg.q_heads * cfg.head_dim * e
        dec_bytes32 = dec_bytes * 4 / e
        # the schedule an engine computes from the key counts it holds on the host
        dec_order = torch.from_numpy(ops.decode_token_order(ctx)).to(dev)
    attn_small = None
    if "attn_decode_small" in only:  # 4 sequences x 32768 keys of context: the split decode path
        sctx, sB = 32768, 4
        snb = sctx // bs_kv
        stab = torch.arange(sB * snb, dtype=torch.int32).view(sB, snb)
        stab = stab[:, torch.randperm(snb, generator=torch.Generator().manual_seed(cfg.seed + 3))].contiguous()
        srows = sB * snb * bs_kv
        attn_small = (randn((sB, cfg.q_heads, cfg.head_dim)), randn((srows, cfg.kv_heads, cfg.head_dim)),
                      randn((srows, cfg.kv_heads, cfg.head_dim)), torch.arange(sB, dtype=torch.int32, device=dev),
                      torch.full((sB,), sctx, dtype=torch.int32, device=dev), stab.to(dev))
        small_bytes = float(sB * sctx) * cfg.kv_heads * cfg.head_dim * 2 * e
    layer = None
    layer_dec = None
    layer_b1 = None
    if {"layer", "layer_decode", "layer_b1", "layer_b1_graph"} & only:  # one whole decoder layer on this library's kernels

        def q8w(n_, k_, lo=1e-3, hi=1e-2):  # random Q8_0 weight planes
            return (torch.randint(-127, 128, (n_ * k_,), generator=g, device=dev, dtype=torch.int8),
                    torch.empty(n_ * k_ // 32, device=dev).uniform_(lo, hi, generator=g).half().view(torch.int16))
        lw = {"w_in": randn((Hd,), 1.0, 0.1), "w_post": randn((Hd,), 1.0, 0.1),
              # (o adds into the residual on every call: small scales keep it within fp16)
              "qkv": q8w(qs + 2 * ks, Hd), "o": q8w(Hd, qs, 1e-5, 1e-4), "gu": q8w(2 * I, Hd), "down": q8w(Hd, I),
              # Qwen3 (config 3): per-head QK-norm gammas, no qkv bias (model.cpp:611-616);
              # Qwen2.5: the fp32 qkv bias (model.cpp:768-772), no QK-norm
              "qn": randn((cfg.head_dim,), 1.0, 0.1) if cfg.qk_norm else None,
              "kn": randn((cfg.head_dim,), 1.0, 0.1) if cfg.qk_norm else None,
              "bias": None if cfg.qk_norm else torch.randn(qs + 2 * ks, generator=g, device=dev) * 0.5}
        model_name = cfg.name.split(" ")[0].replace("qwen", "Qwen").replace("b", "B")

        def build_layer(lpos, lseq, seq_ctx, mql, seed):
            """Activations, a paged KV cache and metadata for tokens at positions lpos
            of sequences lseq (sequence s holds seq_ctx[s] keys once they are stored)."""
            n_ = len(lpos)
            lnb = [-(-int(c) // bs_kv) for c in seq_ctx]
            ltab = np.full((len(seq_ctx), max(lnb)), -1, np.int32)
            lperm = np.random.default_rng(seed).permutation(sum(lnb)).astype(np.int32)
            o_ = 0
            for s_, nb in enumerate(lnb):
                ltab[s_, :nb] = lperm[o_:o_ + nb]
                o_ += nb
            # host-side guard: every key a query attends has a block
            assert ((lpos + 1) <= np.array(lnb)[lseq] * bs_kv).all(), "layer inputs: keys past the block tables"
            lslots = (ltab[lseq, lpos // bs_kv].astype(np.int64) * bs_kv + lpos % bs_kv).astype(np.int32)
            lrows = sum(lnb) * bs_kv
            return dict(lw, T=n_, mql=mql, h=randn((n_, Hd)), r=randn((n_, Hd)), r2=torch.empty(n_, Hd, dtype=tdt, device=dev),
                        pos=torch.from_numpy(lpos.astype(np.int64)).to(dev),
                        kc=torch.zeros(lrows, cfg.kv_heads, cfg.head_dim, dtype=tdt, device=dev),
                        vc=torch.zeros(lrows, cfg.kv_heads, cfg.head_dim, dtype=tdt, device=dev),
                        qseq=torch.from_numpy(lseq.astype(np.int32)).to(dev),
                        qlen=torch.from_numpy((lpos + 1).astype(np.int32)).to(dev),
                        tab=torch.from_numpy(ltab).to(dev), slots=torch.from_numpy(lslots).to(dev),
                        qkv_out=torch.empty(n_, qs + 2 * ks, dtype=tdt, device=dev),
                        attn_out=torch.empty(n_, cfg.q_heads, cfg.head_dim, dtype=tdt, device=dev),
                        o_out=torch.empty(n_, Hd, dtype=tdt, device=dev),
                        gu_out=torch.empty(n_, 2 * I, dtype=tdt, device=dev),
                        down_out=torch.empty(n_, Hd, dtype=tdt, device=dev))

        def layer_flops(n_, lpos):
            return (2.0 * n_ * Hd * (qs + 2 * ks + 2 * I) + 2.0 * n_ * qs * Hd + 2.0 * n_ * I * Hd,
                    4.0 * cfg.q_heads * cfg.head_dim * float((lpos + 1).sum()))
        if "layer" in only:  # the config's prefill
            lpos = cfg.positions()
            lcu = cfg.cu_seqlens()
            llens = [int(n) for n in np.diff(lcu)]
            lseq = np.repeat(np.arange(len(llens), dtype=np.int32), llens)
            lctx = [int(lpos[lcu[s_]:lcu[s_ + 1]].max()) + 1 for s_ in range(len(llens))]  # keys each sequence holds
            layer = build_layer(lpos, lseq, lctx, 0, cfg.seed + 5)
            layer["cu"] = lcu  # the prefill's packing, held on the host like the engine's
            layer_ops, layer_attn_flops = layer_flops(T, lpos)
        if "layer_decode" in only:  # a decode step: 256 sequences, one new token each, context U[1, 4096]
            dctx = np.random.default_rng(cfg.seed + 7).integers(1, 4097, 256)
            layer_dec = build_layer(dctx - 1, np.arange(256), dctx, 1, cfg.seed + 8)
            # the decode kernel's schedule from the key counts the engine holds on the host
            layer_dec["order"] = torch.from_numpy(ops.decode_token_order(dctx)).to(dev)
            dec_ops, dec_attn_flops = layer_flops(256, dctx - 1)
            dec_kv_bytes = float(dctx.sum()) * cfg.kv_heads * cfg.head_dim * 2 * e
        if {"layer_b1", "layer_b1_graph"} & only:  # latency: one sequence, one new token, 4096 keys of context
            layer_b1 = build_layer(np.array([4095]), np.array([0]), [4096], 1, cfg.seed + 9)
    # the same inputs as fp32 caches (the reference's KV dtype; the drop-in's path)
    f32ize = (lambda tup: tuple(x.float() if x.is_floating_point() else x for x in tup))
    attn_in32 = f32ize(attn_in) if "attn_f32" in only else None
    attn_dec32 = f32ize(attn_dec) if "attn_decode_f32" in only else None
    copy_pair = None
    if {"copy", "copy12"} & only:  # 1 GiB plain copy: the attainable-bandwidth and traffic-counter reference
        copy_pair = (torch.ones(1 << 28, dtype=torch.int32, device=dev),
                     torch.empty(1 << 28, dtype=torch.int32, device=dev))
    # the gather's 1:2 read:write mix (nvf_stream_expand): 0.5 GiB in / 1 GiB out, and at the
    # gather's own size (T*H bytes in, T*H*2 out) rotating over >= 1 GiB of sets like the gather
    exp_sets = [(torch.ones(T * Hd // 4, dtype=torch.int32, device=dev), torch.empty(T * Hd // 2, dtype=torch.int32,
                                                                                    device=dev))
                for _ in range(nsets(3 * T * Hd))] if "copy12_emb" in only else []
    torch.cuda.synchronize()

    def run_emb(i):
        ids, out = emb_sets[i % len(emb_sets)]
        if emb_fmt == "q8_0":
            ops.embedding_q8_0(ids, w8, ws, Hd, V, out=out)
        elif emb_fmt == "q8_0_blocks":
            ops.embedding_q8_0_blocks(ids, blocks, Hd, V, out=out)
        elif emb_fmt == "f16":
            ops.embedding(ids, f16_table, V, out=out)
        else:
            kind = {"q4_k": ops.Q4_K, "q5_k": ops.Q5_K, "q6_k": ops.Q6_K}[emb_fmt]
            ops.embedding_qk(ids, blocks, Hd, kind, V, out=out)

    def run_rms(i):
        x, r, out = rms_sets[i % len(rms_sets)]
        ops.rms_norm_add(x, r, gamma, cfg.eps, out=out)

    def run_rope(i):
        q, k = rope_sets[i % len(rope_sets)]
        ops.qk_norm_rope(q, k, pos, qw, kw, inv, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.eps)

    def run_silu(i):
        gu, out = silu_sets[i % len(silu_sets)]
        ops.silu_and_mul(gu, out=out)

    def run_rms_q8(i):
        x, r, out, sc, q = q8_sets[i % len(q8_sets)]
        ops._check(ops.lib().nvf_rms_norm_q8(x.data_ptr(), r.data_ptr(), gamma.data_ptr(), out.data_ptr(),
                                             sc.data_ptr(), q.data_ptr(), T, Hd, cfg.eps, ops._dt(x), ops._stream()),
                   "rms_norm_q8")

    def run_emb_rms(i):
        ids, res, out = er_sets[i % len(er_sets)]
        fmt = {"q8_0": ops.EMB_Q8_0, "q8_0_blocks": ops.EMB_Q8_0_BLOCKS, "q4_k": ops.EMB_Q4_K,
               "q5_k": ops.EMB_Q5_K, "q6_k": ops.EMB_Q6_K}[emb_fmt]
        tab = w8 if emb_fmt == "q8_0" else blocks
        sc = ws if emb_fmt == "q8_0" else None
        ops._check(ops.lib().nvf_embedding_rms_norm(ids.data_ptr(), fmt, tab.data_ptr(),
                                                    sc.data_ptr() if sc is not None else None, T, Hd, V,
                                                    gamma.data_ptr(), res.data_ptr(), out.data_ptr(), cfg.eps,
                                                    ops._dt(out), ops._stream()), "embedding_rms_norm")

    def run_gemm(i):
        xq_, sc_, w8_, ws_, out_ = gemm_in
        ops.matmul_q8_0(xq_, sc_, w8_, ws_, 2 * I, out=out_)

    def run_silu_q8(i):
        gu, sc, q = sq_sets[i % len(sq_sets)]
        ops._check(ops.lib().nvf_silu_and_mul_q8(gu.data_ptr(), None, sc.data_ptr(), q.data_ptr(), T, I, ops._dt(gu),
                                                 ops._stream()), "silu_and_mul_q8")

    def run_gemv_shape(name):
        def f(i):
            xq_, sc_, sets_, n_, o_ = gemv_in[name]
            w8_, ws_ = sets_[i % len(sets_)]
            ops.matmul_q8_0(xq_, sc_, w8_, ws_, n_, out=o_)
        return f
    run_gemv = run_gemv_shape("gemv")

    def run_lm(name):
        def f(i):
            w_, wf_, x_, o_ = lm_sets[name]
            ops.matmul(x_, w_, V, wf_, out_dtype=torch.float32, out=o_)
        return f

    def run_moe(i):
        m = moe_in
        ops._check(ops.lib().nvf_moe_ffn_ws(m["x"].data_ptr(), ops._dt(m["x"]), m["idx"].data_ptr(), m["sc"].data_ptr(),
                                            m["gu"].data_ptr(), m["dn"].data_ptr(), 1, m["slot"].data_ptr(), m["rows"],
                                            m["H"], m["I"], m["K"], m["E"], m["out"].data_ptr(), ops._dt(m["out"]),
                                            m["work"].data_ptr(), m["wb"], ops._stream()), "moe_ffn")

    def run_split(i):
        blk_, w8_, ws_ = split_sets[i % len(split_sets)]
        ops._check(ops.lib().nvf_q8_0_split_blocks(blk_.data_ptr(), nb_split, w8_.data_ptr(), ws_.data_ptr(),
                                                   ops._stream()), "q8_0_split_blocks")

    def run_attn(i):
        q_, kc_, vc_, qs_, ql_, tb_ = attn_in
        # the engine holds the batch's cu_seqlens on the host (model_runner.cpp:43-128)
        ops.paged_attention(q_, kc_, vc_, qs_, ql_, tb_, bs_kv, cfg.head_dim ** -0.5, out=attn_out,
                            cu_seqlens=cfg.cu_seqlens())

    def run_attn_decode(i):
        q_, kc_, vc_, qs_, ql_, tb_ = attn_dec
        ops.paged_attention(q_, kc_, vc_, qs_, ql_, tb_, bs_kv, cfg.head_dim ** -0.5, out=dec_out, max_query_len=1)

    def run_attn_decode_ordered(i):
        q_, kc_, vc_, qs_, ql_, tb_ = attn_dec
        ops.paged_attention(q_, kc_, vc_, qs_, ql_, tb_, bs_kv, cfg.head_dim ** -0.5, out=dec_out, max_query_len=1,
                            token_order=dec_order)

    def run_attn_decode_small(i):
        q_, kc_, vc_, qs_, ql_, tb_ = attn_small
        ops.paged_attention(q_, kc_, vc_, qs_, ql_, tb_, bs_kv, cfg.head_dim ** -0.5, out=small_out, max_query_len=1)

    small_out = torch.empty_like(attn_small[0]) if attn_small is not None else None

    def run_layer_on(L_):
        # model.cpp:758-833's per-layer sequence: input RMSNorm (writing the qkv GEMM's int8 rows),
        # qkv, then in one launch the qkv bias (Qwen2.5) or the QK-norm (Qwen3), RoPE on the q and k
        # columns of the packed row and the KV store, paged attention, o (quantize + GEMM),
        # post-attention residual-add RMSNorm (int8 rows), gate_up, SwiGLU (int8 rows), down
        # (decode GEMV, n <= 16 rows: the input norm runs in the qkv GEMV's prologue, its
        # residual going to r2, and the o and down projections quantize their own rows; the
        # post-attention norm stays a launch of its own: fused into gate_up's 592 workgroups it
        # measured no faster)
        n_ = L_["T"]
        if n_ <= 16:
            qkv = ops.matmul_q8_0_rms(L_["h"], L_["w_in"], cfg.eps, *L_["qkv"], qs + 2 * ks, residual=L_["r"],
                                      residual_out=L_["r2"], out=L_["qkv_out"])
        else:
            _, sc, xq = ops.rms_norm_q8(L_["h"], L_["w_in"], cfg.eps, residual=L_["r"], want_out=False)
            qkv = ops.matmul_q8_0(xq, sc, *L_["qkv"], qs + 2 * ks, tdt, out=L_["qkv_out"])
        ops.qk_norm_rope_store_kv(qkv[:, :qs], qkv[:, qs:qs + ks], qkv[:, qs + ks:], L_["pos"], L_["qn"], L_["kn"],
                                  inv, cfg.q_heads, cfg.kv_heads, cfg.head_dim, L_["kc"], L_["vc"], L_["slots"],
                                  cfg.eps, qkv_bias=L_["bias"])
        att = ops.paged_attention(qkv[:, :qs].view(n_, cfg.q_heads, cfg.head_dim), L_["kc"], L_["vc"], L_["qseq"],
                                  L_["qlen"], L_["tab"], bs_kv, cfg.head_dim ** -0.5, out=L_["attn_out"],
                                  max_query_len=L_["mql"], cu_seqlens=L_.get("cu"), token_order=L_.get("order"),
                                  # decode: the split's partials in the static scratch (a scheduled
                                  # 256-sequence step never splits)
                                  noalloc=L_["mql"] == 1 and L_.get("order") is None)
        if n_ <= 16:
            o = ops.matmul_q8_0_act(att.view(n_, qs), *L_["o"], Hd, out=L_["o_out"])
        else:
            sc2, xq2 = ops.q8_quantize_rows(att.view(n_, qs))
            o = ops.matmul_q8_0(xq2, sc2, *L_["o"], Hd, tdt, out=L_["o_out"])
        _, sc3, xq3 = ops.rms_norm_q8(o, L_["w_post"], cfg.eps, residual=L_["r2"] if n_ <= 16 else L_["r"],
                                      want_out=False)
        gu = ops.matmul_q8_0(xq3, sc3, *L_["gu"], 2 * I, tdt, out=L_["gu_out"])
        if n_ <= 16:  # SwiGLU + its quantizer inside the down GEMV
            ops.matmul_q8_0_act(gu, *L_["down"], Hd, swiglu=True, out=L_["down_out"])
        else:
            _, sc4, xq4 = ops.silu_and_mul_q8(gu)
            ops.matmul_q8_0(xq4, sc4, *L_["down"], Hd, tdt, out=L_["down_out"])

    def run_layer(i):
        run_layer_on(layer)

    def run_layer_decode(i):
        run_layer_on(layer_dec)

    def run_layer_b1(i):
        run_layer_on(layer_b1)

    b1_graph = None
    if "layer_b1_graph" in only:  # the same step captured once into a HIP graph, then replayed
        cs = torch.cuda.Stream()
        cs.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cs):
            for _ in range(3):  # warm: one-time attribute calls and allocator pools before capture
                run_layer_on(layer_b1)
        torch.cuda.current_stream().wait_stream(cs)
        torch.cuda.synchronize()
        b1_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(b1_graph):
            run_layer_on(layer_b1)
        torch.cuda.synchronize()

    def run_layer_b1_graph(i):
        b1_graph.replay()

    def run_attn_f32(i):
        q_, kc_, vc_, qs_, ql_, tb_ = attn_in32
        ops.paged_attention(q_, kc_, vc_, qs_, ql_, tb_, bs_kv, cfg.head_dim ** -0.5, out=attn_out32)

    def run_attn_decode_f32(i):
        q_, kc_, vc_, qs_, ql_, tb_ = attn_dec32
        ops.paged_attention(q_, kc_, vc_, qs_, ql_, tb_, bs_kv, cfg.head_dim ** -0.5, out=dec_out32, max_query_len=1)

    attn_out32 = torch.empty_like(attn_in32[0]) if attn_in32 is not None else None
    dec_out32 = torch.empty_like(attn_dec32[0]) if attn_dec32 is not None else None
    attn_out = torch.empty_like(attn_in[0]) if attn_in is not None else None
    dec_out = torch.empty_like(attn_dec[0]) if attn_dec is not None else None

    def run_copy(i):
        ops.stream_copy(copy_pair[1], copy_pair[0])

    def run_copy12(i):
        ops.stream_expand(copy_pair[1], copy_pair[0][:1 << 27])

    def run_copy12_emb(i):
        src_, dst_ = exp_sets[i % len(exp_sets)]
        ops.stream_expand(dst_, src_)

    table = [("emb", run_emb), ("rms", run_rms), ("rope", run_rope), ("silu", run_silu), ("emb_rms", run_emb_rms),
             ("rms_q8", run_rms_q8), ("silu_q8", run_silu_q8), ("copy", run_copy),
             ("copy12", run_copy12), ("copy12_emb", run_copy12_emb), ("gemm", run_gemm),
             ("gemv", run_gemv), ("gemv_down", run_gemv_shape("gemv_down")), ("gemv_qkv", run_gemv_shape("gemv_qkv")),
             ("gemv_o", run_gemv_shape("gemv_o")), ("split", run_split), ("lm_head", run_lm("lm_head")),
             ("lm_head_q4k", run_lm("lm_head_q4k")), ("moe", run_moe), ("attn", run_attn), ("attn_decode", run_attn_decode),
             ("attn_decode_ordered", run_attn_decode_ordered),
             ("attn_f32", run_attn_f32), ("attn_decode_f32", run_attn_decode_f32), ("attn_decode_small", run_attn_decode_small),
             ("layer", run_layer), ("layer_decode", run_layer_decode), ("layer_b1", run_layer_b1),
             ("layer_b1_graph", run_layer_b1_graph)]
    active = [(n, f) for n, f in table if n in only]

    for i in range(args.warmup):
        for _, f in active:
            f(i)
    torch.cuda.synchronize()

    # Per-op timing.  The GPU is first held by a spin kernel (torch.cuda._sleep) while the
    # host enqueues n >= 200 launches in groups of 25 with an event between groups, so the
    # launches then run back to back with no host gap between them (a Python launch costs
    # ~15-25 us of host time, more than some of these kernels take).  "us" is the mean over
    # all n launches, "p50_us" the median of the 8 groups' mean launch times (the timing rule),
    # p10/p90 their spread.  An op whose enqueue outran the spin is retried with a longer
    # spin; "eager_us" is the plain back-to-back mean with the host in the loop.
    stream = torch.cuda.current_stream()
    res_ops = {}
    act_name = {H.F16: "fp16", H.BF16: "bf16", H.F32: "fp32"}[dt]
    _lens = np.diff(cfg.cu_seqlens())
    batch_desc = (f"{len(_lens)} one-token queries at random positions" if int(_lens.max()) == 1
                  else f"causal prefill {len(_lens)} x {T // len(_lens)} tokens")
    group = 25
    n_launch = -(-max(args.steps, 200) // group) * group
    cyc_per_us = sleep_rate(torch, stream)
    for n, f in active:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record(stream)
        for i in range(args.steps):
            f(args.warmup + i)
        b.record(stream)
        b.synchronize()
        eager_us = a.elapsed_time(b) * 1e3 / args.steps
        if n == "layer_b1":  # host in the loop by design: eager launches (against layer_b1_graph's replays)
            per, t_us = None, eager_us
        else:
            per, ahead = timed_launches(torch, stream, f, args.warmup, n_launch, cyc_per_us, group)
            t_us = float(per.mean())
        entry = {"us": round(t_us, 2)}
        if per is not None and not ahead:
            entry["host_bound"] = True
        if per is not None:
            entry.update({"p10_us": round(float(np.percentile(per, 10)), 2),
                          "p50_us": round(float(np.percentile(per, 50)), 2),
                          "p90_us": round(float(np.percentile(per, 90)), 2), "launches": n_launch,
                          "p_over": f"groups of {group} back-to-back launches",
                          "eager_us": round(eager_us, 2)})
        if n in nbytes:
            gbs = nbytes[n] / (t_us * 1e-6) / 1e9
            entry.update({"bytes": nbytes[n], "GB_s": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
                          "frac_of_peak_p50": round(nbytes[n] / (entry["p50_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                          "tokens_per_s": round(T / (t_us * 1e-6), 1)})
        if n in gemv_in:
            entry.pop("tokens_per_s")
            gnn, gk, gproj = gemv_shapes(cfg)[n]
            entry["shape"] = f"m={GEMV_M} n={gnn} k={gk} ({gproj}, decode)"
        elif n == "moe":
            m = moe_in
            wbytes = m["experts"] * 3 * m["H"] * m["I"] * 2
            flops = 2.0 * m["rows"] * m["K"] * 3 * m["H"] * m["I"]
            entry.update({"shape": f"MoE FFN, {m['rows']} rows, top {m['K']} of {m['E']} experts, H {m['H']}, expert "
                                   f"intermediate {m['I']}, bf16 experts, fp32 activations (Qwen3-30B-A3B's shape)",
                          "expert_weight_GB_s": round(wbytes / (t_us * 1e-6) / 1e9, 1),
                          "TFLOP_s": round(flops / (t_us * 1e-6) / 1e12, 1),
                          "frac_of_fp32_peak": round(flops / (t_us * 1e-6) / FP32_PEAK_FLOPS, 4)})
        elif n in ("lm_head", "lm_head_q4k"):
            entry.pop("tokens_per_s")
            entry["shape"] = (f"m=1 n={V} k={Hd} (LM head at decode, {'Q4_K' if n == 'lm_head_q4k' else 'bf16'} "
                              "weights, fp32 logits)")
        elif n == "split":
            entry.pop("tokens_per_s")
            entry["shape"] = f"{2 * I * Hd // 32} Q8_0 blocks (gate_up [{2 * I}, {Hd}])"
        elif n == "gemm":
            ops_n = 2.0 * T * (2 * I) * Hd
            entry.update({"shape": f"m={T} n={2 * I} k={Hd} (gate_up)", "TOP_s": round(ops_n / (t_us * 1e-6) / 1e12, 1),
                          "frac_of_int8_peak": round(ops_n / (t_us * 1e-6) / INT8_PEAK_OPS, 4)})
        elif n == "attn":
            entry.update({"shape": f"{batch_desc}, {cfg.q_heads}/{cfg.kv_heads} heads x {cfg.head_dim}, KV block {bs_kv}",
                          "TFLOP_s": round(attn_flops / (t_us * 1e-6) / 1e12, 1),
                          "frac_of_16bit_peak": round(attn_flops / (t_us * 1e-6) / 2.5e15, 4)})
        elif n == "attn_f32":
            entry.update({"shape": f"as attn, fp32 cache and activations (the drop-in hip_paged_attention)",
                          "TFLOP_s": round(attn_flops / (t_us * 1e-6) / 1e12, 1),
                          "frac_of_fp32_peak": round(attn_flops / (t_us * 1e-6) / FP32_PEAK_FLOPS, 4)})
        elif n in ("attn_decode", "attn_decode_ordered", "attn_decode_f32"):
            db = dec_bytes32 if n == "attn_decode_f32" else dec_bytes
            entry.update({"shape": f"decode 256 sequences, context uniform in 1..4096, {cfg.q_heads}/{cfg.kv_heads} "
                                   f"heads x {cfg.head_dim}" + (", fp32 cache" if n == "attn_decode_f32" else "") +
                                   (", host-computed token order (nvf_decode_token_order)"
                                    if n == "attn_decode_ordered" else ""),
                          "bytes": int(db), "GB_s": round(db / (t_us * 1e-6) / 1e9, 1),
                          "frac_of_peak": round(db / (t_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        elif n == "attn_decode_small":
            entry.update({"shape": f"decode 4 sequences x 32768 keys, {cfg.q_heads}/{cfg.kv_heads} heads x "
                                   f"{cfg.head_dim} (split decode)", "bytes": int(small_bytes),
                          "GB_s": round(small_bytes / (t_us * 1e-6) / 1e9, 1),
                          "frac_of_peak": round(small_bytes / (t_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        elif n == "layer_decode":
            entry.update({"shape": f"one {model_name} decoder layer, decode step of 256 sequences (context U[1, 4096]), "
                                   f"Q8_0 weights, {act_name} activations and KV cache",
                          "tokens_per_s": round(256 / (t_us * 1e-6), 1),
                          "weights_and_kv_GB_s": round((dec_ops / 2 / 256 * 34 / 32 + dec_kv_bytes) / (t_us * 1e-6) / 1e9,
                                                       1)})
        elif n in ("layer_b1", "layer_b1_graph"):
            entry["shape"] = (f"one {model_name} decoder layer, decode step of 1 sequence with 4096 keys of context"
                              + (", replayed from a captured HIP graph" if n == "layer_b1_graph" else ", eager launches"))
        elif n == "layer":
            entry.update({"shape": f"one {model_name} decoder layer, {T} tokens ({batch_desc}), Q8_0 weights, "
                                   f"{act_name} activations and KV cache",
                          "tokens_per_s": round(T / (t_us * 1e-6), 1),
                          "gemm_TOP_s": round(layer_ops / (t_us * 1e-6) / 1e12, 1),
                          "effective_TOP_s_incl_attention": round((layer_ops + layer_attn_flops) / (t_us * 1e-6) / 1e12, 1)})
        elif n in ("copy", "copy12", "copy12_emb"):
            nb = {"copy": 2 << 30, "copy12": 3 << 29, "copy12_emb": 3 * T * Hd}[n]
            entry.update({"bytes": nb, "GB_s": round(nb / (t_us * 1e-6) / 1e9, 1),
                          "frac_of_peak": round(nb / (t_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        res_ops[n] = entry

    # The step: the whole chain, `steps` times, bracketed by synchronize + events.
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    a.record(stream)
    for i in range(args.steps):
        for n, f in active:
            if n in ("emb", "rms", "rope", "silu"):
                f(args.warmup + i)
    b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_us = a.elapsed_time(b) * 1e3 / args.steps

    chain_ops = [n for n in ("emb", "rms", "rope", "silu") if n in res_ops]
    ms_per_step = wall / args.steps * 1e3
    dom = max(chain_ops, key=lambda n: nbytes[n]) if chain_ops else None
    roofline = None
    if dom:
        roofline = {"kernel": {"emb": "embedding", "rms": "rms_norm_add", "rope": "qk_norm_rope",
                               "silu": "silu_and_mul"}[dom],
                    "bound": "hbm", "achieved": res_ops[dom]["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": res_ops[dom]["frac_of_peak"], "traffic": traffic_from_profiles(dom, args.config)}

    cpu = (cpu_baseline(cfg, args.cpu_seconds, H)
           if args.cpu_seconds > 0 and chain_ops == ["emb", "rms", "rope", "silu"] and emb_fmt == cfg.emb else None)

    line = {
        "metric": METRIC,
        "value": round(T / (step_us * 1e-6), 1) if chain_ops else None,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {H.F16: "f16", H.BF16: "bf16", H.F32: "f32"}[dt],
        "data": "synthetic (seeded; BASELINE value distributions)",
        "config": {"workload": f"BASELINE config {args.config}: {cfg.name}; one step = "
                               f"{emb_fmt} embedding gather + residual-add RMSNorm + "
                               f"{'QK-norm + ' if cfg.qk_norm else ''}NeoX RoPE q/k + SwiGLU",
                   "tokens": T, "hidden": Hd, "intermediate": I, "vocab": V, "q_heads": cfg.q_heads,
                   "kv_heads": cfg.kv_heads, "head_dim": cfg.head_dim, "value_is": "tokens / GPU time of one step (HIP events around all timed steps)",
                   "step_us": round(step_us, 2)},
        "ops": {k: v for k, v in res_ops.items() if k in ("emb", "rms", "rope", "silu")},
        "fused_ops": {k: v for k, v in res_ops.items() if k in ("emb_rms", "rms_q8", "silu_q8")} or None,
        "attainable": ({"kernel": "nvf_stream_copy (1 GiB, 16 B non-temporal loads/stores)",
                        "GB_s": res_ops["copy"]["GB_s"],
                        "frac_of_peak": round(res_ops["copy"]["GB_s"] / HBM_PEAK_GBS, 4),
                        **({"read1_write2_1GiB": {k_: res_ops["copy12"][k_] for k_ in ("us", "GB_s", "frac_of_peak")}}
                           if "copy12" in res_ops else {}),
                        **({"read1_write2_at_emb_size": {k_: res_ops["copy12_emb"][k_]
                                                         for k_ in ("us", "GB_s", "frac_of_peak")}}
                           if "copy12_emb" in res_ops else {})}
                       if "copy" in res_ops else None),
        "roofline": roofline,
        "q8_gemm": res_ops.get("gemm"),
        "q8_gemv": res_ops.get("gemv"),
        "q8_gemv_shapes": {k: res_ops[k] for k in ("gemv_down", "gemv_qkv", "gemv_o") if k in res_ops} or None,
        "q8_0_split": res_ops.get("split"),
        "weight_gemv": {k: res_ops[k] for k in ("lm_head", "lm_head_q4k") if k in res_ops} or None,
        "moe_ffn": res_ops.get("moe"),
        "layer": res_ops.get("layer"),
        "layer_decode": res_ops.get("layer_decode"),
        "layer_b1": res_ops.get("layer_b1"),
        "layer_b1_graph": res_ops.get("layer_b1_graph"),
        "paged_attention": {k: res_ops[k] for k in ("attn", "attn_decode", "attn_decode_ordered", "attn_f32",
                                                    "attn_decode_f32",
                                                    "attn_decode_small") if k in res_ops} or None,
        "cpu_baseline": cpu,
    }
    extra = [int(c_) for c_ in args.configs.split(",") if c_.strip() != "" and int(c_) != args.config]
    if extra and chain_ops == ["emb", "rms", "rope", "silu"] and not args.emb:
        # free the headline's sets first: config 4's SwiGLU alone holds ~7 GB
        del emb_sets, rms_sets, rope_sets, silu_sets
        torch.cuda.empty_cache()
        line["configs"] = {f"c{c_}": bench_chain(c_, args, torch, ops, H, stream, cyc_per_us, group, n_launch)
                           for c_ in extra}
    print(json.dumps(line), flush=True)
    return 0


def bench_chain(ci: int, args, torch, ops, H, stream, cyc_per_us: float, group: int, n_launch: int) -> dict:
    """The four chain ops of BASELINE config ci at its full size, inputs resident in HBM and
    rotated over >= 1 GiB per op like the headline's, timed the same way (timed_launches);
    then the chain back to back for `steps` steps, and the C oracle on this host
    (cpu_baseline: config 0's whole 64-token chain, the others a bounded sample)."""
    cfg = H.CONFIGS[ci]
    dev = torch.device("cuda:0")
    tdt = H.torch_dtype(cfg.dtype)
    e = 2 if cfg.dtype != H.F32 else 4
    T, Hd, I, V = cfg.tokens, cfg.hidden, cfg.inter, cfg.vocab
    qs, ks = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    g = torch.Generator(device=dev).manual_seed(cfg.seed)
    nbytes = op_bytes(cfg, e, cfg.emb)

    def nsets(b: int) -> int:
        return max(2, -(-POOL_BYTES // b))

    def randn(shape, mean=0.0, std=1.0):
        return (torch.randn(shape, generator=g, device=dev) * std + mean).to(tdt)

    if cfg.emb == "q8_0":
        w8 = torch.randint(-127, 128, (V * Hd,), generator=g, device=dev, dtype=torch.int8)
        ws = torch.empty(V * Hd // 32, device=dev).uniform_(1e-3, 1e-2, generator=g).half().view(torch.int16)
    else:
        blocks = torch.from_numpy(H.gen_q4_k(np.random.default_rng(cfg.seed), V * Hd // 256)).to(dev)
    sets = {
        "emb": [(torch.randint(0, V, (T,), generator=g, device=dev), torch.empty(T, Hd, dtype=tdt, device=dev))
                for _ in range(nsets(nbytes["emb"]))],
        "rms": [(randn((T, Hd)), randn((T, Hd)), torch.empty(T, Hd, dtype=tdt, device=dev))
                for _ in range(nsets(nbytes["rms"]))],
        "rope": [(randn((T, qs)), randn((T, ks))) for _ in range(nsets(nbytes["rope"]))],
        "silu": [(randn((T, 2 * I)), torch.empty(T, I, dtype=tdt, device=dev)) for _ in range(nsets(nbytes["silu"]))],
    }
    gamma = randn((Hd,), 1.0, 0.1)
    pos = torch.from_numpy(cfg.positions()).to(dev)
    inv = ops.rope_inv_freq(cfg.theta, cfg.head_dim, dev)
    qw = randn((cfg.head_dim,), 1.0, 0.1) if cfg.qk_norm else None
    kw = randn((cfg.head_dim,), 1.0, 0.1) if cfg.qk_norm else None

    def run_emb(i):
        ids, out = sets["emb"][i % len(sets["emb"])]
        if cfg.emb == "q8_0":
            ops.embedding_q8_0(ids, w8, ws, Hd, V, out=out)
        else:
            ops.embedding_qk(ids, blocks, Hd, ops.Q4_K, V, out=out)

    def run_rms(i):
        x, r, out = sets["rms"][i % len(sets["rms"])]
        ops.rms_norm_add(x, r, gamma, cfg.eps, out=out)

    def run_rope(i):
        q, k = sets["rope"][i % len(sets["rope"])]
        ops.qk_norm_rope(q, k, pos, qw, kw, inv, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.eps)

    def run_silu(i):
        gu, out = sets["silu"][i % len(sets["silu"])]
        ops.silu_and_mul(gu, out=out)

    fns = {"emb": run_emb, "rms": run_rms, "rope": run_rope, "silu": run_silu}
    for i in range(args.warmup):
        for f in fns.values():
            f(i)
    torch.cuda.synchronize()
    res = {}
    for n, f in fns.items():
        per, ahead = timed_launches(torch, stream, f, args.warmup, n_launch, cyc_per_us, group)
        t_us, p50 = float(per.mean()), float(np.percentile(per, 50))
        gbs = nbytes[n] / (t_us * 1e-6) / 1e9
        res[n] = {"us": round(t_us, 2), "p50_us": round(p50, 2), "bytes": nbytes[n], "GB_s": round(gbs, 1),
                  "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
                  "frac_of_peak_p50": round(nbytes[n] / (p50 * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                  "tokens_per_s": round(T / (t_us * 1e-6), 1), **({} if ahead else {"host_bound": True})}
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for i in range(args.steps):
        for f in fns.values():
            f(args.warmup + i)
    b.record(stream)
    torch.cuda.synchronize()
    step_us = a.elapsed_time(b) * 1e3 / args.steps
    del sets
    if cfg.emb == "q8_0":
        del w8, ws
    else:
        del blocks
    torch.cuda.empty_cache()
    out = {"workload": f"BASELINE config {ci}: {cfg.name}; {cfg.emb} embedding gather + residual-add RMSNorm + "
                       f"{'QK-norm + ' if cfg.qk_norm else ''}NeoX RoPE q/k + SwiGLU",
           "tokens": T, "dtype": {H.F16: "f16", H.BF16: "bf16", H.F32: "f32"}[cfg.dtype],
           "step_us": round(step_us, 2), "tokens_per_s": round(T / (step_us * 1e-6), 1), "ops": res}
    if args.cpu_seconds > 0:
        # config 0 is the CPU reference's own case: its whole chain (all 64 tokens, the full table)
        out["cpu_baseline"] = cpu_baseline(cfg, 3.0 if ci == 0 else 2.0, H, full=ci == 0, all_cores=ci == 0)
        out["gpu_over_cpu"] = round(out["tokens_per_s"] / out["cpu_baseline"]["value"], 1)
    return out


def sleep_rate(torch, stream) -> float:
    """Spin-kernel cycles per microsecond (torch.cuda._sleep), measured with events."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(1000)  # load the kernel
    torch.cuda.synchronize()
    a.record(stream)
    torch.cuda._sleep(1_000_000)
    b.record(stream)
    b.synchronize()
    return 1_000_000 / (a.elapsed_time(b) * 1e3)


def timed_launches(torch, stream, f, first: int, n: int, cyc_per_us: float, group: int = 25):
    """n launches f(first), f(first + 1), ... (n a multiple of group) run back to back
    behind a spin kernel that holds the GPU while the host enqueues them.  An event
    sits between groups of `group` launches only (an event record between every two
    launches adds ~2 us to each).  Returns the mean launch time of each group (us) and
    whether the GPU stayed behind the host.  If the GPU reached the first event before
    the host finished enqueueing, the spin was too short: retry with a longer one; a
    host slower still (under a tracing profiler) gives the last attempt's groups, marked
    host-bound."""
    import time as _t
    host_us = 0.0
    ng = n // group
    groups = None
    for _attempt in range(6):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(ng + 1)]
        torch.cuda.synchronize()
        # spin for twice the host time of the previous attempt (or 2 ms), at most 200 ms
        spin_us = min(200_000.0, max(2_000.0, 2.0 * host_us))
        torch.cuda._sleep(int(spin_us * cyc_per_us))
        t0 = _t.perf_counter()
        for g_ in range(ng):
            evs[g_].record(stream)
            for i in range(group):
                f(first + g_ * group + i)
        evs[ng].record(stream)
        host_us = (_t.perf_counter() - t0) * 1e6
        overran = evs[0].query()  # the GPU already passed the first event: the spin ended too early
        evs[ng].synchronize()
        groups = np.array([evs[g_].elapsed_time(evs[g_ + 1]) * 1e3 / group for g_ in range(ng)])
        if not overran:
            return groups, True
    print("timed_launches: the host could not stay ahead of the GPU; groups marked host-bound", file=sys.stderr)
    return groups, False

# the chain's kernels as rocprofv3 names them (prefix of the mangled name) -> bench op
CHAIN_KERNELS = {"emb": "_ZN3nvf17embed_rows_kernel", "rms": "_ZN3nvf19rms_norm_vec_kernel",
                 "rope": "_ZN3nvf19qk_norm_rope_kernel", "silu": "_ZN3nvf19silu_mul_vec_kernel",
                 "copy": "nvf::stream_copy_kernel"}
LIB_PATH = ROOT / "nano_vllm_cpp_amd" / "lib" / "libnvf_ops.so"


def _kernel_in_library(name: str) -> bool:
    """True if the built library holds a kernel of this (mangled) name: its code object
    names each kernel's descriptor, so the bytes of the name appear in the .so."""
    try:
        return name.encode() in LIB_PATH.read_bytes()
    except OSError:
        return False


def traffic_from_profiles(op: str, config: int):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary,
    or None when there is none for this op, or when the kernel it was counted on is not
    a kernel of the library built now (a summary of an older binary is not used)."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        e = json.loads(f.read_text()).get(f"c{config}", {}).get(op, {})
    except (ValueError, AttributeError):
        return None
    name = e.get("kernel", "")
    if not name or not _kernel_in_library(name):
        return None
    return e.get("hbm_bytes_per_launch")


def write_traffic(prof_dir: str, config: int, source_commit: str = "") -> dict:
    """Builds profiles/traffic.json from two rocprofv3 passes over the chain and the copy,
    <prof_dir>/FETCH_SIZE/*counter_collection.csv and <prof_dir>/WRITE_SIZE/..., made by
      rocprofv3 --pmc FETCH_SIZE -f csv -d <prof_dir>/FETCH_SIZE -o FETCH_SIZE -- \
          python3 bench.py --config <c> --only emb,rms,rope,silu,copy --steps 10 --warmup 2 --cpu-seconds 0
    (and the same with WRITE_SIZE).  Per op: the mean counter over the dispatches of the
    op's kernel at its largest grid (the bench's launch), scaled by what the counter reads
    for the 1 GiB copy against the bytes it moves.  Records the source commit."""
    import csv
    import subprocess

    cfg_ops = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        files = sorted(Path(prof_dir, counter).glob("*counter_collection.csv"))
        if not files:
            raise SystemExit(f"no {counter} counter_collection.csv under {prof_dir}/{counter}")
        per = {}
        for row in csv.DictReader(open(files[0])):
            if row["Counter_Name"] != counter:
                continue
            for op, prefix in CHAIN_KERNELS.items():
                if row["Kernel_Name"].startswith(prefix):
                    per.setdefault(op, {}).setdefault(int(row["Grid_Size"]), (row["Kernel_Name"], []))[1].append(
                        float(row["Counter_Value"]))
        for op, grids in per.items():
            g = max(grids)
            name, vals = grids[g]
            cfg_ops.setdefault(op, {"kernel": name, "grid": g})[counter] = sum(vals) / len(vals)
    copy_bytes = 1 << 30
    cal = cfg_ops.pop("copy")
    ff = copy_bytes / (cal["FETCH_SIZE"] * 1024)
    wf = copy_bytes / (cal["WRITE_SIZE"] * 1024)
    from tests import harness as H
    cfg = H.CONFIGS[config]
    alg = op_bytes(cfg, 2 if cfg.dtype != H.F32 else 4, cfg.emb)
    try:
        head = subprocess.run(["git", "-C", str(ROOT), "rev-parse", "HEAD"], capture_output=True, text=True,
                              check=True).stdout.strip()
        dirty = bool(subprocess.run(["git", "-C", str(ROOT), "status", "--porcelain", "--", "nano_vllm_cpp_amd/csrc"],
                                    capture_output=True, text=True).stdout.strip())
    except (OSError, subprocess.CalledProcessError):
        head, dirty = "unknown", True
    out = {"_source": {"commit": head, "kernel_sources_modified": dirty,
                       "command": "rocprofv3 --pmc <FETCH_SIZE|WRITE_SIZE> -f csv -d <dir>/<counter> -o <counter> -- "
                                  f"python3 bench.py --config {config} --only emb,rms,rope,silu,copy --steps 10 "
                                  "--warmup 2 --cpu-seconds 0 --configs ''"},
           "_calibration": {"reference": "nvf_stream_copy of 1 GiB (16 B non-temporal loads/stores)",
                            "copy_fetch_kib": round(cal["FETCH_SIZE"], 1), "copy_write_kib": round(cal["WRITE_SIZE"], 1),
                            "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)},
           "_note": "hbm_bytes_per_launch = FETCH_SIZE[KiB]*1024*fetch_factor + WRITE_SIZE[KiB]*1024*write_factor"}
    entry = {}
    if source_commit:  # the profiled tree's commit, given; its kernel sources compared with the working tree's
        try:
            head = subprocess.run(["git", "-C", str(ROOT), "rev-parse", source_commit], capture_output=True,
                                  text=True, check=True).stdout.strip()
            dirty = subprocess.run(["git", "-C", str(ROOT), "diff", "--quiet", head, "--", "nano_vllm_cpp_amd/csrc"],
                                   capture_output=True).returncode != 0
        except (OSError, subprocess.CalledProcessError):
            head, dirty = source_commit, None
        out["_source"].update({"commit": head, "kernel_sources_modified": dirty})
    for op, d in sorted(cfg_ops.items()):
        hbm = d["FETCH_SIZE"] * 1024 * ff + d["WRITE_SIZE"] * 1024 * wf
        entry[op] = {"kernel": d["kernel"], "grid": d["grid"], "fetch_kib_raw": round(d["FETCH_SIZE"], 1),
                     "write_kib_raw": round(d["WRITE_SIZE"], 1), "hbm_bytes_per_launch": int(hbm),
                     "algorithmic_bytes": alg[op], "ratio_to_algorithmic": round(hbm / alg[op], 4)}
    f = ROOT / "profiles" / "traffic.json"
    try:
        whole = json.loads(f.read_text())
    except (OSError, ValueError):
        whole = {}
    whole.update({k: v for k, v in out.items()})
    whole[f"c{config}"] = entry
    f.write_text(json.dumps(whole, indent=1) + "\n")
    return whole


def cpu_chain_sample(cfg, H, seed: int, full: bool = False, table=None):
    """Buffers for one S-token sample of the chain and a function running it once
    through the C oracle; returns (run, S, table).  run() returns the four ops' seconds.
    full: the config's own tokens (all of them) over its whole table.  table: the
    embedding table of an earlier call to share (threads read it, none writes it)."""
    o = H.oracle()
    r = np.random.default_rng(seed)
    S = cfg.tokens if full else min(256, cfg.tokens)  # sample tokens per chain call
    Hd, I, dt = cfg.hidden, cfg.inter, cfg.dtype
    # gathered rows come from a 4096-row slice of the table (same per-row work), or the whole table
    Vs = cfg.vocab if full else 4096
    ids = r.integers(0, Vs, S).astype(np.int64)
    if table is None:
        table = H.gen_q8_0(r, Vs, Hd) if cfg.emb == "q8_0" else H.gen_q4_k(r, Vs * Hd // 256)
    if cfg.emb == "q8_0":
        w8, ws = table
    else:
        blocks = table
    emb = np.empty((S, Hd), H.NP_STORAGE[dt])
    x, res = H.gen_act(r, (S, Hd), dt), H.gen_act(r, (S, Hd), dt)
    w = H.gen_act(r, (Hd,), dt, 1.0, 0.1)
    out = np.empty_like(x)
    qs, ks = cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    q, k = H.gen_act(r, (S, qs), dt), H.gen_act(r, (S, ks), dt)
    pos = np.ascontiguousarray(cfg.positions()[:S])
    inv = np.empty(cfg.head_dim // 2, np.float32)
    o.orc_inv_freq(cfg.theta, cfg.head_dim, H.ptr(inv))
    qw = H.gen_act(r, (cfg.head_dim,), dt, 1.0, 0.1) if cfg.qk_norm else None
    kw = H.gen_act(r, (cfg.head_dim,), dt, 1.0, 0.1) if cfg.qk_norm else None
    gu = H.gen_act(r, (S, 2 * I), dt)
    so = np.empty((S, I), H.NP_STORAGE[dt])

    def run():
        t = time.perf_counter()
        if cfg.emb == "q8_0":
            o.orc_embedding_q8_split(H.ptr(ids), H.ptr(w8), H.ptr(ws), S, Hd, H.ptr(emb), dt)
        else:
            o.orc_embedding_qk(H.ptr(ids), H.ptr(blocks), S, Hd, 12, H.GGML, H.ptr(emb), dt)
        t1 = time.perf_counter()
        o.orc_rms_norm_add(H.ptr(x), H.ptr(res), H.ptr(w), H.ptr(out), S, Hd, cfg.eps, dt)
        t2 = time.perf_counter()
        o.orc_qk_norm_rope(H.ptr(q), H.ptr(k), H.ptr(pos), H.ptr(qw), H.ptr(kw), H.ptr(inv), S, cfg.q_heads,
                           cfg.kv_heads, cfg.head_dim, qs, ks, cfg.eps, dt)
        t3 = time.perf_counter()
        o.orc_silu_and_mul(H.ptr(gu), H.ptr(so), S, I, dt)
        t4 = time.perf_counter()
        return t1 - t, t2 - t1, t3 - t2, t4 - t3

    return run, S, table


def cpu_baseline(cfg, budget_s: float, H, full: bool = False, all_cores: bool = True) -> dict:
    """The C oracle (scalar, 1 thread, -O2) on a bounded sample of the same chain (full:
    the config's whole chain, repeated), then the same oracle on every host core the box
    gives this job (threads, each on its own sample; ctypes releases the GIL), reported
    under "all_cores"."""
    run, S, table = cpu_chain_sample(cfg, H, cfg.seed, full)
    per = {"emb": 0.0, "rms": 0.0, "rope": 0.0, "silu": 0.0}
    calls = 0
    t_start = time.perf_counter()
    while True:
        d = run()
        for k_, v in zip(per, d):
            per[k_] += v
        calls += 1
        if time.perf_counter() - t_start >= budget_s:
            break
    total = sum(per.values())
    e = 2 if cfg.dtype != H.F32 else 4
    scale = {k_: v * S / cfg.tokens for k_, v in op_bytes(cfg, e, cfg.emb).items()}  # bytes of one S-token call
    cpu_model = ""
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                cpu_model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    result = {"value": round(calls * S / total, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
              "sample": f"{calls} x the {S}-token chain of the same config ("
                        f"{'the whole table' if full else 'table rows from a 4096-row slice'}), "
                        f"{total:.1f} s of single-thread C oracle (-O2) on {cpu_model or 'this host'}, "
                        f"nproc={os.cpu_count()}",
              "ops_GB_s": {k_: round(scale[k_] * calls / per[k_] / 1e9, 3) for k_ in per}}

    if not all_cores:
        return result
    # all cores: at most 16 threads (the box's CPU share per GPU), half the budget
    import concurrent.futures as cf
    n = max(1, min(16, os.cpu_count() or 1))
    runs = [cpu_chain_sample(cfg, H, cfg.seed + 1 + i, full, table)[0] for i in range(n)]
    all_budget = budget_s / 2

    def worker(fn):
        c, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < all_budget:
            fn()
            c += 1
        return c

    t0 = time.perf_counter()
    with cf.ThreadPoolExecutor(max_workers=n) as ex:
        counts = list(ex.map(worker, runs))
    wall = time.perf_counter() - t0
    result["all_cores"] = {"value": round(sum(counts) * S / wall, 1), "unit": "tokens/s", "cores": n,
                           "kind": "port",
                           "sample": f"{sum(counts)} x the {S}-token chain over {n} threads, {wall:.1f} s wall"}
    return result


if __name__ == "__main__":
    sys.exit(main())
