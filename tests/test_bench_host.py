"""Host-side legs of bench.py that run without a GPU: the algorithmic byte
model and the CPU baseline (the oracle timed on a bounded sample)."""
from __future__ import annotations

import subprocess
import sys

import pytest

import bench
from tests import harness as H


@pytest.mark.parametrize("fmt", sorted(bench.TABLE_BYTES_PER_ELEM))
def test_op_bytes_all_formats(fmt):
    cfg = H.CONFIGS[2]
    b = bench.op_bytes(cfg, 2, fmt)
    assert set(b) == {"emb", "rms", "rope", "silu", "emb_rms", "rms_q8", "silu_q8", "gemv", "gemv_down", "gemv_qkv",
                      "gemv_o", "split", "lm_head", "lm_head_q4k"}
    # a decode GEMV streams its Q8_0 weights once (34 bytes per 32) plus m int8 rows, their
    # scales and m fp16 output rows; down is [hidden, inter], o is [hidden, q heads x head_dim]
    m, Hd, I = bench.GEMV_M, cfg.hidden, cfg.inter
    assert b["gemv_down"] == Hd * I // 32 * 34 + m * I + 4 * m + m * Hd * 2
    qd = cfg.q_heads * cfg.head_dim
    assert b["gemv_o"] == Hd * qd // 32 * 34 + m * qd + 4 * m + m * Hd * 2
    assert b["gemv"] == 2 * I * Hd // 32 * 34 + m * Hd + 4 * m + m * 2 * I * 2
    # the decode LM head streams the [vocab, hidden] weights once: 2 bytes (bf16) or 144 per 256 (Q4_K)
    assert b["lm_head"] - b["lm_head_q4k"] == cfg.vocab * cfg.hidden * 2 - cfg.vocab * cfg.hidden // 256 * 144
    # the fused SwiGLU reads gate_up once and writes one int8 row and a scale per token
    assert b["silu_q8"] == 2 * cfg.tokens * cfg.inter * 2 + cfg.tokens * cfg.inter + 4 * cfg.tokens
    # the residual-add + RMSNorm moves x, residual in/out and out: 4 rows of fp16
    assert b["rms"] == 4 * cfg.tokens * cfg.hidden * 2 + cfg.hidden * 2
    # the fused layer-0 op writes one more row than the bare gather
    assert b["emb_rms"] - b["emb"] == cfg.tokens * cfg.hidden * 2 + cfg.hidden * 2


def test_cpu_baseline_leg():
    cb = bench.cpu_baseline(H.CONFIGS[2], 0.05, H)
    assert cb["kind"] == "port" and cb["cores"] == 1 and cb["unit"] == "tokens/s"
    assert cb["value"] > 0 and set(cb["ops_GB_s"]) == {"emb", "rms", "rope", "silu"}


def test_multi_gpu_request_exits_with_message():
    p = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert p.returncode == 2 and "one GPU" in p.stdout
