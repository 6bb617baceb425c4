"""Runs tests/cpp/dropin_chain: a C++ program that calls the drop-in C ABI in
the order src/model.cpp:756-844 does -- a whole layer: embedding, norms, the Q8_0
projections, QK-norm, RoPE, KV store, paged attention, SwiGLU, final norm, the last
rows gathered, lm_head with Q8_0 / Q4_K / bf16 tables -- beside it Qwen2.5's qkv bias
and the mixture-of-experts branch (router, routing, shared expert and its gate, routed
experts, :789-826), then a decode step over a longer cache that the drop-in splits over
its own workspace, and checks every stage against the C oracle (bit-exact gathers,
residuals, cache writes, bias and routing; the stated tolerance or bound elsewhere)."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "_build" / "dropin_chain"


def test_cpp_model_call_sequence(gpu):
    if not BIN.exists():
        pytest.fail(f"{BIN} not built (run __graft_entry__.build())")
    print("[case] C++ drop-in chain", flush=True)
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "DROPIN CHAIN OK" in r.stdout
