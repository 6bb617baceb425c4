"""Writes tests/golden/reference_vectors.npz from the reference's OWN host code.

Run in the build container, where oracle/_ref/libref_host.so has been compiled
from the reference sources (make -C oracle ref):
  * GGUFLoader::dequant_block_f32("Q4_K" / "Q6_K", ...)  src/gguf.cpp:566-571
  * fp16_to_float / float_to_fp16                         include/nanovllm/common.hpp:28-91
Inputs are seeded; only inputs and the reference's outputs are stored.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from tests import harness as H  # noqa: E402


def special_q4k(r: np.random.Generator) -> np.ndarray:
    """Edge-case Q4_K blocks: subnormal / zero / max-normal d and dmin, all-63 scales, 0x00/0xFF nibbles."""
    out = []
    for d, dmin, sc, qs in [
        (np.float16(6e-8), np.float16(1e-7), 63, 0xFF),      # subnormal scales
        (np.float16(0.0), np.float16(2.0), 63, 0x0F),
        (np.float16(65504.0), np.float16(1.0), 63, 0xF0),    # max fp16
        (np.float16(-0.5), np.float16(-0.25), 17, 0x5A),     # negative scales
        (np.float16(1.0), np.float16(0.0), 1, 0x00),
    ]:
        b = np.zeros(144, np.uint8)
        b[0:2] = np.array([d], np.float16).view(np.uint8)
        b[2:4] = np.array([dmin], np.float16).view(np.uint8)
        b[4:16] = H.pack_q4k_scales(np.full(8, sc) - np.arange(8) % 3, np.full(8, sc)[::-1] - np.arange(8) % 2)
        b[16:] = qs
        out.append(b)
    # distinct per-group scales and a nibble ramp: a wrong group or nibble index changes the output
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([np.float16(1.0)], np.float16).view(np.uint8)
    b[2:4] = np.array([np.float16(1.0)], np.float16).view(np.uint8)
    b[4:16] = H.pack_q4k_scales(np.array([1, 2, 4, 8, 16, 32, 63, 5]), np.array([0, 1, 2, 3, 40, 50, 60, 63]))
    b[16:] = (np.arange(128) % 16) | ((15 - np.arange(128) % 16) << 4)
    out.append(b)
    return np.concatenate(out)


def main() -> None:
    ref = H.ref_host()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_host.so not built: make -C oracle ref")
    r = np.random.default_rng(20260101)

    q4k = np.concatenate([special_q4k(r), H.gen_q4_k(r, 26)])
    q6k = H.gen_raw_blocks(r, 32, 210, (208,))
    q6k[q6k.size - 2:] = np.array([np.float16(3e-7)], np.float16).view(np.uint8)  # subnormal d

    def deq(kind: str, blocks: np.ndarray, bb: int) -> np.ndarray:
        n = blocks.size // bb
        y = np.empty(n * 256, np.float32)
        for i in range(n):
            blk = np.ascontiguousarray(blocks[i * bb:(i + 1) * bb])
            assert ref.ref_dequant_block_f32(kind.encode(), H.ptr(blk), y[i * 256:].ctypes.data) == 1
        return y

    codes = np.concatenate([np.arange(0, 0x400), np.arange(0x8000, 0x8400),          # +-0 and subnormals
                            np.arange(0x7C00, 0x7C10), np.arange(0xFC00, 0xFC10),    # inf / nan
                            r.integers(0, 65536, 512)]).astype(np.uint16)
    dec = np.array([ref.ref_fp16_to_float(int(c)) for c in codes], np.float32)

    f = np.concatenate([
        r.normal(0, 1, 512), r.normal(0, 1e-5, 256), r.uniform(-70000, 70000, 128),
        # exact RNE midpoints between fp16 neighbours (ties) and just off them
        (np.arange(1, 200, dtype=np.float64) + 0.5) * 2.0 ** -24,
        (1024 + np.arange(64) + 0.5) * 2.0 ** -10, 65520.0 * np.ones(1), 65519.0 * np.ones(1),
    ]).astype(np.float32)
    enc = np.array([ref.ref_float_to_fp16(float(v)) for v in f], np.uint16)

    np.savez_compressed(HERE / "reference_vectors.npz",
                        q4k_blocks=q4k, q4k_expected=deq("Q4_K", q4k, 144),
                        q6k_blocks=q6k, q6k_expected=deq("Q6_K", q6k, 210),
                        fp16_codes=codes, fp16_decoded=dec, f32_values=f, fp16_encoded=enc)
    print("wrote", HERE / "reference_vectors.npz")


if __name__ == "__main__":
    main()
