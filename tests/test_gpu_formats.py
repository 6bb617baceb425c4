"""GPU parity of the on-device Q8_0 block split (nvf_q8_0_split_blocks), the
device form of the reference's host upload_q8_split (src/model.cpp:396-405).

Bar: bit-exact planes against the oracle's split, over random bytes (every bit
pattern of scale and value bytes), block counts that end inside a 16-byte load
and inside a workgroup's chunk, and the full gate_up matrix of config 2 checked
by the size-independent round trip join(split(blocks)) == blocks.  The split
planes then feed the GEMM and the gather to the same results as planes split on
the host.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_vllm_cpp_amd import ops
from tests import harness as H

pytestmark = pytest.mark.gpu


def case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def oracle_split(raw: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    nb = raw.size // 34
    w8 = np.empty(nb * 32, np.int8)
    ws = np.empty(nb, np.uint16)
    H.oracle().orc_q8_0_split_blocks(H.ptr(raw), nb, H.ptr(w8), H.ptr(ws))
    return w8, ws


@pytest.mark.parametrize("nblocks", [1, 2, 3, 7, 8, 9, 255, 256, 257, 511, 512, 513, 1023, 1024, 1025, 4099, 100003])
def test_split_bitexact(gpu, nblocks):
    r = H.rng(nblocks)
    raw = r.integers(0, 256, nblocks * 34, dtype=np.uint8)
    case(f"q8_0_split_blocks nblocks={nblocks}")
    w8, ws = ops.q8_0_split_blocks(torch.from_numpy(raw).to(gpu))
    e8, es = oracle_split(raw)
    H.assert_bitexact(w8.cpu().numpy(), e8, "w8")
    H.assert_bitexact(ws.cpu().numpy().view(np.uint16), es, "ws")


def test_split_does_not_write_past_the_planes(gpu):
    """Outputs carved from larger buffers: the bytes after w8 and ws keep their
    sentinel values (the last workgroup's chunk is partial)."""
    nb = 517
    raw = H.rng(9).integers(0, 256, nb * 34, dtype=np.uint8)
    w8buf = torch.full((nb * 32 + 64,), -7, dtype=torch.int8, device=gpu)
    wsbuf = torch.full((nb + 8,), 0x1234, dtype=torch.int16, device=gpu)
    case("q8_0_split_blocks sentinels")
    rc = ops.lib().nvf_q8_0_split_blocks(torch.from_numpy(raw).to(gpu).data_ptr(), nb, w8buf.data_ptr(),
                                         wsbuf.data_ptr(), None)
    assert rc == 0
    torch.cuda.synchronize()
    e8, es = oracle_split(raw)
    g8 = w8buf.cpu().numpy()
    gs = wsbuf.cpu().numpy().view(np.uint16)
    H.assert_bitexact(g8[:nb * 32], e8, "w8")
    H.assert_bitexact(gs[:nb], es, "ws")
    assert (g8[nb * 32:] == -7).all() and (gs[nb:] == 0x1234).all()


def test_split_full_gate_up_round_trip(gpu):
    """Config 2's gate_up weights [37888, 3584] as GGUF blocks (144 MB): the
    device split, re-joined on the device, reproduces the uploaded bytes."""
    n, k = 37888, 3584
    nb = n * k // 32
    g = torch.Generator(device=gpu)
    g.manual_seed(5)
    raw = torch.randint(0, 256, (nb * 34,), dtype=torch.uint8, device=gpu, generator=g)
    case("q8_0_split_blocks gate_up round trip")
    w8, ws = ops.q8_0_split_blocks(raw)
    joined = torch.empty((nb, 34), dtype=torch.uint8, device=gpu)
    joined[:, :2] = ws.view(torch.uint8).view(nb, 2)
    joined[:, 2:] = w8.view(torch.uint8).view(nb, 32)
    assert torch.equal(joined.view(-1), raw)


def test_split_planes_feed_gemm_and_gather(gpu):
    """Blocks split on the device give the same GEMM output and gather as the
    planes split by the oracle."""
    m, n, k = 24, 320, 512
    r = H.rng(41)
    w8h, wsh = H.gen_q8_0(r, n, k)
    raw = H.q8_split_to_blocks(w8h, wsh)
    case("split planes feed gemm / gather")
    w8, ws = ops.q8_0_split_blocks(torch.from_numpy(raw).to(gpu))
    x = torch.from_numpy(r.standard_normal((m, k)).astype(np.float32)).to(gpu)
    a = ops.matmul_q8(x, w8, ws, n)
    b = ops.matmul_q8(x, H.to_dev(w8h, gpu), H.to_dev(wsh, gpu), n)
    assert torch.equal(a, b)
    ids = torch.from_numpy(r.integers(0, n, 17).astype(np.int64)).to(gpu)
    ga = ops.embedding_q8_0(ids, w8, ws, k)
    gb = ops.embedding_q8_0(ids, H.to_dev(w8h, gpu), H.to_dev(wsh, gpu), k)
    assert torch.equal(ga, gb)
