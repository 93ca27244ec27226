"""The HBM read probe (a measurement helper of bench.py, include/mipaged_probe.h) reads every
chunk it is given exactly once on each of its read paths: the XOR of its sink equals the XOR of
every 32-bit word of the chunks, computed on the host."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("chunk,n,grid", [(2048, 3000, 64), (8192, 700, 96), (1024, 5, 512)])
@pytest.mark.parametrize("order", ["random", "sequential"])
def test_probe_reads_every_chunk(gpu, mode, chunk, n, grid, order):
    from engine import _native

    announce(f"read probe mode {mode} chunk {chunk} n {n} grid {grid} {order}")
    lib = _native.load()
    total = 4 * n
    rng = np.random.default_rng(chunk + n + mode)
    data = rng.integers(0, 2**32, size=total * chunk // 4, dtype=np.uint32)
    ids = rng.permutation(total)[:n] if order == "random" else np.arange(n)
    ids = ids.astype(np.int32)
    buf = torch.from_numpy(data.view(np.int32)).to(gpu)
    ids_t = torch.from_numpy(ids).to(gpu)
    sink = torch.zeros(grid * 256, dtype=torch.int32, device=gpu)
    st = torch.cuda.current_stream(gpu).cuda_stream
    rc = lib.mip_hbm_read_probe(buf.data_ptr(), total * chunk, ids_t.data_ptr(), n, chunk, sink.data_ptr(), grid,
                                mode, st)
    assert rc == _native.MIP_OK, rc
    torch.cuda.synchronize()
    words = data.reshape(total, chunk // 4)[ids]
    want = np.bitwise_xor.reduce(words.ravel())
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == want
