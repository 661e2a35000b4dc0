"""The streaming-read probe (``mt_stream_read``) reads every 16-byte chunk of its buffer once,
whatever the grid: with 1, 2, 4 or 8 loads per thread in one batch (grids sized to the buffer)
and in several batches (a fixed grid smaller than the buffer), including a ragged last batch.

Each case plants the probe's sentinel word in one chunk of an all-zero buffer. The thread that
reads that chunk folds it into its XOR alone (every other word it reads is zero), so its
block, and only its block, stores the sentinel to the sink."""

from __future__ import annotations

import pytest
import torch

from metile_amd import _lib

pytestmark = pytest.mark.gpu

SENTINEL = 0x9E3779B9


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)


# (bytes, blocks): one batch of 1, 2, 4 and 8 loads per thread; several batches of 8 with a
# ragged end; a buffer smaller than one grid span
CASES = [(4096 * 64, 64), (4096 * 64 * 2, 64), (4096 * 64 * 4 - 4096, 64), (4096 * 64 * 8, 64),
         (4096 * 64 * 8 * 3 + 16 * 300, 64), (4096 * 3 + 48, 8)]


@pytest.mark.parametrize("nbytes,blocks", CASES)
def test_probe_reads_every_chunk(nbytes, blocks):
    lib = _lib.lib()
    chunks = nbytes // 16
    span = blocks * 256  # chunks the grid reads per step
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device="cuda")
    sink = torch.zeros(blocks, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    sentinel = torch.tensor(SENTINEL, dtype=torch.int64).to(torch.int32).item()
    for c in sorted({0, 1, 255, 256, span - 1, span, chunks // 2, chunks - 1}):
        if c >= chunks:
            continue
        print(f"[probe] bytes {nbytes} blocks {blocks} chunk {c}", flush=True)
        buf.zero_()
        sink.zero_()
        buf[4 * c] = sentinel
        _lib.check(lib.mt_stream_read(buf.data_ptr(), nbytes, sink.data_ptr(), blocks, stream))
        torch.cuda.synchronize()
        owner = (c % span) // 256
        expect = torch.zeros_like(sink)
        expect[owner] = sentinel
        assert torch.equal(sink, expect), (nbytes, blocks, c)
