"""The streaming-read probe (``mt_stream_read``, and ``mt_stream_read_blocked`` whose blocks
each read a contiguous run) reads every 16-byte chunk of its buffer once, whatever the grid: with 1, 2, 4 or 8 loads per thread in one batch (grids sized to the buffer)
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


def _loads_per_thread(nbytes, blocks):
    steps = -(-nbytes // (blocks * 4096))
    return 1 if steps <= 1 else 2 if steps <= 2 else 4 if steps <= 4 else 8


@pytest.mark.parametrize("blocked", [False, True], ids=["grid-stride", "blocked"])
@pytest.mark.parametrize("nbytes,blocks", CASES)
def test_probe_reads_every_chunk(nbytes, blocks, blocked):
    lib = _lib.lib()
    fn = lib.mt_stream_read_blocked if blocked else lib.mt_stream_read
    chunks = nbytes // 16
    u = _loads_per_thread(nbytes, blocks)
    # grid-stride: block b reads chunks [256 b, 256 b + 256) of every grid step of 256 blocks
    # chunks; blocked: block b reads the run [256 u b, 256 u (b + 1)) of every span of
    # 256 u blocks chunks
    span = blocks * 256 * (u if blocked else 1)
    run = 256 * (u if blocked else 1)
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device="cuda")
    sink = torch.zeros(blocks, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    sentinel = torch.tensor(SENTINEL, dtype=torch.int64).to(torch.int32).item()
    for c in sorted({0, 1, 255, 256, run - 1, run, span - 1, span, chunks // 2, chunks - 1}):
        if c >= chunks:
            continue
        print(f"[probe] bytes {nbytes} blocks {blocks} blocked {blocked} chunk {c}", flush=True)
        buf.zero_()
        sink.zero_()
        buf[4 * c] = sentinel
        _lib.check(fn(buf.data_ptr(), nbytes, sink.data_ptr(), blocks, stream))
        torch.cuda.synchronize()
        owner = (c % span) // run
        expect = torch.zeros_like(sink)
        expect[owner] = sentinel
        assert torch.equal(sink, expect), (nbytes, blocks, c)
