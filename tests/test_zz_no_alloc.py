"""mt_affine_mlp_noalloc, the MLP entry point that allocates nothing: its workspace is a 16 MiB
device array inside the library (one per GPU, kept until the process ends).

On the GPU (through the C ABI): the process's first call made under graph capture and replayed
three times, and two eager calls in a row, the second with fewer rows, each bit-identical to
mt_affine_mlp with a caller workspace (same kernels and plans), so the split-K counters it shares
between calls are left at zero and its hidden activation and partial sums are not stale; the
eager calls leave the device's free memory unchanged. On the CPU: sizes beyond the array and
invalid shapes are rejected before any device work.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from metile_amd import _lib
from oracle import affine as O
from tests.helpers import act_to_torch, affine_to_torch

H, I, G, BITS = 1536, 8960, 64, 4


def _dummy():
    return ctypes.c_void_p(256)  # never dereferenced: every case below fails validation first


def test_noalloc_rejects_calls_beyond_its_array_without_device_work():
    lib = _lib.lib()
    need = lib.mt_affine_mlp_workspace_bytes(32, 8192, 28672, 64, 4)
    assert need > 16 << 20
    p = _dummy()
    st = lib.mt_affine_mlp_noalloc(p, p, p, p, p, p, p, p, p, p, None, p, 32, 8192, 28672, 64, 4,
                                   _lib.MT_BF16, None)
    assert st == _lib.MT_ERR_WORKSPACE
    msg = lib.mt_last_error().decode()
    assert "mt_affine_mlp_noalloc" in msg and str(16 << 20) in msg and str(need) in msg


def test_noalloc_rejects_invalid_shapes_like_the_workspace_entry_point():
    lib = _lib.lib()
    p = _dummy()
    st = lib.mt_affine_mlp_noalloc(p, p, p, p, p, p, p, p, p, p, None, p, 1, 100, 8960, 64, 4,
                                   _lib.MT_BF16, None)
    assert st == _lib.MT_ERR_INVALID_ARGUMENT
    assert "mt_affine_mlp_noalloc" in lib.mt_last_error().decode()


def _weights():
    gate = affine_to_torch(O.make_affine_weight(I, H, BITS, G, 31, 10), "bf16")
    up = affine_to_torch(O.make_affine_weight(I, H, BITS, G, 31, 12), "bf16")
    down = affine_to_torch(O.make_affine_weight(H, I, BITS, G, 31, 14), "bf16")
    return [t.data_ptr() for triple in (gate, up, down) for t in triple], (gate, up, down)


def _reference(lib, ptrs, x, r, m, stream):
    want = torch.empty(m, H, dtype=torch.bfloat16, device="cuda")
    need = lib.mt_affine_mlp_workspace_bytes(m, H, I, G, BITS)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    _lib.check(lib.mt_affine_mlp(x.data_ptr(), *ptrs, r.data_ptr(), want.data_ptr(), m, H, I, G,
                                 BITS, _lib.MT_BF16, ws.data_ptr(), need, stream))
    torch.cuda.synchronize()
    return want


# First in the file, so that the process's first call of the entry point (the one that resolves
# the array's device address) is made under graph capture, whether the file runs alone or after
# the rest of the suite.
@pytest.mark.gpu
def test_noalloc_first_call_under_graph_capture_replays_bit_identical():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)
    lib = _lib.lib()
    ptrs, keep = _weights()
    m = 16  # both projections split K: the counters and partials live in the array
    x = act_to_torch(O.make_activations(m, H, 40), "bf16")
    r = act_to_torch(O.make_activations(m, H, 40, tensor_id=3), "bf16")
    want = _reference(lib, ptrs, x, r, m, torch.cuda.current_stream().cuda_stream)
    got = torch.full((m, H), float("nan"), dtype=torch.bfloat16, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    print("[noalloc] first call under capture", flush=True)
    with torch.cuda.graph(graph, stream=side):
        _lib.check(lib.mt_affine_mlp_noalloc(x.data_ptr(), *ptrs, r.data_ptr(), got.data_ptr(), m,
                                             H, I, G, BITS, _lib.MT_BF16, side.cuda_stream))
    for replay in range(3):
        got.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), replay
    del graph


@pytest.mark.gpu
def test_noalloc_matches_mt_affine_mlp_on_two_calls_second_smaller():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    torch.cuda.set_device(0)
    lib = _lib.lib()
    ptrs, keep = _weights()
    stream = torch.cuda.current_stream().cuda_stream
    for m in (16, 3):  # 16 rows: both projections split K; then a smaller call over the array
        print(f"[noalloc] M={m}", flush=True)
        x = act_to_torch(O.make_activations(m, H, 31 + m), "bf16")
        r = act_to_torch(O.make_activations(m, H, 31 + m, tensor_id=3), "bf16")
        want = _reference(lib, ptrs, x, r, m, stream)
        got = torch.full((m, H), float("nan"), dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info()[0]
        _lib.check(lib.mt_affine_mlp_noalloc(x.data_ptr(), *ptrs, r.data_ptr(), got.data_ptr(), m,
                                             H, I, G, BITS, _lib.MT_BF16, stream))
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free_before, "the call allocated device memory"
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), m
