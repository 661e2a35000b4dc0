"""The C-ABI library loads without a GPU and exports every function include/*.h declares."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from metile_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        for m in re.finditer(r"\b(mt_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_header_declares_the_bound_signatures():
    assert declared_functions() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(declared_functions()) if not hasattr(handle, n)]
    assert not missing, missing


def test_version_and_error_reporting_without_gpu():
    lib = _lib.lib()
    assert lib.mt_version().decode().startswith("metile_amd")
    # argument validation runs on the host, before any HIP call
    st = lib.mt_affine_qmv(None, None, None, None, None, None, 1, 100, 64, 64, 4, 0, None, 0,
                           None)
    assert st == _lib.MT_ERR_INVALID_ARGUMENT
    assert "group_size" in lib.mt_last_error().decode()
    st = lib.mt_affine_qmv(None, None, None, None, None, None, 1, 128, 64, 64, 3, 0, None, 0,
                           None)
    assert st == _lib.MT_ERR_INVALID_ARGUMENT and "bits" in lib.mt_last_error().decode()


def test_workspace_sizes_are_row_independent_plans():
    lib = _lib.lib()
    # split-K partials scale with rows (capped at one 32-row chunk), the plan does not change
    w1 = lib.mt_affine_qmv_workspace_bytes(1, 8960, 1536, 64, 4, 1)
    w32 = lib.mt_affine_qmv_workspace_bytes(32, 8960, 1536, 64, 4, 1)
    w64 = lib.mt_affine_qmv_workspace_bytes(64, 8960, 1536, 64, 4, 1)
    assert 0 < w1 < w32 == w64
    assert lib.mt_affine_mlp_workspace_bytes(4, 1536, 8960, 64, 4) >= 4 * 8960 * 2
    assert lib.mt_affine_qmv_workspace_bytes(1, 100, 64, 64, 4, 1) == 0  # invalid K


def test_repack_argument_checks_without_gpu():
    lib = _lib.lib()
    buf = ctypes.c_void_p(256)  # never dereferenced: every case fails validation first
    assert lib.mt_affine_repack(buf, buf, 16, 128, 3, None) == _lib.MT_ERR_INVALID_ARGUMENT
    assert "bits" in lib.mt_last_error().decode()
    assert lib.mt_affine_repack(buf, buf, 16, 100, 4, None) == _lib.MT_ERR_INVALID_ARGUMENT
    assert "multiple of 64" in lib.mt_last_error().decode()
    assert lib.mt_affine_repack(None, buf, 16, 128, 4, None) == _lib.MT_ERR_INVALID_ARGUMENT
    assert "null" in lib.mt_last_error().decode()
    assert lib.mt_affine_repack(ctypes.c_void_p(264), buf, 16, 128, 4, None) == \
        _lib.MT_ERR_INVALID_ARGUMENT
    assert "aligned" in lib.mt_last_error().decode()


def test_mlp_layouts_argument_checks_without_gpu():
    lib = _lib.lib()
    args = [None] * 12 + [1, 1536, 8960, 64, 4, 0]
    # an unknown layout is refused before anything else is read
    for up, down in ((2, 0), (0, -1)):
        st = lib.mt_affine_mlp_layouts(*args, up, down, None, 0, None)
        assert st == _lib.MT_ERR_INVALID_ARGUMENT
        assert "MT_LAYOUT_MLX or MT_LAYOUT_REPACKED" in lib.mt_last_error().decode()
    # valid layouts reach the usual shape and pointer checks
    st = lib.mt_affine_mlp_layouts(*args, _lib.MT_LAYOUT_REPACKED, _lib.MT_LAYOUT_MLX, None, 0,
                                   None)
    assert st != 0 and "LAYOUT" not in lib.mt_last_error().decode()


def test_stream_read_argument_checks_without_gpu():
    lib = _lib.lib()
    buf = ctypes.c_void_p(256)  # never dereferenced: every case fails validation first
    for p, nbytes, sink, blocks in ((None, 4096, buf, 1), (buf, 0, buf, 1), (buf, 1 << 31, buf, 1),
                                    (buf, 4096, None, 1), (buf, 4096, buf, 0),
                                    (buf, 4096, buf, 65537)):
        for fn in (lib.mt_stream_read, lib.mt_stream_read_blocked):
            assert fn(p, nbytes, sink, blocks, None) == _lib.MT_ERR_INVALID_ARGUMENT
            assert "below 2 GiB" in lib.mt_last_error().decode()


def test_dense_workspace_covers_both_row_chunks():
    """Dense dispatches of more than 64 rows run as two 64-row grid chunks, each with its own
    split-K partials and counters: the workspace of 65..128 rows holds 128 rows of partials,
    and a dispatch's workspace never depends on more than 128 rows."""
    lib = _lib.lib()
    k, n = 8192, 2048  # the config-2 down projection: split along K
    ws = {m: lib.mt_dense_workspace_bytes(m, k, n, 1) for m in (1, 64, 65, 100, 128, 129, 1000)}
    counters = 64 * 1024
    per_row = (ws[64] - counters) // 64
    assert ws[1] == counters + per_row
    assert ws[65] == ws[100] == ws[128] == counters + 128 * per_row
    assert ws[129] == ws[1000] == ws[128]
    assert lib.mt_dense_workspace_bytes(4, 2048, 8192, 2) == 0  # gate/up: one K split
