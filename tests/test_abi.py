"""The C-ABI library loads and exports every entry point include/lq_api.h declares
(no compute calls: this runs without a GPU)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lq_api.h")


def declared_symbols() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "lq_quantize_per_tensor_f32" in syms and "lq_minmax_f32" in syms
    assert len(syms) >= 30


def test_library_exports_every_declared_symbol():
    from lucid_amd import _C

    lib = ctypes.CDLL(_C.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"declared in lq_api.h but not exported: {missing}"


def test_python_binding_declares_only_exported_symbols():
    from lucid_amd import _C

    L = _C.lib()  # raises if a registered signature is not exported
    assert L.lq_abi_version() == 1
    assert L.lq_backend_name() == b"hip-gfx950"


def test_device_count_without_gpu_is_not_an_error():
    from lucid_amd import _C

    assert _C.device_count() >= 0


def test_cpu_tensor_ops_fail_loudly():
    import numpy as np

    import lucid_amd as L
    import lucid_amd.quantization as Q

    x = L.tensor(np.ones(4, np.float32))
    with pytest.raises(L.LucidError, match="GPU tensors"):
        Q.quantize(x, 0.1, 0, Q.qint8)
    with pytest.raises(L.LucidError, match="GPU tensors"):
        Q.MinMaxObserver()(x)


def test_workspace_queries_on_degenerate_shapes():
    """Host-side planning of empty / tiny shapes (no GPU call): sizes are finite and the
    query does not divide by zero for an empty channel extent."""
    from lucid_amd import _C

    L = _C.lib()
    for outer, C, inner in ((1, 2, 0), (0, 3, 5), (0, 1, 100), (4, 1, 0), (2, 4096, 1)):
        assert L.lq_minmax_per_channel_workspace_size(outer, C, inner) >= 0
    assert L.lq_minmax_workspace_size(0) > 0
    for M, N, K in ((0, 0, 0), (1, 1, 1), (4096, 4096, 4096), (128, 4096, 4096)):
        assert L.lq_gemm_w8a8_workspace_size(M, N, K) >= 0
    # split-K partials are only planned for mid-size M with few 128x128 tiles
    assert L.lq_gemm_w8a8_workspace_size(128, 4096, 4096) >= 128 * 4096 * 4
