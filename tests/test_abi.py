"""The C ABI (include/sqx.h) against the built libsqx_hip.so — CPU only, no kernel launches.

Checks that the library loads in a torch process, exports every entry point the header declares,
that the ctypes table covers exactly those names, and that argument validation rejects bad calls
with the documented status codes before anything reaches the GPU."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from scratch_llm_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "sqx.h"


def _declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"\b(sqx_[a-z0-9_]+)\s*\(", text)


def test_header_declares_entry_points():
    names = _declared()
    assert len(names) == len(set(names)), "duplicate declarations"
    assert "sqx_int4_linear" in names and "sqx_last_error" in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in sqx.h but not exported"


def test_ctypes_table_matches_header():
    assert sorted(_lib.exported_names()) == sorted(_declared())


def test_abi_version_and_error_string():
    lib = _lib.load()
    assert lib.sqx_abi_version() >= 1
    assert isinstance(lib.sqx_last_error(), bytes)


def test_argument_validation_without_device():
    lib = _lib.load()
    null = None
    # indivisible group -> SQX_E_ARG with the reference's message
    rc = lib.sqx_int4_quantize_sym(null, 0, 4, 100, 128, null, null, null)
    assert rc == -1
    rc = lib.sqx_int4_quantize_sym(ctypes.c_void_p(16), 0, 4, 100, 128, ctypes.c_void_p(16), ctypes.c_void_p(16), null)
    assert rc == -1 and b"not divisible by group_size" in lib.sqx_last_error()
    # unsupported tiled group size
    assert lib.sqx_int4_tile(null, 0, null, null, 0, 16, 96, 96, null, null, null, null) == -1
    assert b"group_size" in lib.sqx_last_error()
    # activations must be bf16/fp16
    rc = lib.sqx_int4_linear(null, null, null, 0, null, 0, null, null, 1, 16, 128, 128, 1, null)
    assert rc == -1 and b"BF16 or F16" in lib.sqx_last_error()
    # more than 16 k-slices per tile
    rc = lib.sqx_int4_linear(
        ctypes.c_void_p(256), ctypes.c_void_p(256), null, 0, ctypes.c_void_p(256), 1, ctypes.c_void_p(256), null,
        1, 64, 4096, 128, 17, null,
    )
    assert rc == -1 and b"k_slices" in lib.sqx_last_error()
    # misaligned weight tiles
    rc = lib.sqx_int4_linear(
        ctypes.c_void_p(8), ctypes.c_void_p(256), null, 0, ctypes.c_void_p(256), 1, ctypes.c_void_p(256), null,
        1, 64, 4096, 128, 0, null,
    )
    assert rc == -1 and b"aligned" in lib.sqx_last_error()


def test_size_queries():
    lib = _lib.load()
    assert lib.sqx_int4_tiled_weight_bytes(4096, 4096) == 4096 * 4096 // 2
    assert lib.sqx_int4_tiled_weight_bytes(1000, 96) == 63 * 1 * 1024
    assert lib.sqx_int4_tiled_param_count(4096, 4096, 128) == 4096 * 32
    assert lib.sqx_int4_tiled_param_count(4096, 4096, 96) == -1
    for rows, cols in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336), (128256, 4096), (16, 128)):
        s = lib.sqx_int4_linear_default_kslices(1, rows, cols)
        assert 1 <= s <= 16 and s <= max(1, cols // 256)


def test_python_layer_rejects_cpu_tensors():
    from scratch_llm_amd.quant import int4_group

    with pytest.raises(RuntimeError, match="device tensors"):
        int4_group.quantize_groupwise_int4(torch.randn(4, 128))
    with pytest.raises(RuntimeError, match="device tensors"):
        int4_group.pack_int4(torch.zeros(4, dtype=torch.int8))
    with pytest.raises(ValueError, match="1-D"):
        int4_group.pack_int4(torch.zeros(2, 2, dtype=torch.int8))
    with pytest.raises(ValueError, match="not divisible by group_size"):
        int4_group.quantize_groupwise_int4(torch.randn(4, 100))
    with pytest.raises(ValueError, match="2-D"):
        int4_group.quantize_groupwise_int4(torch.randn(128))
