"""The C ABI: the built library loads without a GPU and exports every declared symbol."""

import ctypes
import re
from pathlib import Path

import pytest

from cxldsagr_amd import _native

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = []
    for header in sorted((ROOT / "include").glob("*.h")):
        text = header.read_text()
        names += re.findall(r"^\s*int\s+(dsa_\w+)\s*\(", text, flags=re.M)
    return names


def test_header_declares_entry_points():
    names = declared_functions()
    assert "dsa_last_error" in names and "dsa_topk_radix" in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    if not _native.LIBRARY_PATH.exists():
        pytest.fail("libdsa_gfx950.so not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(_native.LIBRARY_PATH))
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, f"undeclared exports missing: {missing}"


def test_python_binding_covers_every_declared_symbol():
    assert set(declared_functions()) == set(_native.SIGNATURES)


def test_abi_version_and_error_channel_without_gpu():
    lib = _native.library()
    assert lib.dsa_abi_version() == _native.ABI_VERSION
    # An argument error is reported before any device work.
    status = lib.dsa_topk_radix(None, 1, 0, 0, 1, None, None, 1, None)
    assert status == 1
    assert "nonempty" in _native.last_error()
    status = lib.dsa_topk_radix(None, 1, 8, 8, 4096, None, None, 8, None)
    assert status == 1 and "k must" in _native.last_error()


def test_operators_refuse_cpu_tensors():
    import torch

    from cxldsagr_amd import indexer

    with pytest.raises(NotImplementedError):
        indexer.exact_topk(torch.ones(2, 7), 3)
    with pytest.raises(NotImplementedError):
        indexer.quantize_index(torch.ones(2, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="CUDA Q"):
        indexer.logits(torch.zeros(1, 64, 128), torch.zeros(8, 128), None, None, 7)


def test_topk_workspace_query_without_gpu():
    import ctypes

    size = ctypes.c_int64()
    _native.call("dsa_topk_workspace_bytes", 128, ctypes.byref(size))
    assert size.value == 128 * 2 * 2048 * 8
    with pytest.raises(ValueError, match="workspace query"):
        _native.call("dsa_topk_workspace_bytes", -1, ctypes.byref(size))
