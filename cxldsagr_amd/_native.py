"""ctypes binding of libdsa_gfx950.so (the C ABI declared in include/dsa_gfx950.h).

The library is built in-tree by ``cxldsagr_amd.csrc.build``. Loading fails
loudly when it is missing: there is no CPU or eager fallback for any
operator.
"""

import ctypes
from functools import cache
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libdsa_gfx950.so"
ABI_VERSION = 1

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float

# name -> argument types (restype is int for every entry point)
SIGNATURES = {
    "dsa_last_error": [ctypes.c_char_p, ctypes.c_size_t],
    "dsa_abi_version": [],
    "dsa_quantize_fp8_rows": [_ptr, _int, _i64, _i64, _i64, _ptr, _ptr, _int, _ptr],
    "dsa_quantize_fp8_rows_fold": [_ptr, _int, _i64, _i64, _i64, _ptr, _ptr, _int, _ptr, _ptr,
                                   _ptr],
    "dsa_indexer_logits_fp8": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr,
                               _ptr],
    "dsa_indexer_logits_fp8_folded": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64,
                                      _ptr, _ptr, _ptr],
    "dsa_topk_radix": [_ptr, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr],
    "dsa_topk_workspace_bytes": [_i64, ctypes.POINTER(ctypes.c_int64)],
    "dsa_topk_radix_split": [_ptr, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _i64, _ptr],
    "dsa_topk_radix_split_static": [_ptr, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr],
    "dsa_indexer_logits_fp8_counted": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64,
                                       _i64, _ptr, _ptr, _ptr, _ptr],
    "dsa_topk_radix_digits": [_ptr, _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _i64, _ptr],
    "dsa_indexer_topk_workspace_bytes": [_i64, _i64, ctypes.POINTER(ctypes.c_int64)],
    "dsa_indexer_topk_fp8": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr,
                             _ptr, _i64, _ptr, _ptr, _i64, _ptr, _i64, _ptr],
    "dsa_indexer_select_workspace_bytes": [_i64, _i64, _i64, ctypes.POINTER(ctypes.c_int64)],
    "dsa_indexer_floors_fp8": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64, _ptr,
                               _ptr],
    "dsa_indexer_logits_fp8_emit": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _i64,
                                    _ptr, _ptr, _i64, _ptr, _i64, _ptr],
    "dsa_indexer_emit_topk": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _ptr, _ptr,
                              _i64, _ptr, _ptr, _i64, _i64, _ptr, _i64, _ptr],
    "dsa_indexer_select_fp8": [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _i64, _ptr, _ptr,
                               _i64, _ptr, _ptr, _i64, _ptr, _i64, _ptr],
    "dsa_kv_pack_fp8": [_ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _ptr],
    "dsa_layer_prologue_fp8": [_ptr, _i64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _ptr, _ptr,
                               _ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _ptr],
    "dsa_layer_prologue_floors_fp8": [_ptr, _i64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _ptr,
                                      _ptr, _ptr, _i64, _i64, _ptr, _i64, _ptr, _ptr, _ptr, _ptr,
                                      _i64, _i64, _ptr, _ptr],
    "dsa_index_producer_fp8": [_ptr, _i64, _ptr, _f32, _f32, _ptr, _ptr, _ptr, _f32, _ptr, _i64,
                               _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _ptr, _i64,
                               _ptr, _ptr, _ptr],
    "dsa_index_producer_floors_fp8": [_ptr, _i64, _ptr, _f32, _f32, _ptr, _ptr, _ptr, _f32, _ptr,
                                      _i64, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64,
                                      _ptr, _i64, _ptr, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _ptr],
    "dsa_sparse_mla_bf16": [_ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _f32, _ptr, _ptr],
    "dsa_sparse_mla_fp8_paged": [_ptr, _i64, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64, _f32,
                                 _ptr, _ptr],
    "dsa_gather_records": [_ptr, _i64, _ptr, _i64, _i64, _ptr, _ptr, _i64, _ptr, _int, _i64, _ptr,
                           _ptr],
    "dsa_copy_records_h2d": [_ptr, _ptr, _i64, _ptr],
    "dsa_pool_workspace_bytes": [_i64, _i64, ctypes.POINTER(ctypes.c_int64)],
    "dsa_pool_recall": [_ptr, _i64, _ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr, _i64, _i64,
                        _ptr, _ptr, _ptr, _i64, _i64, _ptr, _i64, _i64, _int, _ptr, _ptr, _ptr,
                        _ptr],
    "dsa_pool_recall_pipelined": [_ptr, _i64, _ptr, _i64, _i64, _i64, _i64, _ptr, _i64, _ptr,
                                  _i64, _i64, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _i64, _i64,
                                  _int, _ptr, _ptr, _ptr, _i64, _i64, _ptr, _ptr],
    "dsa_pool_release_rows": [_ptr, _i64, _i64, _ptr, _ptr, _ptr, _i64, _ptr, _ptr],
}

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


class NativeError(RuntimeError):
    """A C-ABI entry point returned a nonzero status."""


@cache
def library():
    if not LIBRARY_PATH.exists():
        raise RuntimeError(
            f"{LIBRARY_PATH.name} is not built; run `python -c \"import __graft_entry__ as g; "
            "g.build()\"` (hipcc --offload-arch=gfx950). There is no fallback path."
        )
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    version = lib.dsa_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libdsa_gfx950 ABI {version} != expected {ABI_VERSION}")
    return lib


def last_error():
    buf = ctypes.create_string_buffer(512)
    library().dsa_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def call(name, *args):
    status = getattr(library(), name)(*args)
    if status != 0:
        message = last_error()
        if status == 1:
            raise ValueError(message)
        raise NativeError(f"{name} failed ({status}): {message}")


def ptr(tensor):
    """Device (or host) address of a tensor, or None for a missing tensor."""
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gfx950(device, what):
    """The native kernels are built for gfx950 only."""
    if device.type != "cuda" or not torch.cuda.is_available():
        raise NotImplementedError(f"{what} requires an MI355X (gfx950) HIP device")
    arch = torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]
    if arch != "gfx950":
        raise NotImplementedError(f"{what} requires an MI355X (gfx950) HIP device, got {arch}")
