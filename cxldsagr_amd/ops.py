"""The hot-path operators in one flat namespace, with the reference's names
and argument order (what a caller of the reference's operator modules
imports):

* quantize_index   - operators/deepseek_v32/indexer/quantization.py:63
* logits           - operators/deepseek_v32/indexer/echo.py:299 (prefetch must be None)
* exact_topk       - operators/deepseek_v32/indexer/selection.py:62
* sparse_mla       - operators/deepseek_v32/attention/device_only/mla.py:90
* sparse_mla_from_pool - operators/deepseek_v32/attention/offload/mla.py:12
* gather_host_records  - operators/common/kv_transfer.py:21
* copy_host_records_async - operators/common/kv_transfer.py (contiguous span copy)

plus the operators of the fp8 paged KV record (656 bytes per token), which
the reference does not have: sparse_mla_fp8_paged and pack_kv_fp8.
"""

from .attention import pack_kv_fp8, sparse_mla, sparse_mla_fp8_paged, sparse_mla_from_pool
from .indexer import exact_topk, logits, quantize_index
from .kv_transfer import copy_host_records_async, gather_host_records

__all__ = [
    "quantize_index",
    "logits",
    "exact_topk",
    "sparse_mla",
    "sparse_mla_from_pool",
    "sparse_mla_fp8_paged",
    "pack_kv_fp8",
    "gather_host_records",
    "copy_host_records_async",
]
