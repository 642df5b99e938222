"""CPU oracle for the DeepSeek-V3.2 DSA prefill hot path.

TEST INFRASTRUCTURE ONLY. This package is a numpy (and, for the timed CPU
baseline, torch CPU) restatement of the reference algorithms and exists to check the HIP kernels. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker (or as the timed CPU baseline). The product path in
``cxldsagr_amd`` never imports it and fails loudly when the HIP library is
missing.

Modules and the reference code each one restates (paths relative to the
reference checkout):

* ``fp8``        - OCP float8 e4m3fn encode/decode, the conversion used by
                   ``tensor.to(torch.float8_e4m3fn)`` (RNE, no infinities).
* ``quantize``   - ``operators/deepseek_v32/indexer/quantization.py:12-21,34-60``.
* ``logits``     - ``operators/deepseek_v32/indexer/echo.py:299-410`` and the
                   oracle in ``indexer/tests/test_echo_indexer.py:86-109``.
* ``topk``       - ``operators/deepseek_v32/indexer/selection.py:62-113``.
* ``sparse_mla`` - ``operators/deepseek_v32/attention/reference/torch.py:13-28``,
                   ``attention/_validation.py:8-24``, ``device_only/mla.py:58-115``.
* ``kv_fp8``     - the 656-byte paged fp8 KV record (no reference counterpart;
                   built from the A1 quantiser rule).
* ``recall``     - ``cache/sparse_token_cache.py:483-569`` and
                   ``operators/common/kv_transfer.py:21-68``.
* ``layer``      - the CPU DSA layer in the order of
                   ``models/deepseek_v32/attention.py:276-425``.
* ``torch_layer`` - the same layer on torch's CPU kernels, multi-threaded: the
                   timed CPU baseline of ``bench.py`` (pinned to ``layer``).

Every function is pinned by a check in ``tests/test_oracle_*.py`` that does not
retype its formula (golden vectors, library routines, closed forms, brute
force). Pinning status per function is listed in each module header.
"""
