"""Argument validation of the host-record transfers (CPU; no device needed).

Mirrors the validation half of the reference's
operators/common/tests/test_kv_transfer.py: every contract violation raises
``ValueError`` with the reference message before anything is launched.
"""

import pytest
import torch

from cxldsagr_amd import kv_transfer


def _ids(n=4):
    return torch.arange(n, dtype=torch.int64)


@pytest.mark.parametrize("max_ctas", [0, -1, 2**31, 1.5, True])
def test_gather_rejects_bad_grid_bounds(max_ctas):
    host = torch.zeros(8, 16, dtype=torch.uint8)
    with pytest.raises(ValueError, match="max_ctas must be a positive CUDA grid size"):
        kv_transfer.gather_host_records(host, host, _ids(), _ids(), max_ctas=max_ctas)


def test_gather_requires_pinned_host_records():
    host = torch.zeros(8, 16, dtype=torch.uint8)  # pageable
    with pytest.raises(ValueError, match="host records must use pinned CPU memory"):
        kv_transfer.gather_host_records(host, host, _ids(), _ids())


@pytest.mark.parametrize(
    "kwargs,message",
    [
        ({"host_start": -1, "device_start": 0, "count": 1}, "host_start must be a nonnegative integer"),
        ({"host_start": 0, "device_start": 1.0, "count": 1}, "device_start must be a nonnegative integer"),
        ({"host_start": 0, "device_start": 0, "count": -2}, "count must be a nonnegative integer"),
    ],
)
def test_copy_rejects_bad_spans(kwargs, message):
    host = torch.zeros(8, 16, dtype=torch.uint8)
    with pytest.raises(ValueError, match=message):
        kv_transfer.copy_host_records_async(host, host, **kwargs)


def test_copy_requires_pinned_host_records():
    host = torch.zeros(8, 16, dtype=torch.uint8)
    with pytest.raises(ValueError, match="host records must use pinned CPU memory"):
        kv_transfer.copy_host_records_async(host, host, host_start=0, device_start=0, count=1)
