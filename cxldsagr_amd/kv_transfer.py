"""Pinned-host record transfers: sparse GPU gathers or contiguous async copies.

Drop-in for ``operators/common/kv_transfer.py:21-103`` (same names, argument
order and validation messages). The gather runs in ``csrc/gather.hip``: the
GPU reads the selected host rows over PCIe straight into their HBM slots.
Invalid ids do not trap the GPU (the reference's ``trap``); they are skipped
and flagged in a per-device status word, see ``transfer_status``.
"""

import torch

from cxldsagr_amd import _native

_STATUS = {}


def _status_word(device):
    key = (device.type, device.index)
    word = _STATUS.get(key)
    if word is None:
        word = torch.zeros(1, dtype=torch.int32, device=device)
        _STATUS[key] = word
    return word


def transfer_status(device, *, reset=True):
    """Read (and by default clear) the device's gather status bits.

    Bit 0: a host or device id was out of range (row skipped); bit 1: a
    ``valid_count`` was outside ``[0, len(ids)]`` (nothing copied). Reading it
    synchronises with the device.
    """
    word = _status_word(torch.device(device))
    value = int(word.item())
    if reset:
        word.zero_()
    return value


def gather_host_records(host, device, host_ids, device_ids, *, max_ctas=None, valid_count=None,
                        status=None):
    """Copy complete records on the current stream; ids stay on the GPU.

    ``device[device_ids[r]] = host[host_ids[r]]`` for every ``r`` (or the
    ``valid_count`` prefix, a device int64/uint32 scalar). The caller owns both
    allocations until stream completion. ``max_ctas`` bounds the grid so the
    copy can overlap compute on another stream. ``status`` (int32 ``[1]`` on
    the device) receives the error bits; by default the per-device word of
    ``transfer_status`` does.
    """
    if max_ctas is not None and (type(max_ctas) is not int or not 0 < max_ctas < 2**31):
        raise ValueError("max_ctas must be a positive CUDA grid size")
    if host.device.type != "cpu" or not host.is_pinned():
        raise ValueError("host records must use pinned CPU memory")
    if device.device.type != "cuda" or host.dtype != device.dtype:
        raise ValueError("device records must be CUDA and match host dtype")
    if host.ndim != 2 or device.ndim != 2 or host.shape[1] != device.shape[1]:
        raise ValueError("host/device records must have the same row width")
    if not host.is_contiguous() or not device.is_contiguous():
        raise ValueError("records must be contiguous")
    if host_ids.dtype != torch.int64 or device_ids.dtype != torch.int64:
        raise ValueError("record IDs must be int64")
    if host_ids.device != device.device or device_ids.device != device.device:
        raise ValueError("record IDs must be on the cache GPU")
    if host_ids.ndim != 1 or host_ids.shape != device_ids.shape:
        raise ValueError("host/device IDs must be equal length vectors")
    if not host_ids.is_contiguous() or not device_ids.is_contiguous():
        raise ValueError("record IDs must be contiguous")
    if valid_count is not None and (
        valid_count.device != device.device
        or valid_count.dtype not in (torch.int64, torch.uint32)
        or valid_count.numel() != 1
        or not valid_count.is_contiguous()
    ):
        raise ValueError("valid_count must be a contiguous int64/uint32 scalar on the cache GPU")
    if status is not None and (status.dtype != torch.int32 or status.device != device.device):
        raise ValueError("status must be an int32 tensor on the cache GPU")
    _native.require_gfx950(device.device, "host record gather")
    if not host_ids.numel():
        return
    row_bytes = host.shape[1] * host.element_size()
    if status is None:
        status = _status_word(device.device)
    kind = 1 if valid_count is not None and valid_count.dtype == torch.uint32 else 0
    with torch.cuda.device(device.device):
        _native.call(
            "dsa_gather_records",
            _native.ptr(host), host.shape[0],
            _native.ptr(device), device.shape[0],
            row_bytes,
            _native.ptr(host_ids), _native.ptr(device_ids), host_ids.numel(),
            _native.ptr(valid_count), kind,
            max_ctas or 0,
            _native.ptr(status),
            _native.stream_of(device.device),
        )


def copy_host_records_async(host, device, *, host_start, device_start, count):
    """Copy one contiguous record span with hipMemcpyAsync on the current stream.

    Offsets and count are CPU integers; no synchronisation is performed.
    """
    for name, value in (("host_start", host_start), ("device_start", device_start),
                        ("count", count)):
        if type(value) is not int or value < 0:
            raise ValueError(f"{name} must be a nonnegative integer")
    if host.device.type != "cpu" or not host.is_pinned():
        raise ValueError("host records must use pinned CPU memory")
    if device.device.type != "cuda" or host.dtype != device.dtype:
        raise ValueError("device records must be CUDA and match host dtype")
    if host.ndim != 2 or device.ndim != 2 or host.shape[1] != device.shape[1] or host.shape[1] <= 0:
        raise ValueError("host/device records must have the same positive row width")
    if not host.is_contiguous() or not device.is_contiguous():
        raise ValueError("records must be contiguous")
    if host_start > host.shape[0] or count > host.shape[0] - host_start:
        raise ValueError("host record span exceeds its allocation")
    if device_start > device.shape[0] or count > device.shape[0] - device_start:
        raise ValueError("device record span exceeds its allocation")
    if not count:
        return
    row_bytes = host.shape[1] * host.element_size()
    with torch.cuda.device(device.device):
        _native.call(
            "dsa_copy_records_h2d",
            _native.ptr(host[host_start:]),
            _native.ptr(device[device_start:]),
            count * row_bytes,
            _native.stream_of(device.device),
        )
