"""GPU byte-exactness of the host-record gather and contiguous copy (A11).

Cases follow operators/common/tests/test_kv_transfer.py: storage offsets
smaller than 16 bytes on both sides, bounded grids, counted prefixes whose
tail ids are invalid, guard bytes around both views.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("host_offset,device_offset", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("max_ctas", [None, 1, 2])
@pytest.mark.parametrize("dtype,width", [(torch.bfloat16, 8), (torch.bfloat16, 576),
                                         (torch.float32, 19), (torch.uint8, 656)])
def test_gather_storage_offsets_preserve_other_bytes(gpu, dtype, width, host_offset,
                                                     device_offset, max_ctas):
    from cxldsagr_amd.kv_transfer import gather_host_records, transfer_status

    rows = 4
    host_storage = torch.arange(rows * width + 8, dtype=torch.float32).to(dtype).pin_memory()
    host = host_storage[host_offset:host_offset + rows * width].view(rows, width)
    device_storage = torch.full((rows * width + 8,), 17, dtype=dtype, device=gpu)
    device = device_storage[device_offset:device_offset + rows * width].view(rows, width)
    expected = device_storage.cpu()
    before = host_storage.clone()
    host_ids = torch.tensor([3, 0, 2], dtype=torch.int64, device=gpu)
    device_ids = torch.tensor([1, 3, 0], dtype=torch.int64, device=gpu)
    expected[device_offset:device_offset + rows * width].view(rows, width)[[1, 3, 0]] = host[[3, 0, 2]]
    gather_host_records(host, device, host_ids, device_ids, max_ctas=max_ctas)
    torch.cuda.synchronize()
    assert torch.equal(device_storage.cpu(), expected)
    assert torch.equal(host_storage, before)
    assert transfer_status(gpu) == 0


@pytest.mark.parametrize("count_dtype", [torch.int64, torch.uint32])
@pytest.mark.parametrize("count", [0, 1, 3])
@pytest.mark.parametrize("max_ctas", [None, 1])
def test_counted_gather_never_reads_uninitialized_tail(gpu, count_dtype, count, max_ctas):
    from cxldsagr_amd.kv_transfer import gather_host_records, transfer_status

    host = torch.arange(6 * 576, dtype=torch.float32).bfloat16().reshape(6, 576).pin_memory()
    device = torch.full((6, 576), -17, dtype=host.dtype, device=gpu)
    host_ids = torch.full((8,), -1, dtype=torch.int64, device=gpu)
    device_ids = torch.full_like(host_ids, -1)
    host_ids[:count] = torch.tensor([4, 1, 5][:count], device=gpu)
    device_ids[:count] = torch.tensor([1, 3, 2][:count], device=gpu)
    valid_count = torch.tensor([count], dtype=count_dtype, device=gpu)
    expected = device.cpu()
    expected[[1, 3, 2][:count]] = host[[4, 1, 5][:count]]
    gather_host_records(host, device, host_ids, device_ids, max_ctas=max_ctas,
                        valid_count=valid_count)
    torch.cuda.synchronize()
    assert torch.equal(device.cpu(), expected)
    assert transfer_status(gpu) == 0  # invalid tail ids were never touched


def test_invalid_ids_are_flagged_not_trapped(gpu):
    from cxldsagr_amd.kv_transfer import gather_host_records, transfer_status

    host = torch.arange(4 * 16, dtype=torch.uint8).reshape(4, 16).pin_memory()
    device = torch.zeros(4, 16, dtype=torch.uint8, device=gpu)
    host_ids = torch.tensor([1, 9, 2], dtype=torch.int64, device=gpu)
    device_ids = torch.tensor([0, 1, 5], dtype=torch.int64, device=gpu)
    gather_host_records(host, device, host_ids, device_ids)
    assert transfer_status(gpu) == 1
    expected = torch.zeros(4, 16, dtype=torch.uint8)
    expected[0] = host[1]
    assert torch.equal(device.cpu(), expected)
    bad = torch.tensor([9], dtype=torch.int64, device=gpu)
    gather_host_records(host, device, host_ids, device_ids, valid_count=bad)
    assert transfer_status(gpu) == 2


def test_large_fp8_record_gather_matches_index_copy(gpu):
    from cxldsagr_amd.kv_transfer import gather_host_records

    gen = torch.Generator().manual_seed(3)
    host = torch.randint(0, 256, (20000, 656), dtype=torch.uint8, generator=gen).pin_memory()
    device = torch.zeros(5001, 656, dtype=torch.uint8, device=gpu)
    host_ids = torch.randperm(20000, generator=gen)[:4000]
    device_ids = torch.randperm(5000, generator=gen)[:4000] + 1
    gather_host_records(host, device, host_ids.to(gpu), device_ids.to(gpu), max_ctas=128)
    expected = torch.zeros(5001, 656, dtype=torch.uint8)
    expected[device_ids] = host[host_ids]
    assert torch.equal(device.cpu(), expected)


@pytest.mark.parametrize("dtype,width", [(torch.bfloat16, 576), (torch.float32, 7), (torch.uint8, 13)])
@pytest.mark.parametrize("count", [0, 3])
def test_contiguous_copy_on_private_stream(gpu, dtype, width, count):
    from cxldsagr_amd.kv_transfer import copy_host_records_async

    host_storage = torch.arange(8 * width + 3, dtype=torch.float32).to(dtype).pin_memory()
    host = host_storage[1:1 + 8 * width].view(8, width)
    device_storage = torch.full((8 * width + 5,), 17, dtype=dtype, device=gpu)
    device = device_storage[2:2 + 8 * width].view(8, width)
    expected = device_storage.cpu()
    expected[2:2 + 8 * width].view(8, width)[3:3 + count] = host[1:1 + count]
    producer = torch.cuda.Stream()
    consumer = torch.cuda.Stream()
    producer.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(producer):
        copy_host_records_async(host, device, host_start=1, device_start=3, count=count)
        ready = torch.cuda.Event()
        ready.record()
    with torch.cuda.stream(consumer):
        consumer.wait_event(ready)
        observed = device_storage.clone()
    consumer.synchronize()
    assert torch.equal(observed.cpu(), expected)


@pytest.mark.parametrize("host_start,device_start,count", [(4, 0, 1), (0, 4, 1), (3, 0, 2), (0, 3, 2)])
def test_contiguous_copy_rejects_out_of_bounds_span(gpu, host_start, device_start, count):
    from cxldsagr_amd.kv_transfer import copy_host_records_async

    host = torch.zeros(4, 7, pin_memory=True)
    device = torch.zeros_like(host, device=gpu)
    with pytest.raises(ValueError, match="span exceeds"):
        copy_host_records_async(host, device, host_start=host_start, device_start=device_start,
                                count=count)
