"""Runtime tables (reference: test/test_runtime.py:7-53)."""
import pytest
import torch

import llaisys_amd as L


def _roundtrip(api, size):
    a = torch.randint(0, 255, (size,), dtype=torch.uint8)
    b = torch.zeros_like(a)
    da, db = api.malloc_device(size), api.malloc_device(size)
    api.memcpy_sync(da, a.data_ptr(), size, L.MemcpyKind.H2D)
    api.memcpy_sync(db, da, size, L.MemcpyKind.D2D)
    api.memcpy_sync(b.data_ptr(), db, size, L.MemcpyKind.D2H)
    api.free_device(da)
    api.free_device(db)
    assert torch.equal(a, b)


def test_cpu_runtime_memcpy():
    api = L.RuntimeAPI(L.DeviceType.CPU)
    assert api.get_device_count() == 1
    _roundtrip(api, 1 << 20)


def test_nvidia_slot_reports_no_devices():
    assert L.RuntimeAPI(L.DeviceType.NVIDIA).get_device_count() == 0


@pytest.mark.gpu
def test_amd_runtime_memcpy_and_streams():
    api = L.RuntimeAPI(L.DeviceType.AMD)
    n = api.get_device_count()
    assert n >= 1
    for i in range(n):
        api.set_device(i)
        _roundtrip(api, 1 << 20)
    s = api.create_stream()
    h = api.malloc_host(4096)
    d = api.malloc_device(4096)
    api.memcpy_async(d, h, 4096, L.MemcpyKind.H2D, s)
    api.stream_synchronize(s)
    api.destroy_stream(s)
    api.free_device(d)
    api.free_host(h)
    api.device_synchronize()


@pytest.mark.gpu
def test_amd_is_default_device_and_cpu_tensors_are_host_memory():
    t = L.Tensor((4,), dtype=L.DataType.F32, device=L.DeviceType.AMD)
    assert t.device_type() == L.DeviceType.AMD
    c = L.Tensor((4,), dtype=L.DataType.F32, device=L.DeviceType.CPU)
    assert c.device_type() == L.DeviceType.CPU
    x = torch.arange(4, dtype=torch.float32)
    c.load(x.data_ptr())
    t.load(x.data_ptr())
    from utils import to_torch

    assert torch.equal(to_torch(t).cpu(), x) and torch.equal(to_torch(c), x)
