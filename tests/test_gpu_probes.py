"""bench.py's device-ceiling probes (bench_probes.so): they run, measure finite rates and touch what they claim."""
import ctypes as C
import math
import os

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    L = C.CDLL(os.path.join(ROOT, "bench_probes.so"))
    L.probe_last_error.restype = C.c_char_p
    L.probe_stream_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_double), C.c_void_p]
    L.probe_random_lines.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_void_p, C.c_size_t,
                                     C.POINTER(C.c_double), C.c_void_p]
    L.probe_atomic_lines.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.POINTER(C.c_double), C.c_void_p]
    return L


def test_stream_copy_probe_copies(lib):
    src = torch.arange(1 << 22, dtype=torch.float32, device="cuda")
    dst = torch.zeros_like(src)
    r = C.c_double(0)
    assert lib.probe_stream_copy(src.data_ptr(), dst.data_ptr(), src.numel() * 4, 3, C.byref(r), 0) == 0
    torch.cuda.synchronize()
    assert torch.equal(src, dst) and math.isfinite(r.value) and r.value > 1e10
    assert lib.probe_stream_copy(src.data_ptr(), dst.data_ptr(), 17, 3, C.byref(r), 0) != 0  # not a multiple of 16


@pytest.mark.parametrize("part", [0, 1])
def test_random_lines_probe_reads_inside_the_table(lib, part):
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    table = torch.full((1 << 23,), -1, dtype=torch.int32, device="cuda")   # 32 MiB of 0xffffffff
    sink = torch.zeros(cus * 16 * 256, dtype=torch.int32, device="cuda")
    r = C.c_double(0)
    assert lib.probe_random_lines(table.data_ptr(), table.numel() * 4, part, 3, sink.data_ptr(), sink.numel() * 4,
                                  C.byref(r), 0) == 0
    torch.cuda.synchronize()
    assert bool((sink == -1).all()), "every lane xor-ed three words of the table"
    assert math.isfinite(r.value) and r.value > 1e9
    assert lib.probe_random_lines(table.data_ptr(), table.numel() * 4, part, 3, sink.data_ptr(), 64, C.byref(r),
                                  0) != 0


def test_atomic_lines_probe_adds_every_request(lib):
    buf = torch.zeros(1 << 22, dtype=torch.float32, device="cuda")  # 16 MiB
    rates = {}
    for dw in (1, 4, 16):
        r = C.c_double(0)
        assert lib.probe_atomic_lines(buf.data_ptr(), buf.numel() * 4, dw, C.byref(r), 0) == 0
        assert math.isfinite(r.value) and r.value > 1e8, (dw, r.value)
        rates[dw] = r.value
    torch.cuda.synchronize()
    lanes = torch.cuda.get_device_properties(0).multi_processor_count * 256
    expected = sum(6 * lanes * max(1, ((1 << 24) * dw) // lanes) for dw in (1, 4, 16))
    assert int(buf.double().sum().item()) == expected
    assert lib.probe_atomic_lines(buf.data_ptr(), buf.numel() * 4, 3, C.byref(r), 0) != 0
