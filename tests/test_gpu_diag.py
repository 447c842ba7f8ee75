"""The atomic line-request ceiling probe behind bench.py's scatter roofline (include/graft_diag.h)."""
import ctypes as C
import importlib
import math

import pytest

torch = pytest.importorskip("torch")
P = importlib.import_module("3dmaker_amd")


@pytest.mark.gpu
def test_atomic_line_rate_probe():
    buf = torch.zeros(1 << 22, dtype=torch.float32, device="cuda:0")  # 16 MiB
    sp = torch.cuda.current_stream().cuda_stream
    rates = {}
    for dw in (1, 4, 16):
        r = C.c_double(0.0)
        P.check(P.lib().graft_diag_atomic_line_rate(buf.data_ptr(), buf.numel() * 4, dw, C.byref(r), sp))
        assert math.isfinite(r.value) and r.value > 1e8, (dw, r.value)
        rates[dw] = r.value
    # every lane of the warm-up and 5 timed launches added 1.0 inside the buffer, none lost
    lanes = torch.cuda.get_device_properties(0).multi_processor_count * 256
    expected = sum(6 * lanes * max(1, ((1 << 24) * dw) // lanes) for dw in (1, 4, 16))
    assert int(buf.double().sum().item()) == expected
    # a request's cost does not grow with the dwords it carries (within a factor of 2)
    assert rates[16] > 0.5 * rates[1], rates


@pytest.mark.gpu
def test_atomic_line_rate_probe_rejects_bad_arguments():
    buf = torch.zeros(1 << 10, dtype=torch.float32, device="cuda:0")  # 4 KiB: too small
    r = C.c_double(0.0)
    sp = torch.cuda.current_stream().cuda_stream
    assert P.lib().graft_diag_atomic_line_rate(buf.data_ptr(), buf.numel() * 4, 4, C.byref(r), sp) != 0
    big = torch.zeros(1 << 16, dtype=torch.float32, device="cuda:0")
    assert P.lib().graft_diag_atomic_line_rate(big.data_ptr(), big.numel() * 4, 3, C.byref(r), sp) != 0
    assert P.lib().graft_diag_atomic_line_rate(big.data_ptr(), big.numel() * 4, 32, C.byref(r), sp) != 0
