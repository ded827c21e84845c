"""The measurement probes of the C-ABI (kai_gdn_hip_probe_*): the copy
probe copies exactly, the read and MFMA probes run, flop counts follow the
launch shape, and bad arguments are refused before anything is launched."""
import ctypes

import numpy as np
import pytest

from tests.gpu_util import P, host, stream, torch_mod

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    torch = torch_mod()
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orionsbelt_amd as ob
    return ob.lib()


def test_probe_copy_exact_and_read_runs(L):
    torch = torch_mod()
    sink = torch.empty(L.kai_gdn_hip_probe_sink_bytes() // 4 + 1, dtype=torch.float32, device="cuda")
    for n in (4, 1000, (1 << 20) + 36):  # 16-byte words, with a partial last block
        src = torch.randint(-2**31, 2**31 - 1, (4 * n,), dtype=torch.int32, device="cuda")
        dst = torch.zeros_like(src)
        assert L.kai_gdn_hip_probe_stream(P(src), P(dst), 16 * n, 0, P(sink), stream()) == 0
        assert np.array_equal(host(dst), host(src))
        assert L.kai_gdn_hip_probe_stream(P(src), None, 16 * n, 1, P(sink), stream()) == 0
    torch.cuda.synchronize()


def test_probe_mfma_counts_and_runs(L):
    torch = torch_mod()
    sink = torch.empty(L.kai_gdn_hip_probe_sink_bytes() // 4 + 1, dtype=torch.float32, device="cuda")
    f0, f1 = ctypes.c_ulonglong(0), ctypes.c_ulonglong(0)
    assert L.kai_gdn_hip_probe_mfma_bf16(10, 0, P(sink), ctypes.byref(f0), stream()) == 0
    assert L.kai_gdn_hip_probe_mfma_bf16(10, 1, P(sink), ctypes.byref(f1), stream()) == 0
    torch.cuda.synchronize()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    waves = cus * 16 * 4
    assert f0.value == waves * 10 * 4 * 2 * 32 * 32 * 16
    assert f1.value == waves * 10 * 8 * 2 * 16 * 16 * 32
    assert np.isfinite(host(sink)).all()


def test_probe_rejects_bad_arguments(L):
    torch = torch_mod()
    t = torch.empty(1 << 16, dtype=torch.float32, device="cuda")
    f = ctypes.c_ulonglong(0)
    assert L.kai_gdn_hip_probe_stream(P(t), P(t), 17, 0, P(t), stream()) != 0        # not a multiple of 16
    assert L.kai_gdn_hip_probe_stream(P(t), None, 16, 0, P(t), stream()) != 0        # copy without dst
    assert L.kai_gdn_hip_probe_stream(P(t), P(t), 16, 2, P(t), stream()) != 0        # unknown mode
    assert L.kai_gdn_hip_probe_mfma_bf16(0, 0, P(t), ctypes.byref(f), stream()) != 0
    assert L.kai_gdn_hip_probe_mfma_bf16(1, 2, P(t), ctypes.byref(f), stream()) != 0
