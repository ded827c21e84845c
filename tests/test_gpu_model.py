"""GPU parity of the hybrid decode loop's matmuls through the C-ABI: the
per-output-channel int8 quantiser (bit-exact against the oracle's
restatement of the reference's quantize_weight) and the int8 weight-only
GEMM with fp16 activations (fp32 accumulation in MFMA order against the
oracle's float64 sum: rtol 1e-4 with an absolute floor of 1e-5 of the
output's largest magnitude; deterministic across runs).
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import P, dev, empty, host, stream, torch_mod

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    torch = torch_mod()
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orionsbelt_amd as ob
    return ob.lib()


def gpu_quantize(L, W):
    torch = torch_mod()
    N, K = W.shape
    dW = dev(W)
    q = empty((N, K), torch.int8)
    s = empty((N,), torch.float32)
    assert L.kai_run_gdn_w8_quantize_hip(P(dW), P(q), P(s), N, K, stream()) == 0
    return host(q), host(s)


def gpu_gemm(L, x16, q, s):
    torch = torch_mod()
    M, K = x16.shape
    N = q.shape[0]
    dx, dq, ds = dev(x16.view(np.int16)), dev(q), dev(s)
    y = empty((M, N), torch.float32)
    nb = L.kai_gdn_w8a16_gemm_workspace_bytes(M, N, K)
    ws = empty((max(nb, 16) // 4,), torch.float32)
    assert L.kai_run_gdn_w8a16_gemm_hip(P(dx), P(dq), P(ds), P(y), M, N, K, P(ws), nb, stream()) == 0
    return host(y)


def test_w8_quantize_bit_exact(L):
    rs = np.random.RandomState(1)
    W = rs.randn(300, 1024).astype(np.float32)
    W[7] = 0.0
    W[11, :4] = [127.0, 63.5, -63.5, 0.5]       # halves of the scale 1.0 round away from zero
    W[11, 4:] = 0.0
    q, s = gpu_quantize(L, W)
    rq, rs_ = orc.w8_quantize(W)
    assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs_.view(np.uint32))
    assert list(q[11, :4]) == [127, 64, -64, 1]


@pytest.mark.parametrize("M,N,K", [(1, 48, 256), (5, 2560, 4096), (16, 8192, 2560), (3, 32, 2560),
                                   (16, 2560, 9216), (1, 9216, 2560)])
def test_w8a16_gemm_vs_oracle(L, M, N, K):
    rs = np.random.RandomState(M * 7 + N)
    x = rs.randn(M, K).astype(np.float16)
    W = (rs.randn(N, K) * rs.uniform(0.01, 2.0, (N, 1))).astype(np.float32)
    q, s = orc.w8_quantize(W)
    y = gpu_gemm(L, x.view(np.uint16), q, s)
    ref = orc.w8_gemm(x.view(np.uint16), q, s)
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    y2 = gpu_gemm(L, x.view(np.uint16), q, s)
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))       # deterministic


def test_w8a16_gemm_rejects_bad_args(L):
    torch = torch_mod()
    t = empty((16 * 2560,), torch.float32)
    fn = L.kai_run_gdn_w8a16_gemm_hip
    assert fn(P(t), P(t), P(t), P(t), 17, 32, 256, P(t), 1 << 20, stream()) != 0    # M > 16
    assert fn(P(t), P(t), P(t), P(t), 1, 33, 256, P(t), 1 << 20, stream()) != 0    # N % 16
    assert fn(P(t), P(t), P(t), P(t), 1, 32, 200, P(t), 1 << 20, stream()) != 0    # K % 256
    nb = L.kai_gdn_w8a16_gemm_workspace_bytes(4, 2560, 4096)
    assert nb > 0
    assert fn(P(t), P(t), P(t), P(t), 4, 2560, 4096, P(t), nb - 4, stream()) != 0  # workspace short
    off = ctypes.c_void_p(t.data_ptr() + 8)
    assert fn(off, P(t), P(t), P(t), 1, 32, 256, P(t), 1 << 20, stream()) != 0    # misaligned x
    assert fn(None, None, None, None, 0, 32, 256, None, 0, stream()) == 0         # nothing to do
