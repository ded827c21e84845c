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


def gpu_gemm_tiled(L, x16, q, s, reps=1):
    """Tile Wq on the device, run the tiled GEMM `reps` times on one zeroed
    workspace; returns the outputs and the workspace's counters after."""
    torch = torch_mod()
    M, K = x16.shape
    N = q.shape[0]
    dx, dq, ds = dev(x16.view(np.int16)), dev(q), dev(s)
    wt = torch.empty_like(dq)
    assert L.kai_run_gdn_w8_tile_hip(P(dq), P(wt), N, K, stream()) == 0
    nb = L.kai_gdn_w8a16_gemm_tiled_workspace_bytes(M, N, K)
    ws = torch.zeros(max(nb, 256) // 4, dtype=torch.float32, device="cuda")
    ys = []
    for _ in range(reps):
        y = empty((M, N), torch.float32)
        assert L.kai_run_gdn_w8a16_gemm_tiled_hip(P(dx), P(wt), P(ds), P(y), M, N, K, P(ws), nb, stream()) == 0
        ys.append(host(y))
    cnt = host(ws.view(torch.int32))[-(N // 64):] if nb else np.zeros(1, np.int32)
    return ys, cnt


@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (5, 2560, 4096), (16, 12352, 2560), (3, 2560, 9216),
                                   (16, 1024, 512), (1, 18432, 2560),
                                   # M <= 3: the small-batch form (8 waves per tile at K = 2560,
                                   # 16 at 4096 and 9216)
                                   (1, 2560, 4096), (2, 12352, 2560), (3, 640, 2560), (1, 2560, 9216),
                                   (2, 10240, 2560), (3, 2560, 4096),
                                   # M > 16: the prefill GEMM (128-row blocks: ragged row tails,
                                   # a half channel block when N % 128 == 64, the 4B shapes)
                                   (17, 64, 256), (100, 192, 512), (300, 2560, 9216), (129, 18432, 2560),
                                   # M >= 512: its 256 x 256 form (ragged rows, blocks with 1-3 of
                                   # their four 64-channel groups; 4, 8 and 12 k steps end its
                                   # three-step buffer ring after its first, second and third slot)
                                   (1000, 12352, 2560), (513, 2560, 9216), (600, 192, 512),
                                   (2048, 10240, 2560), (520, 64, 256), (777, 320, 768),
                                   # 16 and 32 row blocks
                                   (4096, 320, 768), (8192, 192, 512)])
def test_w8a16_gemm_tiled_vs_oracle(L, M, N, K):
    """The tiled-weight GEMM (the hybrid loop's): against the oracle at the
    row-major GEMM's bar, deterministic over calls that share one workspace
    (split shapes: down and out_proj), and the workspace's counters are back
    at zero after every call."""
    rs = np.random.RandomState(M * 11 + N)
    x = rs.randn(M, K).astype(np.float16)
    W = (rs.randn(N, K) * rs.uniform(0.01, 2.0, (N, 1))).astype(np.float32)
    q, s = orc.w8_quantize(W)
    (y, y2), cnt = gpu_gemm_tiled(L, x.view(np.uint16), q, s, reps=2)
    ref = orc.w8_gemm(x.view(np.uint16), q, s)
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))
    assert not cnt.any()


def test_w8a16_gemm_tiled_rejects_bad_args(L):
    torch = torch_mod()
    t = empty((16 * 4096,), torch.float32)
    assert L.kai_run_gdn_w8_tile_hip(P(t), P(t), 64, 256, stream()) != 0          # in place
    assert L.kai_run_gdn_w8_tile_hip(P(t), None, 64, 256, stream()) != 0
    u = empty((16 * 4096,), torch.float32)
    assert L.kai_run_gdn_w8_tile_hip(P(t), P(u), 48, 256, stream()) != 0          # N % 64
    fn = L.kai_run_gdn_w8a16_gemm_tiled_hip
    assert fn(P(t), P(u), P(t), P(t), -1, 64, 256, P(t), 1 << 20, stream()) != 0  # M < 0
    assert fn(P(t), P(u), P(t), P(t), 17, 64, 200, P(t), 1 << 20, stream()) != 0  # K % 256 (many rows)
    assert fn(P(t), P(u), P(t), P(t), 1, 48, 256, P(t), 1 << 20, stream()) != 0   # N % 64
    assert fn(P(t), P(u), P(t), P(t), 1, 64, 200, P(t), 1 << 20, stream()) != 0   # K % 256
    nb = L.kai_gdn_w8a16_gemm_tiled_workspace_bytes(4, 2560, 4096)
    assert nb > 0
    assert fn(P(t), P(u), P(t), P(t), 4, 2560, 4096, None, nb, stream()) != 0      # split needs a workspace
    assert fn(P(t), P(u), P(t), P(t), 4, 2560, 4096, P(t), nb - 4, stream()) != 0


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


# ---- attention decode --------------------------------------------------------

def gpu_attn(L, q16, k16, v16, length, scaling):
    torch = torch_mod()
    B, Hq, D = q16.shape
    Hkv, Tmax = k16.shape[1], k16.shape[2]
    dq, dk, dv = (dev(a.view(np.int16)) for a in (q16, k16, v16))
    out = empty((B, Hq, D), torch.float32)
    nb = L.kai_gdn_attn_decode_workspace_bytes(B, Hq, length)
    ws = empty((nb // 4,), torch.float32)
    rc = L.kai_run_gdn_attn_decode_f16kv_hip(P(dq), P(dk), P(dv), P(out), B, Hq, Hkv, Tmax, length,
                                              scaling, P(ws), nb, stream())
    assert rc == 0, rc
    return host(out)


@pytest.mark.parametrize("B,Hq,Hkv,Tmax,length", [(1, 4, 1, 64, 1), (2, 16, 4, 300, 300),
                                                   (3, 8, 4, 1000, 777), (1, 16, 4, 4096, 4096),
                                                   (16, 16, 4, 640, 513), (16, 16, 4, 4200, 4100)])
def test_attn_decode_vs_oracle(L, B, Hq, Hkv, Tmax, length):
    """Up to 16 sequences, GQA groups of 1 to 4 query heads, lengths that end
    inside a 16-position group and inside a 256-position span."""
    rs = np.random.RandomState(length + B)
    D = 256
    q = (rs.randn(B, Hq, D) * 0.5).astype(np.float16)
    k = rs.randn(B, Hkv, Tmax, D).astype(np.float16)
    v = rs.randn(B, Hkv, Tmax, D).astype(np.float16)
    k[:, :, length:] = np.float16(1e4)                            # past the length: must not count
    out = gpu_attn(L, q.view(np.uint16), k.view(np.uint16), v.view(np.uint16), length, 1 / 16)
    ref = orc.attn_decode(q.view(np.uint16), k.view(np.uint16), v.view(np.uint16), length, 1 / 16)
    np.testing.assert_allclose(out, ref, rtol=2e-5, atol=2e-5)


def test_attn_decode_peaked_and_long(L):
    """A dominant key selects its value (the softmax's max tracking across
    spans and waves), at 32K positions."""
    torch = torch_mod()
    B, Hq, Hkv, T, D = 1, 16, 4, 32768, 256
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    k = (torch.randn(B, Hkv, T, D, generator=gen, device="cuda") * 0.1).half()
    v = torch.randn(B, Hkv, T, D, generator=gen, device="cuda").half()
    q = torch.zeros(B, Hq, D, device="cuda").half()
    q[:, :, :] = 1.0
    hot = [123, 20000, 32767, 5]                                 # one per kv head
    for kv, t in enumerate(hot):
        k[0, kv, t] = 2.0
    out = torch.empty(B, Hq, D, device="cuda")
    nb = L.kai_gdn_attn_decode_workspace_bytes(B, Hq, T)
    ws = torch.empty(nb // 4, device="cuda")
    assert L.kai_run_gdn_attn_decode_f16kv_hip(P(q), P(k), P(v), P(out), B, Hq, Hkv, T, T, 1 / 16,
                                               P(ws), nb, stream()) == 0
    torch.cuda.synchronize()
    for h in range(Hq):
        kv = h // 4
        assert torch.allclose(out[0, h], v[0, kv, hot[kv]].float(), rtol=1e-3, atol=1e-3)


def test_attn_decode_rejects_bad_args(L):
    torch = torch_mod()
    t = empty((1 << 16,), torch.float32)
    fn = L.kai_run_gdn_attn_decode_f16kv_hip
    args = [P(t), P(t), P(t), P(t), 1, 16, 4, 64, 64, 0.0625, P(t), 1 << 18, stream()]
    bad = list(args); bad[5] = 15                                 # Hq % Hkv
    assert fn(*bad) != 0
    bad = list(args); bad[5] = 32                                 # Hq / Hkv > 4
    assert fn(*bad) != 0
    bad = list(args); bad[8] = 65                                 # length > max_len
    assert fn(*bad) != 0
    bad = list(args); bad[11] = 16                                # workspace short
    assert fn(*bad) != 0
    bad = list(args); bad[4] = 0                                  # nothing to do
    assert fn(*bad) == 0
