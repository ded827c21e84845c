"""GPU parity of the layer glue around the recurrence, through the C-ABI:
the gating prologue (conv output -> L2-normalised q, k, v and the gates) and
the gated RMSNorm epilogue, against the oracle (pinned to HF
transformers' own functions by tests/test_oracle.py) and against the HF
golden vectors directly.

Bars (written per test):
  fp32 outputs   rtol 2e-6 (q, k, g, beta: reduction order, 1-ulp expf /
                 log1pf / sqrtf differences), v bit-exact (a copy);
  bf16 outputs   within one bf16 ulp of the oracle's bf16 rounding: an fp32
                 ulp of difference before the rounding can move it by one.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.gdn_inputs import bf16_to_f32, prefill_inputs, rel_errors
from tests.gpu_util import P, dev, empty, host, host_u16, stream, torch_mod, u16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    torch = torch_mod()
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orionsbelt_amd as ob
    return ob.lib()


def ulp_bf16_diff(a16, b16):
    def key(u):
        u = np.asarray(u, np.uint16).astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - (u & 0x7FFF), u + 0x8000)
    return np.abs(key(a16) - key(b16))


def prologue_inputs(seed, rows, Hk, Hv):
    rs = np.random.RandomState(seed)
    H = 2 * Hk + Hv
    x = rs.randn(rows, H * 128).astype(np.float32)
    x *= rs.uniform(0.05, 5.0, (rows, 1)).astype(np.float32)   # row scales
    a = (3 * rs.randn(rows, Hv)).astype(np.float32)
    b = (4 * rs.randn(rows, Hv)).astype(np.float32)
    A_log = np.log(rs.uniform(0.5, 16, Hv)).astype(np.float32)
    dt_bias = rs.randn(Hv).astype(np.float32)
    return x, a, b, A_log, dt_bias


def gpu_prologue(L, x, a, b, A_log, dt_bias, rows, Hk, Hv, bf16):
    torch = torch_mod()
    dx, da, db_, dA, ddt = (dev(t) for t in (x, a, b, A_log, dt_bias))
    odt = torch.int16 if bf16 else torch.float32
    q = empty((rows, Hk, 128), odt)
    k = empty((rows, Hk, 128), odt)
    v = empty((rows, Hv, 128), odt)
    g = empty((rows, Hv), torch.float32)
    beta = empty((rows, Hv), torch.float32)
    fn = L.kai_run_gdn_gating_prologue_bf16_hip if bf16 else L.kai_run_gdn_gating_prologue_f32_hip
    rc = fn(P(dx), P(da), P(db_), P(dA), P(ddt), P(q), P(k), P(v), P(g), P(beta), rows, Hk, Hv,
            stream())
    assert rc == 0, rc
    get = host_u16 if bf16 else host
    return get(q), get(k), get(v), host(g), host(beta)


@pytest.mark.parametrize("rows,Hk,Hv", [(1, 1, 1), (37, 2, 4), (64, 16, 32), (5, 3, 9)])
def test_gating_prologue_f32_vs_oracle(L, rows, Hk, Hv):
    x, a, b, A_log, dt = prologue_inputs(rows + Hk, rows, Hk, Hv)
    q, k, v, g, beta = gpu_prologue(L, x, a, b, A_log, dt, rows, Hk, Hv, bf16=False)
    rq, rk, rv, rg, rb = orc.gating_prologue(x, a, b, A_log, dt, rows, Hk, Hv)
    np.testing.assert_allclose(q, rq, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(k, rk, rtol=2e-6, atol=1e-7)
    assert np.array_equal(v.view(np.uint32), rv.view(np.uint32))
    np.testing.assert_allclose(g, rg, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(beta, rb, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("rows,Hk,Hv", [(37, 2, 4), (64, 16, 32)])
def test_gating_prologue_bf16_vs_oracle(L, rows, Hk, Hv):
    x, a, b, A_log, dt = prologue_inputs(100 + rows, rows, Hk, Hv)
    q, k, v, g, beta = gpu_prologue(L, x, a, b, A_log, dt, rows, Hk, Hv, bf16=True)
    rq, rk, rv, rg, rb = orc.gating_prologue(x, a, b, A_log, dt, rows, Hk, Hv)
    for got, ref in ((q, rq), (k, rk)):
        assert ulp_bf16_diff(got, orc.f32_to_bf16_bits(ref)).max() <= 1
    assert np.array_equal(v, orc.f32_to_bf16_bits(rv))       # RNE of the copy
    np.testing.assert_allclose(g, rg, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(beta, rb, rtol=2e-6, atol=1e-7)


def test_gating_prologue_vs_hf_golden(L, golden):
    """The HF fixture itself (zero q heads, large rows, softplus threshold)."""
    d = golden("hf_layer.npz")
    rows, Hk, Hv = (int(t) for t in d["gp_dims"])
    q, k, v, g, beta = gpu_prologue(L, d["gp_x"], d["gp_a"], d["gp_b"], d["gp_A_log"],
                                    d["gp_dt_bias"], rows, Hk, Hv, bf16=False)
    np.testing.assert_allclose(q, d["gp_q"], rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(k, d["gp_k"], rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(v, d["gp_v"], rtol=0, atol=0)
    np.testing.assert_allclose(g, d["gp_g"], rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(beta, d["gp_beta"], rtol=2e-6, atol=1e-7)


def test_gating_prologue_full_size_properties(L):
    """B=1, T=16384, Hk=16, Hv=32: every q and k head row has unit norm and
    keeps its direction; v is the rounded copy; gates in range."""
    torch = torch_mod()
    rows, Hk, Hv = 16384, 16, 32
    gen = torch.Generator(device="cuda")
    gen.manual_seed(9)
    x = torch.randn(rows, (2 * Hk + Hv) * 128, generator=gen, device="cuda")
    a = torch.randn(rows, Hv, generator=gen, device="cuda") * 3
    b = torch.randn(rows, Hv, generator=gen, device="cuda") * 4
    A_log = torch.log(torch.rand(Hv, generator=gen, device="cuda") * 15 + 0.5)
    dt = torch.randn(Hv, generator=gen, device="cuda")
    q = torch.empty(rows, Hk, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.empty_like(q)
    v = torch.empty(rows, Hv, 128, dtype=torch.bfloat16, device="cuda")
    g = torch.empty(rows, Hv, device="cuda")
    beta = torch.empty_like(g)
    rc = L.kai_run_gdn_gating_prologue_bf16_hip(P(x), P(a), P(b), P(A_log), P(dt), P(q), P(k),
                                                P(v), P(g), P(beta), rows, Hk, Hv, stream())
    assert rc == 0
    xs = x.view(rows, 2 * Hk + Hv, 128)
    for t, src in ((q, xs[:, :Hk]), (k, xs[:, Hk:2 * Hk])):
        n = t.float().norm(dim=-1)
        assert (n - 1).abs().max().item() < 4e-3                 # bf16 rounding of 128 values
        cos = (t.float() * src).sum(-1) / src.norm(dim=-1)
        assert (cos - 1).abs().max().item() < 4e-3
    assert torch.equal(v, xs[:, 2 * Hk:].to(torch.bfloat16))     # RNE, as torch rounds
    # sigmoid(b) rounds to 1.0 for b > ~17 in fp32 (as torch's does)
    assert (g <= 0).all().item() and (beta >= 0).all().item() and (beta <= 1).all().item()


def test_gating_prologue_rejects_bad_args(L):
    torch = torch_mod()
    t = empty((64, 8 * 128), torch.float32)
    s = empty((64, 8), torch.float32)
    o = empty((64, 8, 128), torch.int16)
    good = [P(t), P(s), P(s), P(s), P(s), P(o), P(o), P(o), P(s), P(s), 64, 2, 4, stream()]
    fn = L.kai_run_gdn_gating_prologue_bf16_hip
    bad = list(good); bad[12] = 3          # Hv % Hk != 0
    assert fn(*bad) != 0
    bad = list(good); bad[0] = ctypes_ptr_off(t, 4)   # misaligned x
    assert fn(*bad) != 0
    bad = list(good); bad[5] = None        # null q
    assert fn(*bad) != 0
    bad = list(good); bad[10] = 0          # nothing to do
    assert fn(*bad) == 0


def ctypes_ptr_off(t, nbytes):
    import ctypes
    return ctypes.c_void_p(t.data_ptr() + nbytes)


# ---- gated RMSNorm ----------------------------------------------------------

def gpu_rmsnorm(L, o, z, w, eps, bf16):
    torch = torch_mod()
    if bf16:
        do, dz, dw = u16(o), u16(z), u16(w)
        y = empty(o.shape, torch.int16)
        rc = L.kai_run_gdn_gated_rmsnorm_bf16_hip(P(do), P(dz), P(dw), P(y), o.size // 128, eps,
                                                 stream())
        assert rc == 0
        return host_u16(y)
    do, dz, dw = dev(o), dev(z), dev(w)
    y = empty(o.shape, torch.float32)
    rc = L.kai_run_gdn_gated_rmsnorm_f32_hip(P(do), P(dz), P(dw), P(y), o.size // 128, eps, stream())
    assert rc == 0
    return host(y)


@pytest.mark.parametrize("rows", [1, 63, 64, 65, 1000])
def test_gated_rmsnorm_f32_vs_oracle(L, rows):
    rs = np.random.RandomState(rows)
    o = (rs.randn(rows, 128) * rs.uniform(1e-3, 10, (rows, 1))).astype(np.float32)
    z = (3 * rs.randn(rows, 128)).astype(np.float32)
    w = (1 + 0.3 * rs.randn(128)).astype(np.float32)
    y = gpu_rmsnorm(L, o, z, w, 1e-6, bf16=False)
    np.testing.assert_allclose(y, orc.gated_rmsnorm_f32(o, z, w, 1e-6), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("rows", [1, 65, 1000])
def test_gated_rmsnorm_bf16_vs_oracle(L, rows):
    rs = np.random.RandomState(50 + rows)
    o = orc.f32_to_bf16_bits(rs.randn(rows, 128) * rs.uniform(1e-3, 10, (rows, 1)))
    z = orc.f32_to_bf16_bits(3 * rs.randn(rows, 128))
    w = orc.f32_to_bf16_bits(1 + 0.3 * rs.randn(128))
    y = gpu_rmsnorm(L, o, z, w, 1e-6, bf16=True)
    diff = ulp_bf16_diff(y, orc.gated_rmsnorm_bf16(o, z, w, 1e-6))
    assert diff.max() <= 1 and (diff > 0).mean() < 0.02


def test_gated_rmsnorm_vs_hf_golden(L, golden):
    d = golden("hf_layer.npz")
    y = gpu_rmsnorm(L, d["rn_f32_o"], d["rn_f32_z"], d["rn_f32_w"], 1e-6, bf16=False)
    np.testing.assert_allclose(y, d["rn_f32_y"], rtol=3e-6, atol=1e-7)
    y16 = gpu_rmsnorm(L, d["rn_bf16_o"], d["rn_bf16_z"], d["rn_bf16_w"], 1e-6, bf16=True)
    diff = ulp_bf16_diff(y16, d["rn_bf16_y"])
    assert diff.max() <= 1 and (diff > 0).mean() < 0.05


def test_gated_rmsnorm_rejects_bad_args(L):
    torch = torch_mod()
    t = empty((64, 128), torch.float32)
    fn = L.kai_run_gdn_gated_rmsnorm_f32_hip
    assert fn(P(t), P(t), P(t), P(t), 64, -1.0, stream()) != 0          # eps < 0
    assert fn(P(t), P(t), P(t), P(t), 64, float("nan"), stream()) != 0  # eps NaN
    assert fn(ctypes_ptr_off(t, 8), P(t), P(t), P(t), 64, 1e-6, stream()) != 0
    assert fn(None, P(t), P(t), P(t), 64, 1e-6, stream()) != 0
    assert fn(None, None, None, None, 0, 1e-6, stream()) == 0


# ---- the three steps together -------------------------------------------------

def test_prologue_prefill_epilogue_chain(L):
    """conv output -> prologue (bf16) -> chunked prefill -> gated RMSNorm
    (bf16), against the same chain on the oracle (fp32 prefill on the
    bf16-rounded q, k, v), at T = 200 (a partial last chunk), Hk=2, Hv=4."""
    torch = torch_mod()
    T, Hk, Hv = 200, 2, 4
    x, a, b, A_log, dt = prologue_inputs(7, T, Hk, Hv)
    q16, k16, v16, g, beta = gpu_prologue(L, x, a, b, A_log, dt, T, Hk, Hv, bf16=True)
    rs = np.random.RandomState(8)
    S0 = (0.02 * rs.randn(1, Hv, 128, 128)).astype(np.float32)
    dq, dk_, dv_ = (u16(t) for t in (q16, k16, v16))
    dg, dbeta, dS = dev(g), dev(beta), dev(S0)
    do = empty((1, T, Hv, 128), torch.int16)
    rc = L.kai_run_gdn_chunk_delta_rule_bf16_f32_hip(P(dq), P(dk_), P(dv_), P(dg), P(dbeta), P(do),
                                                      P(dS), 1, T, Hv, Hk, 1 / math.sqrt(128),
                                                      stream())
    assert rc == 0
    z = orc.f32_to_bf16_bits(3 * rs.randn(T * Hv, 128))
    w = orc.f32_to_bf16_bits(1 + 0.3 * rs.randn(128))
    dz, dw = u16(z), u16(w)
    y = empty((T * Hv, 128), torch.int16)
    rc = L.kai_run_gdn_gated_rmsnorm_bf16_hip(P(do), P(dz), P(dw), P(y), T * Hv, 1e-6, stream())
    assert rc == 0
    y = host_u16(y)
    # oracle chain
    rq, rk, rv, rg, rb = orc.gating_prologue(x, a, b, A_log, dt, T, Hk, Hv)
    bf = lambda t: bf16_to_f32(orc.f32_to_bf16_bits(t))  # noqa: E731
    ro, _ = orc.chunk_gdr(bf(rq).reshape(1, T, Hk, 128), bf(rk).reshape(1, T, Hk, 128),
                          bf(rv).reshape(1, T, Hv, 128), rg.reshape(1, T, Hv), rb.reshape(1, T, Hv),
                          S0, 1, T, Hv, Hk, 128, 128, 64)
    ry = orc.gated_rmsnorm_f32(ro.reshape(T * Hv, 128), bf16_to_f32(z), bf16_to_f32(w), 1e-6)
    mx, l2 = rel_errors(bf16_to_f32(y), ry)
    assert mx <= 3e-2 and l2 <= 1.5e-2, (mx, l2)
