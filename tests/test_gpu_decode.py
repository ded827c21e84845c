"""GPU parity of the single-token matrix-state delta-rule decode.

Oracle: orc_delta_rule_decode_f32 (ref_delta_rule, gpu/gdn_gpu_validate.c:
100-118, with per-head gates and the HF q scale).  Bar: BASELINE's <= 1e-4
relative on the final state and outputs, applied element-wise as
|got - ref| <= 1e-4 * |ref| + 1e-6 (the 1e-6 floor covers outputs that
cancel to ~0).  The reference validator's own rule (fail iff max_abs > 1e-4
and max_rel > 1e-3, gdn_gpu_validate.c:57-58) is checked on its own cases.
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.gdn_inputs import decode_inputs, validator_pass
from tests.gpu_util import P, dev, empty, host, host_u16, stream, torch_mod

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    torch = torch_mod()
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orionsbelt_amd as ob
    return ob.lib()


def gpu_decode(L, S, q, k, v, g, beta, B, Hv, Hk, dk, dv, q_scale, steps=1, f16=False):
    import orionsbelt_amd as ob
    torch = torch_mod()
    dS = dev(S.view(np.int16) if f16 else S)
    dq, dk_, dv_, dg, db = dev(q), dev(k), dev(v), dev(g), dev(beta)
    do = empty((B, Hv, dv), torch.float32)
    fn = L.kai_run_gdn_delta_rule_decode_f16state_hip if f16 else \
        L.kai_run_gdn_delta_rule_decode_f32_hip
    for _ in range(steps):
        ob.check(fn(P(dS), P(dq), P(dk_), P(dv_), P(dg), P(db), P(do), B, Hv, Hk, dk, dv,
                    q_scale, stream()), "decode")
    return (host_u16(dS) if f16 else host(dS)), host(do)


def assert_rel(got, ref, rtol=1e-4, atol=1e-6, label=""):
    d = np.abs(np.asarray(got, np.float64) - ref)
    bad = d > rtol * np.abs(ref) + atol
    assert not bad.any(), f"{label}: {int(bad.sum())} elements off, max diff {d.max():.3e}"


@pytest.mark.parametrize("B,Hv,Hk,dk,dv", [(64, 32, 16, 128, 128), (3, 4, 2, 128, 128),
                                          (2, 8, 8, 64, 64), (5, 4, 1, 32, 32),
                                          (2, 4, 2, 128, 64), (2, 2, 2, 32, 128)])
def test_decode_vs_oracle(L, B, Hv, Hk, dk, dv):
    S, q, k, v, g, beta = decode_inputs(B * 7 + dk, B, Hv, Hk, dk, dv)
    qs = 1.0 / math.sqrt(dk)
    Sg, og = gpu_decode(L, S, q, k, v, g, beta, B, Hv, Hk, dk, dv, qs)
    Sr, orf = orc.delta_rule_decode(S, q, k, v, g, beta, B, Hv, Hk, dk, dv, qs)
    assert_rel(Sg, Sr, label="state")
    assert_rel(og, orf, label="output")


def test_decode_multi_step_state_carry(L):
    B, Hv, Hk, d = 4, 8, 4, 128
    S, q, k, v, g, beta = decode_inputs(31, B, Hv, Hk, d, d)
    qs = 1.0 / math.sqrt(d)
    Sg, og = gpu_decode(L, S, q, k, v, g, beta, B, Hv, Hk, d, d, qs, steps=8)
    Sr = S
    for _ in range(8):
        Sr, orf = orc.delta_rule_decode(Sr, q, k, v, g, beta, B, Hv, Hk, d, d, qs)
    assert_rel(Sg, Sr, rtol=2e-4, label="state after 8 steps")
    assert_rel(og, orf, rtol=2e-4, atol=2e-6, label="output after 8 steps")


# The reference validator's delta-rule cases (gdn_gpu_validate.c:621-640):
# scalar beta/decay for all heads, no q scale, S in [-0.01, 0.01],
# k, q L2-normalised U(-1, 1), v in [-0.5, 0.5].
VALIDATOR_CASES = [
    ("delta_0.8B", 16, 128, 0.5, 0.9), ("delta_4B_32heads", 32, 128, 0.5, 0.9),
    ("delta_decay_0.01", 16, 128, 0.5, 0.01), ("delta_decay_0.99", 16, 128, 0.5, 0.99),
    ("delta_decay_1.0", 16, 128, 0.5, 1.0), ("delta_beta_0", 16, 128, 0.0, 0.9),
    ("delta_beta_1", 16, 128, 1.0, 0.9), ("delta_64x64", 8, 64, 0.5, 0.9),
    ("delta_32x32", 4, 32, 0.5, 0.9),
]


@pytest.mark.parametrize("name,H,d,beta,decay", VALIDATOR_CASES)
def test_decode_validator_cases(L, name, H, d, beta, decay):
    rs = np.random.RandomState(abs(hash(name)) % 2**31)
    S = rs.uniform(-0.01, 0.01, (1, H, d, d)).astype(np.float32)
    k = rs.uniform(-1, 1, (1, H, d))
    q = rs.uniform(-1, 1, (1, H, d))
    k = (k / np.linalg.norm(k, axis=-1, keepdims=True)).astype(np.float32)
    q = (q / np.linalg.norm(q, axis=-1, keepdims=True)).astype(np.float32)
    v = rs.uniform(-0.5, 0.5, (1, H, d)).astype(np.float32)
    g = np.full((1, H), np.log(np.float32(decay)) if decay > 0 else -np.inf, np.float32)
    bt = np.full((1, H), beta, np.float32)
    Sg, og = gpu_decode(L, S, q, k, v, g, bt, 1, H, H, d, d, 1.0)
    # reference loop: ref_delta_rule per head with the same decay value
    Sr = S.copy()
    orf = np.empty((1, H, d), np.float32)
    dec = float(np.exp(np.float32(g[0, 0]))) if decay > 0 else 0.0
    for h in range(H):
        Sh, oh = orc.delta_rule_head(Sr[0, h].ravel(), k[0, h], v[0, h], q[0, h], beta, dec, d, d)
        Sr[0, h] = Sh.reshape(d, d)
        orf[0, h] = oh
    ok_o, *_ = validator_pass(og, orf)
    ok_s, *_ = validator_pass(Sg, Sr)
    assert ok_o and ok_s, name
    assert_rel(Sg, Sr, label=name + " state")
    assert_rel(og, orf, label=name + " out")


def test_decode_f16_state(L):
    B, Hv, Hk, d = 8, 32, 16, 128
    S, q, k, v, g, beta = decode_inputs(77, B, Hv, Hk, d, d)
    S16 = S.astype(np.float16).view(np.uint16)
    qs = 1.0 / math.sqrt(d)
    Sg, og = gpu_decode(L, S16, q, k, v, g, beta, B, Hv, Hk, d, d, qs, f16=True)
    Sr, orf = orc.delta_rule_decode_f16state(S16, q, k, v, g, beta, B, Hv, Hk, d, d, qs)
    # identical arithmetic up to summation order: the narrowed states agree to
    # one fp16 ulp, the outputs to 1e-4
    a = Sg.view(np.float16).astype(np.float32)
    r = Sr.view(np.float16).astype(np.float32)
    ulp = np.spacing(np.abs(r).astype(np.float16)).astype(np.float32)
    assert np.all(np.abs(a - r) <= ulp), "f16 state differs by more than 1 ulp"
    assert_rel(og, orf, rtol=1e-4, atol=1e-5, label="f16-state output")


def test_decode_rejects_bad_shapes(L):
    """Argument errors return a code and enqueue nothing."""
    rc = L.kai_run_gdn_delta_rule_decode_f32_hip(None, None, None, None, None, None, None,
                                                 1, 3, 2, 128, 128, 1.0, None)
    assert rc != 0
    rc = L.kai_run_gdn_delta_rule_decode_f32_hip(None, None, None, None, None, None, None,
                                                 1, 2, 2, 96, 128, 1.0, None)
    assert rc != 0
