"""GPU parity of the prefill -> decode hand-off: the decode-step conv on
HF's cache layout, the conv-state remaps and the recurrent-state format
conversion, through the C-ABI, against the oracle (pinned to HF's own
causal_conv1d_update and LinearAttentionLayer.update_conv_state by
tests/test_oracle.py).

Bars: bit-exact for the index work, the RNE conversions and the conv
without SiLU (a 4-tap dot product in the kai reference's order, no
contraction).  The SiLU epilogue uses the device expf, which can differ from
the host's by an ulp: with SiLU the outputs are within BASELINE's 1e-5
relative of the oracle (the state stays bit-exact), and bit-exact against
the kai conv on the device.  HF's conv sums in its own order (rtol 1e-5).
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.gdn_inputs import decode_inputs, prefill_inputs, bf16_bits
from tests.gpu_util import P, dev, empty, host, host_u16, stream, torch_mod, u16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    torch = torch_mod()
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orionsbelt_amd as ob
    return ob.lib()


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def gpu_conv_update(L, x, state, w, silu):
    torch = torch_mod()
    B, T, C = x.shape
    dx, dst, dw = dev(x), dev(state), dev(w)
    out = empty((B, T, C), torch.float32)
    rc = L.kai_run_gdn_causal_conv1d_update_f32_hip(P(dx), P(dst), P(dw), P(out), B, T, C, int(silu),
                                                    stream())
    assert rc == 0, rc
    return host(out), host(dst)


@pytest.mark.parametrize("B,T,C,silu", [(3, 1, 40, True), (2, 3, 24, False), (64, 1, 8192, True),
                                        (1, 5, 300, True)])
def test_conv_update_vs_oracle(L, B, T, C, silu):
    rs = np.random.RandomState(B * 7 + T)
    x = rs.randn(B, T, C).astype(np.float32)
    st = rs.randn(B, C, 4).astype(np.float32)
    w = (0.5 * rs.randn(C, 4)).astype(np.float32)
    out, st_new = gpu_conv_update(L, x, st, w, silu)
    r_out, r_st = orc.causal_conv1d_update(x, st, w, silu)
    if silu:
        np.testing.assert_allclose(out, r_out, rtol=1e-5, atol=1e-6)
    else:
        assert np.array_equal(bits(out), bits(r_out))
    assert np.array_equal(bits(st_new), bits(r_st))


def test_conv_update_vs_hf_golden(L, golden):
    d = golden("hf_state.npz")
    for name in ("cu_t1", "cu_t3"):
        out, st = gpu_conv_update(L, d[f"{name}_x"], d[f"{name}_state0"], d[f"{name}_w"],
                                  bool(d[f"{name}_silu"]))
        np.testing.assert_allclose(out, d[f"{name}_out"], rtol=1e-5, atol=1e-6)
        assert np.array_equal(bits(st), bits(d[f"{name}_state"]))


def test_prefill_conv_then_decode_steps_bit_identical(L):
    """The kai conv (+SiLU) over T tokens, its history converted to HF's
    state, then N decode-step updates, equals the kai conv over T + N
    tokens bit for bit (C = 8192, the Qwen3.5 conv width)."""
    torch = torch_mod()
    T, N, C = 50, 4, 8192
    rs = np.random.RandomState(21)
    x = rs.randn(T + N, C).astype(np.float32)
    w_kai = (0.5 * rs.randn(4, C)).astype(np.float32)
    dx, dw = dev(x), dev(w_kai)
    full = empty((T + N, C), torch.float32)
    hist0 = dev(np.zeros((3, C), np.float32))
    assert L.kai_run_gdn_causal_dwconv1d_silu_f32_k4_hip(P(dx), P(dw), P(full), P(hist0), T + N, C,
                                                         stream()) == 0
    pre = empty((T, C), torch.float32)
    hist = dev(np.zeros((3, C), np.float32))
    assert L.kai_run_gdn_causal_dwconv1d_silu_f32_k4_hip(P(dx), P(dw), P(pre), P(hist), T, C,
                                                         stream()) == 0
    st = empty((1, C, 4), torch.float32)
    assert L.kai_run_gdn_conv_hist_to_state_f32_hip(P(hist), P(st), 1, C, stream()) == 0
    w_hf = dev(np.ascontiguousarray(w_kai.T))
    outs = empty((N, C), torch.float32)
    for i in range(N):
        xi = dx[T + i:T + i + 1]
        oi = outs[i:i + 1]
        assert L.kai_run_gdn_causal_conv1d_update_f32_hip(P(xi), P(st), P(w_hf), P(oi), 1, 1, C, 1,
                                                          stream()) == 0
    got = np.concatenate([host(pre), host(outs)])
    assert np.array_equal(bits(got), bits(host(full)))
    ref, _ = orc.conv_f32(x.ravel(), w_kai.ravel(), np.zeros(3 * C, np.float32), T + N, C, silu=True)
    np.testing.assert_allclose(got, ref.reshape(T + N, C), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("T", [0, 2, 7, 300])
def test_conv_state_from_inputs(L, T):
    torch = torch_mod()
    B, C = 3, 200
    x = np.random.RandomState(T).randn(B, max(T, 1), C).astype(np.float32)[:, :T]
    dx = dev(x) if T else dev(np.zeros((1,), np.float32))
    st = empty((B, C, 4), torch.float32)
    st.fill_(7.0)
    assert L.kai_run_gdn_conv_state_from_inputs_f32_hip(P(dx), P(st), B, T, C, stream()) == 0
    assert np.array_equal(bits(host(st)), bits(orc.conv_state_from_inputs(x)))


def test_conv_state_from_inputs_vs_hf_cache(L, golden):
    torch = torch_mod()
    d = golden("hf_state.npz")
    for name in ("cs_t2", "cs_t7"):
        x = d[f"{name}_x"]
        B, T, C = x.shape
        dx = dev(x)
        st = empty((B, C, 4), torch.float32)
        assert L.kai_run_gdn_conv_state_from_inputs_f32_hip(P(dx), P(st), B, T, C, stream()) == 0
        assert np.array_equal(bits(host(st)), bits(d[f"{name}_state"]))


def test_conv_hist_state_remaps(L):
    torch = torch_mod()
    B, C = 5, 1000
    rs = np.random.RandomState(3)
    st = rs.randn(B, C, 4).astype(np.float32)
    dst = dev(st)
    hist = empty((B, 3, C), torch.float32)
    assert L.kai_run_gdn_conv_state_to_hist_f32_hip(P(dst), P(hist), B, C, stream()) == 0
    h = host(hist)
    assert np.array_equal(bits(h), bits(orc.conv_state_to_hist(st)))
    back = empty((B, C, 4), torch.float32)
    assert L.kai_run_gdn_conv_hist_to_state_f32_hip(P(hist), P(back), B, C, stream()) == 0
    assert np.array_equal(bits(host(back)), bits(orc.conv_hist_to_state(h)))


# ---- recurrent state formats ------------------------------------------------

def gpu_convert(L, src_t, sf, df, n):
    torch = torch_mod()
    dst = empty((n,), torch.float32 if df == 0 else torch.int16)
    assert L.kai_run_gdn_state_convert_hip(P(src_t), sf, P(dst), df, n, stream()) == 0
    return host(dst) if df == 0 else host_u16(dst)


def test_state_convert_matches_rne(L):
    import orionsbelt_amd as ob
    rs = np.random.RandomState(8)
    x = np.concatenate([rs.randn(5000) * 10.0 ** rs.uniform(-9, 6, 5000),
                        [0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-8, np.inf, -np.inf]]).astype(np.float32)
    n = x.size
    dx = dev(x)
    f16 = gpu_convert(L, dx, ob.FMT_F32, ob.FMT_F16, n)
    with np.errstate(over="ignore"):  # values past 65504 round to infinity, as they should
        ref16 = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(f16, ref16)          # IEEE RNE
    b16 = gpu_convert(L, dx, ob.FMT_F32, ob.FMT_BF16, n)
    assert np.array_equal(b16, orc.f32_to_bf16_bits(x))                        # reference rule
    back = gpu_convert(L, u16(f16), ob.FMT_F16, ob.FMT_F32, n)
    assert np.array_equal(bits(back), bits(f16.view(np.float16).astype(np.float32)))
    back = gpu_convert(L, u16(b16), ob.FMT_BF16, ob.FMT_F32, n)
    assert np.array_equal(bits(back), bits(orc.bf16_bits_to_f32(b16)))
    f16_from_b = gpu_convert(L, u16(b16), ob.FMT_BF16, ob.FMT_F16, n)
    with np.errstate(over="ignore"):
        ref = orc.bf16_bits_to_f32(b16).astype(np.float16).view(np.uint16)
    assert np.array_equal(f16_from_b, ref)


def test_prefill_state_to_f16_decode(L):
    """Hand-off: a prefill leaves an fp32 state; converted to fp16 it feeds
    the fp16-state decode step, which then matches the oracle's step on the
    same fp16 state; a full decode-size state (64 x 32 x 128 x 128) converts
    exactly as torch's RNE .half()."""
    import orionsbelt_amd as ob
    torch = torch_mod()
    T, Hv, Hk = 100, 4, 2
    q, k, v, g, beta, S = prefill_inputs(17, 1, T, Hv, Hk)
    dq, dk_, dv_ = (u16(bf16_bits(t)) for t in (q, k, v))
    dS = dev(S)
    do = empty((1, T, Hv, 128), torch.int16)
    assert L.kai_run_gdn_chunk_delta_rule_bf16_f32_hip(P(dq), P(dk_), P(dv_), P(dev(g)), P(dev(beta)),
                                                       P(do), P(dS), 1, T, Hv, Hk, 1 / math.sqrt(128),
                                                       stream()) == 0
    n = Hv * 128 * 128
    S16 = empty((1, Hv, 128, 128), torch.int16)
    assert L.kai_run_gdn_state_convert_hip(P(dS), ob.FMT_F32, P(S16), ob.FMT_F16, n, stream()) == 0
    S16_h = host_u16(S16)
    assert np.array_equal(S16_h.ravel(), host(dS).astype(np.float16).view(np.uint16).ravel())
    _, q1, k1, v1, g1, b1 = decode_inputs(5, 1, Hv, Hk, 128, 128)
    o = empty((1, Hv, 128), torch.float32)
    assert L.kai_run_gdn_delta_rule_decode_f16state_hip(P(S16), P(dev(q1)), P(dev(k1)), P(dev(v1)),
                                                        P(dev(g1)), P(dev(b1)), P(o), 1, Hv, Hk, 128,
                                                        128, 1 / math.sqrt(128), stream()) == 0
    rS, ro = orc.delta_rule_decode_f16state(S16_h, q1, k1, v1, g1, b1, 1, Hv, Hk, 128, 128,
                                            1 / math.sqrt(128))
    np.testing.assert_allclose(host(o), ro, rtol=1e-4, atol=1e-6)
    big = torch.randn(64 * 32 * 128 * 128, device="cuda") * 0.3
    out = empty((big.numel(),), torch.int16)
    assert L.kai_run_gdn_state_convert_hip(P(big), ob.FMT_F32, P(out), ob.FMT_F16, big.numel(),
                                           stream()) == 0
    assert torch.equal(out, big.half().view(torch.int16))


def test_state_formats_reject_bad_args(L):
    torch = torch_mod()
    t = empty((64, 16, 4), torch.float32)
    fn = L.kai_run_gdn_causal_conv1d_update_f32_hip
    assert fn(P(t), P(t), P(t), P(t), -1, 1, 16, 1, stream()) != 0             # batch < 0
    assert fn(P(t), P(t), P(t), P(t), 70000, 1, 16, 1, stream()) != 0          # batch > 65535
    assert fn(P(t), None, P(t), P(t), 2, 1, 16, 1, stream()) != 0              # null state
    import ctypes
    off = ctypes.c_void_p(t.data_ptr() + 4)
    assert fn(P(t), off, P(t), P(t), 2, 1, 16, 1, stream()) != 0               # misaligned state
    assert fn(P(t), P(t), P(t), P(t), 2, -1, 16, 1, stream()) != 0             # seq_len < 0
    assert fn(None, None, None, None, 0, 1, 16, 1, stream()) == 0              # nothing to do
    cv = L.kai_run_gdn_state_convert_hip
    assert cv(P(t), 0, P(t), 3, 16, stream()) != 0                             # bad format
    assert cv(P(t), 0, off, 1, 16, stream()) != 0                              # overlap
    assert cv(P(t), 0, P(t), 0, 16, stream()) == 0                             # same array, format
