"""Pins the CPU oracle (oracle/gdn_oracle.c) before anything is compared
against it.  CPU only.

Each oracle function is checked against (a) the reference's own sources
compiled in oracle/_ref (bit-identical), (b) the committed golden fixtures in
tests/golden (bit-identical for the kai / gdn_sve vectors, tolerance for the
HuggingFace delta-rule vectors), and (c) closed forms and brute force chosen
so that a dropped term, a wrong index or a transposed operand fails.
"""
import math
import os

import numpy as np
import pytest

from oracle import oracle as orc

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module", autouse=True)
def _built():
    orc.lib()  # raises if liborb_oracle.so is missing


def bits_equal(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape
    return np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                          b.view(np.uint32) if b.dtype == np.float32 else b)


# --------------------------------------------------------------------------
# kai ukernels vs the reference golden vectors (kai_ref.npz)
# --------------------------------------------------------------------------

def test_kai_golden_cumdecay(golden):
    d = golden("kai_ref.npz")
    for n in ("cd1", "cd2"):
        seq, ch = d[f"{n}_shape"]
        assert bits_equal(orc.cumdecay_f32(d[f"{n}_a"], seq, ch), d[f"{n}_out"])


def test_kai_golden_gated_scan(golden):
    d = golden("kai_ref.npz")
    for n in ("sc1", "sc2"):
        seq, ch = d[f"{n}_shape"]
        s, st = orc.gated_scan_f32(d[f"{n}_g"], d[f"{n}_x"], d[f"{n}_state"], seq, ch)
        assert bits_equal(s, d[f"{n}_s"]) and bits_equal(st, d[f"{n}_state_out"])


def test_kai_golden_conv(golden):
    d = golden("kai_ref.npz")
    for n in ("cv1", "cv2", "cv3"):
        seq, ch = d[f"{n}_shape"]
        out, h = orc.conv_f32(d[f"{n}_in"], d[f"{n}_w"], d[f"{n}_hist"], seq, ch)
        assert bits_equal(out, d[f"{n}_out"]) and bits_equal(h, d[f"{n}_hist_out"])


def test_kai_golden_gemv(golden):
    d = golden("kai_ref.npz")
    for n in ("gv1", "gv2"):
        k, nn = d[f"{n}_shape"]
        assert bits_equal(orc.gemv_f32(d[f"{n}_a"], d[f"{n}_b"], k, nn), d[f"{n}_c"])


def test_delta_matmul_golden(golden):
    """orc_delta_rule_matmul_f32 against the reference gdn_delta_matmul.c's
    outputs on its test's inputs (tests/golden/delta_matmul.npz)."""
    d = golden("delta_matmul.npz")
    for n in ("mm1", "mm2"):
        m, k, nn = (int(x) for x in d[f"{n}_shape"])
        got = orc.delta_rule_matmul(d[f"{n}_A"], d[f"{n}_B"], m, k, nn)
        assert bits_equal(got.ravel(), d[f"{n}_C"])


def test_delta_matmul_bounds_and_live_reference():
    """Against a float64 product: each element within the fp32 sum's error
    bound (k * 2^-24 * sum |a b|, with slack 2); K = 0 gives zeros; a
    transposed operand or a dropped k term fails the bound.  Bit-identical to
    the live reference build when oracle/_ref holds it, at the reference
    test's shapes (test_gdn_delta_matmul.c:87-96)."""
    rs = np.random.RandomState(3)
    ref = orc.ref_matmul()
    for m, k, n in [(1, 128, 128), (64, 128, 128), (1, 128, 2048), (64, 128, 2048), (1, 128, 130),
                    (64, 128, 130), (5, 7, 3)]:
        A = rs.uniform(-1, 1, m * k).astype(np.float32)
        B = rs.uniform(-1, 1, k * n).astype(np.float32)
        C = orc.delta_rule_matmul(A, B, m, k, n)
        A2, B2 = A.reshape(m, k).astype(np.float64), B.reshape(k, n).astype(np.float64)
        exact = A2 @ B2
        bound = 2 * k * 2.0 ** -24 * (np.abs(A2) @ np.abs(B2))
        assert np.all(np.abs(C - exact) <= bound + 1e-30)
        if k > 1:  # a dropped last term is far outside the bound somewhere
            drop = A2[:, :-1] @ B2[:-1, :]
            assert np.any(np.abs(drop - exact) > bound)
        if k == n:  # so is a transposed operand
            assert np.any(np.abs(A2 @ B2.T - exact) > bound)
        if ref is not None:
            assert bits_equal(C.ravel(), orc.delta_rule_matmul(A, B, m, k, n, L=ref).ravel())
    z = orc.delta_rule_matmul(np.zeros(1, np.float32), np.zeros(1, np.float32), 2, 0, 3)
    assert np.all(z == 0)


def test_oracle_under_sanitizers():
    """make -C oracle asan: the oracle rebuilt with AddressSanitizer and
    UBSan runs this file's tests (and the reference kai test, when the
    reference tree is present) without a report.  Skipped inside that run."""
    if os.environ.get("ORB_ORACLE_LIB"):
        pytest.skip("already running under the sanitizer build")
    import subprocess
    r = subprocess.run(["make", "-s", "-C", os.path.join(REPO, "oracle"), "asan"], capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "passed" in r.stdout and "ERROR: AddressSanitizer" not in r.stderr + r.stdout


# --------------------------------------------------------------------------
# kai ukernels vs the live reference build (oracle/_ref), full test sweep
# --------------------------------------------------------------------------

REF_SEQS = [1, 4, 16, 64]                                  # test_kai_gdn.c:167
REF_CHANS = [1, 3, 7, 8, 12, 16, 17, 32, 33, 128]          # test_kai_gdn.c:168


@pytest.fixture(scope="module")
def refkai():
    L = orc.ref_kai()
    if L is None:
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    return L


def test_ref_sweep_bit_identical(refkai):
    rs = np.random.RandomState(7)
    for seq in REF_SEQS:
        for ch in REF_CHANS + [129, 255, 2051]:
            n = seq * ch
            a = rs.uniform(0.1, 1.5, n).astype(np.float32)
            assert bits_equal(orc.cumdecay_f32(a, seq, ch), orc.cumdecay_f32(a, seq, ch, L=refkai))
            g = rs.uniform(-0.99, 0.99, n).astype(np.float32)
            x = rs.uniform(-2, 2, n).astype(np.float32)
            st = rs.uniform(-1, 1, ch).astype(np.float32)
            r1 = orc.gated_scan_f32(g, x, st, seq, ch)
            r2 = orc.gated_scan_f32(g, x, st, seq, ch, L=refkai)
            assert bits_equal(r1[0], r2[0]) and bits_equal(r1[1], r2[1])
            w = rs.uniform(-1, 1, 4 * ch).astype(np.float32)
            h = rs.uniform(-1, 1, 3 * ch).astype(np.float32)
            c1 = orc.conv_f32(x, w, h, seq, ch)
            c2 = orc.conv_f32(x, w, h, seq, ch, L=refkai)
            assert bits_equal(c1[0], c2[0]) and bits_equal(c1[1], c2[1])
    for k in (0, 1, 4, 128, 1024):
        for n in (1, 3, 7, 130, 257):
            a = rs.uniform(-1, 1, max(k, 1)).astype(np.float32)
            b = rs.uniform(-1, 1, max(k * n, 1)).astype(np.float32)
            assert bits_equal(orc.gemv_f32(a, b, k, n), orc.gemv_f32(a, b, k, n, L=refkai))


def test_ref_sve_narrow_sweep_bit_identical():
    """fp16/bf16 decay and scan against the live gdn_sve.c build over the
    same ragged sizes (channel counts off the oracle's 16-channel groups,
    and sizes above its OpenMP threshold)."""
    L = orc.ref_sve()
    if L is None:
        pytest.skip("oracle/_ref not built (needs the reference tree)")
    rs = np.random.RandomState(8)
    for seq in REF_SEQS:
        for ch in REF_CHANS + [129, 255, 2051]:
            n = seq * ch
            a = rs.uniform(0.1, 1.5, n).astype(np.float32)
            g = rs.uniform(-0.99, 0.99, n).astype(np.float32)
            x = rs.uniform(-2, 2, n).astype(np.float32)
            for fmt in ("f16", "bf16"):
                st = rs.randint(0, 0x3C00, ch).astype(np.uint16)
                assert np.array_equal(orc.cumdecay_narrow(a, seq, ch, fmt),
                                      orc.cumdecay_narrow(a, seq, ch, fmt, L=L, prefix="gdn_")), (seq, ch, fmt)
                r1 = orc.gated_scan_narrow(g, x, st, seq, ch, fmt)
                r2 = orc.gated_scan_narrow(g, x, st, seq, ch, fmt, L=L, prefix="gdn_")
                assert bits_equal(r1[0], r2[0]) and np.array_equal(r1[1], r2[1]), (seq, ch, fmt)


def test_gdn2_scan_vs_reference_and_closed_forms():
    """orc_gdn2_gated_scan_f32 against the live gdn_sve.c build (bit for
    bit, ragged channel counts, sizes above the OpenMP threshold); with
    b = w = 1 it is the GDN-1 scan bit for bit (test_gdn2_scan.c:29); with
    w = 0 the state decays by the products g * b alone."""
    rs = np.random.RandomState(9)
    L = orc.ref_sve()
    for seq in REF_SEQS + [100]:
        for ch in REF_CHANS + [2051]:
            n = seq * ch
            g = rs.uniform(-0.99, 0.99, n).astype(np.float32)
            b = rs.uniform(0, 1, n).astype(np.float32)
            w = rs.uniform(0, 1, n).astype(np.float32)
            x = rs.uniform(-2, 2, n).astype(np.float32)
            st = rs.uniform(-1, 1, ch).astype(np.float32)
            r1 = orc.gdn2_scan_f32(g, b, w, x, st, seq, ch)
            if L is not None:
                r2 = orc.gdn2_scan_f32(g, b, w, x, st, seq, ch, L=L, name="gdn2_gated_scan_f32")
                assert bits_equal(r1[0], r2[0]) and bits_equal(r1[1], r2[1]), (seq, ch)
            ones = np.ones(n, np.float32)
            a1 = orc.gdn2_scan_f32(g, ones, ones, x, st, seq, ch)
            a2 = orc.gated_scan_f32(g, x, st, seq, ch)
            assert bits_equal(a1[0], a2[0]) and bits_equal(a1[1], a2[1]), (seq, ch)
    seq, ch = 5, 3
    g = np.full(seq * ch, 0.5, np.float32)
    b = np.full(seq * ch, 0.5, np.float32)
    st = np.array([1.0, -2.0, 4.0], np.float32)
    s, stf = orc.gdn2_scan_f32(g, b, np.zeros(seq * ch, np.float32), np.ones(seq * ch, np.float32), st, seq, ch)
    expect = np.array([[v * 0.25 ** (t + 1) for v in st] for t in range(seq)], np.float32).ravel()
    assert bits_equal(s, expect) and bits_equal(stf, expect[-ch:])


def test_degenerate_writes_nothing():
    """seq=0 / channels=0 leave outputs and state untouched
    (test_kai_gdn.c:520-637)."""
    L = orc.lib()
    sentinel = np.full(8, 42.0, np.float32)
    out = sentinel.copy()
    L.orc_cumdecay_f32(orc.P(sentinel), orc.P(out), orc._sz(0), orc._sz(8))
    assert bits_equal(out, sentinel)
    st = np.array([1, -2, 3, -4], np.float32)
    s = orc.gated_scan_f32(sentinel, sentinel, st, 0, 4)[1]
    assert bits_equal(s, st)
    hist = np.arange(6, dtype=np.float32)
    assert bits_equal(orc.conv_f32(sentinel, sentinel, hist, 0, 2)[1], hist)
    assert np.all(orc.gemv_f32(sentinel, sentinel, 0, 8) == 0.0)


# --------------------------------------------------------------------------
# Closed forms
# --------------------------------------------------------------------------

def test_cumdecay_closed_form_powers_of_two():
    seq, ch = 100, 5
    a = np.full(seq * ch, 0.5, np.float32)
    d = orc.cumdecay_f32(a, seq, ch).reshape(seq, ch)
    expect = np.ldexp(np.float32(1), -(np.arange(seq) + 1)).astype(np.float32)
    assert bits_equal(d, np.repeat(expect[:, None], ch, axis=1))


def test_scan_closed_forms():
    seq, ch = 50, 3
    x = np.random.RandomState(1).randint(-8, 8, seq * ch).astype(np.float32)
    st = np.array([1, 2, 3], np.float32)
    s, st2 = orc.gated_scan_f32(np.ones(seq * ch, np.float32), x, st, seq, ch)
    expect = np.cumsum(x.reshape(seq, ch), axis=0) + st  # integer-valued: exact
    assert bits_equal(s.reshape(seq, ch), expect.astype(np.float32))
    assert bits_equal(st2, expect[-1].astype(np.float32))
    s0, _ = orc.gated_scan_f32(np.zeros(seq * ch, np.float32), x, st, seq, ch)
    assert bits_equal(s0, x)


def test_conv_impulse_returns_taps():
    seq, ch = 8, 4
    w = np.random.RandomState(2).randn(4 * ch).astype(np.float32)
    x = np.zeros((seq, ch), np.float32)
    x[0] = 1.0
    out, hist = orc.conv_f32(x.ravel(), w, np.zeros(3 * ch, np.float32), seq, ch)
    out = out.reshape(seq, ch)
    # out[t] = w[3 - t] for t < 4, then 0
    for t in range(4):
        assert bits_equal(out[t], w.reshape(4, ch)[3 - t])
    assert np.all(out[4:] == 0)


def test_conv_silu_epilogue_matches_torch():
    torch = pytest.importorskip("torch")
    rs = np.random.RandomState(3)
    seq, ch = 33, 65
    x = rs.randn(seq * ch).astype(np.float32)
    w = (0.25 * rs.randn(4 * ch)).astype(np.float32)
    h = rs.randn(3 * ch).astype(np.float32)
    plain, h1 = orc.conv_f32(x, w, h, seq, ch)
    silu, h2 = orc.conv_f32(x, w, h, seq, ch, silu=True)
    assert bits_equal(h1, h2)
    ref = torch.nn.functional.silu(torch.from_numpy(plain)).numpy()
    np.testing.assert_allclose(silu, ref, rtol=2e-6, atol=1e-7)


# --------------------------------------------------------------------------
# Narrow formats (gdn_sve.c mixed precision)
# --------------------------------------------------------------------------

def test_f16_conversion_matches_numpy():
    rs = np.random.RandomState(4)
    bits = rs.randint(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    vals = np.concatenate([
        bits.view(np.float32),
        np.float32([0.0, -0.0, 65504, 65520, 65519.99, 6.1035156e-05, 5.9604645e-08,
                    2.9802322e-08, 2.9802326e-08, 8.940697e-08, 1e-10, np.inf, -np.inf]),
        (rs.randn(20000) * 1e-5).astype(np.float32),
    ])
    vals = vals[~np.isnan(vals)]
    L = orc.lib()
    got = np.array([L.orc_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    h = h[(h & 0x7C00) != 0x7C00]  # finite halves
    back = np.array([L.orc_f16_to_f32(int(x)) for x in h], np.float32)
    assert bits_equal(back, h.view(np.float16).astype(np.float32))


def test_bf16_conversion_rne():
    L = orc.lib()
    # halfway cases round to even; above-half rounds up
    cases = {0x3F808000: 0x3F80, 0x3F818000: 0x3F82, 0x3F808001: 0x3F81, 0x3F807FFF: 0x3F80}
    for u, b in cases.items():
        f = np.array([u], np.uint32).view(np.float32)[0]
        assert L.orc_f32_to_bf16(float(f)) == b
        assert orc.f32_to_bf16_bits(np.array([f], np.float32))[0] == b


def test_mixed_precision_vs_reference_gdn_sve(golden):
    d = golden("sve_mixed.npz")
    T, C = d["shape"]
    for scen in ("warm", "cold"):
        for fmt in ("f16", "bf16"):
            cd = orc.cumdecay_narrow(d[f"{scen}_a"], T, C, fmt)
            assert np.array_equal(cd, d[f"{scen}_cd_{fmt}"]), (scen, fmt)
            s, st = orc.gated_scan_narrow(d[f"{scen}_g"], d[f"{scen}_x"],
                                          d[f"{scen}_st16_{fmt}"], T, C, fmt)
            assert bits_equal(s, d[f"{scen}_scan_s_{fmt}"]), (scen, fmt)
            assert np.array_equal(st, d[f"{scen}_scan_st_{fmt}"]), (scen, fmt)


# --------------------------------------------------------------------------
# Matrix-state delta rule
# --------------------------------------------------------------------------

def test_delta_rule_hand_computed():
    """d=2: S0=0, beta=1 -> S = k (x) v and o = S^T q."""
    k = np.float32([0.8, 0.6])
    v = np.float32([1.0, 2.0])
    q = np.float32([0.6, 0.8])
    S, o = orc.delta_rule_head(np.zeros(4, np.float32), k, v, q, 1.0, 0.7, 2, 2)
    np.testing.assert_allclose(S.reshape(2, 2), [[0.8, 1.6], [0.6, 1.2]], rtol=1e-7)
    np.testing.assert_allclose(o, [0.96, 1.92], rtol=1e-6)


def test_delta_rule_known_answers():
    rs = np.random.RandomState(5)
    dk, dv = 16, 12
    S0 = rs.randn(dk * dv).astype(np.float32)
    q = rs.randn(dk).astype(np.float32)
    v = rs.randn(dv).astype(np.float32)
    # k = e_i, beta = 1, decay = 1: row i becomes v (to rounding), others kept
    i = 5
    k = np.zeros(dk, np.float32)
    k[i] = 1.0
    S, _ = orc.delta_rule_head(S0, k, v, q, 1.0, 1.0, dk, dv)
    S, S0m = S.reshape(dk, dv), S0.reshape(dk, dv)
    np.testing.assert_allclose(S[i], v, rtol=0, atol=4 * np.finfo(np.float32).eps * 4)
    assert bits_equal(np.delete(S, i, 0), np.delete(S0m, i, 0))
    # beta = 0: pure decay, o = (decay S)^T q
    kk = rs.randn(dk).astype(np.float32)
    S, o = orc.delta_rule_head(S0, kk, v, q, 0.0, 0.75, dk, dv)
    assert bits_equal(S, (S0 * np.float32(0.75)).astype(np.float32))
    np.testing.assert_allclose(o, (S0m.astype(np.float64) * 0.75).T @ q, rtol=1e-5)
    # decay = 0: S = beta k (x) v, o = beta (k.q) v
    S, o = orc.delta_rule_head(S0, kk, v, q, 0.4, 0.0, dk, dv)
    np.testing.assert_allclose(S.reshape(dk, dv), 0.4 * np.outer(kk, v), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(o, 0.4 * float(kk @ q) * v, rtol=1e-5, atol=1e-6)


def _delta_rule_f64(S, k, v, q, beta, decay):
    S = S * decay
    kv = S.T @ k
    S = S + np.outer(k, (v - kv) * beta)
    return S, S.T @ q


def test_delta_rule_brute_force_f64():
    rs = np.random.RandomState(6)
    for d in (2, 3, 5, 8, 32, 128):
        S0 = rs.randn(d, d)
        k, v, q = rs.randn(d), rs.randn(d), rs.randn(d)
        k /= np.linalg.norm(k)
        S, o = orc.delta_rule_head(S0.astype(np.float32).ravel(), k.astype(np.float32),
                                   v.astype(np.float32), q.astype(np.float32), 0.6, 0.9, d, d)
        S2, o2 = _delta_rule_f64(S0.astype(np.float32).astype(np.float64),
                                 k.astype(np.float32).astype(np.float64),
                                 v.astype(np.float32).astype(np.float64),
                                 q.astype(np.float32).astype(np.float64), 0.6, 0.9)
        np.testing.assert_allclose(S.reshape(d, d), S2, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(o, o2, rtol=1e-4, atol=1e-4 * np.abs(S2).sum() / d)


def _unpack(d, name):
    B, T, Hk, Hv, dk, dv, chunk = (int(x) for x in d[f"{name}_dims"])
    return (d[f"{name}_q"], d[f"{name}_k"], d[f"{name}_v"], d[f"{name}_g"],
            d[f"{name}_beta"], d[f"{name}_S0"], B, T, Hk, Hv, dk, dv, chunk)


def test_decode_vs_hf_recurrent(golden):
    d = golden("hf_gdr.npz")
    for name in ("rc_step", "rc_multi"):
        q, k, v, g, beta, S0, B, T, Hk, Hv, dk, dv, _ = _unpack(d, name)
        S = S0.copy()
        o = np.empty((B, T, Hv, dv), np.float32)
        for t in range(T):
            S, ot = orc.delta_rule_decode(
                S, np.ascontiguousarray(q[:, t]), np.ascontiguousarray(k[:, t]),
                np.ascontiguousarray(v[:, t]), np.ascontiguousarray(g[:, t]),
                np.ascontiguousarray(beta[:, t]), B, Hv, Hk, dk, dv, 1.0 / math.sqrt(dk))
            o[:, t] = ot
        np.testing.assert_allclose(o, d[f"{name}_o"], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(S, d[f"{name}_S"], rtol=1e-5, atol=1e-6)


def test_decode_unscaled_equals_reference_loop():
    """q_scale=1 is the reference's ref_delta_rule looped over heads, with
    v-head h reading k-head h // (Hv/Hk)."""
    rs = np.random.RandomState(8)
    B, Hv, Hk, dk, dv = 2, 4, 2, 8, 8
    S0 = rs.randn(B, Hv, dk, dv).astype(np.float32)
    q, k = rs.randn(B, Hk, dk).astype(np.float32), rs.randn(B, Hk, dk).astype(np.float32)
    v = rs.randn(B, Hv, dv).astype(np.float32)
    g, beta = -rs.rand(B, Hv).astype(np.float32), rs.rand(B, Hv).astype(np.float32)
    S, o = orc.delta_rule_decode(S0, q, k, v, g, beta, B, Hv, Hk, dk, dv, 1.0)
    import ctypes
    expf = ctypes.CDLL("libm.so.6").expf
    expf.restype, expf.argtypes = ctypes.c_float, [ctypes.c_float]
    for b in range(B):
        for h in range(Hv):
            Sh, oh = orc.delta_rule_head(S0[b, h].ravel(), k[b, h // 2], v[b, h], q[b, h // 2],
                                         float(beta[b, h]), expf(float(g[b, h])),
                                         dk, dv)
            assert bits_equal(Sh, S[b, h].ravel()) and bits_equal(oh, o[b, h])


def test_decode_f16state_is_widen_step_narrow():
    """The fp16-state step is the fp32 step (pinned above against HF) on the
    widened state, narrowed once by round-to-nearest-even; numpy's float16
    conversion is the independent check of both conversions."""
    rs = np.random.RandomState(9)
    B, Hv, Hk, dk, dv = 2, 4, 2, 16, 8
    S16 = (rs.randn(B, Hv, dk, dv) * 0.3).astype(np.float16).view(np.uint16)
    q, k = rs.randn(B, Hk, dk).astype(np.float32), rs.randn(B, Hk, dk).astype(np.float32)
    v = rs.randn(B, Hv, dv).astype(np.float32)
    g, beta = -rs.rand(B, Hv).astype(np.float32), rs.rand(B, Hv).astype(np.float32)
    S16n, o16 = orc.delta_rule_decode_f16state(S16, q, k, v, g, beta, B, Hv, Hk, dk, dv, 0.25)
    S32 = S16.view(np.float16).astype(np.float32)
    S32n, o32 = orc.delta_rule_decode(S32, q, k, v, g, beta, B, Hv, Hk, dk, dv, 0.25)
    assert bits_equal(o16, o32)
    assert np.array_equal(S16n, S32n.astype(np.float16).view(np.uint16))
    assert not np.array_equal(S16n, S16)  # the step changed the state


# --------------------------------------------------------------------------
# Chunkwise prefill
# --------------------------------------------------------------------------

@pytest.mark.parametrize("precision", ["f32", "f64"])
def test_chunk_vs_hf(golden, precision):
    d = golden("hf_gdr.npz")
    for name in ("ck_small", "ck_tail", "ck_b2"):
        q, k, v, g, beta, S0, B, T, Hk, Hv, dk, dv, chunk = _unpack(d, name)
        o, S = orc.chunk_gdr(q, k, v, g, beta, S0, B, T, Hv, Hk, dk, dv, chunk,
                             precision=precision)
        scale_o = np.abs(d[f"{name}_o"]).max()
        np.testing.assert_allclose(o, d[f"{name}_o"], rtol=1e-4, atol=2e-5 * scale_o)
        np.testing.assert_allclose(S, d[f"{name}_S"], rtol=1e-4, atol=2e-5 * np.abs(S).max())


def test_chunk_equals_stepped_recurrence():
    """The WY chunk form and T single-token steps compute the same recurrence
    (exact in real arithmetic); in double they agree to ~1e-6."""
    from tests.golden.gen_golden import _inputs
    rs = np.random.RandomState(9)
    B, T, Hk, Hv, dk, dv = 1, 70, 1, 2, 16, 16
    q, k, v, g, beta, S0 = _inputs(rs, B, T, Hk, Hv, dk, dv)
    oc, Sc = orc.chunk_gdr(q, k, v, g, beta, S0, B, T, Hv, Hk, dk, dv, 32, precision="f64")
    S = S0.copy()
    for t in range(T):
        S, ot = orc.delta_rule_decode(
            S, np.ascontiguousarray(q[:, t]), np.ascontiguousarray(k[:, t]),
            np.ascontiguousarray(v[:, t]), np.ascontiguousarray(g[:, t]),
            np.ascontiguousarray(beta[:, t]), B, Hv, Hk, dk, dv, 1.0 / math.sqrt(dk))
        np.testing.assert_allclose(oc[:, t], ot, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(Sc, S, rtol=1e-4, atol=1e-5)


def test_chunk_state_carry_two_calls():
    """Splitting at a chunk boundary and carrying S gives bit-identical
    results (same chunks, same operation order)."""
    from tests.golden.gen_golden import _inputs
    rs = np.random.RandomState(10)
    B, T, Hk, Hv, dk, dv, C = 1, 96, 1, 2, 16, 16, 16
    q, k, v, g, beta, S0 = _inputs(rs, B, T, Hk, Hv, dk, dv)
    o, S = orc.chunk_gdr(q, k, v, g, beta, S0, B, T, Hv, Hk, dk, dv, C)
    T1 = 48
    sl = [lambda x, a=a, b=b: np.ascontiguousarray(x[:, a:b]) for a, b in ((0, T1), (T1, T))]
    o1, S1 = orc.chunk_gdr(*(sl[0](x) for x in (q, k, v, g, beta)), S0, B, T1, Hv, Hk, dk, dv, C)
    o2, S2 = orc.chunk_gdr(*(sl[1](x) for x in (q, k, v, g, beta)), S1, B, T - T1, Hv, Hk, dk,
                           dv, C)
    assert bits_equal(np.concatenate([o1, o2], axis=1), o) and bits_equal(S2, S)


def test_chunk_gate_sensitivity():
    """A dropped decay mask or a dropped beta would be caught: perturbing
    either input changes the HF-pinned output well beyond the tolerance."""
    from tests.golden.gen_golden import _inputs
    rs = np.random.RandomState(11)
    B, T, Hk, Hv, dk, dv = 1, 40, 1, 1, 8, 8
    q, k, v, g, beta, S0 = _inputs(rs, B, T, Hk, Hv, dk, dv)
    o, _ = orc.chunk_gdr(q, k, v, g, beta, S0, B, T, Hv, Hk, dk, dv, 16)
    o_nog, _ = orc.chunk_gdr(q, k, v, np.zeros_like(g), beta, S0, B, T, Hv, Hk, dk, dv, 16)
    o_nob, _ = orc.chunk_gdr(q, k, v, g, np.ones_like(beta), S0, B, T, Hv, Hk, dk, dv, 16)
    assert np.abs(o - o_nog).max() > 1e-2 * np.abs(o).max()
    assert np.abs(o - o_nob).max() > 1e-2 * np.abs(o).max()


# --------------------------------------------------------------------------
# layer glue: gating prologue and gated RMSNorm (hf_layer.npz)
# --------------------------------------------------------------------------

def ulp_bf16_diff(a16, b16):
    """Distance in bf16 units in the last place between two bit arrays
    (monotone integer mapping of the bit patterns)."""
    def key(u):
        u = np.asarray(u, np.uint16).astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - (u & 0x7FFF), u + 0x8000)
    return np.abs(key(a16) - key(b16))


def test_gating_prologue_vs_hf(golden):
    d = golden("hf_layer.npz")
    rows, Hk, Hv = (int(t) for t in d["gp_dims"])
    q, k, v, g, beta = orc.gating_prologue(d["gp_x"], d["gp_a"], d["gp_b"], d["gp_A_log"],
                                           d["gp_dt_bias"], rows, Hk, Hv)
    np.testing.assert_allclose(q, d["gp_q"], rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(k, d["gp_k"], rtol=2e-6, atol=1e-7)
    assert bits_equal(v, d["gp_v"])
    np.testing.assert_allclose(g, d["gp_g"], rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(beta, d["gp_beta"], rtol=2e-6, atol=1e-7)


def test_gating_prologue_closed_forms():
    rows, Hk, Hv = 3, 1, 2
    rs = np.random.RandomState(5)
    x = rs.randn(rows, (2 * Hk + Hv) * 128).astype(np.float32)
    x[2, :128] = 3.0                                   # constant q head
    a = np.array([[0, 0], [30, -40], [0, 0]], np.float32)
    b = np.array([[0, 0], [50, -50], [0, 0]], np.float32)
    A_log = np.array([0.0, math.log(2.0)], np.float32)
    dt = np.zeros(Hv, np.float32)
    q, k, v, g, beta = orc.gating_prologue(x, a, b, A_log, dt, rows, Hk, Hv)
    # unit rows (|x|^2 >> eps), v untouched and in the v channels, k from the k channels
    np.testing.assert_allclose(np.linalg.norm(q, axis=-1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(np.linalg.norm(k, axis=-1), 1.0, rtol=1e-6)
    assert bits_equal(v.reshape(rows, -1), x[:, 2 * Hk * 128:])
    np.testing.assert_allclose(k[0, 0] * np.linalg.norm(x[0, 128:256]), x[0, 128:256], rtol=1e-5)
    np.testing.assert_allclose(q[2, 0], np.full(128, 1 / math.sqrt(128), np.float32), rtol=1e-6)
    # softplus(0) = ln 2, scaled by exp(A_log) = 1 and 2; beyond the
    # threshold softplus(y) = y; far below, exp(y)
    np.testing.assert_allclose(g[0], [-math.log(2.0), -2 * math.log(2.0)], rtol=1e-6)
    assert g[1, 0] == np.float32(-30.0)
    np.testing.assert_allclose(g[1, 1], -2 * math.exp(-40.0), rtol=1e-5)
    np.testing.assert_allclose(beta[0], [0.5, 0.5], rtol=0)
    assert beta[1, 0] == 1.0 and 0 < beta[1, 1] < 1e-20


def test_gated_rmsnorm_vs_hf(golden):
    d = golden("hf_layer.npz")
    y = orc.gated_rmsnorm_f32(d["rn_f32_o"], d["rn_f32_z"], d["rn_f32_w"], 1e-6)
    np.testing.assert_allclose(y, d["rn_f32_y"], rtol=3e-6, atol=1e-7)
    y16 = orc.gated_rmsnorm_bf16(d["rn_bf16_o"], d["rn_bf16_z"], d["rn_bf16_w"], 1e-6)
    # the three bf16 roundings of HF's bf16 module; rsqrt/exp differ by an
    # fp32 ulp, which can move a rounding by one bf16 ulp
    diff = ulp_bf16_diff(y16, d["rn_bf16_y"])
    assert diff.max() <= 1 and (diff > 0).mean() < 0.02


def test_gated_rmsnorm_closed_forms():
    n = 128
    w = np.linspace(0.5, 1.5, n).astype(np.float32)
    # a constant row c: o / rms(o) = sign(c) exactly up to eps; z large -> silu(z) ~ z
    o = np.full((2, n), 2.0, np.float32)
    z = np.full((2, n), 30.0, np.float32)
    z[1] = 0.0
    y = orc.gated_rmsnorm_f32(o, z, w, 0.0)
    np.testing.assert_allclose(y[0], w * 30.0, rtol=1e-6)
    assert np.all(y[1] == 0)
    # scaling o does not change the result (eps = 0); scaling w scales y
    rs = np.random.RandomState(3)
    o = rs.randn(4, n).astype(np.float32)
    z = rs.randn(4, n).astype(np.float32)
    y1 = orc.gated_rmsnorm_f32(o, z, w, 0.0)
    np.testing.assert_allclose(orc.gated_rmsnorm_f32(o * 8, z, w, 0.0), y1, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(orc.gated_rmsnorm_f32(o, z, 2 * w, 0.0), 2 * y1, rtol=1e-6, atol=1e-7)
    # a plain-numpy restatement in float64 (mean of squares, rsqrt, silu)
    ref = (o / np.sqrt((o.astype(np.float64) ** 2).mean(-1, keepdims=True))) * w * (z / (1 + np.exp(-z.astype(np.float64))))
    np.testing.assert_allclose(y1, ref, rtol=2e-6, atol=1e-7)


# --------------------------------------------------------------------------
# state hand-off formats (hf_state.npz)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["cu_t1", "cu_t3"])
def test_conv_update_vs_hf(golden, name):
    d = golden("hf_state.npz")
    out, st = orc.causal_conv1d_update(d[f"{name}_x"], d[f"{name}_state0"], d[f"{name}_w"],
                                       bool(d[f"{name}_silu"]))
    # HF's F.conv1d sums the four taps in its own order: a few fp32 ulps
    np.testing.assert_allclose(out, d[f"{name}_out"], rtol=1e-5, atol=1e-6)
    assert bits_equal(st, d[f"{name}_state"])   # the state is a pure shift


def test_conv_update_continues_kai_conv():
    """A sequence prefilled by the kai conv and continued by decode steps on
    the HF state layout is bit-identical to the kai conv over the whole
    sequence (both in the reference's tap order)."""
    rs = np.random.RandomState(12)
    T, N, C = 37, 5, 19
    x = rs.randn(T + N, C).astype(np.float32)
    w_kai = rs.randn(4, C).astype(np.float32)          # kai layout [4][C]
    full, _ = orc.conv_f32(x.ravel(), w_kai.ravel(), np.zeros(3 * C, np.float32), T + N, C, silu=True)
    pre, hist = orc.conv_f32(x[:T].ravel(), w_kai.ravel(), np.zeros(3 * C, np.float32), T, C, silu=True)
    st = orc.conv_hist_to_state(hist.reshape(1, 3, C))
    expect = orc.conv_state_from_inputs(x[None, :T])
    expect[:, :, 0] = 0.0                      # the dead entry hist -> state writes
    assert bits_equal(st, expect)
    outs = []
    for t in range(T, T + N):
        o, st = orc.causal_conv1d_update(x[None, t:t + 1], st, np.ascontiguousarray(w_kai.T), True)
        outs.append(o[0, 0])
    assert bits_equal(np.concatenate([pre.reshape(T, C), np.stack(outs)]), full.reshape(T + N, C))


@pytest.mark.parametrize("name", ["cs_t2", "cs_t7"])
def test_conv_state_from_inputs_vs_hf_cache(golden, name):
    d = golden("hf_state.npz")
    assert bits_equal(orc.conv_state_from_inputs(d[f"{name}_x"]), d[f"{name}_state"])


def test_conv_hist_state_round_trip():
    rs = np.random.RandomState(4)
    st = rs.randn(3, 11, 4).astype(np.float32)
    hist = orc.conv_state_to_hist(st)
    assert hist.shape == (3, 3, 11) and bits_equal(hist[:, 0, :], st[:, :, 1])
    assert bits_equal(hist[:, 2, :], st[:, :, 3])
    back = orc.conv_hist_to_state(hist)
    assert bits_equal(back[:, :, 1:], st[:, :, 1:]) and np.all(back[:, :, 0] == 0)


# --------------------------------------------------------------------------
# int8 weight-only matmul of the hybrid decode loop
# --------------------------------------------------------------------------

def test_w8_quantize_closed_forms():
    W = np.array([[0.5, -1.0, 0.25, 0.0],      # max 1 -> scale 1/127
                  [0.0, 0.0, 0.0, 0.0],        # zero row -> scale 1, q = 0
                  [3.0, -3.0, 1.5, 0.01]], np.float32)
    q, s = orc.w8_quantize(W)
    assert s[1] == 1.0 and np.all(q[1] == 0)
    assert q[0, 1] == -127 and q[2, 0] == 127 and q[2, 1] == -127
    assert s[0] == np.float32(1.0) / np.float32(127.0)
    # 0.5 * 127 = 63.5 rounds away from zero (lroundf), 0.25 * 127 = 31.75 -> 32
    assert q[0, 0] == 64 and q[0, 2] == 32
    assert q[2, 2] == 64                        # 1.5 / (3/127) = 63.5 -> 64
    rs = np.random.RandomState(2)
    W = rs.randn(40, 96).astype(np.float32)
    q, s = orc.w8_quantize(W)
    assert np.all(np.abs(q).max(axis=1) == 127)
    np.testing.assert_allclose(q * s[:, None], W, atol=0.5 * s.max() * 1.0001)


def test_w8_gemm_vs_numpy():
    rs = np.random.RandomState(3)
    M, N, K = 5, 48, 256
    x = rs.randn(M, K).astype(np.float16)
    W = rs.randn(N, K).astype(np.float32)
    q, s = orc.w8_quantize(W)
    y = orc.w8_gemm(x.view(np.uint16), q, s)
    ref = (x.astype(np.float64) @ q.astype(np.float64).T).astype(np.float32) * s
    assert np.array_equal(y, ref)
    # a transposed operand or a dropped scale fails
    assert not np.allclose(y, (x.astype(np.float64) @ q.astype(np.float64).T).astype(np.float32))


def test_attn_decode_closed_forms():
    rs = np.random.RandomState(6)
    B, Hq, Hkv, T, D = 1, 4, 2, 5, 16
    q = rs.randn(B, Hq, D).astype(np.float16)
    k = rs.randn(B, Hkv, T, D).astype(np.float16)
    v = rs.randn(B, Hkv, T, D).astype(np.float16)
    bits = lambda a: a.view(np.uint16)  # noqa: E731
    # one position: the output is its value row (each query head's own kv head)
    o = orc.attn_decode(bits(q), bits(k), bits(v), 1, 0.25)
    np.testing.assert_allclose(o[0, 0], v[0, 0, 0].astype(np.float32), rtol=1e-6)
    np.testing.assert_allclose(o[0, 3], v[0, 1, 0].astype(np.float32), rtol=1e-6)
    # equal scores (zero keys): the mean of the values
    o = orc.attn_decode(bits(q), bits(np.zeros_like(k)), bits(v), T, 0.25)
    np.testing.assert_allclose(o[0, 1], v[0, 0].astype(np.float64).mean(0), rtol=1e-6)
    # float64 numpy restatement
    o = orc.attn_decode(bits(q), bits(k), bits(v), T, 0.25)
    kk = np.repeat(k.astype(np.float64), Hq // Hkv, axis=1)
    vv = np.repeat(v.astype(np.float64), Hq // Hkv, axis=1)
    s = np.einsum("bhd,bhtd->bht", q.astype(np.float64), kk) * 0.25
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(o, np.einsum("bht,bhtd->bhd", p, vv), rtol=1e-6, atol=1e-7)


# ---- hybrid decode loop ----------------------------------------------------

def _hybrid_fixture(golden):
    d = golden("hf_hybrid.npz")
    cfg = orc.HybridConfig(*[d["cfg_" + f].item() for f, _ in orc.HybridConfig._fields_])
    return d, cfg


def test_hybrid_oracle_matches_hf_logits(golden):
    """Teacher-forced decode steps of the oracle model from an empty context
    against HF Qwen3_5ForCausalLM (fp32, eager attention) run over the whole
    sequence at once on the same dequantised weights.  The oracle rounds
    every matmul input and the KV cache to fp16, HF keeps fp32: 1e-3 of the
    largest logit bounds that (observed 2.6e-4); a flipped rotary sign, a
    missing output gate, a dropped q scale or a short attention window each
    move the logits by more than 2e-2 of it."""
    d, cfg = _hybrid_fixture(golden)
    m = orc.HybridModel(cfg, int(d["seed"]))
    m.reset(2, 0, 0)
    tokens, ref = d["tokens"], d["logits"]
    for t in range(tokens.shape[1]):
        nxt, lg = m.step(tokens[:, t])
        r = ref[:, t]
        assert np.abs(lg - r).max() <= 1e-3 * np.abs(r).max(), t
        top2 = np.sort(r, 1)[:, -2:]
        clear = top2[:, 1] - top2[:, 0] > 2e-3 * np.abs(r).max()
        assert np.array_equal(nxt[clear], r.argmax(1)[clear])
    assert m.position == tokens.shape[1]


def test_hybrid_oracle_batch_rows_independent(golden):
    """A sequence's logits do not depend on the other rows of the batch, and
    reset(context=0) restores the empty state exactly."""
    d, cfg = _hybrid_fixture(golden)
    m = orc.HybridModel(cfg, int(d["seed"]))
    tokens = d["tokens"]
    m.reset(2, 0, 0)
    both = [m.step(tokens[:, t])[1] for t in range(4)]
    m.reset(1, 0, 0)
    one = [m.step(tokens[1:, t])[1] for t in range(4)]
    for a, b in zip(both, one):
        assert np.array_equal(a[1], b[0])
    m.reset(2, 0, 0)
    again = [m.step(tokens[:, t])[1] for t in range(4)]
    for a, b in zip(both, again):
        assert np.array_equal(a, b)


def test_hybrid_oracle_drawn_context(golden):
    """reset(context > 0) draws the states for the context deterministically
    from the seed; different seeds give different continuations."""
    d, cfg = _hybrid_fixture(golden)
    m = orc.HybridModel(cfg, int(d["seed"]))
    tok = d["tokens"][:, 0]
    m.reset(2, 20, 3)
    a = m.step(tok)[1]
    assert m.position == 21
    m.reset(2, 20, 3)
    assert np.array_equal(a, m.step(tok)[1])
    m.reset(2, 20, 4)
    assert not np.allclose(a, m.step(tok)[1])
