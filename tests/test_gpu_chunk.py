"""GPU parity of the chunkwise (WY) prefill against the oracle's restatement
of HF torch_chunk_gated_delta_rule (fp32), through the C-ABI.

The kernel feeds bf16 operands to MFMA (q/k/v are bf16 inputs; T - I, the
bf16 copy of S, v_new and A are rounded to bf16 once each; R enters as a
bf16 hi + lo pair, or as one bf16 fragment in chunks whose M has 1-norm
below 1/2) and accumulates in fp32; the state stays fp32 and the
output is stored in bf16.  Bounds, relative to the largest reference
magnitude (max) and as a relative 2-norm (l2):
    output  max <= 1.0e-2   l2 <= 5.0e-3
    state   max <= 5.0e-3   l2 <= 3.0e-3
Measured on MI355X for every case below, T = 1 .. 16384 (all 32 value
heads at T = 16384, fp32 and fp16 state alike): output max 3.9e-3 .. 7.9e-3,
l2 2.9e-3 .. 3.1e-3; state max 1.4e-3 .. 3.3e-3, l2 1.5e-3 .. 1.9e-3.  The
fp32 oracle is itself within 1.5e-6 of the fp64 restatement, so these are the
kernel's bf16 roundings.  The bounds are at most 2x the worst measured value
and at the reference's bf16 bound after two chunks, 1e-2
(test_gdn_mixed.c:150-153,176-194); the error does not grow with T (the
gates bound it), so no drift factor is applied (the reference's rule,
docs/CORRECTNESS_TOLERANCES.md:34-49, would allow 1.5x at 8K and 2.25x at
16K).  The rank-1 repeated-key chunks have their own, stated bound.  Long
sequences are cut into segments that run in parallel (their results depend
on the cut, within the bound); calls split inside one segment are checked
bit for bit.  Every check prints the measured errors (pytest -s).
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc
from tests.gdn_inputs import bf16_bits, bf16_to_f32, prefill_inputs, rel_errors, round_bf16
from tests.gpu_util import P, dev, empty, host, host_u16, stream, torch_mod

pytestmark = pytest.mark.gpu

BOUNDS = {"output": (1.0e-2, 5.0e-3), "state": (5.0e-3, 3.0e-3)}


@pytest.fixture(scope="module")
def L():
    torch = torch_mod()
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orionsbelt_amd as ob
    return ob.lib()


def gpu_prefill(L, q, k, v, g, beta, S, f16=False, calls=None):
    """Run the prefill; `calls` splits T into consecutive calls that carry S."""
    import orionsbelt_amd as ob
    torch = torch_mod()
    B, T, Hk, d = q.shape
    Hv = v.shape[2]
    dq, dk_, dv_ = (dev(bf16_bits(x).view(np.int16)) for x in (q, k, v))
    dg, db = dev(g), dev(beta)
    do = empty((B, T, Hv, d), torch.int16)
    if f16:
        dS = dev(S.astype(np.float16).view(np.int16))
        fn = L.kai_run_gdn_chunk_delta_rule_bf16_f16state_hip
    else:
        dS = dev(S)
        fn = L.kai_run_gdn_chunk_delta_rule_bf16_f32_hip
    bounds = calls or [T]
    t0 = 0
    for tlen in bounds:
        sl = slice(t0, t0 + tlen)
        if len(bounds) == 1:
            args = (dq, dk_, dv_, dg, db, do)
        else:
            args = tuple(x[:, sl].contiguous() for x in (dq, dk_, dv_, dg, db)) + \
                (empty((B, tlen, Hv, d), torch.int16),)
        ob.check(fn(*(P(a) for a in args), P(dS), B, tlen, Hv, Hk, 1.0 / math.sqrt(d),
                    stream()), "prefill")
        if len(bounds) > 1:
            do[:, sl] = args[-1]
        t0 += tlen
    o = bf16_to_f32(host_u16(do))
    Sg = host_u16(dS).view(np.float16).astype(np.float32) if f16 else host(dS)
    return o, Sg


def check(got, ref, T, label):
    """`label` starts with "output" or "state" (or names them after a
    prefix): that tensor's bound applies."""
    kind = "state" if "state" in label else "output"
    mx, l2 = rel_errors(got, ref)
    bmx, bl2 = BOUNDS[kind]
    print(f"{label} (T={T}): max_rel {mx:.3e} l2_rel {l2:.3e}", flush=True)
    assert mx <= bmx and l2 <= bl2, f"{label}: max_rel {mx:.3e} l2_rel {l2:.3e} (bound {bmx:.1e} / {bl2:.1e})"
    return mx, l2


@pytest.mark.parametrize("B,T,Hv,Hk", [(1, 64, 2, 1), (1, 200, 4, 2), (2, 130, 2, 2),
                                      (1, 1, 2, 1), (1, 37, 2, 1), (1, 512, 32, 16)])
def test_prefill_vs_oracle(L, B, T, Hv, Hk):
    q, k, v, g, beta, S = prefill_inputs(T * 3 + Hv, B, T, Hv, Hk)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, B, T, Hv, Hk, 128, 128, 64)
    check(o, o_ref, T, "output")
    check(Sg, S_ref, T, "state")


def test_prefill_zero_initial_state(L):
    q, k, v, g, beta, S = prefill_inputs(5, 1, 256, 4, 2, zero_state=True)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, 256, 4, 2, 128, 128, 64)
    check(o, o_ref, 256, "output")
    check(Sg, S_ref, 256, "state")


def test_prefill_multi_segment_vs_oracle(L):
    """T above one 4096-token segment: the state crosses segment launches."""
    q, k, v, g, beta, S = prefill_inputs(9, 1, 4096 + 300, 2, 1)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, 4096 + 300, 2, 1, 128, 128, 64)
    check(o, o_ref, 4396, "output")
    check(Sg, S_ref, 4396, "state")


def test_prefill_segments_vs_oracle(L):
    """A sequence long enough to be cut into segments that run in parallel
    (segment transitions, the combine and the output pass), vs the oracle."""
    for T, Hv, Hk in [(2048 + 37, 4, 2), (64 * 40, 2, 1)]:
        q, k, v, g, beta, S = prefill_inputs(T + Hv, 1, T, Hv, Hk)
        o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
        o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, T, Hv, Hk, 128, 128, 64)
        check(o, o_ref, T, f"output T={T}")
        check(Sg, S_ref, T, f"state T={T}")


@pytest.mark.parametrize("gate", ["weak", "strong", "extreme", "mixed"])
def test_prefill_decay_regimes(L, gate):
    """Decay regimes, as per-token log-gates: weak -0.01 (the state is kept
    for thousands of tokens), strong -1.2 (each chunk decays by about
    e^-77), extreme -5 (e^G underflows to 0 inside a chunk: the state and
    the transitions are forgotten), mixed: chunks alternating between -0.6
    and -0.05.  T = 1000 (16 chunks, one segment) and T = 1600 at 32 heads
    (segments whose start states are composed from those transitions)."""
    for T, Hv, Hk in ((1000, 2, 1), (1600, 32, 16)):
        q, k, v, g, beta, S = prefill_inputs(77, 1, T, Hv, Hk)
        if gate == "weak":
            g[:] = -0.01
        elif gate == "strong":
            g[:] = -1.2
        elif gate == "extreme":
            g[:] = -5.0
        else:
            chunk = np.arange(T) // 64
            g[:] = np.where(chunk % 2 == 0, -0.6, -0.05)[None, :, None]
        o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
        # weak gates keep the state for thousands of tokens: the exact
        # two-pass path; the others forget it within a window
        assert L.kai_gdn_hip_prefill_windowed_heads() == (0 if gate == "weak" else Hv), gate
        o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, T, Hv, Hk, 128, 128, 64)
        check(o, o_ref, T, f"{gate} T={T} output")
        check(Sg, S_ref, T, f"{gate} T={T} state")


def test_prefill_positive_log_gates(L):
    """Log-gates of either sign (the kernel must not assume g <= 0): the
    Gamma factors exp(G_i - G_j) then exceed 1 inside a chunk."""
    q, k, v, g, beta, S = prefill_inputs(31, 1, 200, 2, 1)
    g = np.random.RandomState(32).uniform(-0.3, 0.05, g.shape).astype(np.float32)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, 200, 2, 1, 128, 128, 64)
    check(o, o_ref, 200, "output")
    check(Sg, S_ref, 200, "state")


def test_prefill_repeated_keys(L):
    """Degenerate chunks: every token has the same key, beta near 1, little or
    no decay (a repeated token).  M is then nearly the all-ones strictly lower
    triangle and T = (I + M)^-1 nearly the alternating bidiagonal I - shift:
    T R is a difference of consecutive rows of R that almost cancel, so R
    must enter the T product with more than bf16's 8 bits (the kernel uses a
    hi + lo pair), and the diagonal blocks of T must be exact enough to
    cancel (fp32 substitution).  Rank-1 keys also amplify the bf16 rounding
    of T's off-diagonal blocks and of v_new, so the bound here is looser than
    the generic one: max_rel <= 4e-2 and l2_rel <= 3.5e-2 (measured: output
    1.9e-2 / 1.6e-2, state 2.7e-2 / 2.5e-2 at beta = 1; 1.7e-2 / 1.8e-2 at
    beta = 0.9)."""
    for beta_v, g_v in [(1.0, 0.0), (0.9, -0.01)]:
        q, k, v, g, beta, S = prefill_inputs(41, 1, 256, 2, 1)
        k[:, :] = k[:, :1]
        beta[:] = beta_v
        g[:] = g_v
        o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
        o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, 256, 2, 1, 128, 128, 64)
        for got, ref, what in [(o, o_ref, "output"), (Sg, S_ref, "state")]:
            mx, l2 = rel_errors(got, ref)
            print(f"repeated keys beta={beta_v} {what}: max_rel {mx:.3e} l2_rel {l2:.3e}", flush=True)
            assert mx <= 4e-2 and l2 <= 3.5e-2, f"beta={beta_v} {what}: max_rel {mx:.3e} l2_rel {l2:.3e}"


@pytest.mark.parametrize("beta_v", [0.0075, 0.0085])
def test_prefill_repeated_keys_at_the_norm_bound(L, beta_v):
    """The one-fragment T R product is taken when the chunk's M has 1-norm
    below 1/2.  Identical keys with no decay make column 0 of M sum to
    63 beta |k|^2: 0.47 at beta = 0.0075 (one bf16 fragment of R) and 0.54 at
    0.0085 (the hi + lo pair).  A zero start state leaves the outputs to the
    v products alone; both sides of the bound meet the generic bounds."""
    q, k, v, g, beta, S = prefill_inputs(43, 1, 256, 2, 1)
    k[:, :] = k[:, :1]
    beta[:] = beta_v
    g[:] = 0.0
    S[:] = 0.0
    col0 = 63 * beta_v * float(np.sum(round_bf16(k[0, 0, 0]) ** 2))
    assert (col0 < 0.5) == (beta_v < 0.008)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, 256, 2, 1, 128, 128, 64)
    check(o, o_ref, 256, f"norm-bound beta={beta_v} output")
    check(Sg, S_ref, 256, f"norm-bound beta={beta_v} state")


@pytest.mark.parametrize("seed", range(12))
def test_prefill_random_shapes(L, seed):
    """Seeded random shapes and gate regimes against the oracle: batch 1-3,
    1-2 value heads per key head, ragged T, fp32 or fp16 state, and gates
    that take the windowed path, the exact path, or both within one call
    (every other head slow).  Each case prints its shape and how many heads
    ran windowed."""
    rng = np.random.default_rng(seed)
    B = int(rng.choice([1, 1, 2, 3]))
    Hk = int(rng.choice([1, 2, 4, 8, 16]))
    Hv = Hk * int(rng.choice([1, 2]))
    T = int(rng.integers(1, 6000 if B * Hv <= 8 else 2500))
    regime = ["base", "weak", "slow", "strong", "mixed", "perhead"][seed % 6]
    q, k, v, g, beta, S = prefill_inputs(2000 + seed, B, T, Hv, Hk)
    if regime == "weak":
        g[:] = -0.003
    elif regime == "slow":
        g[:] = -float(rng.uniform(0.008, 0.05))
    elif regime == "strong":
        g[:] = -1.0
    elif regime == "mixed":
        g[:] = np.where((np.arange(T) // 64) % 2 == 0, -0.6, -0.02)[None, :, None]
    elif regime == "perhead":
        g[:] = np.where(np.arange(Hv) % 2 == 0, -0.005, -0.4)[None, None, :]
    f16 = seed % 4 == 3
    if f16:
        S = S.astype(np.float16).astype(np.float32)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S, f16=f16)
    windowed = L.kai_gdn_hip_prefill_windowed_heads()
    print(f"B={B} T={T} Hv={Hv} Hk={Hk} {regime} f16={f16}: {windowed} windowed", flush=True)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, B, T, Hv, Hk, 128, 128, 64)
    check(o, o_ref, T, f"random {seed} output")
    check(Sg, S_ref, T, f"random {seed} state")


def test_prefill_split_calls_bit_identical(L):
    """Calls split at chunk boundaries carry the fp32 state exactly."""
    q, k, v, g, beta, S = prefill_inputs(13, 1, 640, 4, 2)
    o1, S1 = gpu_prefill(L, q, k, v, g, beta, S)
    o2, S2 = gpu_prefill(L, q, k, v, g, beta, S, calls=[128, 64, 448])
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(S1.view(np.uint32), S2.view(np.uint32))


def test_prefill_matches_decode_steps(L):
    """A prefill of T tokens and T GPU decode steps run the same recurrence."""
    import orionsbelt_amd as ob
    torch = torch_mod()
    B, T, Hv, Hk, d = 1, 48, 4, 2, 128
    q, k, v, g, beta, S = prefill_inputs(21, B, T, Hv, Hk)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    dS = dev(S)
    outs = []
    for t in range(T):
        dq, dk_, dv_ = dev(q[:, t]), dev(k[:, t]), dev(v[:, t])
        dg, db = dev(g[:, t]), dev(beta[:, t])
        do = empty((B, Hv, d), torch.float32)
        ob.check(L.kai_run_gdn_delta_rule_decode_f32_hip(
            P(dS), P(dq), P(dk_), P(dv_), P(dg), P(db), P(do), B, Hv, Hk, d, d,
            1.0 / math.sqrt(d), stream()), "decode")
        outs.append(host(do))
    check(o, np.stack(outs, axis=1), T, "prefill vs decode output")
    check(Sg, host(dS), T, "prefill vs decode state")


def test_prefill_f16_state(L):
    q, k, v, g, beta, S = prefill_inputs(17, 1, 300, 4, 2)
    S16 = S.astype(np.float16).astype(np.float32)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S16, f16=True)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S16, 1, 300, 4, 2, 128, 128, 64)
    check(o, o_ref, 300, "output")
    check(Sg, S_ref, 300, "state (fp16)")


def test_prefill_config3_all_heads(L):
    """Config 3 (B=1, T=16384, Hv=32, Hk=16, chunk 64, bf16 q/k/v, fp32
    state): every value head against the oracle over the whole sequence,
    then the properties: finite, and one call agrees with two calls split at
    a chunk boundary (each call cuts its own sequence into segments, so the
    agreement is to the stated bound, not bit for bit)."""
    B, T, Hv, Hk = 1, 16384, 32, 16
    q, k, v, g, beta, S = prefill_inputs(3, B, T, Hv, Hk)
    o1, S1 = gpu_prefill(L, q, k, v, g, beta, S)
    # the config-3 gates decay the state by about e^-22 per chunk: every
    # head runs windowed
    assert L.kai_gdn_hip_prefill_windowed_heads() == B * Hv
    assert np.isfinite(o1).all() and np.isfinite(S1).all()
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, B, T, Hv, Hk, 128, 128, 64)
    check(o1, o_ref, T, "output, all 32 heads")
    check(S1, S_ref, T, "state, all 32 heads")
    o2, S2 = gpu_prefill(L, q, k, v, g, beta, S, calls=[8192, 8192])
    check(o2, o1, T, "two calls vs one, output")
    check(S2, S1, T, "two calls vs one, state")


def test_prefill_rejects_bad_args(L):
    assert L.kai_run_gdn_chunk_delta_rule_bf16_f32_hip(None, None, None, None, None, None, None,
                                                       1, 64, 3, 2, 1.0, None) != 0


@pytest.mark.parametrize("T", [1024, 8192])
def test_prefill_config4_f16_state_all_heads(L, T):
    """Config 4 (fp16 recurrent state, fp32 accumulation) at the 4B head
    shape (Hv=32, Hk=16): every value head against the oracle, which starts
    from the same fp16-rounded state; the kernel's final state is narrowed to
    fp16 once, on exit."""
    B, Hv, Hk = 1, 32, 16
    q, k, v, g, beta, S = prefill_inputs(60 + T, B, T, Hv, Hk)
    S16 = S.astype(np.float16).astype(np.float32)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S16, f16=True)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S16, B, T, Hv, Hk, 128, 128, 64)
    check(o, o_ref, T, f"output T={T}")
    check(Sg, S_ref, T, f"state (fp16) T={T}")


def device_inputs(seed, T, Hv, Hk, d=128):
    """Config-2/3 distributions drawn on the device (long sequences): bf16
    q, k (L2-normalised), v; fp32 g = -softplus(N) * e^U(-2,0), beta =
    sigmoid(N); an fp16 initial state ~ N(0, 0.02)."""
    torch = torch_mod()
    gen = torch.Generator(device="cuda").manual_seed(seed)
    def randn(*shape):
        return torch.randn(*shape, device="cuda", generator=gen)
    q = torch.nn.functional.normalize(randn(1, T, Hk, d), dim=-1).to(torch.bfloat16)
    k = torch.nn.functional.normalize(randn(1, T, Hk, d), dim=-1).to(torch.bfloat16)
    v = randn(1, T, Hv, d).to(torch.bfloat16)
    u = torch.rand(1, T, Hv, device="cuda", generator=gen) * -2.0
    g = (-torch.nn.functional.softplus(randn(1, T, Hv)) * torch.exp(u)).contiguous()
    beta = torch.sigmoid(randn(1, T, Hv)).contiguous()
    S = (0.02 * randn(1, Hv, d, d)).to(torch.float16)
    return q, k, v, g, beta, S


def gpu_prefill_dev(L, q, k, v, g, beta, S16, calls):
    """fp16-state prefill of device tensors over consecutive calls; returns
    (o bf16 [1][T][Hv][128], final fp16 state) on the device."""
    import orionsbelt_amd as ob
    torch = torch_mod()
    _, T, Hk, d = q.shape
    Hv = v.shape[2]
    S = S16.clone()
    o = torch.empty((1, T, Hv, d), dtype=torch.bfloat16, device="cuda")
    t0 = 0
    for tlen in calls:
        sl = slice(t0, t0 + tlen)
        xs = [x[:, sl].contiguous() for x in (q, k, v, g, beta)]
        oc = torch.empty((1, tlen, Hv, d), dtype=torch.bfloat16, device="cuda")
        ob.check(L.kai_run_gdn_chunk_delta_rule_bf16_f16state_hip(
            *(P(x) for x in xs), P(oc), P(S), 1, tlen, Hv, Hk, 1.0 / math.sqrt(d), stream()), "prefill f16")
        o[:, sl] = oc
        t0 += tlen
    torch.cuda.synchronize()
    return o, S


@pytest.mark.parametrize("T", [32768, 131072])
def test_prefill_config4_long_sequences(L, T):
    """Config 4 at T = 32K and 128K: finite; one call agrees with two calls
    split at the middle (a chunk boundary) to the stated bound; the two value
    heads of the last key head agree with the oracle over the whole
    sequence."""
    torch = torch_mod()
    Hv, Hk = 32, 16
    print(f"config 4 fp16 state T={T}", flush=True)
    q, k, v, g, beta, S = device_inputs(T, T, Hv, Hk)
    o1, S1 = gpu_prefill_dev(L, q, k, v, g, beta, S, [T])
    assert torch.isfinite(o1).all().item() and torch.isfinite(S1).all().item()
    o2, S2 = gpu_prefill_dev(L, q, k, v, g, beta, S, [T // 2, T // 2])
    f32 = lambda x: x.float().cpu().numpy()  # noqa: E731
    check(f32(o2), f32(o1), T, "two calls vs one, output")
    check(f32(S2), f32(S1), T, "two calls vs one, state")
    hv = slice(Hv - 2, Hv)  # value heads 30, 31 read key head 15
    sub = [np.ascontiguousarray(f32(x)) for x in (q[:, :, Hk - 1:], k[:, :, Hk - 1:], v[:, :, hv], g[:, :, hv],
                                                   beta[:, :, hv], S[:, hv])]
    o_ref, S_ref = orc.chunk_gdr(*sub, 1, T, 2, 1, 128, 128, 64)
    check(f32(o1[:, :, hv]), o_ref, T, f"output T={T}, heads 30-31")
    check(f32(S1[:, hv]), S_ref, T, f"state (fp16) T={T}, heads 30-31")


def test_prefill_windowed_and_exact_heads_in_one_call(L):
    """Per head, the call picks its path: heads with weak gates (-0.01) run
    the exact two-pass segments, heads with config-3 gates run windowed
    segments, in the same launches; both against the oracle."""
    T, Hv, Hk = 2048 + 37, 8, 4
    q, k, v, g, beta, S = prefill_inputs(T + 11, 1, T, Hv, Hk)
    g[:, :, ::2] = -0.01
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    assert L.kai_gdn_hip_prefill_windowed_heads() == Hv // 2
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, T, Hv, Hk, 128, 128, 64)
    check(o, o_ref, T, "mixed paths output")
    check(Sg, S_ref, T, "mixed paths state")


@pytest.mark.parametrize("g_val,windowed", [(-1.0, False), (-2.0, True)])
def test_prefill_window_bound_counts_key_norms(L, g_val, windowed):
    """Keys of norm 3 with beta = 0.5: one token's state map has norm
    e^g |1 - 4.5| = 3.5 e^g, so g = -1 (3.5 e^-1 > 1: no window bounds the
    state) must take the exact path and g = -2 (0.47 per token) may run
    windowed.  Both against the oracle."""
    T, Hv, Hk = 1600, 4, 2
    q, k, v, g, beta, S = prefill_inputs(91, 1, T, Hv, Hk)
    k = round_bf16(3.0 * k)
    beta[:] = 0.5
    g[:] = g_val
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    assert L.kai_gdn_hip_prefill_windowed_heads() == (Hv if windowed else 0)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, T, Hv, Hk, 128, 128, 64)
    check(o, o_ref, T, f"|k| = 3, g = {g_val} output")
    check(Sg, S_ref, T, f"|k| = 3, g = {g_val} state")


@pytest.mark.parametrize("chunk_log2", [-20.0, -70.0, -120.0])
def test_prefill_window_lengths(L, chunk_log2):
    """Gates whose chunk decays by 2^-20 (two chunks meet the 2^-24 bound),
    2^-70 and 2^-120 (one chunk); the last chunk of the window is where a
    mistake in the window's start would show.  Against the oracle."""
    T, Hv, Hk = 4096 + 64 * 3, 4, 2
    q, k, v, g, beta, S = prefill_inputs(5 + int(-chunk_log2), 1, T, Hv, Hk)
    g[:] = chunk_log2 / 64 * math.log(2.0)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    assert L.kai_gdn_hip_prefill_windowed_heads() == Hv
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, T, Hv, Hk, 128, 128, 64)
    check(o, o_ref, T, f"chunk decay 2^{chunk_log2:.0f} output")
    check(Sg, S_ref, T, f"chunk decay 2^{chunk_log2:.0f} state")


@pytest.mark.parametrize("T,g_val,windowed", [(8192, -0.027, True), (8192, -0.01, False), (16384, -0.01, True)])
def test_prefill_long_windows(L, T, g_val, windowed):
    """Windows up to the planned segment length: with 32 heads the plan has
    8 segments, of 16 chunks at T = 8192 and 32 at T = 16384, and windows
    of up to that many chunks are checked.  g = -0.027 decays a chunk by
    2^-2.49, so ten chunks meet the 2^-24 bound (windowed, ten warm-up
    chunks per segment; the gates read in a second round); g = -0.01 needs
    26: the exact two-pass path at T = 8192, 26-chunk windows at T = 16384
    (the bench's long-memory line).  Against the oracle, all heads."""
    Hv, Hk = 32, 16
    q, k, v, g, beta, S = prefill_inputs(61, 1, T, Hv, Hk)
    g[:] = g_val
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    assert L.kai_gdn_hip_prefill_windowed_heads() == (Hv if windowed else 0)
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, 1, T, Hv, Hk, 128, 128, 64)
    check(o, o_ref, T, f"g={g_val} output")
    check(Sg, S_ref, T, f"g={g_val} state")


def test_prefill_windowed_f16_state(L):
    """The fp16-state variant runs windowed too (its initial state read once,
    its final state narrowed once)."""
    T, Hv, Hk = 4096, 8, 4
    q, k, v, g, beta, S = prefill_inputs(123, 1, T, Hv, Hk)
    S16 = S.astype(np.float16).astype(np.float32)
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S16, f16=True)
    assert L.kai_gdn_hip_prefill_windowed_heads() == Hv
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S16, 1, T, Hv, Hk, 128, 128, 64)
    check(o, o_ref, T, "windowed fp16 output")
    check(Sg, S_ref, T, "windowed fp16 state (fp16)")


def test_prefill_windowed_batch_of_two(L):
    """Two sequences in one call, both windowed but for one head of the
    second sequence, whose weak gates take the exact path: each (sequence,
    head) decides on its own, and the final states land in their own slots.
    Ragged T (not a multiple of 64)."""
    B, T, Hv, Hk = 2, 3000, 4, 2
    q, k, v, g, beta, S = prefill_inputs(202, B, T, Hv, Hk)
    g[1, :, 3] = -0.01
    o, Sg = gpu_prefill(L, q, k, v, g, beta, S)
    assert L.kai_gdn_hip_prefill_windowed_heads() == B * Hv - 1
    o_ref, S_ref = orc.chunk_gdr(q, k, v, g, beta, S, B, T, Hv, Hk, 128, 128, 64)
    check(o, o_ref, T, "B=2 output")
    check(Sg, S_ref, T, "B=2 state")
