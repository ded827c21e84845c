"""GPU parity of the hybrid decode loop (include/kai_gdn_hybrid.h) through the
C-ABI, against the oracle's CPU model (oracle/gdn_hybrid_oracle.c) drawn from
the same seed, and against the HF Qwen3_5ForCausalLM logits fixture.

Tolerance: 1e-3 of the step's largest |logit| for models of up to 8
layers (the device sums the int8 matmuls in fp32 where the oracle sums in
double and uses hardware exp and rsqrt; an fp16 rounding of an activation
that lands the other side of a rounding boundary moves a logit by about 1e-4
of the largest), and the greedy token wherever the oracle's top-2 margin
exceeds twice the tolerance.  Those flips accumulate through the residual
stream: at the 4B widths the measured error is 7e-4 (4 layers), 1.1e-3 (8),
1.6-1.8e-3 (16) and 2.2-2.6e-3 (32 layers), growing as sqrt(layers) and the
same after an empty or an 8192-token context, with the 2-norm error tracking
the maximum.  Deeper models are therefore held to 7e-4 * sqrt(layers) (4e-3
at 32 layers).
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import dev, empty, host, torch_mod

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def hb():
    torch = torch_mod()
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from orionsbelt_amd import hybrid
    return hybrid


@pytest.fixture(scope="module")
def fixture(golden):
    d = golden("hf_hybrid.npz")
    fields = {f: d["cfg_" + f].item() for f, _ in orc.HybridConfig._fields_}
    return d, fields


def models(hb, fields, seed, **over):
    f = dict(fields, **over)
    return hb.HybridModel(hb.config(**f), seed), orc.HybridModel(
        orc.HybridConfig(*[f[n] for n, _ in orc.HybridConfig._fields_]), seed)


def step(gm, tokens, vocab):
    torch = torch_mod()
    nxt = empty((gm.batch,), torch.int32)
    logits = empty((gm.batch, vocab), torch.float32)
    gm.step(dev(np.asarray(tokens, np.int32)), nxt, logits)
    return host(nxt), host(logits)


def tol(layers=8):
    return max(TOL, 7e-4 * np.sqrt(layers))


def assert_close(lg, ref, what, layers=8):
    scale = np.abs(ref).max()
    err = np.abs(lg - ref).max()
    print(f"{what}: max |dlogit| {err:.3e} = {err / scale:.2e} of the largest")
    assert err <= tol(layers) * scale, what


def assert_greedy(nxt, lg, ref, layers=8):
    # the device's token is its own logits' first maximum, exactly
    assert np.array_equal(nxt, lg.argmax(1))
    top2 = np.sort(ref, 1)[:, -2:]
    clear = top2[:, 1] - top2[:, 0] > 2 * tol(layers) * np.abs(ref).max()
    assert np.array_equal(nxt[clear], ref.argmax(1)[clear])


def test_hybrid_teacher_forced_matches_oracle_and_hf(hb, fixture):
    d, fields = fixture
    gm, om = models(hb, fields, int(d["seed"]))
    gm.reset(2, 0, 0)
    om.reset(2, 0, 0)
    tokens = d["tokens"]
    for t in range(tokens.shape[1]):
        nxt, lg = step(gm, tokens[:, t], fields["vocab"])
        onxt, olg = om.step(tokens[:, t])
        assert_close(lg, olg, f"step {t} vs oracle")
        assert_close(lg, d["logits"][:, t], f"step {t} vs HF")
        assert_greedy(nxt, lg, olg)
    assert gm.position == tokens.shape[1]


def test_hybrid_greedy_loop_on_device(hb, fixture):
    """Tokens fed back on the device for 10 steps; the oracle replays the
    device's tokens (teacher-forced) and checks each step's logits."""
    d, fields = fixture
    torch = torch_mod()
    gm, om = models(hb, fields, int(d["seed"]))
    gm.reset(2, 0, 0)
    om.reset(2, 0, 0)
    tok = dev(d["tokens"][:, 0].astype(np.int32))
    logits = empty((2, fields["vocab"]), torch.float32)
    for t in range(10):
        fed = host(tok).copy()
        nxt = empty((2,), torch.int32)
        gm.step(tok, nxt, logits)
        lg = host(logits)
        _, olg = om.step(fed)
        assert_close(lg, olg, f"greedy step {t}")
        assert_greedy(host(nxt), lg, olg)
        tok = nxt


def test_hybrid_drawn_context_two_spans(hb, fixture):
    """Three sequences after a drawn 300-token context (the attention decode
    reads two 256-position spans and combines them), in a cache of 310
    positions (the device rounds its tiled K cache up to 320)."""
    d, fields = fixture
    gm, om = models(hb, fields, 77, max_batch=3, max_context=310)
    gm.reset(3, 300, 9)
    om.reset(3, 300, 9)
    rs = np.random.RandomState(2)
    for t in range(3):
        tok = rs.randint(0, fields["vocab"], 3)
        nxt, lg = step(gm, tok, fields["vocab"])
        _, olg = om.step(tok)
        assert_close(lg, olg, f"context 300 step {t}")
        assert_greedy(nxt, lg, olg)
    assert gm.position == 303


def test_hybrid_batch_rows_independent_and_deterministic(hb, fixture):
    d, fields = fixture
    gm, _ = models(hb, fields, int(d["seed"]))
    tokens = d["tokens"]
    gm.reset(2, 0, 0)
    both = [step(gm, tokens[:, t], fields["vocab"])[1] for t in range(4)]
    gm.reset(1, 0, 0)
    one = [step(gm, tokens[1:, t], fields["vocab"])[1] for t in range(4)]
    gm.reset(2, 0, 0)
    again = [step(gm, tokens[:, t], fields["vocab"])[1] for t in range(4)]
    for a, b, c in zip(both, one, again):
        assert np.array_equal(a[1], b[0])
        assert np.array_equal(a, c)


def test_hybrid_rejects_bad_arguments(hb, fixture):
    d, fields = fixture
    from orionsbelt_amd import HipError
    gm = hb.HybridModel(hb.config(**dict(fields, max_context=4)), 1)
    with pytest.raises(HipError):
        gm.reset(3, 0, 0)   # batch above max_batch
    with pytest.raises(HipError):
        gm.reset(1, 4, 0)   # context must leave room for a step
    gm.reset(1, 3, 0)
    step(gm, [5], fields["vocab"])
    with pytest.raises(HipError):
        step(gm, [5], fields["vocab"])  # the KV cache is full
    import ctypes
    import orionsbelt_amd as ob
    host_tokens = (ctypes.c_int32 * 1)(5)
    assert ob.lib().kai_gdn_hybrid_step(gm._h, ctypes.addressof(host_tokens), None, None, None) != 0  # host memory
    with pytest.raises(HipError):
        hb.HybridModel(hb.config(**dict(fields, hidden=200)), 1)   # hidden % 256
    with pytest.raises(HipError):
        hb.HybridModel(hb.config(**dict(fields, attn_q_heads=8)), 1)   # 8 q heads per kv head
    with pytest.raises(HipError):
        hb.HybridModel(hb.config(**dict(fields, attn_q_heads=0)), 1)
    with pytest.raises(HipError):
        hb.HybridModel(hb.config(**dict(fields, max_context=(1 << 24) + 1)), 1)


def test_hybrid_qwen35_4b_shape(hb):
    """The full Qwen3.5-4B shape at batch 2 after a drawn 4000-token context,
    three greedy steps: finite logits, in-range tokens, bit-identical on a
    replay from the same reset."""
    torch = torch_mod()
    cfg = hb.qwen35_4b(2, 4096)
    assert (cfg.layers, cfg.hidden, cfg.inter, cfg.vocab) == (32, 2560, 9216, 151936)
    gm = hb.HybridModel(cfg, 12345)
    assert gm.weight_bytes > 3.9e9
    outs = []
    for _ in range(2):
        gm.reset(2, 4000, 7)
        nxt = empty((2,), torch.int32)
        logits = empty((2, cfg.vocab), torch.float32)
        run = []
        tok = dev(np.array([17, 151935], np.int32))
        for _t in range(3):
            gm.step(tok, nxt, logits)
            run.append((host(nxt).copy(), host(logits).copy()))
            tok = nxt.clone()
        outs.append(run)
    for (n1, l1), (n2, l2) in zip(*outs):
        assert np.isfinite(l1).all()
        assert ((n1 >= 0) & (n1 < cfg.vocab)).all()
        assert np.array_equal(n1, l1.argmax(1))
        assert np.array_equal(l1, l2) and np.array_equal(n1, n2)
    assert gm.position == 4003
    gm.close()


def oracle_config(cfg):
    return orc.HybridConfig(*[getattr(cfg, n) for n, _ in orc.HybridConfig._fields_])


def test_hybrid_qwen35_4b_vs_oracle(hb):
    """The full Qwen3.5-4B shape (hidden 2560, the 9216-wide MLP, the
    151936-wide LM head) against the CPU model after a drawn 8192-token
    context, two steps each: batch 1 (the small-batch matrices with the
    residual add in the branch matrices' epilogues and the norm formed in
    the reading matrices) and batch 4 (the separate norm kernel, the
    split-k down matrix).  Batches 2 and 3 give batch 1's rows bit for bit
    (test_hybrid_qwen35_4b_rows_same_at_batch_1_2_3)."""
    cfg = hb.qwen35_4b(4, 8200)
    gm = hb.HybridModel(cfg, 2468)
    om = orc.HybridModel(oracle_config(cfg), 2468)
    rs = np.random.RandomState(5)
    for B in (1, 4):
        gm.reset(B, 8192, 31)
        om.reset(B, 8192, 31)
        for t in range(2):
            tok = rs.randint(0, cfg.vocab, B)
            nxt, lg = step(gm, tok, cfg.vocab)
            _, olg = om.step(tok)
            assert_close(lg, olg, f"4B shape B={B} ctx 8192 step {t}", cfg.layers)
            assert_greedy(nxt, lg, olg, cfg.layers)
    gm.close()


def test_hybrid_qwen35_4b_rows_same_at_batch_1_2_3(hb):
    """At the 4B shape a sequence's logits do not depend on the batch: batch
    1 (norm formed inside the reading matrices, residual add in the branch
    matrices' epilogues) and batches 2 and 3 (the norm kernel) give row 0
    bit-identical logits and tokens over three steps from an empty context,
    whatever the other rows are fed."""
    torch = torch_mod()
    cfg = hb.qwen35_4b(3, 64)
    gm = hb.HybridModel(cfg, 97)
    rs = np.random.RandomState(11)
    toks = rs.randint(0, cfg.vocab, (3, 3)).astype(np.int32)
    runs = []
    for B in (1, 2, 3):
        gm.reset(B, 0, 0)
        run = []
        for t in range(3):
            nxt = empty((B,), torch.int32)
            logits = empty((B, cfg.vocab), torch.float32)
            gm.step(dev(toks[t, :B].copy()), nxt, logits)
            run.append((host(nxt)[0], host(logits)[0].copy()))
        runs.append(run)
    for t in range(3):
        assert np.isfinite(runs[0][t][1]).all()
        for B in (2, 3):
            assert np.array_equal(runs[B - 1][t][1], runs[0][t][1]), f"B={B} step {t}"
            assert runs[B - 1][t][0] == runs[0][t][0]
    gm.close()


@pytest.mark.parametrize("batch", [2, 4])
def test_hybrid_reduced_hidden_32k_context_vs_oracle(hb, batch):
    """Attention over a 32K-position drawn context (the spans and their
    combine at the config-5 length) with the 4B head counts and a small
    hidden size, against the CPU model, two steps: batch 2 (a grid sized
    to fill the GPU once) and batch 4 (over 2048 blocks of 256 positions,
    so spans sized for about 2048 blocks: 5 groups of 16 positions per
    wave)."""
    over = dict(layers=8, attn_every=4, hidden=512, inter=1024, vocab=2048, gdn_k_heads=16, gdn_v_heads=32,
                attn_q_heads=16, attn_kv_heads=4, max_batch=batch, max_context=32768 + 8, rope_theta=1e7,
                rms_eps=1e-6)
    gm = hb.HybridModel(hb.config(**over), 97)
    om = orc.HybridModel(orc.HybridConfig(*[over[n] for n, _ in orc.HybridConfig._fields_]), 97)
    gm.reset(batch, 32768, 3)
    om.reset(batch, 32768, 3)
    rs = np.random.RandomState(6)
    for t in range(2):
        tok = rs.randint(0, over["vocab"], batch)
        nxt, lg = step(gm, tok, over["vocab"])
        _, olg = om.step(tok)
        assert_close(lg, olg, f"batch {batch} ctx 32768 step {t}")
        assert_greedy(nxt, lg, olg)
    assert gm.position == 32770
    gm.close()


def test_hybrid_config5_batch16_ctx32k(hb):
    """Config 5's batch-16 decode at the 4B shape after a drawn 32K context
    (the state the bench times): finite logits, each device token its own
    logits' argmax, a replay from the same reset bit-identical, and row 0
    unchanged when every other row is fed different tokens (rows never mix)."""
    torch = torch_mod()
    B = 16
    cfg = hb.qwen35_4b(B, 32768 + 64)
    gm = hb.HybridModel(cfg, 12345)
    rs = np.random.RandomState(8)
    first = rs.randint(0, cfg.vocab, B).astype(np.int32)

    def run(tok0):
        gm.reset(B, 32768, 7)
        nxt = empty((B,), torch.int32)
        logits = empty((B, cfg.vocab), torch.float32)
        tok = dev(tok0)
        out = []
        for _t in range(3):
            gm.step(tok, nxt, logits)
            out.append((host(nxt).copy(), host(logits).copy()))
            tok = nxt.clone()
        return out

    a = run(first)
    b = run(first)
    other = first.copy()
    other[1:] = (other[1:] + 1000) % cfg.vocab
    c = run(other)
    for (n1, l1), (n2, l2), (n3, l3) in zip(a, b, c):
        assert np.isfinite(l1).all()
        assert ((n1 >= 0) & (n1 < cfg.vocab)).all()
        assert np.array_equal(n1, l1.argmax(1))
        assert np.array_equal(l1, l2) and np.array_equal(n1, n2)
        assert np.array_equal(l3[0], l1[0]) and n3[0] == n1[0]
        assert not np.array_equal(l3[1:], l1[1:])
    assert gm.position == 32768 + 3
    gm.close()


def test_e2e_driver_runs(hb):
    """The C driver (orionsbelt_amd/bin/gdn_e2e_decode, the reference e2e
    program's interface) decodes at the 4B shape and prints the reference's
    CSV rows: the decode report, a context sweep and the prefill report,
    with the per-layer-type columns (gdn_e2e_decode.c:2708-2710,2820-2857)
    filled by the library's timing mode: positive numbers, except the conv
    and decay shares of a decode step, which run inside the fused scan kernel
    (0); the decode shares add up to 100%."""
    import os
    import subprocess
    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "orionsbelt_amd", "bin",
                       "gdn_e2e_decode")
    r = subprocess.run([exe, "--tokens", "4", "--csv", "--batch", "2", "--ctx", "300"], capture_output=True,
                       text=True, timeout=240)
    assert r.returncode == 0, r.stderr
    head, row = r.stdout.strip().splitlines()[-2:]
    assert head.startswith("model,tokens,ttft_ms,tok_per_sec_mean,p50_us")
    f = row.split(",")
    assert f[0] == "Qwen3.5-4B" and f[1] == "4" and float(f[3]) > 0 and float(f[7]) > 0
    pct = [float(x) for x in f[8:15]]
    print("decode shares (proj, conv, decay, scan, oproj, full, ffn):", pct)
    assert pct[1] == 0.0 and pct[2] == 0.0
    assert all(pct[i] > 0 for i in (0, 3, 4, 5, 6)) and abs(sum(pct) - 100.0) < 0.5
    r = subprocess.run([exe, "--csv", "--ctx-sweep", "1,300"], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.strip().splitlines()
    assert lines[0].startswith("model,ctx_len,gdn_layer_us,full_attn_us,ffn_us,total_us")
    assert [ln.split(",")[1] for ln in lines[1:]] == ["1", "300"]
    for ln in lines[1:]:
        v = [float(x) for x in ln.split(",")[2:6]]
        print("sweep (gdn, full, ffn, total us):", v)
        assert all(x > 0 for x in v) and v[0] + v[1] + v[2] < 1.5 * v[3]
    # --prefill M: the reference's prefill report (gdn_e2e_decode.c:2708-2710)
    r = subprocess.run([exe, "--csv", "--prefill", "1000", "--batch", "2"], capture_output=True, text=True,
                       timeout=240)
    assert r.returncode == 0, r.stderr
    head, row = r.stdout.strip().splitlines()[-2:]
    assert head == "model,prefill_M,ttft_ms,tok_per_sec_prefill,gdn_us,full_us,ffn_us"
    f = row.split(",")
    assert f[0] == "Qwen3.5-4B" and f[1] == "1000" and float(f[2]) > 0 and float(f[3]) > 0
    gdn, full, ffn = (float(x) for x in f[4:7])
    print("prefill split (gdn, full, ffn us):", gdn, full, ffn, "ttft ms", f[2])
    assert gdn > 0 and full > 0 and ffn > 0 and (gdn + full + ffn) < 1.5 * float(f[2]) * 1e3


def test_hybrid_real_head_counts_vs_oracle(hb, fixture):
    """The 4B model's head counts (GDN 16 key / 32 value heads, attention 16
    query / 4 kv heads, so the in-projection is the 4B's 12352 rows) with a
    small hidden size and vocabulary, 8 layers (two attention), batch 4,
    after a drawn 40-token context: logits against the CPU model."""
    d, fields = fixture
    over = dict(layers=8, hidden=512, inter=1024, vocab=2048, gdn_k_heads=16, gdn_v_heads=32, attn_q_heads=16,
                attn_kv_heads=4, max_batch=4, max_context=64)
    gm, om = models(hb, fields, 4242, **over)
    gm.reset(4, 40, 11)
    om.reset(4, 40, 11)
    rs = np.random.RandomState(9)
    for t in range(5):
        tok = rs.randint(0, over["vocab"], 4)
        nxt, lg = step(gm, tok, over["vocab"])
        _, olg = om.step(tok)
        assert_close(lg, olg, f"4B heads step {t}")
        assert_greedy(nxt, lg, olg)


def test_hybrid_long_context_span_sizes_vs_oracle(hb, fixture):
    """Small attention grids size their spans to fill the GPU in one round
    (16 G positions per wave): batch 4 with 4 kv heads after drawn contexts
    of 3000 (G = 2) and 5000 positions (G = 3, an odd count of groups), and
    batch 1 at 5000 (G = 1 on 128-way span splits) -- logits against the
    CPU model."""
    d, fields = fixture
    over = dict(layers=4, hidden=512, inter=1024, vocab=2048, gdn_k_heads=16, gdn_v_heads=32, attn_q_heads=16,
                attn_kv_heads=4, max_batch=4, max_context=5010)
    gm, om = models(hb, fields, 515, **over)
    rs = np.random.RandomState(5)
    for batch, ctx in ((4, 3000), (4, 5000), (1, 5000)):
        gm.reset(batch, ctx, 3)
        om.reset(batch, ctx, 3)
        for t in range(2):
            tok = rs.randint(0, over["vocab"], batch)
            nxt, lg = step(gm, tok, over["vocab"])
            _, olg = om.step(tok)
            assert_close(lg, olg, f"batch {batch} context {ctx} step {t}")
            assert_greedy(nxt, lg, olg)


def test_hybrid_fused_and_separate_norms_agree(hb, fixture):
    """At batch 1 the residual add runs in the branch matrices' epilogues and
    the RMSNorm in every block of the matrices that read it (in-projections,
    gate|up, lm_head); from batch 2 both run in a kernel of their own, with
    the same arithmetic in the same order.  The same sequence stepped alone
    and as row 0 of batch 2 and batch 3 gives bit-identical logits and
    greedy tokens."""
    d, fields = fixture
    gm, _ = models(hb, fields, int(d["seed"]), max_batch=3)
    tokens = d["tokens"]
    gm.reset(1, 0, 0)
    one = [step(gm, tokens[:1, t], fields["vocab"]) for t in range(6)]
    gm.reset(2, 0, 0)
    two = [step(gm, tokens[:, t], fields["vocab"]) for t in range(6)]
    gm.reset(3, 0, 0)
    three = [step(gm, np.concatenate([tokens[:, t], tokens[:1, t]]), fields["vocab"]) for t in range(6)]
    for t, ((n1, l1), (n2, l2), (n3, l3)) in enumerate(zip(one, two, three)):
        assert np.array_equal(l2[:1], l1) and np.array_equal(l3[:1], l1), f"step {t}"
        assert n2[0] == n1[0] and n3[0] == n1[0], f"step {t}"
