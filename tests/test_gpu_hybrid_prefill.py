"""GPU parity of the hybrid model's prefill (kai_gdn_hybrid_prefill): every
position of a prompt through each layer at once (int8 GEMMs on MFMA, the
conv and gating glue, the chunked delta rule on bf16 MFMA, causal attention
that fills the KV cache), against
  - HF Qwen3_5ForCausalLM's logits of the same prompt (the golden fixture:
    HF runs the chunked GDN form and causal-masked attention, a prefill);
  - the CPU model stepping the prompt token by token;
and the decode steps that continue from the prefilled states.

Tolerance: the prefill feeds the delta rule bf16 q, k, v and stores its
output in bf16 (the decode step keeps them fp32: the chunked kernel's own
error against the fp32 oracle is about 3e-3 in 2-norm, test_gpu_chunk.py),
so its logits carry that rounding through every GDN layer on top of the
decode loop's error.  Bounds, as fractions of the largest logit, at about
twice what was measured on MI355X:
  fixture model (4 layers, hidden 256, one attention layer): 2e-3
      (measured 4e-4 .. 8e-4 after prompts of 1 .. 2000 tokens; the decode
      steps that follow 1.2e-4 .. 2.9e-4);
  4B widths, 4 attention layers: 2.5e-3 (measured 1.06e-3, as the decode
      loop's 9.9e-4: the attention prefill adds nothing measurable);
  4B widths, 4 GDN layers: 1.2e-2 against the CPU model with the delta
      rule's q, k, v and output rounded to bf16 as the prefill hands them on
      (measured 5.9e-3: the kernels' own error, chiefly the bf16 state in the
      MFMA products), 1.6e-2 against the all-fp32 CPU model (measured 7.8e-3;
      the two CPU models differ by 7.8e-3, so this is the format's share);
  the full 4B model (24 GDN + 8 attention layers): 5e-2 against either CPU
      model (measured 2.4e-2 and 2.3e-2, the two CPU models differ by 2.4e-2:
      32 random-init layers amplify a 1e-3 perturbation of one layer's output
      20-fold, so at this depth the kernel and format shares are of one
      size); the logit rows' relative 2-norm and their top-10 overlap are
      held as well, which do not loosen with the max-abs bound;
  32K-token prompts at the 4B head counts (hidden 256): two GDN layers 1.2e-3
      against the rounded CPU model (measured 5.4e-4); two GDN and two
      attention layers 1.6e-3 against the GPU decode loop stepping the prompt
      (measured 7.0e-4); the whole 4B model, prefill of T then a step against
      a prefill of T + 1: 3e-2 (measured 1.4e-2).
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import dev, empty, host, torch_mod

pytestmark = pytest.mark.gpu

FIXTURE_TOL = 2e-3
# Bounds of the tests at the 4B head counts, as fractions of the largest
# logit (measured values in each test's output and in the module docstring).
TOL_4B_GDN, FMT_4B_GDN = 1.2e-2, 1.6e-2
TOL_4B, FMT_4B = 5e-2, 5e-2
TOL_32K_GDN = 1.2e-3
TOL_32K_ATT = 1.6e-3
TOL_4B_32K_STEP = 3e-2
# Agreement of whole logit rows that does not loosen with the max-abs
# bound: relative 2-norm of the difference (measured 2.55e-2 for the 4B
# model's 70-token prefill against the rounded CPU model), and how many of
# the reference's 10 largest logits are among the device's 10 largest
# (measured 9).
REL2_4B, TOP10_4B = 5e-2, 7


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


def close(lg, ref, what, tol=FIXTURE_TOL):
    scale = np.abs(ref).max()
    err = np.abs(lg - ref).max()
    print(f"{what}: max |dlogit| {err:.3e} = {err / scale:.2e} of the largest", flush=True)
    assert err <= tol * scale, what


def greedy(nxt, lg, ref, tol=FIXTURE_TOL):
    assert np.array_equal(nxt, lg.argmax(1))  # the device's token is its logits' first maximum
    top2 = np.sort(ref, 1)[:, -2:]
    clear = top2[:, 1] - top2[:, 0] > 2 * tol * np.abs(ref).max()
    assert np.array_equal(nxt[clear], ref.argmax(1)[clear])


def prefill(gm, tokens, vocab):
    torch = torch_mod()
    B = tokens.shape[0]
    nxt = empty((B,), torch.int32)
    lg = empty((B, vocab), torch.float32)
    gm.prefill(dev(np.ascontiguousarray(tokens, dtype=np.int32)), nxt, lg)
    return host(nxt), host(lg)


def step(gm, tokens, vocab):
    torch = torch_mod()
    nxt = empty((gm.batch,), torch.int32)
    lg = empty((gm.batch, vocab), torch.float32)
    gm.step(dev(np.asarray(tokens, np.int32)), nxt, lg)
    return host(nxt), host(lg)


@pytest.mark.parametrize("T", [1, 7, 12])
def test_prefill_matches_hf_and_oracle(hb, fixture, T):
    """Prompts of 1, 7 and 12 tokens of the fixture's two sequences, then
    the decode steps through the rest of the fixture from the prefilled
    states, each against HF and the CPU model."""
    d, fields = fixture
    gm, om = models(hb, fields, int(d["seed"]))
    tokens = d["tokens"]
    nxt, lg = prefill(gm, tokens[:, :T], fields["vocab"])
    assert gm.position == T
    om.reset(2, 0, 0)
    for t in range(T):
        _, olg = om.step(tokens[:, t])
    close(lg, olg, f"prefill {T} vs oracle")
    close(lg, d["logits"][:, T - 1], f"prefill {T} vs HF")
    greedy(nxt, lg, olg)
    for t in range(T, tokens.shape[1]):
        nxt, lg = step(gm, tokens[:, t], fields["vocab"])
        _, olg = om.step(tokens[:, t])
        close(lg, olg, f"prefill {T}, step {t} vs oracle")
        close(lg, d["logits"][:, t], f"prefill {T}, step {t} vs HF")
        greedy(nxt, lg, olg)


def test_prefill_long_prompt_vs_oracle(hb, fixture):
    """2000-token prompts of two sequences (32 chunks: the delta rule runs
    as parallel segments; 63 key blocks of the attention, ragged at both
    ends) with two attention layers, against the CPU model stepping the
    prompt; then three decode steps."""
    d, fields = fixture
    gm, om = models(hb, fields, 5150, attn_every=2, max_context=2100)
    rs = np.random.RandomState(11)
    T = 2000
    tokens = rs.randint(0, fields["vocab"], (2, T)).astype(np.int32)
    nxt, lg = prefill(gm, tokens, fields["vocab"])
    om.reset(2, 0, 0)
    for t in range(T):
        _, olg = om.step(tokens[:, t])
    close(lg, olg, f"prefill {T} vs oracle")
    greedy(nxt, lg, olg)
    for t in range(3):
        tok = rs.randint(0, fields["vocab"], 2)
        nxt, lg = step(gm, tok, fields["vocab"])
        _, olg = om.step(tok)
        close(lg, olg, f"after prefill {T}, step {t}")
        greedy(nxt, lg, olg)
    assert gm.position == T + 3


def test_prefill_rows_independent_and_replayable(hb, fixture):
    """A batch's sequences do not interact (batch 2 equals each sequence
    prefilled alone, bit for bit), a repeated prefill reproduces itself, and
    a prefill resets whatever the model held before."""
    d, fields = fixture
    gm, _ = models(hb, fields, 321, max_context=300)
    rs = np.random.RandomState(3)
    tokens = rs.randint(0, fields["vocab"], (2, 250)).astype(np.int32)
    n2, l2 = prefill(gm, tokens, fields["vocab"])
    step(gm, [1, 2], fields["vocab"])  # state moved on
    n2b, l2b = prefill(gm, tokens, fields["vocab"])
    assert np.array_equal(l2.view(np.uint32), l2b.view(np.uint32)) and np.array_equal(n2, n2b)
    for b in range(2):
        n1, l1 = prefill(gm, tokens[b:b + 1], fields["vocab"])
        assert np.array_equal(l1[0].view(np.uint32), l2[b].view(np.uint32))


def test_prefill_rejects_bad_arguments(hb, fixture):
    import orionsbelt_amd as ob
    torch = torch_mod()
    d, fields = fixture
    gm, _ = models(hb, fields, 1)
    L = ob.lib()
    tok = dev(np.zeros((2, 8), np.int32))
    assert L.kai_gdn_hybrid_prefill(gm._h, tok.data_ptr(), 3, 8, None, None, None) != 0        # batch > max
    assert L.kai_gdn_hybrid_prefill(gm._h, tok.data_ptr(), 2, 0, None, None, None) != 0        # empty prompt
    assert L.kai_gdn_hybrid_prefill(gm._h, tok.data_ptr(), 2, fields["max_context"], None, None, None) != 0
    host_tok = np.zeros((2, 8), np.int32)
    assert L.kai_gdn_hybrid_prefill(gm._h, host_tok.ctypes.data, 2, 8, None, None, None) != 0  # host memory
    assert L.kai_gdn_hybrid_prefill(gm._h, tok.data_ptr(), 2, 8, None, None, None) == 0
    torch.cuda.synchronize()
    assert gm.position == 8


def rel_err(lg, ref):
    return float(np.abs(lg - ref).max() / np.abs(ref).max())


def agreement(lg, ref, what, rel2_tol, top10_min):
    """Relative 2-norm of lg - ref per row and the overlap of the rows' 10
    largest entries."""
    for r in range(ref.shape[0]):
        rel2 = float(np.linalg.norm(lg[r] - ref[r]) / np.linalg.norm(ref[r]))
        top = len(set(np.argsort(lg[r])[-10:]) & set(np.argsort(ref[r])[-10:]))
        print(f"{what}, row {r}: relative 2-norm {rel2:.2e}, top-10 overlap {top}/10", flush=True)
        assert rel2 <= rel2_tol and top >= top10_min, what


def prefill_vs_oracle(hb, fields, seed, T, tol, what, steps=0, fmt_tol=None, rows=None):
    """The device prefill of a T-token prompt against the CPU model stepping
    it with the recurrence's operands and output rounded to bf16 (the
    prefill's formats: what remains is the kernels' own error, held to
    `tol`), and against the all-fp32 CPU model (format + kernel error,
    held to `fmt_tol`); then `steps` greedy decode steps against the
    rounded model continuing from its state."""
    gm, om = models(hb, fields, seed)
    _, om32 = models(hb, fields, seed) if fmt_tol else (None, None)
    rs = np.random.RandomState(5)
    tokens = rs.randint(0, fields["vocab"], (1, T)).astype(np.int32)
    nxt, lg = prefill(gm, tokens, fields["vocab"])
    om.reset(1, 0, 0)
    om.set_gdn_bf16_io(True)
    if om32:
        om32.reset(1, 0, 0)
    for t in range(T):
        _, olg = om.step(tokens[:, t])
        if om32:
            _, olg32 = om32.step(tokens[:, t])
    close(lg, olg, f"{what}: prefill {T} vs oracle (bf16 delta-rule I/O)", tol)
    greedy(nxt, lg, olg, tol)
    if rows:
        agreement(lg, olg, f"{what}: prefill {T} vs oracle (bf16 delta-rule I/O)", *rows)
    if om32:
        close(lg, olg32, f"{what}: prefill {T} vs fp32 oracle (format bound)", fmt_tol)
        close(olg, olg32, f"{what}: bf16-I/O oracle vs fp32 oracle", fmt_tol)
    om.set_gdn_bf16_io(False)  # the decode step keeps the recurrence in fp32
    for t in range(steps):
        tok = nxt.copy()
        nxt, lg = step(gm, tok, fields["vocab"])
        _, olg = om.step(tok)
        close(lg, olg, f"{what}: after prefill, step {t}", tol)
    gm.close()


def widths_4b(**over):
    f = dict(layers=4, attn_every=4, hidden=2560, inter=9216, vocab=2048, gdn_k_heads=16, gdn_v_heads=32,
             attn_q_heads=16, attn_kv_heads=4, max_batch=1, max_context=128, rope_theta=1e7, rms_eps=1e-6)
    f.update(over)
    return f


def test_prefill_4b_widths_attention_layers(hb):
    """Four attention layers at the 4B widths (16 query / 4 kv heads: four
    kv heads' blocks), a 70-token prompt, against the CPU model."""
    prefill_vs_oracle(hb, widths_4b(attn_every=1), 2468, 70, 2.5e-3, "4B widths, attention", steps=2)


def test_prefill_4b_widths_gdn_layers(hb):
    """Four GDN layers at the 4B widths (16 key / 32 value heads, conv
    width 8192), a 70-token prompt (two chunks), against the CPU model."""
    prefill_vs_oracle(hb, widths_4b(attn_every=100), 2468, 70, TOL_4B_GDN, "4B widths, GDN", steps=2,
                      fmt_tol=FMT_4B_GDN)


def test_prefill_qwen35_4b_vs_oracle(hb):
    """The whole 4B model (32 layers, hidden 2560, vocab 151936): a 70-token
    prompt against the CPU model stepping it, then two decode steps."""
    cfg = hb.qwen35_4b(1, 128)
    fields = {n: getattr(cfg, n) for n, _ in orc.HybridConfig._fields_}
    prefill_vs_oracle(hb, fields, 2468, 70, TOL_4B, "4B", steps=2, fmt_tol=FMT_4B, rows=(REL2_4B, TOP10_4B))


def reduced_4b_heads(**over):
    """The 4B head counts (GDN 16 key / 32 value heads, attention 16 query /
    4 kv heads) at hidden 256, for 32K-token prompts."""
    f = dict(layers=2, attn_every=100, hidden=256, inter=512, vocab=2048, gdn_k_heads=16, gdn_v_heads=32,
             attn_q_heads=16, attn_kv_heads=4, max_batch=1, max_context=32800, rope_theta=1e7, rms_eps=1e-6)
    f.update(over)
    return f


def test_prefill_32k_reduced_gdn_vs_oracle(hb):
    """A 32,768-token prompt (512 chunks: the delta rule's segmented
    parallel form over the whole sequence, the many-row GEMMs at M = 32768)
    through two GDN layers with the 4B head counts, against the CPU model
    stepping the prompt with the recurrence's I/O in bf16, then two decode
    steps from the prefilled states.  (The CPU model's attention costs
    O(T^2) in double precision, so the attention layers are checked against
    the device decode loop below.)"""
    f = reduced_4b_heads()
    gm, om = models(hb, f, 90210)
    rs = np.random.RandomState(17)
    T = 32768
    tokens = rs.randint(0, f["vocab"], (1, T)).astype(np.int32)
    nxt, lg = prefill(gm, tokens, f["vocab"])
    om.reset(1, 0, 0)
    om.set_gdn_bf16_io(True)
    for t in range(T):
        _, olg = om.step(tokens[:, t])
        if (t + 1) % 8192 == 0:
            print(f"CPU model: {t + 1} tokens stepped", flush=True)
    close(lg, olg, f"32K reduced GDN: prefill {T} vs oracle (bf16 delta-rule I/O)", TOL_32K_GDN)
    greedy(nxt, lg, olg, TOL_32K_GDN)
    om.set_gdn_bf16_io(False)
    for t in range(2):
        tok = nxt.copy()
        nxt, lg = step(gm, tok, f["vocab"])
        _, olg = om.step(tok)
        close(lg, olg, f"32K reduced GDN: after prefill, step {t}", TOL_32K_GDN)
        greedy(nxt, lg, olg, TOL_32K_GDN)
    gm.close()


def test_prefill_32k_reduced_attention_vs_decode_loop(hb):
    """A 32,768-token prompt through two GDN and two attention layers with
    the 4B head counts: the prefill (chunked delta rule, causal attention
    over up to 32K keys, the KV cache it writes) against the same model's
    decode loop stepping the prompt one token at a time on the GPU (fp32
    delta rule, the decode attention; that loop is checked against the CPU
    model and HF elsewhere); then two steps from each, which read the KV
    caches the two paths wrote."""
    f = reduced_4b_heads(layers=4, attn_every=2)
    gm = hb.HybridModel(hb.config(**f), 4711)
    rs = np.random.RandomState(23)
    T = 32768
    tokens = rs.randint(0, f["vocab"], (1, T)).astype(np.int32)
    nxt_p, lg_p = prefill(gm, tokens, f["vocab"])
    follow = rs.randint(0, f["vocab"], 2)
    after_p = [step(gm, [x], f["vocab"]) for x in follow]
    torch = torch_mod()
    gm.reset(1, 0, 0)
    dtok = dev(tokens[0])
    for t in range(T - 1):
        gm.step(dtok[t:t + 1])
        if (t + 1) % 8192 == 0:
            torch.cuda.synchronize()
            print(f"decode loop: {t + 1} tokens stepped", flush=True)
    nxt_s, lg_s = step(gm, tokens[0, T - 1:], f["vocab"])  # the last prompt position
    close(lg_p, lg_s, "32K reduced with attention: prefill vs decode loop, last position", TOL_32K_ATT)
    greedy(nxt_p, lg_p, lg_s, TOL_32K_ATT)
    after_s = [step(gm, [x], f["vocab"]) for x in follow]
    for i, ((np_, lp), (ns, ls)) in enumerate(zip(after_p, after_s)):
        close(lp, ls, f"32K reduced with attention: step {i} after prefill vs after decode loop", TOL_32K_ATT)
        greedy(np_, lp, ls, TOL_32K_ATT)
    assert np.isfinite(lg_p).all() and nxt_p[0] == lg_p[0].argmax()
    gm.close()


def test_prefill_qwen35_4b_32k(hb):
    """The BASELINE workload's prefill: the whole 4B model, batch 1, a
    32,768-token prompt of uniform-random ids, then three greedy steps.
    Finite logits; every token is its logits' argmax; a second prefill of
    the same prompt is bit-identical; and a prefill of T tokens followed by
    one step fed token x agrees with a prefill of the T + 1 tokens ending in
    x (chunked and recurrent forms of the same last position)."""
    torch = torch_mod()
    T = 32768
    cfg = hb.qwen35_4b(1, T + 8)
    gm = hb.HybridModel(cfg, 12345)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2026)
    prompt = torch.randint(0, cfg.vocab, (1, T + 1), dtype=torch.int32, device="cuda", generator=gen)
    nxt = empty((1,), torch.int32)
    lg = empty((1, cfg.vocab), torch.float32)
    gm.prefill(prompt[:, :T].contiguous(), nxt, lg)
    n1, l1 = host(nxt), host(lg)
    assert np.isfinite(l1).all() and n1[0] == l1[0].argmax()
    gm.prefill(prompt[:, :T].contiguous(), nxt, lg)
    n2, l2 = host(nxt), host(lg)
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32)) and n1[0] == n2[0]
    x = prompt[0, T:T + 1].contiguous()
    ns, ls = step(gm, host(x), cfg.vocab)
    for i in range(2):
        ns2, ls2 = step(gm, ns, cfg.vocab)
        assert np.isfinite(ls2).all() and ns2[0] == ls2[0].argmax(), i
        ns = ns2
    assert gm.position == T + 3
    gm.prefill(prompt.contiguous(), nxt, lg)
    nT1, lT1 = host(nxt), host(lg)
    assert np.isfinite(lT1).all() and nT1[0] == lT1[0].argmax()
    close(ls, lT1, "4B 32K: prefill(T) + step(x) vs prefill(T + 1)", TOL_4B_32K_STEP)
    agreement(ls, lT1, "4B 32K: prefill(T) + step(x) vs prefill(T + 1)", REL2_4B, TOP10_4B)
    gm.close()
