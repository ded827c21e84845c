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
  4B widths, 4 GDN layers: 1.6e-2 (measured 7.8e-3, against 8.9e-4 for the
      decode loop: the bf16 rounding of the delta rule's operands);
  the full 4B model (24 GDN + 8 attention layers): 6e-2 (measured 2.3e-2
      .. 3.0e-2; 1.1e-2 at 8 layers, 2.3e-2 at 16: roughly sqrt(layers)).
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gpu_util import dev, empty, host, torch_mod

pytestmark = pytest.mark.gpu

FIXTURE_TOL = 2e-3


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


def prefill_vs_oracle(hb, fields, seed, T, tol, what, steps=0):
    gm, om = models(hb, fields, seed)
    rs = np.random.RandomState(5)
    tokens = rs.randint(0, fields["vocab"], (1, T)).astype(np.int32)
    nxt, lg = prefill(gm, tokens, fields["vocab"])
    om.reset(1, 0, 0)
    for t in range(T):
        _, olg = om.step(tokens[:, t])
    close(lg, olg, f"{what}: prefill {T} vs oracle", tol)
    greedy(nxt, lg, olg, tol)
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
    prefill_vs_oracle(hb, widths_4b(attn_every=100), 2468, 70, 1.6e-2, "4B widths, GDN", steps=2)


def test_prefill_qwen35_4b_vs_oracle(hb):
    """The whole 4B model (32 layers, hidden 2560, vocab 151936): a 70-token
    prompt against the CPU model stepping it, then two decode steps."""
    cfg = hb.qwen35_4b(1, 128)
    fields = {n: getattr(cfg, n) for n, _ in orc.HybridConfig._fields_}
    prefill_vs_oracle(hb, fields, 2468, 70, 6e-2, "4B", steps=2)
