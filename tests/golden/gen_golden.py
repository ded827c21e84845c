"""Generate the golden fixtures under tests/golden/.  Run in the build
container (needs /root/reference for the kai / gdn_sve vectors and the
installed HuggingFace transformers for the delta-rule vectors):

    python tests/golden/gen_golden.py

Seven fixture files, each a numpy .npz (no pickles):

delta_matmul.npz  the reference's gdn_delta_rule_matmul
                (src/orionsbelt/engines/cpu/kernels/gdn_delta_matmul.c,
                portable branch) from oracle/_ref/libdelta_matmul_ref.so on
                the inputs of its test (test_gdn_delta_matmul.c:50-52: rand_r
                seed 42, values in [-1, 1) in steps of 1e-3), at M=3 and 64,
                K=128, N=130 and 17.
kai_ref.npz     inputs and outputs of the reference kai ukernels
                (kleidiai_submission/kai/ukernels/gdn/*.c, scalar branch),
                compiled from the reference sources by oracle/Makefile into
                oracle/_ref/libkai_ref.so.  Inputs come from the reference
                test's LCG (kleidiai_submission/test_kai_gdn.c:45-51, seed
                0x5EED1234) with the value ranges that test uses.
sve_mixed.npz   the reference gdn_sve.c fp16/bf16 variants
                (src/orionsbelt/engines/cpu/kernels/gdn_sve.c:442-766) from
                oracle/_ref/libgdn_sve_ref.so on T=64, C=35 warm/cold gates
                (the scenarios of test_gdn_mixed.c).
hf_layer.npz    HuggingFace transformers (v5.15.0): the gate expressions and
                l2norm of Qwen3_5GatedDeltaNet.forward and Qwen3_5RMSNormGated
                (modeling_qwen3_5.py:168-184,242-245,497-499), fp32 and bf16
                (`python tests/golden/gen_golden.py layer` rewrites only
                it and hf_state.npz).
hf_state.npz    HuggingFace transformers (v5.15.0): causal_conv1d_update
                (modeling_qwen3_5.py:199-217) and the conv cache of
                LinearAttentionLayer.update_conv_state (cache_utils.py:
                1032-1070).
hf_gdr.npz      HuggingFace transformers (v5.15.0, third-party, not part of
                the reference) torch_chunk_gated_delta_rule and
                torch_recurrent_gated_delta_rule
                (transformers/models/qwen3_5/modeling_qwen3_5.py:248-380), the
                published definition the reference documents for the GDN
                prefill/decode (docs/GDN_ARCHITECTURE_AUDIT.md:142-153), on
                small shapes with BASELINE config-2 distributions.
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import oracle as orc  # noqa: E402


class LCG:
    """The linear congruential generator of test_kai_gdn.c:45-51."""

    def __init__(self, seed=0x5EED1234):
        self.s = seed

    def uniform(self, n, lo, hi):
        out = np.empty(n, np.float32)
        lo32, hi32 = np.float32(lo), np.float32(hi)
        for i in range(n):
            self.s = (self.s * 1103515245 + 12345) & 0xFFFFFFFF
            r = np.float32((self.s >> 8) & 0xFFFFFF) / np.float32(0xFFFFFF)
            out[i] = lo32 + r * (hi32 - lo32)
        return out


def gen_kai():
    L = orc.ref_kai()
    assert L is not None, "oracle/_ref/libkai_ref.so missing: run make -C oracle ref"
    rng = LCG()
    d = {}
    # cumdecay, a in [0.5, 1.5] and tail range [0.1, 0.99]
    for name, seq, ch, lo, hi in [("cd1", 16, 17, 0.5, 1.5), ("cd2", 64, 33, 0.1, 0.99)]:
        a = rng.uniform(seq * ch, lo, hi)
        d[f"{name}_a"] = a
        d[f"{name}_out"] = orc.cumdecay_f32(a, seq, ch, L=L)
        d[f"{name}_shape"] = np.array([seq, ch], np.int64)
    # gated scan, g in [-0.99, 0.99], x in [-2, 2], state in [-1, 1]
    for name, seq, ch in [("sc1", 16, 33), ("sc2", 64, 7)]:
        g = rng.uniform(seq * ch, -0.99, 0.99)
        x = rng.uniform(seq * ch, -2.0, 2.0)
        st = rng.uniform(ch, -1.0, 1.0)
        s, st2 = orc.gated_scan_f32(g, x, st, seq, ch, L=L)
        d.update({f"{name}_g": g, f"{name}_x": x, f"{name}_state": st, f"{name}_s": s,
                  f"{name}_state_out": st2, f"{name}_shape": np.array([seq, ch], np.int64)})
    # conv, all in [-1, 1]; includes seq < 3 (history straddles the call)
    for name, seq, ch in [("cv1", 16, 17), ("cv2", 2, 12), ("cv3", 64, 129)]:
        x = rng.uniform(seq * ch, -1.0, 1.0)
        w = rng.uniform(4 * ch, -1.0, 1.0)
        h = rng.uniform(3 * ch, -1.0, 1.0)
        out, h2 = orc.conv_f32(x, w, h, seq, ch, L=L)
        d.update({f"{name}_in": x, f"{name}_w": w, f"{name}_hist": h, f"{name}_out": out,
                  f"{name}_hist_out": h2, f"{name}_shape": np.array([seq, ch], np.int64)})
    # gemv, a and b in [-1, 1]
    for name, k, n in [("gv1", 128, 33), ("gv2", 7, 130)]:
        a = rng.uniform(k, -1.0, 1.0)
        b = rng.uniform(k * n, -1.0, 1.0)
        d.update({f"{name}_a": a, f"{name}_b": b, f"{name}_c": orc.gemv_f32(a, b, k, n, L=L),
                  f"{name}_shape": np.array([k, n], np.int64)})
    np.savez_compressed(os.path.join(HERE, "kai_ref.npz"), **d)


def _rand_r(seed):
    """glibc rand_r (the generator of test_gdn_delta_matmul.c:50-52)."""
    state = [seed & 0xFFFFFFFF]

    def step():
        nxt = state[0]
        nxt = (nxt * 1103515245 + 12345) & 0xFFFFFFFF
        result = (nxt // 65536) % 2048
        nxt = (nxt * 1103515245 + 12345) & 0xFFFFFFFF
        result = (result << 10) ^ ((nxt // 65536) % 1024)
        nxt = (nxt * 1103515245 + 12345) & 0xFFFFFFFF
        result = (result << 10) ^ ((nxt // 65536) % 1024)
        state[0] = nxt
        return result

    return step


def gen_matmul():
    L = orc.ref_matmul()
    assert L is not None, "oracle/_ref/libdelta_matmul_ref.so missing: run make -C oracle ref"
    d = {}
    for name, m, k, n in [("mm1", 3, 128, 130), ("mm2", 64, 128, 17)]:
        r = _rand_r(42)
        A = np.array([((r() % 2000) - 1000) / 1000.0 for _ in range(m * k)], np.float32)
        B = np.array([((r() % 2000) - 1000) / 1000.0 for _ in range(k * n)], np.float32)
        d[f"{name}_A"], d[f"{name}_B"] = A, B
        d[f"{name}_C"] = orc.delta_rule_matmul(A, B, m, k, n, L=L).ravel()
        d[f"{name}_shape"] = np.array([m, k, n], np.int64)
    np.savez_compressed(os.path.join(HERE, "delta_matmul.npz"), **d)


def gen_sve():
    L = orc.ref_sve()
    assert L is not None, "oracle/_ref/libgdn_sve_ref.so missing: run make -C oracle ref"
    rs = np.random.RandomState(42)
    T, C = 64, 35
    d = {"shape": np.array([T, C], np.int64)}
    for scen, (alo, ahi) in {"warm": (0.90, 0.99), "cold": (0.5, 0.5)}.items():
        a = rs.uniform(alo, ahi, T * C).astype(np.float32)
        g = rs.uniform(0.5, 0.9, T * C).astype(np.float32)
        x = (rs.uniform(0, 1, T * C) - 0.5).astype(np.float32)
        st = (rs.uniform(0, 1, C) - 0.5).astype(np.float32)
        d[f"{scen}_a"], d[f"{scen}_g"], d[f"{scen}_x"], d[f"{scen}_st"] = a, g, x, st
        for fmt in ("f16", "bf16"):
            d[f"{scen}_cd_{fmt}"] = orc.cumdecay_narrow(a, T, C, fmt, L=L, prefix="gdn_")
            if fmt == "f16":
                st16 = np.array([orc.lib().orc_f32_to_f16(float(v)) for v in st], np.uint16)
            else:
                st16 = orc.f32_to_bf16_bits(st)
            s, st_out = orc.gated_scan_narrow(g, x, st16, T, C, fmt, L=L, prefix="gdn_")
            d[f"{scen}_st16_{fmt}"] = st16
            d[f"{scen}_scan_s_{fmt}"] = s
            d[f"{scen}_scan_st_{fmt}"] = st_out
    np.savez_compressed(os.path.join(HERE, "sve_mixed.npz"), **d)


def _inputs(rs, B, T, Hk, Hv, dk, dv, zero_state=False):
    """BASELINE config-2 distributions; q/k/v rounded to bf16-representable
    values so the same numbers serve the bf16 kernels."""
    def bf(x):
        return orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(x.astype(np.float32)))

    q = rs.randn(B, T, Hk, dk)
    k = rs.randn(B, T, Hk, dk)
    q = bf(q / np.linalg.norm(q, axis=-1, keepdims=True))
    k = bf(k / np.linalg.norm(k, axis=-1, keepdims=True))
    v = bf(rs.randn(B, T, Hv, dv))
    beta = (1.0 / (1.0 + np.exp(-rs.randn(B, T, Hv)))).astype(np.float32)
    g = (-np.log1p(np.exp(rs.randn(B, T, Hv))) * np.exp(rs.uniform(-2, 0, (B, T, Hv))))
    g = g.astype(np.float32)
    S0 = np.zeros((B, Hv, dk, dv), np.float32) if zero_state else \
        (0.02 * rs.randn(B, Hv, dk, dv)).astype(np.float32)
    return q, k, v, g, beta, S0


def gen_hf():
    import torch
    from transformers.models.qwen3_5 import modeling_qwen3_5 as m

    torch.set_num_threads(4)
    rs = np.random.RandomState(2024)
    d = {}
    cases = [
        # name,      kind,        B, T,   Hk, Hv, dk, dv, chunk, zero_state
        ("ck_small", "chunk",     1, 37,  2,  4,  16, 16, 16, False),
        ("ck_tail",  "chunk",     1, 100, 1,  2,  32, 32, 64, False),
        ("ck_b2",    "chunk",     2, 20,  1,  1,  8,  12, 8,  True),
        ("rc_step",  "recurrent", 3, 1,   2,  4,  32, 32, 0,  False),
        ("rc_multi", "recurrent", 1, 9,   1,  2,  16, 16, 0,  False),
    ]
    for name, kind, B, T, Hk, Hv, dk, dv, chunk, zs in cases:
        q, k, v, g, beta, S0 = _inputs(rs, B, T, Hk, Hv, dk, dv, zs)
        rep = Hv // Hk
        tq = torch.from_numpy(q).repeat_interleave(rep, dim=2)
        tk = torch.from_numpy(k).repeat_interleave(rep, dim=2)
        args = (tq, tk, torch.from_numpy(v), torch.from_numpy(g), torch.from_numpy(beta))
        with torch.no_grad():
            if kind == "chunk":
                o, S = m.torch_chunk_gated_delta_rule(
                    *args, chunk_size=chunk, initial_state=None if zs else torch.from_numpy(S0),
                    output_final_state=True, use_qk_l2norm_in_kernel=False)
            else:
                o, S = m.torch_recurrent_gated_delta_rule(
                    *args, initial_state=torch.from_numpy(S0), output_final_state=True,
                    use_qk_l2norm_in_kernel=False)
        d.update({f"{name}_q": q, f"{name}_k": k, f"{name}_v": v, f"{name}_g": g,
                  f"{name}_beta": beta, f"{name}_S0": S0,
                  f"{name}_o": o.numpy().astype(np.float32),
                  f"{name}_S": S.numpy().astype(np.float32),
                  f"{name}_dims": np.array([B, T, Hk, Hv, dk, dv, chunk], np.int64)})
    np.savez_compressed(os.path.join(HERE, "hf_gdr.npz"), **d)


def gen_layer():
    """The layer glue around the recurrence, from HF transformers v5.15.0:
    the gate expressions of Qwen3_5GatedDeltaNet.forward
    (modeling_qwen3_5.py:497-499), its l2norm (:242-245, applied to q and k
    with use_qk_l2norm_in_kernel, :262-264) after the split of the conv
    output into q, k, v heads (:481-492), and Qwen3_5RMSNormGated
    (:168-184) in fp32 and in bf16."""
    import torch
    import torch.nn.functional as F
    from transformers.models.qwen3_5 import modeling_qwen3_5 as m

    torch.set_num_threads(4)
    rs = np.random.RandomState(77)
    d = {}
    rows, Hk, Hv, D = 6, 2, 4, 128
    x = rs.randn(rows, (2 * Hk + Hv) * D).astype(np.float32)
    x[1, :Hk * D] = 0.0                      # zero q heads: l2norm of 0 is 0
    x[2] *= 40.0                             # large rows
    a = rs.randn(rows, Hv).astype(np.float32) * 3
    a[3] = [25.0, -30.0, 0.0, 19.5]          # softplus threshold (20) both sides
    b = rs.randn(rows, Hv).astype(np.float32) * 4
    A_log = np.log(rs.uniform(0.5, 16, Hv)).astype(np.float32)
    dt_bias = rs.randn(Hv).astype(np.float32)
    with torch.no_grad():
        tx, ta, tb = (torch.from_numpy(t) for t in (x, a, b))
        query, key, value = torch.split(tx, [Hk * D, Hk * D, Hv * D], dim=-1)
        query = m.l2norm(query.reshape(rows, Hk, D), dim=-1, eps=1e-6)
        key = m.l2norm(key.reshape(rows, Hk, D), dim=-1, eps=1e-6)
        value = value.reshape(rows, Hv, D)
        beta = tb.sigmoid()
        g = -torch.from_numpy(A_log).float().exp() * F.softplus(ta.float() + torch.from_numpy(dt_bias))
    d.update(gp_x=x, gp_a=a, gp_b=b, gp_A_log=A_log, gp_dt_bias=dt_bias,
             gp_q=query.numpy(), gp_k=key.numpy(), gp_v=value.numpy(), gp_g=g.numpy(),
             gp_beta=beta.numpy(), gp_dims=np.array([rows, Hk, Hv], np.int64))

    n, nrows = 128, 9
    o = rs.randn(nrows, n).astype(np.float32)
    o[1] = 0.0                               # zero row: eps keeps it finite
    o[2] *= 1e-3
    z = (rs.randn(nrows, n) * 3).astype(np.float32)
    z[3] = 0.0                               # silu(0) = 0
    w = (1.0 + 0.2 * rs.randn(n)).astype(np.float32)
    for dt, tag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        norm = m.Qwen3_5RMSNormGated(n, eps=1e-6)
        with torch.no_grad():
            norm.weight.copy_(torch.from_numpy(w))
            norm = norm.to(dt)
            to, tz = torch.from_numpy(o).to(dt), torch.from_numpy(z).to(dt)
            y = norm(to, tz)
        if dt == torch.float32:
            d.update(rn_f32_o=o, rn_f32_z=z, rn_f32_w=w, rn_f32_y=y.numpy())
        else:
            bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
            d.update(rn_bf16_o=bits(to), rn_bf16_z=bits(tz), rn_bf16_w=bits(norm.weight.data),
                     rn_bf16_y=bits(y))
    np.savez_compressed(os.path.join(HERE, "hf_layer.npz"), **d)


def gen_state():
    """The decode-step conv and the conv cache of HF transformers v5.15.0:
    causal_conv1d_update (modeling_qwen3_5.py:199-217, torch fallback) and
    LinearAttentionLayer.update_conv_state (cache_utils.py:1032-1070) after a
    prefill, on small shapes.  Tensors are stored token-major ([B][T][C]) as
    the kernels take them; HF's own calls use [B][C][T]."""
    import torch
    from transformers import cache_utils
    from transformers.models.qwen3_5 import modeling_qwen3_5 as m

    rs = np.random.RandomState(91)
    d = {}
    for name, B, T, C, silu in (("cu_t1", 3, 1, 40, True), ("cu_t3", 2, 3, 24, False)):
        x = rs.randn(B, T, C).astype(np.float32)
        st = rs.randn(B, C, 4).astype(np.float32)
        w = (0.5 * rs.randn(C, 4)).astype(np.float32)
        ts = torch.from_numpy(st.copy())
        with torch.no_grad():
            out = m.causal_conv1d_update(torch.from_numpy(x).transpose(1, 2).contiguous(), ts,
                                         torch.from_numpy(w), None, "silu" if silu else None)
        d.update({f"{name}_x": x, f"{name}_state0": st, f"{name}_w": w,
                  f"{name}_out": out.transpose(1, 2).contiguous().numpy(),
                  f"{name}_state": ts.numpy(), f"{name}_silu": np.array(int(silu))})
    for name, B, T, C in (("cs_t2", 2, 2, 16), ("cs_t7", 2, 7, 16)):
        x = rs.randn(B, T, C).astype(np.float32)
        layer = cache_utils.LinearAttentionLayer()
        layer.update_conv_state(torch.from_numpy(x).transpose(1, 2).contiguous(), 0,
                                conv_kernel_size=4)
        d.update({f"{name}_x": x, f"{name}_state": layer.conv_states[0].numpy().copy()})
    np.savez_compressed(os.path.join(HERE, "hf_state.npz"), **d)


# The tiny hybrid model of the logits fixture: every shape constraint of the
# device model holds (hidden, inter % 256; vocab, projections % 16), layer 3
# is full attention, and the GDN and attention head dims are the real ones.
HYBRID_TINY = dict(layers=4, attn_every=4, hidden=256, inter=512, vocab=1024, gdn_k_heads=8,
                   gdn_v_heads=16, attn_q_heads=4, attn_kv_heads=1, max_batch=2, max_context=64,
                   rope_theta=1.0e7, rms_eps=1e-6)
HYBRID_SEED = 20260
HYBRID_T = 12


def gen_hybrid():
    """HF Qwen3_5ForCausalLM (fp32, eager attention, no cache) on the
    dequantised weights of the oracle's drawn tiny model: logits of every
    position of two token sequences, run over the whole sequence at once
    (chunked GDN form, causal-masked attention)."""
    import torch
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM

    c = HYBRID_TINY
    m = orc.HybridModel(orc.HybridConfig(*[c[f] for f, _ in orc.HybridConfig._fields_]), HYBRID_SEED)
    cfg = Qwen3_5TextConfig(
        vocab_size=c["vocab"], hidden_size=c["hidden"], intermediate_size=c["inter"],
        num_hidden_layers=c["layers"], num_attention_heads=c["attn_q_heads"],
        num_key_value_heads=c["attn_kv_heads"], head_dim=256, rms_norm_eps=c["rms_eps"],
        linear_num_key_heads=c["gdn_k_heads"], linear_num_value_heads=c["gdn_v_heads"],
        linear_key_head_dim=128, linear_value_head_dim=128, linear_conv_kernel_dim=4,
        full_attention_interval=c["attn_every"], tie_word_embeddings=False,
        rope_parameters={"rope_type": "default", "rope_theta": c["rope_theta"],
                         "partial_rotary_factor": 0.25, "mrope_section": [11, 11, 10],
                         "mrope_interleaved": True},
        max_position_embeddings=c["max_context"])
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    hf = Qwen3_5ForCausalLM(cfg).float().eval()
    sd = {}
    for name, t in hf.state_dict().items():
        parts = name.split(".")
        if parts[1] == "layers":
            layer = int(parts[2])
            key = parts[4] if parts[3] in ("linear_attn", "self_attn", "mlp") else parts[3]
            if parts[3] in ("linear_attn", "self_attn") and parts[4] == "norm":
                key = "norm"
            v = m.tensor(layer, key)
        elif parts[0] == "lm_head":
            v = m.tensor(-1, "lm_head")
        else:
            v = m.tensor(-1, parts[1])
        assert v is not None and v.size == t.numel(), (name, None if v is None else v.size, t.shape)
        sd[name] = torch.from_numpy(v.reshape(t.shape).copy())
    hf.load_state_dict(sd)
    rs = np.random.RandomState(5)
    tokens = rs.randint(0, c["vocab"], size=(2, HYBRID_T)).astype(np.int32)
    with torch.no_grad():
        logits = hf(input_ids=torch.from_numpy(tokens.astype(np.int64)), use_cache=False).logits
    d = {"tokens": tokens, "logits": logits.float().numpy(), "seed": np.int64(HYBRID_SEED)}
    for k, v in c.items():
        d["cfg_" + k] = np.asarray(v)
    np.savez_compressed(os.path.join(HERE, "hf_hybrid.npz"), **d)


if __name__ == "__main__":
    orc.build()
    if len(sys.argv) > 1 and sys.argv[1] == "layer":
        gen_layer()
        gen_state()
        sys.exit(0)
    if len(sys.argv) > 1 and sys.argv[1] == "hybrid":
        gen_hybrid()
        sys.exit(0)
    if len(sys.argv) > 1 and sys.argv[1] == "matmul":
        gen_matmul()
        sys.exit(0)
    gen_kai()
    gen_matmul()
    gen_sve()
    gen_hf()
    gen_layer()
    gen_state()
    gen_hybrid()
    for f in ("kai_ref.npz", "delta_matmul.npz", "sve_mixed.npz", "hf_gdr.npz", "hf_layer.npz", "hf_state.npz",
              "hf_hybrid.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
