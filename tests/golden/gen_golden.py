"""Generate the golden fixtures under tests/golden/.  Run in the build
container (needs /root/reference for the kai / gdn_sve vectors and the
installed HuggingFace transformers for the delta-rule vectors):

    python tests/golden/gen_golden.py

Three fixture files, each a numpy .npz (no pickles):

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


if __name__ == "__main__":
    orc.build()
    gen_kai()
    gen_sve()
    gen_hf()
    for f in ("kai_ref.npz", "sve_mixed.npz", "hf_gdr.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
