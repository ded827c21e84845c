"""Seeded synthetic inputs with the BASELINE distributions, and comparison
helpers shared by the parity tests and bench.py's checks.

Distributions (N(0, s) means standard deviation s):
  conv:   x ~ N(0, 1), w ~ N(0, 0.25), zero history
  decode: q, k = L2-normalised N(0, 1); v ~ N(0, 1); beta = sigmoid(N(0, 1));
          g = -softplus(N(0, 1)) * exp(U(-2, 0)); S ~ N(0, 0.02)
  prefill: the decode distributions with q/k/v rounded to bf16.
"""
from __future__ import annotations

import numpy as np


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(bf16_bits(x))


def l2norm(x: np.ndarray) -> np.ndarray:
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def gates(rs, shape):
    """beta = sigmoid(N(0,1)), g = -softplus(N(0,1)) * exp(U(-2,0))."""
    beta = (1.0 / (1.0 + np.exp(-rs.randn(*shape)))).astype(np.float32)
    g = (-np.log1p(np.exp(rs.randn(*shape))) * np.exp(rs.uniform(-2, 0, shape))).astype(np.float32)
    return g, beta


def conv_inputs(seed, seq, ch):
    rs = np.random.RandomState(seed)
    x = rs.randn(seq * ch).astype(np.float32)
    w = (0.25 * rs.randn(4 * ch)).astype(np.float32)
    return x, w, np.zeros(3 * ch, np.float32)


def decode_inputs(seed, B, Hv, Hk, dk, dv):
    rs = np.random.RandomState(seed)
    q = l2norm(rs.randn(B, Hk, dk)).astype(np.float32)
    k = l2norm(rs.randn(B, Hk, dk)).astype(np.float32)
    v = rs.randn(B, Hv, dv).astype(np.float32)
    g, beta = gates(rs, (B, Hv))
    S = (0.02 * rs.randn(B, Hv, dk, dv)).astype(np.float32)
    return S, q, k, v, g, beta


def prefill_inputs(seed, B, T, Hv, Hk, d=128, zero_state=False):
    """Returns float32 arrays whose q/k/v values are exactly bf16."""
    rs = np.random.RandomState(seed)
    q = round_bf16(l2norm(rs.randn(B, T, Hk, d)).astype(np.float32))
    k = round_bf16(l2norm(rs.randn(B, T, Hk, d)).astype(np.float32))
    v = round_bf16(rs.randn(B, T, Hv, d).astype(np.float32))
    g, beta = gates(rs, (B, T, Hv))
    S = np.zeros((B, Hv, d, d), np.float32) if zero_state else \
        (0.02 * rs.randn(B, Hv, d, d)).astype(np.float32)
    return q, k, v, g, beta, S


def kai_approx_eq(got, ref, abs_tol, rel_tol):
    """Element-wise rule of the reference test (test_kai_gdn.c:57-62):
    |a-b| <= abs_tol, or |a-b| <= rel_tol * max(|a|, |b|)."""
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    diff = np.abs(got - ref)
    mag = np.maximum(np.abs(got), np.abs(ref))
    return (diff <= abs_tol) | (diff <= rel_tol * mag)


def assert_kai_close(got, ref, abs_tol, rel_tol, label=""):
    ok = kai_approx_eq(got, ref, abs_tol, rel_tol)
    if not ok.all():
        i = int(np.argmin(ok.ravel()))
        g, r = np.ravel(got)[i], np.ravel(ref)[i]
        raise AssertionError(f"{label}: {int((~ok).sum())} mismatches; first at {i}: "
                             f"got {g!r} ref {r!r} diff {abs(g - r):.3e}")


def validator_pass(got, ref, atol=1e-4, rtol=1e-3, floor=1e-2):
    """Pass rule of the reference GPU validator (gpu/gdn_gpu_validate.c:57-58,
    132-148): fail only if max_abs > atol AND max_rel > rtol, max_rel taken
    over |ref| > floor."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    d = np.abs(got - ref)
    max_abs = d.max() if d.size else 0.0
    big = np.abs(ref) > floor
    max_rel = (d[big] / np.abs(ref[big])).max() if big.any() else 0.0
    return not (max_abs > atol and max_rel > rtol), max_abs, max_rel


def rel_errors(got, ref):
    """(max |got-ref| / max |ref|, ||got-ref||_2 / ||ref||_2)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = got - ref
    scale = np.abs(ref).max()
    return (np.abs(d).max() / scale if scale > 0 else np.abs(d).max(),
            np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30))
