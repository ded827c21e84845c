"""ctypes binding of the CPU oracle (liborb_oracle.so) and of the reference
builds in oracle/_ref.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker; the product library never uses it.
All array arguments are numpy arrays (C-contiguous, float32 / uint16).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ORB_ORACLE_LIB selects another build of the same sources (the sanitizer
# build of `make asan`).
LIB_PATH = os.environ.get("ORB_ORACLE_LIB") or os.path.join(HERE, "liborb_oracle.so")
REF_DIR = os.path.join(HERE, "_ref")

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_sz = ctypes.c_size_t
_int = ctypes.c_int
_flt = ctypes.c_float


def build() -> None:
    """Compile liborb_oracle.so (and oracle/_ref when the reference tree is
    present).  Raises CalledProcessError on a compiler error."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if os.path.isdir("/root/reference"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _load(path: str) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built (run oracle/Makefile)")
    return ctypes.CDLL(path)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load(LIB_PATH)
        _lib.orc_f32_to_f16.restype = ctypes.c_uint16
        _lib.orc_f32_to_f16.argtypes = [_flt]
        _lib.orc_f16_to_f32.restype = ctypes.c_float
        _lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        _lib.orc_f32_to_bf16.argtypes = [_flt]
        _lib.orc_bf16_to_f32.restype = ctypes.c_float
        _lib.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.orc_num_threads.restype = ctypes.c_int
    return _lib


def ref_kai() -> ctypes.CDLL | None:
    """The reference kai ukernels compiled from /root/reference (scalar
    branch), or None when oracle/_ref was not built."""
    p = os.path.join(REF_DIR, "libkai_ref.so")
    return ctypes.CDLL(p) if os.path.exists(p) else None


def ref_sve() -> ctypes.CDLL | None:
    """The reference gdn_sve.c compiled from /root/reference, or None."""
    p = os.path.join(REF_DIR, "libgdn_sve_ref.so")
    return ctypes.CDLL(p) if os.path.exists(p) else None


def P(a: np.ndarray):
    """Pointer to the data of a C-contiguous float32 or uint16 array."""
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    if a.dtype == np.float32:
        return a.ctypes.data_as(_f32p)
    if a.dtype == np.uint16:
        return a.ctypes.data_as(_u16p)
    raise TypeError(f"unsupported dtype {a.dtype}")


# ---- kai-shaped entry points (the same argument order as the kai ABI) -----

def cumdecay_f32(a, seq, ch, L=None):
    L = L or lib()
    out = np.empty(seq * ch, np.float32)
    fn = getattr(L, "orc_cumdecay_f32", None) or L.kai_run_gdn_cumdecay_f32_sve
    fn(P(a), P(out), _sz(seq), _sz(ch))
    return out


def gated_scan_f32(g, x, state, seq, ch, L=None):
    L = L or lib()
    s = np.empty(seq * ch, np.float32)
    st = np.array(state, np.float32, copy=True)
    fn = getattr(L, "orc_gated_scan_f32", None) or L.kai_run_gdn_gated_scan_f32_sve
    fn(P(g), P(x), P(s), P(st), _sz(seq), _sz(ch))
    return s, st


def gdn2_scan_f32(g, b, w, x, state, seq, ch, L=None, name="orc_gdn2_gated_scan_f32"):
    L = L or lib()
    s = np.empty(seq * ch, np.float32)
    st = np.array(state, np.float32, copy=True)
    getattr(L, name)(P(g), P(b), P(w), P(x), P(s), P(st), _sz(seq), _sz(ch))
    return s, st


def conv_f32(inp, w, hist, seq, ch, silu=False, L=None):
    L = L or lib()
    out = np.empty(seq * ch, np.float32)
    h = np.array(hist, np.float32, copy=True)
    if silu:
        fn = L.orc_causal_dwconv1d_silu_f32_k4
    else:
        fn = getattr(L, "orc_causal_dwconv1d_f32_k4", None) or \
            L.kai_run_gdn_causal_dwconv1d_f32_k4_sve
    fn(P(inp), P(w), P(out), P(h), _sz(seq), _sz(ch))
    return out, h


def gemv_f32(a, b, k, n, L=None):
    L = L or lib()
    c = np.empty(max(n, 1), np.float32)
    fn = getattr(L, "orc_gemv_f32", None) or L.kai_run_gdn_gemv_f32_f32_f32_1x4_neon
    fn(P(a), P(b), P(c), _sz(k), _sz(n))
    return c[:n]


def delta_rule_matmul(A, B, m, k, n, L=None):
    """C = A.B (orc_delta_rule_matmul_f32, or the reference's own
    gdn_delta_rule_matmul when L is ref_matmul())."""
    L = L or lib()
    c = np.empty(max(m * n, 1), np.float32)
    fn = getattr(L, "orc_delta_rule_matmul_f32", None) or L.gdn_delta_rule_matmul
    fn(P(A), P(B), P(c), _sz(m), _sz(k), _sz(n))
    return c[:m * n].reshape(m, n)


def ref_matmul() -> ctypes.CDLL | None:
    """The reference's gdn_delta_matmul.c (portable branch, no KleidiAI)
    compiled from its source into oracle/_ref, or None when not built."""
    p = os.path.join(REF_DIR, "libdelta_matmul_ref.so")
    return ctypes.CDLL(p) if os.path.exists(p) else None


def cumdecay_narrow(a, seq, ch, fmt, L=None, prefix="orc_"):
    L = L or lib()
    out = np.empty(seq * ch, np.uint16)
    getattr(L, f"{prefix}cumdecay_{fmt}")(P(a), P(out), _sz(seq), _sz(ch))
    return out


def gated_scan_narrow(g, x, state16, seq, ch, fmt, L=None, prefix="orc_"):
    L = L or lib()
    s = np.empty(seq * ch, np.float32)
    st = np.array(state16, np.uint16, copy=True)
    getattr(L, f"{prefix}gated_scan_{fmt}")(P(g), P(x), P(s), P(st), _sz(seq), _sz(ch))
    return s, st


# ---- matrix-state delta rule ----------------------------------------------

def delta_rule_head(S, k, v, q, beta, decay, hkd, hvd):
    S = np.array(S, np.float32, copy=True)
    out = np.empty(hvd, np.float32)
    lib().orc_delta_rule_head(P(S), P(k), P(v), P(q), _flt(beta), _flt(decay), P(out),
                              _sz(hkd), _sz(hvd))
    return S, out


def delta_rule_decode(S, q, k, v, g, beta, B, Hv, Hk, dk, dv, q_scale):
    """One decode step; returns (S_new, o).  S is [B][Hv][dk][dv] fp32."""
    S = np.array(S, np.float32, copy=True)
    o = np.empty((B, Hv, dv), np.float32)
    lib().orc_delta_rule_decode_f32(P(S), P(q), P(k), P(v), P(g), P(beta), P(o),
                                    _int(B), _int(Hv), _int(Hk), _int(dk), _int(dv),
                                    _flt(q_scale))
    return S, o


def delta_rule_decode_f16state(S16, q, k, v, g, beta, B, Hv, Hk, dk, dv, q_scale):
    S16 = np.array(S16, np.uint16, copy=True)
    o = np.empty((B, Hv, dv), np.float32)
    lib().orc_delta_rule_decode_f16state(P(S16), P(q), P(k), P(v), P(g), P(beta), P(o),
                                         _int(B), _int(Hv), _int(Hk), _int(dk), _int(dv),
                                         _flt(q_scale))
    return S16, o


def chunk_gdr(q, k, v, g, beta, S0, B, T, Hv, Hk, dk, dv, chunk=64, q_scale=None,
              precision="f32"):
    """HF chunkwise gated delta rule; returns (o [B][T][Hv][dv], S_final)."""
    if q_scale is None:
        q_scale = 1.0 / np.sqrt(dk)
    S = np.array(S0, np.float32, copy=True)
    o = np.empty((B, T, Hv, dv), np.float32)
    fn = lib().orc_chunk_gdr_f32 if precision == "f32" else lib().orc_chunk_gdr_f64
    fn(P(np.ascontiguousarray(q, np.float32)), P(np.ascontiguousarray(k, np.float32)),
       P(np.ascontiguousarray(v, np.float32)), P(np.ascontiguousarray(g, np.float32)),
       P(np.ascontiguousarray(beta, np.float32)), P(o), P(S), _int(B), _int(T), _int(Hv),
       _int(Hk), _int(dk), _int(dv), _int(chunk), _flt(q_scale))
    return o, S


# ---- layer glue ------------------------------------------------------------

def gating_prologue(x, a, b, A_log, dt_bias, rows, Hk, Hv):
    """HF gate expressions and q/k l2norm; returns (q [rows][Hk][128],
    k [rows][Hk][128], v [rows][Hv][128], g [rows][Hv], beta [rows][Hv])."""
    q = np.empty((rows, Hk, 128), np.float32)
    k = np.empty((rows, Hk, 128), np.float32)
    v = np.empty((rows, Hv, 128), np.float32)
    g = np.empty((rows, Hv), np.float32)
    beta = np.empty((rows, Hv), np.float32)
    c = lambda t: np.ascontiguousarray(t, np.float32)  # noqa: E731
    lib().orc_gating_prologue_f32(P(c(x)), P(c(a)), P(c(b)), P(c(A_log)), P(c(dt_bias)),
                                  P(q), P(k), P(v), P(g), P(beta), _sz(rows), _int(Hk),
                                  _int(Hv))
    return q, k, v, g, beta


def gated_rmsnorm_f32(o, z, w, eps=1e-6):
    """HF Qwen3_5RMSNormGated in an fp32 model over the last axis."""
    o = np.ascontiguousarray(o, np.float32)
    n = o.shape[-1]
    y = np.empty_like(o)
    lib().orc_gated_rmsnorm_f32(P(o), P(np.ascontiguousarray(z, np.float32)),
                                P(np.ascontiguousarray(w, np.float32)), P(y),
                                _sz(o.size // n), _int(n), _flt(eps))
    return y


def gated_rmsnorm_bf16(o16, z16, w16, eps=1e-6):
    """HF Qwen3_5RMSNormGated in a bf16 model (bf16 bit patterns)."""
    o16 = np.ascontiguousarray(o16, np.uint16)
    n = o16.shape[-1]
    y = np.empty_like(o16)
    lib().orc_gated_rmsnorm_bf16(P(o16), P(np.ascontiguousarray(z16, np.uint16)),
                                 P(np.ascontiguousarray(w16, np.uint16)), P(y),
                                 _sz(o16.size // n), _int(n), _flt(eps))
    return y


# ---- state hand-off formats ----------------------------------------------

def causal_conv1d_update(x, conv_state, w, silu):
    """HF causal_conv1d_update on x [B][T][C] (token-major), conv_state
    [B][C][4], w [C][4]; returns (out [B][T][C], new conv_state)."""
    x = np.ascontiguousarray(x, np.float32)
    B, T, C = x.shape
    st = np.array(conv_state, np.float32, copy=True)
    out = np.empty_like(x)
    lib().orc_causal_conv1d_update_f32(P(x), P(st), P(np.ascontiguousarray(w, np.float32)),
                                       P(out), _int(B), _int(T), _sz(C), _int(int(silu)))
    return out, st


def conv_state_from_inputs(x):
    """The HF conv state [B][C][4] after a prefill over x [B][T][C]: the
    last four inputs, newest last, zero-padded when T < 4 (index work)."""
    x = np.asarray(x, np.float32)
    B, T, C = x.shape
    st = np.zeros((B, C, 4), np.float32)
    n = min(T, 4)
    if n:
        st[:, :, 4 - n:] = np.transpose(x[:, T - n:, :], (0, 2, 1))
    return st


def conv_state_to_hist(conv_state):
    """[B][C][4] -> kai history [B][3][C] (entries 1..3, oldest first)."""
    return np.ascontiguousarray(np.transpose(np.asarray(conv_state, np.float32)[:, :, 1:], (0, 2, 1)))


def conv_hist_to_state(hist):
    """kai history [B][3][C] -> [B][C][4] with entry 0 (unused) = 0."""
    h = np.asarray(hist, np.float32)
    st = np.zeros((h.shape[0], h.shape[2], 4), np.float32)
    st[:, :, 1:] = np.transpose(h, (0, 2, 1))
    return st


# ---- hybrid decode loop matmuls ----------------------------------------------

_i8p = ctypes.POINTER(ctypes.c_int8)


def w8_quantize(W):
    """Per-output-channel symmetric int8 of W [N][K] fp32 -> (Wq int8, scale)."""
    W = np.ascontiguousarray(W, np.float32)
    N, K = W.shape
    Wq = np.empty((N, K), np.int8)
    sc = np.empty(N, np.float32)
    lib().orc_w8_quantize(P(W), Wq.ctypes.data_as(_i8p), P(sc), _int(N), _int(K))
    return Wq, sc


def w8_gemm(x16, Wq, scale):
    """y [M][N] fp32 from x [M][K] fp16 bits, Wq [N][K] int8, scale [N]."""
    x16 = np.ascontiguousarray(x16, np.uint16)
    Wq = np.ascontiguousarray(Wq, np.int8)
    M, K = x16.shape
    N = Wq.shape[0]
    y = np.empty((M, N), np.float32)
    lib().orc_w8_gemm(P(x16), Wq.ctypes.data_as(_i8p), P(np.ascontiguousarray(scale, np.float32)),
                      P(y), _int(M), _int(N), _int(K))
    return y


def attn_decode(q16, k16, v16, L, scaling):
    """softmax(scaling q K^T) V over the first L positions; q [B][Hq][D],
    k, v [B][Hkv][Tmax][D] fp16 bits -> out [B][Hq][D] fp32."""
    q16 = np.ascontiguousarray(q16, np.uint16)
    k16 = np.ascontiguousarray(k16, np.uint16)
    v16 = np.ascontiguousarray(v16, np.uint16)
    B, Hq, D = q16.shape
    Hkv, Tmax = k16.shape[1], k16.shape[2]
    out = np.empty((B, Hq, D), np.float32)
    lib().orc_attn_decode(P(q16), P(k16), P(v16), P(out), _int(B), _int(Hq), _int(Hkv), _int(Tmax),
                          _int(L), _int(D), _flt(scaling))
    return out


def num_threads() -> int:
    return lib().orc_num_threads()


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


# ---- hybrid decode loop ----------------------------------------------------

class HybridConfig(ctypes.Structure):
    """orc_hybrid_config (field order of kai_gdn_hybrid_config)."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "layers", "attn_every", "hidden", "inter", "vocab", "gdn_k_heads", "gdn_v_heads",
        "attn_q_heads", "attn_kv_heads", "max_batch", "max_context")] + [
        ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float)]


# Tensor ids of orc_hybrid_tensor: per layer, and model-level (layer -1).
HYBRID_LAYER_TENSORS = {
    "input_layernorm": 0, "post_attention_layernorm": 1, "in_proj_qkv": 2, "in_proj_z": 3,
    "in_proj_b": 4, "in_proj_a": 5, "out_proj": 6, "conv1d": 7, "dt_bias": 8, "A_log": 9,
    "norm": 10, "q_proj": 11, "k_proj": 12, "v_proj": 13, "o_proj": 14, "q_norm": 15,
    "k_norm": 16, "gate_proj": 17, "up_proj": 18, "down_proj": 19}
HYBRID_MODEL_TENSORS = {"embed_tokens": 1, "norm": 2, "lm_head": 3}


class HybridModel:
    """The CPU restatement of the hybrid decode model (gdn_hybrid_oracle.c)."""

    def __init__(self, cfg: HybridConfig, seed: int):
        self._h = None
        L = lib()
        L.orc_hybrid_create.restype = ctypes.c_void_p
        L.orc_hybrid_create.argtypes = [ctypes.POINTER(HybridConfig), ctypes.c_uint64]
        L.orc_hybrid_reset.argtypes = [ctypes.c_void_p, _int, _int, ctypes.c_uint64]
        L.orc_hybrid_step.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, _f32p]
        L.orc_hybrid_position.argtypes = [ctypes.c_void_p]
        L.orc_hybrid_tensor.restype = ctypes.c_long
        L.orc_hybrid_tensor.argtypes = [ctypes.c_void_p, _int, _int, _f32p]
        L.orc_hybrid_destroy.argtypes = [ctypes.c_void_p]
        L.orc_hybrid_set_gdn_bf16_io.argtypes = [ctypes.c_void_p, _int]
        self.cfg = cfg
        self._h = L.orc_hybrid_create(ctypes.byref(cfg), ctypes.c_uint64(seed))
        self.batch = cfg.max_batch

    def reset(self, batch: int, context: int, seed: int) -> None:
        lib().orc_hybrid_reset(self._h, batch, context, ctypes.c_uint64(seed))
        self.batch = batch

    def set_gdn_bf16_io(self, on: bool) -> None:
        """Round the delta rule's q, k, v and output to bf16 (the device
        prefill's formats) from now on."""
        lib().orc_hybrid_set_gdn_bf16_io(self._h, int(bool(on)))

    def step(self, tokens):
        """-> (next tokens [batch] int32, logits [batch][vocab] fp32)."""
        tok = np.ascontiguousarray(tokens, np.int32)
        assert tok.shape == (self.batch,)
        nxt = np.empty(self.batch, np.int32)
        logits = np.empty((self.batch, self.cfg.vocab), np.float32)
        lib().orc_hybrid_step(self._h, tok.ctypes.data, nxt.ctypes.data, P(logits))
        return nxt, logits

    @property
    def position(self) -> int:
        return lib().orc_hybrid_position(self._h)

    def tensor(self, layer: int, name: str) -> np.ndarray | None:
        """A drawn tensor as fp32 (matrices dequantised), None if absent."""
        tid = HYBRID_MODEL_TENSORS[name] if layer < 0 else HYBRID_LAYER_TENSORS[name]
        n = lib().orc_hybrid_tensor(self._h, layer, tid, None)
        if n < 0:
            return None
        out = np.empty(n, np.float32)
        lib().orc_hybrid_tensor(self._h, layer, tid, P(out))
        return out

    def close(self) -> None:
        if self._h:
            lib().orc_hybrid_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


# ---- narrow-format helpers -------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (vectorised form
    of orc_f32_to_bf16)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    return ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)
