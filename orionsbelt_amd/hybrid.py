"""Host-side handle of the hybrid decode model in libkai_gdn_hip.so
(include/kai_gdn_hybrid.h): a random-init, Qwen3.5-shaped stack of Gated
DeltaNet and full-attention layers with int8 weights, stepped one token per
sequence on the GPU.

Only plumbing: every call goes to the C-ABI; token and logit buffers are torch
tensors on the model's device, passed by address.
"""
from __future__ import annotations

import ctypes

from . import HybridConfig, check, lib


def qwen35_4b(max_batch: int, max_context: int) -> HybridConfig:
    """The Qwen3.5-4B shape (32 layers, every fourth full attention)."""
    return lib().kai_gdn_hybrid_qwen35_4b(max_batch, max_context)


def config(**kw) -> HybridConfig:
    c = HybridConfig()
    for name, _ in HybridConfig._fields_:
        setattr(c, name, kw[name])
    return c


class HybridModel:
    def __init__(self, cfg: HybridConfig, seed: int):
        self.cfg = cfg
        self._h = None
        h = ctypes.c_void_p()
        check(lib().kai_gdn_hybrid_create(ctypes.byref(cfg), seed, ctypes.byref(h)),
              "kai_gdn_hybrid_create")
        self._h = h
        self.batch = cfg.max_batch

    def reset(self, batch: int, context: int, seed: int) -> None:
        check(lib().kai_gdn_hybrid_reset(self._h, batch, context, seed), "kai_gdn_hybrid_reset")
        self.batch = batch

    def step(self, tokens, next_tokens=None, logits=None, stream=None) -> None:
        """tokens [batch] int32 on the device; next_tokens [batch] int32 and
        logits [batch][vocab] fp32 (device tensors or None)."""
        assert tokens.is_cuda and tokens.dtype.itemsize == 4 and tokens.numel() >= self.batch
        for t, n in ((next_tokens, self.batch), (logits, self.batch * self.cfg.vocab)):
            assert t is None or (t.is_cuda and t.is_contiguous() and t.numel() >= n)
        st = stream.cuda_stream if stream is not None else None
        check(lib().kai_gdn_hybrid_step(
            self._h, tokens.data_ptr(), None if next_tokens is None else next_tokens.data_ptr(),
            None if logits is None else logits.data_ptr(), st), "kai_gdn_hybrid_step")

    def prefill(self, tokens, next_tokens=None, logits=None, stream=None) -> None:
        """tokens [batch][length] int32 on the device: start `batch`
        sequences from empty states and run their prompts; next_tokens and
        logits of the last position as for step."""
        assert tokens.is_cuda and tokens.dtype.itemsize == 4 and tokens.dim() == 2 and tokens.is_contiguous()
        batch, length = tokens.shape
        for t, n in ((next_tokens, batch), (logits, batch * self.cfg.vocab)):
            assert t is None or (t.is_cuda and t.is_contiguous() and t.numel() >= n)
        st = stream.cuda_stream if stream is not None else None
        check(lib().kai_gdn_hybrid_prefill(
            self._h, tokens.data_ptr(), batch, length, None if next_tokens is None else next_tokens.data_ptr(),
            None if logits is None else logits.data_ptr(), st), "kai_gdn_hybrid_prefill")
        self.batch = batch

    @property
    def position(self) -> int:
        return lib().kai_gdn_hybrid_position(self._h)

    @property
    def device_bytes(self) -> int:
        return lib().kai_gdn_hybrid_device_bytes(self._h)

    @property
    def weight_bytes(self) -> int:
        return lib().kai_gdn_hybrid_weight_bytes(self._h)

    def close(self) -> None:
        if self._h:
            lib().kai_gdn_hybrid_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
