"""orionsbelt_amd -- MI355X (gfx950) implementation of the OrionsBelt GDN hot path.

The product is the C-ABI library ``orionsbelt_amd/lib/libkai_gdn_hip.so``
(declared in ``include/kai/ukernels/gdn/*.h``, ``include/kai_gdn_hip.h`` and
``include/kai_gdn_hybrid.h``).
This module only loads it through ctypes so Python tests and the benchmark
can call the same entry points a C caller would.  There is no fallback: if the
library is missing, :func:`lib` raises.
"""
from __future__ import annotations

import ctypes
import os

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "lib", "libkai_gdn_hip.so")

# Every symbol the headers in include/ declare.
KAI_SYMBOLS = (
    "kai_run_gdn_cumdecay_f32_sve",
    "kai_run_gdn_gated_scan_f32_sve",
    "kai_run_gdn_causal_dwconv1d_f32_k4_sve",
    "kai_run_gdn_gemv_f32_f32_f32_1x4_neon",
)
HIP_SYMBOLS = (
    "kai_run_gdn_cumdecay_f32_hip",
    "kai_run_gdn_cumdecay_f32_noalloc_hip",
    "kai_run_gdn_gated_scan_f32_hip",
    "kai_run_gdn_causal_dwconv1d_f32_k4_hip",
    "kai_run_gdn_causal_dwconv1d_silu_f32_k4_hip",
    "kai_run_gdn_gemv_f32_f32_f32_hip",
    "kai_run_gdn_delta_rule_matmul_f32_hip",
    "kai_run_gdn_cumdecay_f16_hip",
    "kai_run_gdn_cumdecay_bf16_hip",
    "kai_run_gdn_gated_scan_f16_hip",
    "kai_run_gdn_gated_scan_bf16_hip",
    "kai_run_gdn2_gated_scan_f32_hip",
    "kai_run_gdn_delta_rule_decode_f32_hip",
    "kai_run_gdn_delta_rule_decode_f16state_hip",
    "kai_run_gdn_chunk_delta_rule_bf16_f32_hip",
    "kai_run_gdn_chunk_delta_rule_bf16_f16state_hip",
    "kai_run_gdn_gating_prologue_bf16_hip",
    "kai_run_gdn_gating_prologue_f32_hip",
    "kai_run_gdn_gated_rmsnorm_bf16_hip",
    "kai_run_gdn_gated_rmsnorm_f32_hip",
    "kai_run_gdn_causal_conv1d_update_f32_hip",
    "kai_run_gdn_conv_state_from_inputs_f32_hip",
    "kai_run_gdn_conv_state_to_hist_f32_hip",
    "kai_run_gdn_conv_hist_to_state_f32_hip",
    "kai_run_gdn_state_convert_hip",
    "kai_gdn_w8a16_gemm_workspace_bytes",
    "kai_run_gdn_w8a16_gemm_hip",
    "kai_run_gdn_w8_tile_hip",
    "kai_gdn_w8a16_gemm_tiled_workspace_bytes",
    "kai_run_gdn_w8a16_gemm_tiled_hip",
    "kai_run_gdn_w8_quantize_hip",
    "kai_gdn_attn_decode_workspace_bytes",
    "kai_run_gdn_attn_decode_f16kv_hip",
    "kai_gdn_hybrid_qwen35_4b",
    "kai_gdn_hybrid_create",
    "kai_gdn_hybrid_reset",
    "kai_gdn_hybrid_step",
    "kai_gdn_hybrid_prefill",
    "kai_gdn_hybrid_set_timing",
    "kai_gdn_hybrid_phase_times",
    "kai_gdn_hybrid_position",
    "kai_gdn_hybrid_device_bytes",
    "kai_gdn_hybrid_weight_bytes",
    "kai_gdn_hybrid_destroy",
    "kai_gdn_hip_init",
    "kai_gdn_hip_error_string",
    "kai_gdn_hip_check_device_error",
    "kai_gdn_hip_prefill_workspace_bytes",
    "kai_gdn_hip_device_bytes_held",
    "kai_gdn_hip_prefill_windowed_heads",
    "kai_gdn_hip_probe_sink_bytes",
    "kai_gdn_hip_probe_stream",
    "kai_gdn_hip_probe_mfma_bf16",
)
# The reference's internal gdn_* ABI (include/gdn_sve.h).
SVE_SYMBOLS = (
    "gdn_cumdecay_f32",
    "gdn_gated_scan_f32",
    "gdn_causal_dwconv1d_f32",
    "gdn_cumdecay_f16",
    "gdn_gated_scan_f16",
    "gdn_cumdecay_bf16",
    "gdn_gated_scan_bf16",
    "gdn2_gated_scan_f32",
)
# The reference's delta-rule matmul (include/gdn_delta_matmul.h).
MATMUL_SYMBOLS = ("gdn_delta_rule_matmul",)
ALL_SYMBOLS = KAI_SYMBOLS + HIP_SYMBOLS + SVE_SYMBOLS + MATMUL_SYMBOLS

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i = ctypes.c_int
_f = ctypes.c_float



class HybridConfig(ctypes.Structure):
    """kai_gdn_hybrid_config (include/kai_gdn_hybrid.h)."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "layers", "attn_every", "hidden", "inter", "vocab", "gdn_k_heads", "gdn_v_heads",
        "attn_q_heads", "attn_kv_heads", "max_batch", "max_context")] + [
        ("rope_theta", ctypes.c_float), ("rms_eps", ctypes.c_float)]


# Element formats of kai_run_gdn_state_convert_hip (KAI_GDN_FMT_* in kai_gdn_hip.h).
FMT_F32, FMT_F16, FMT_BF16 = 0, 1, 2

_SIGS = {
    "kai_run_gdn_cumdecay_f32_sve": (None, [_vp, _vp, _sz, _sz]),
    "kai_run_gdn_gated_scan_f32_sve": (None, [_vp, _vp, _vp, _vp, _sz, _sz]),
    "kai_run_gdn_causal_dwconv1d_f32_k4_sve": (None, [_vp, _vp, _vp, _vp, _sz, _sz]),
    "kai_run_gdn_gemv_f32_f32_f32_1x4_neon": (None, [_vp, _vp, _vp, _sz, _sz]),
    "kai_run_gdn_cumdecay_f32_hip": (_i, [_vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_cumdecay_f32_noalloc_hip": (_i, [_vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_cumdecay_f16_hip": (_i, [_vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_cumdecay_bf16_hip": (_i, [_vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_gated_scan_f32_hip": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_gated_scan_f16_hip": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_gated_scan_bf16_hip": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn2_gated_scan_f32_hip": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_causal_dwconv1d_f32_k4_hip": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_causal_dwconv1d_silu_f32_k4_hip": (_i, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_gemv_f32_f32_f32_hip": (_i, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "kai_run_gdn_delta_rule_matmul_f32_hip": (_i, [_vp, _vp, _vp, _sz, _sz, _sz, _vp]),
    "gdn_delta_rule_matmul": (None, [_vp, _vp, _vp, _sz, _sz, _sz]),
    "kai_run_gdn_delta_rule_decode_f32_hip":
        (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp]),
    "kai_run_gdn_delta_rule_decode_f16state_hip":
        (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp]),
    "kai_run_gdn_chunk_delta_rule_bf16_f32_hip":
        (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp]),
    "kai_run_gdn_chunk_delta_rule_bf16_f16state_hip":
        (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp]),
    "kai_run_gdn_gating_prologue_bf16_hip":
        (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _vp]),
    "kai_run_gdn_gating_prologue_f32_hip":
        (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _i, _i, _vp]),
    "kai_run_gdn_gated_rmsnorm_bf16_hip": (_i, [_vp, _vp, _vp, _vp, _sz, _f, _vp]),
    "kai_run_gdn_gated_rmsnorm_f32_hip": (_i, [_vp, _vp, _vp, _vp, _sz, _f, _vp]),
    "kai_run_gdn_causal_conv1d_update_f32_hip": (_i, [_vp, _vp, _vp, _vp, _i, _i, _sz, _i, _vp]),
    "kai_run_gdn_conv_state_from_inputs_f32_hip": (_i, [_vp, _vp, _i, _sz, _sz, _vp]),
    "kai_run_gdn_conv_state_to_hist_f32_hip": (_i, [_vp, _vp, _i, _sz, _vp]),
    "kai_run_gdn_conv_hist_to_state_f32_hip": (_i, [_vp, _vp, _i, _sz, _vp]),
    "kai_run_gdn_state_convert_hip": (_i, [_vp, _i, _vp, _i, _sz, _vp]),
    "kai_gdn_w8a16_gemm_workspace_bytes": (_sz, [_i, _i, _i]),
    "kai_run_gdn_w8a16_gemm_hip": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "kai_run_gdn_w8_tile_hip": (_i, [_vp, _vp, _i, _i, _vp]),
    "kai_gdn_w8a16_gemm_tiled_workspace_bytes": (_sz, [_i, _i, _i]),
    "kai_run_gdn_w8a16_gemm_tiled_hip": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "kai_run_gdn_w8_quantize_hip": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "kai_gdn_attn_decode_workspace_bytes": (_sz, [_i, _i, _i]),
    "kai_run_gdn_attn_decode_f16kv_hip":
        (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp]),
    "kai_gdn_hybrid_qwen35_4b": (HybridConfig, [_i, _i]),
    "kai_gdn_hybrid_create": (_i, [ctypes.POINTER(HybridConfig), ctypes.c_ulonglong,
                                   ctypes.POINTER(_vp)]),
    "kai_gdn_hybrid_reset": (_i, [_vp, _i, _i, ctypes.c_ulonglong]),
    "kai_gdn_hybrid_step": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "kai_gdn_hybrid_prefill": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp]),
    "kai_gdn_hybrid_set_timing": (_i, [_vp, _i]),
    "kai_gdn_hybrid_phase_times": (_i, [_vp, ctypes.POINTER(ctypes.c_double), _i]),
    "kai_gdn_hybrid_position": (_i, [_vp]),
    "kai_gdn_hybrid_device_bytes": (_sz, [_vp]),
    "kai_gdn_hybrid_weight_bytes": (_sz, [_vp]),
    "kai_gdn_hybrid_destroy": (None, [_vp]),
    "kai_gdn_hip_init": (_i, []),
    "kai_gdn_hip_error_string": (ctypes.c_char_p, [_i]),
    "kai_gdn_hip_check_device_error": (_i, []),
    "kai_gdn_hip_prefill_workspace_bytes": (_sz, [_i, _i, _i]),
    "kai_gdn_hip_device_bytes_held": (_sz, []),
    "kai_gdn_hip_prefill_windowed_heads": (_i, []),
    "kai_gdn_hip_probe_sink_bytes": (_sz, []),
    "kai_gdn_hip_probe_stream": (_i, [_vp, _vp, _sz, _i, _vp, _vp]),
    "kai_gdn_hip_probe_mfma_bf16": (_i, [_i, _i, _vp, ctypes.POINTER(ctypes.c_ulonglong), _vp]),
}

_lib = None


class HipError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Load libkai_gdn_hip.so (built by ``python -m orionsbelt_amd.build``).

    torch is imported first when it is installed so that the library binds to
    the same HIP runtime (libamdhip64.so.7) torch already loaded."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(
            f"{LIB_PATH} not built: run `python -m orionsbelt_amd.build` (no CPU fallback exists)")
    try:
        import torch  # noqa: F401  (shares the HIP runtime)
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc: int, what: str = "") -> None:
    """Raise HipError for a non-zero return code of a *_hip entry point."""
    if rc != 0:
        msg = lib().kai_gdn_hip_error_string(rc).decode()
        raise HipError(f"{what}: {msg} ({rc})")
