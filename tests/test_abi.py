"""CPU checks of the drop-in boundary: the library exists, loads, and exports
every symbol the headers in include/ declare, with the kai prototypes
unchanged from the reference.  No compute calls (no GPU here)."""
import ctypes
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(REPO, "include")


def declared_symbols():
    names = set()
    for root, _, files in os.walk(INCLUDE):
        for f in files:
            if f.endswith(".h"):
                txt = open(os.path.join(root, f)).read()
                txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
                names.update(re.findall(r"\b((?:kai|gdn2?)_[a-z0-9_]+)\s*\(", txt))
    return names


def test_headers_declare_expected_entry_points():
    import orionsbelt_amd as ob
    assert declared_symbols() == set(ob.ALL_SYMBOLS)


def test_library_exports_every_declared_symbol():
    import orionsbelt_amd as ob
    assert os.path.exists(ob.LIB_PATH), "run python -m orionsbelt_amd.build"
    out = subprocess.run(["nm", "-D", "--defined-only", ob.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = declared_symbols() - exported
    assert not missing, f"not exported: {sorted(missing)}"


def test_library_loads_and_binds():
    import orionsbelt_amd as ob
    L = ob.lib()
    for name in ob.ALL_SYMBOLS:
        assert isinstance(getattr(L, name), ctypes._CFuncPtr)


def _proto(path, name):
    txt = re.sub(r"/\*.*?\*/|//[^\n]*", "", open(path).read(), flags=re.S)
    m = re.search(r"void\s+" + name + r"\s*\(([^)]*)\)", txt)
    return re.sub(r"\s+", " ", m.group(1)).strip() if m else None


@pytest.mark.parametrize("hdr,name", [
    ("kai_gdn_cumdecay_f32_sve.h", "kai_run_gdn_cumdecay_f32_sve"),
    ("kai_gdn_gated_scan_f32_sve.h", "kai_run_gdn_gated_scan_f32_sve"),
    ("kai_gdn_causal_dwconv1d_f32_k4_sve.h", "kai_run_gdn_causal_dwconv1d_f32_k4_sve"),
    ("kai_gdn_gemv_f32_f32_f32_1x4_neon.h", "kai_run_gdn_gemv_f32_f32_f32_1x4_neon"),
])
def test_kai_prototypes_identical_to_reference(hdr, name):
    ref = os.path.join("/root/reference/kleidiai_submission/kai/ukernels/gdn", hdr)
    if not os.path.exists(ref):
        pytest.skip("reference tree not present")
    ours = os.path.join(INCLUDE, "kai", "ukernels", "gdn", hdr)
    assert _proto(ours, name) == _proto(ref, name)


@pytest.mark.parametrize("name", ["gdn_cumdecay_f32", "gdn_gated_scan_f32", "gdn_causal_dwconv1d_f32",
                                  "gdn_cumdecay_f16", "gdn_gated_scan_f16", "gdn_cumdecay_bf16",
                                  "gdn_gated_scan_bf16", "gdn2_gated_scan_f32"])
def test_gdn_sve_prototypes_match_reference(name):
    """include/gdn_sve.h against the reference's gdn_sve.h:30-86: the same
    parameters in the same order, once this header's spelling macros
    (restrict, and __fp16 where the compiler has it) are read as the
    reference writes them."""
    ref = "/root/reference/src/orionsbelt/engines/cpu/kernels/gdn_sve.h"
    if not os.path.exists(ref):
        pytest.skip("reference tree not present")
    ours = _proto(os.path.join(INCLUDE, "gdn_sve.h"), name)
    ours = ours.replace("GDN_SVE_RESTRICT", "restrict").replace("GDN_SVE_F16", "__fp16")
    assert ours == _proto(ref, name)


def test_c_harnesses_built():
    for b in ("test_kai_gdn", "bench_kai_gdn", "gdn_e2e_decode"):
        assert os.access(os.path.join(REPO, "orionsbelt_amd", "bin", b), os.X_OK), b


def test_e2e_driver_cli():
    """The hybrid decode driver keeps the reference program's flags: --help
    runs without a GPU, bad token counts are rejected before any HIP call."""
    exe = os.path.join(REPO, "orionsbelt_amd", "bin", "gdn_e2e_decode")
    r = subprocess.run([exe, "--help"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0
    for flag in ("--tokens", "--csv", "--ctx-sweep", "--batch", "--ctx"):
        assert flag in r.stdout
    r = subprocess.run([exe, "--tokens", "0"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "--tokens must be >= 1" in r.stderr
    for bad in ("0", "-3", "abc", "12x"):
        r = subprocess.run([exe, "--prefill", bad], capture_output=True, text=True, timeout=60)
        assert r.returncode == 1 and "--prefill must be an integer" in r.stderr, bad


def test_bench_line_is_compact_with_prefill_last():
    """bench.py's JSON line keeps the figures only and ends with the T=16K
    prefill entry (its own roofline and cpu_baseline), so a reader of the
    output's tail sees the prefill half of the metric."""
    import json
    import sys
    sys.path.insert(0, REPO)
    import bench
    sec = {
        "conv": {"us": 47.0, "hbm_frac": 0.71, "cpu_baseline": {"value": 0.4, "kind": "reference",
                                                                  "port_all_cores": {"value": 10.0}}},
        "cumdecay": {"us": 46.0, "hbm_frac": 0.72},
        "scans": {"gated_scan_f32": {"us": 71.0, "hbm_frac": 0.7}},
        "decode_f16_state": {"ms_per_step": 0.6, "tokens_per_s": 1.0e5, "launch_us": 24.0, "hbm_frac": 0.7},
        "prefill_f16_state": {"lengths": [{"T": 1024, "ms": 0.05, "tokens_per_s": 2e7,
                                           "state_bytes_per_layer": 1 << 20}]},
        "hybrid_decode": {"runs": [{"batch": 1, "ms_per_step": 1.7, "tokens_per_s": 576.0, "hbm_frac": 0.37,
                                    "ttft_ms": 372.0, "device_bytes": 1}]},
        "prefill": {"ms": 0.2309, "ms_20_warmups": 0.277, "tokens_per_s": 7.1e7, "mfma_frac": 0.1637,
                    "achieved_tflops": 409.3, "flop_per_launch": 94489280512, "windowed_heads": 32,
                    "ms_long_memory": 0.19, "long_memory_windowed_heads": 32,
                    "ms_exact_path": 0.2433, "mfma_frac_exact_path": 0.1554,
                    "cpu_baseline": {"value": 15302.8, "unit": "tokens/s", "cores": 16, "kind": "port",
                                     "sample": "598 x T=256 (32 heads, OpenMP over heads), 10.0 s"}},
    }
    c = bench.compact_secondary(sec)
    assert list(c)[-1] == "prefill"
    p = c["prefill"]
    assert p["roofline"]["bound"] == "mfma" and p["roofline"]["frac"] == 0.1637
    assert p["cpu_baseline"]["kind"] == "port" and p["cpu_baseline"]["sample"] == "598 x T=256"
    assert p["windowed_heads"] == 32 and p["ms_exact_path"] == 0.2433 and p["ms_long_memory"] == 0.19
    text = json.dumps({"secondary": c}, separators=(",", ":"))
    assert text.index('"prefill":{') > text.index('"hybrid_decode"') and len(text) < 1500


def test_bench_refuses_multi_gpu():
    r = subprocess.run(["python", os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_generated_substitution_steps_up_to_date():
    """gdn_subst_steps.inc is the output of its generator, unedited."""
    import importlib.util
    csrc = os.path.join(REPO, "orionsbelt_amd", "csrc")
    spec = importlib.util.spec_from_file_location("gen_subst_steps", os.path.join(csrc, "gen_subst_steps.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    with open(os.path.join(csrc, "gdn_subst_steps.inc")) as f:
        assert f.read() == gen.render()


def test_prefill_workspace_query_needs_no_device():
    """The carry-buffer query is host arithmetic over the segment plan:
    three 128x128 fp32 slots per (sequence, head, segment), no carry for
    one segment (short sequences, and batches that fill the device by
    themselves), flat in T once the plan stops growing.  The planner picks
    the segment count whose plan has the lowest modelled time, up to what
    fills the device (1 + ceil(256 / (B*Hv))) with at least 4 chunks per
    segment: 9 for 32 heads from T = 8K, 4 at T = 1K; 24 for 4 heads at
    T = 16K, where 64 would compose too long a chain."""
    import orionsbelt_amd as ob
    L = ob.lib()
    slot = 3 * 128 * 128 * 4
    assert L.kai_gdn_hip_prefill_workspace_bytes(1, 640, 4) == 0
    assert L.kai_gdn_hip_prefill_workspace_bytes(16, 32768, 32) == 0
    assert L.kai_gdn_hip_prefill_workspace_bytes(1, 1024, 32) == 4 * 32 * slot
    for T in (8192, 16384, 131072):
        assert L.kai_gdn_hip_prefill_workspace_bytes(1, T, 32) == 9 * 32 * slot
    assert L.kai_gdn_hip_prefill_workspace_bytes(1, 16384, 4) == 23 * 4 * slot
    for bad in ((0, 16384, 32), (1, 0, 32), (1, 16384, 0), (-1, 16384, 32)):
        assert L.kai_gdn_hip_prefill_workspace_bytes(*bad) == 0
