"""The drop-in claim, observed on the GPU: the kai test and bench harness
programs run against libkai_gdn_hip.so and keep the reference harnesses'
observable contract (kleidiai_submission/test_kai_gdn.c:84-96,665-675:
`[ RUN      ]` lines, a `Tests run:` summary, `ALL TESTS PASSED`, exit 0;
bench_kai_gdn.c:249-256,298: `--repeats N`, `--csv` and the CSV header that
scripts/verify_kleidiai_kernels.sh:74-79 parses).

Programs:
- orionsbelt_amd/bin/test_kai_gdn: this build's harness (host and device
  pointer suites);
- oracle/_ref/test_kai_gdn_on_hip: the reference's own test_kai_gdn.c,
  compiled unchanged against include/ and linked to the HIP library
  (oracle/Makefile), when that build exists;
- orionsbelt_amd/bin/bench_kai_gdn: the bench harness, CSV mode;
- oracle/_ref/test_gdn_{mixed,2_scan,sve}_on_hip: the reference's tests of
  its gdn_sve.h kernels, compiled unchanged against this library;
- oracle/_ref/test_gdn_delta_matmul_on_hip: the reference's test of its
  delta-rule matmul, compiled unchanged against this library."""
import os
import subprocess

import pytest

from tests.gpu_util import torch_mod

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSV_HEADER = "kernel,shape,seq,channels,repeats,p50_us,gib_per_s_p50"


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch_mod().cuda.is_available():
        pytest.skip("no GPU")


def run(exe, *args, timeout=180):
    print(f"running {os.path.relpath(exe, REPO)} {' '.join(args)}", flush=True)
    return subprocess.run([exe, *args], capture_output=True, text=True, timeout=timeout)


def check_test_output(r):
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    out = r.stdout
    assert "[ RUN      ]" in out and "[       OK ]" in out
    assert "[  FAILED  ]" not in out
    assert "Tests run:" in out
    assert "ALL TESTS PASSED" in out


def test_kai_test_harness_passes():
    check_test_output(run(os.path.join(REPO, "orionsbelt_amd", "bin", "test_kai_gdn")))


def test_reference_test_program_on_hip_library():
    exe = os.path.join(REPO, "oracle", "_ref", "test_kai_gdn_on_hip")
    if not os.access(exe, os.X_OK):
        pytest.skip("oracle/_ref/test_kai_gdn_on_hip not built (needs the reference tree at build time)")
    r = run(exe)
    check_test_output(r)
    print(r.stdout.strip().splitlines()[-3:])


@pytest.mark.parametrize("prog", ["test_gdn_mixed_on_hip", "test_gdn2_scan_on_hip"])
def test_reference_gdn_sve_tests_on_hip_library(prog):
    """The reference's tests of its gdn_sve.h kernels (test_gdn_mixed.c:
    fp16/bf16 decay and scan against its fp32 reference, bounds and a
    determinism check; test_gdn2_scan.c: the GDN-2 scan against its float
    and double references, the reduction to GDN-1, state continuity and
    determinism), compiled unchanged and linked to this library by
    oracle/Makefile."""
    exe = os.path.join(REPO, "oracle", "_ref", prog)
    if not os.access(exe, os.X_OK):
        pytest.skip(f"oracle/_ref/{prog} not built (needs the reference tree at build time)")
    r = run(exe)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    assert "ALL TESTS PASSED" in r.stdout
    print(r.stdout.strip().splitlines()[-1])


def test_reference_delta_matmul_test_on_hip_library():
    """test_gdn_delta_matmul.c (naive fp32 loop against gdn_delta_rule_matmul
    at M in {1, 64}, K = 128, N in {128, 2048, 130}, rel < 1e-4 each,
    test_gdn_delta_matmul.c:70,87-96) with host pointers, through the
    library's staging path."""
    exe = os.path.join(REPO, "oracle", "_ref", "test_gdn_delta_matmul_on_hip")
    if not os.access(exe, os.X_OK):
        pytest.skip("oracle/_ref/test_gdn_delta_matmul_on_hip not built (needs the reference tree at build time)")
    r = run(exe)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if "max_rel" in ln]
    assert len(lines) == 6 and all(ln.rstrip().endswith("PASS") for ln in lines), r.stdout
    assert "ALL PASS" in r.stdout
    print("\n".join(lines))


def test_reference_gdn_sve_report_on_hip_library():
    """test_gdn_sve.c prints the scan, decay and conv against its
    precision-matched float reference and has no pass/fail exit, so its
    verdict lines are read here: at its shape (64 rows, one row tile of each
    scan) the scan and the decay are bit-identical to the reference's
    sequential loops, and the conv over two chunks equals the conv over the
    whole sequence."""
    exe = os.path.join(REPO, "oracle", "_ref", "test_gdn_sve_on_hip")
    if not os.access(exe, os.X_OK):
        pytest.skip("oracle/_ref/test_gdn_sve_on_hip not built (needs the reference tree at build time)")
    r = run(exe)
    assert r.returncode == 0, r.stderr[-2000:]
    print(r.stdout)
    out = r.stdout
    assert "gated_scan bit-identical to matched reference: YES" in out
    assert "cumdecay bit-identical to matched reference: YES" in out
    assert "conv streaming bit-identical: YES" in out
    assert "nan" not in out.lower()


def test_kai_bench_harness_csv():
    r = run(os.path.join(REPO, "orionsbelt_amd", "bin", "bench_kai_gdn"), "--repeats", "3", "--csv")
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.strip().splitlines() if ln]
    assert lines[0] == CSV_HEADER
    rows = [ln.split(",") for ln in lines[1:]]
    assert len(rows) >= 4
    kernels = {f[0] for f in rows}
    for k in ("cumdecay", "gated_scan", "conv1d", "gemv"):
        assert any(k in name for name in kernels), (k, sorted(kernels))
    for f in rows:
        assert len(f) == 7, f
        assert int(f[4]) == 3
        assert float(f[5]) > 0 and float(f[6]) > 0
