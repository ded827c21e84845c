"""The drop-in claim, observed on the GPU: the kai test and bench harness
programs run against libkai_gdn_hip.so and keep the reference harnesses'
observable contract (kleidiai_submission/test_kai_gdn.c:84-96,665-675:
`[ RUN      ]` lines, a `Tests run:` summary, `ALL TESTS PASSED`, exit 0;
bench_kai_gdn.c:249-256,298: `--repeats N`, `--csv` and the CSV header that
scripts/verify_kleidiai_kernels.sh:74-79 parses).

Three programs:
- orionsbelt_amd/bin/test_kai_gdn: this build's harness (host and device
  pointer suites);
- oracle/_ref/test_kai_gdn_on_hip: the reference's own test_kai_gdn.c,
  compiled unchanged against include/ and linked to the HIP library
  (oracle/Makefile), when that build exists;
- orionsbelt_amd/bin/bench_kai_gdn: the bench harness, CSV mode."""
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
