"""The no-allocation cumulative decay (kai_run_gdn_cumdecay_f32_noalloc_hip)
against the allocating entry point (kai_run_gdn_cumdecay_f32_hip) and the CPU
oracle, through the C-ABI.

Bars: a single 128-row tile keeps the reference's operation order, so those
results are bit-identical to both; across tiles only the carry into a tile is
re-associated, so results are held to the fp32 decay tolerance (1e-5
relative) of the kai test rule.  Shapes past the fixed scratch are refused
with hipErrorInvalidValue and nothing is written."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests.gdn_inputs import assert_kai_close
from tests.gpu_util import P, dev, empty, host, stream, torch_mod

pytestmark = pytest.mark.gpu

HIP_ERROR_INVALID_VALUE = 1


@pytest.fixture(scope="module")
def L():
    torch = torch_mod()
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import orionsbelt_amd as ob
    return ob.lib()


def gates(seq, ch, seed):
    rs = np.random.RandomState(seed)
    g = -np.log1p(np.exp(rs.randn(seq * ch))) * np.exp(rs.uniform(-2, 0, seq * ch))
    return np.exp(g).astype(np.float32)


def run(L, fn, a, seq, ch):
    import orionsbelt_amd as ob
    da = dev(a)
    out = empty(seq * ch, torch_mod().float32)
    ob.check(fn(P(da), P(out), seq, ch, stream()), "cumdecay")
    return host(out)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_noalloc_matches_allocating_entry_point_twice(L):
    # the largest shape the scratch covers, then a smaller ragged one, then a
    # single-tile one: each call reuses the scratch the previous one left
    for seq, ch, seed in [(4096, 8192, 1), (1000, 513, 2), (100, 300, 3)]:
        print(f"no-alloc cumdecay seq={seq} ch={ch}", flush=True)
        a = gates(seq, ch, seed)
        got = run(L, L.kai_run_gdn_cumdecay_f32_noalloc_hip, a, seq, ch)
        want = run(L, L.kai_run_gdn_cumdecay_f32_hip, a, seq, ch)
        ref = orc.cumdecay_f32(a, seq, ch)
        if seq <= 128:
            assert np.array_equal(bits(got), bits(want)), (seq, ch)
            assert np.array_equal(bits(got), bits(ref)), (seq, ch)
        else:
            assert_kai_close(got, want, 1e-6, 1e-5, "no-alloc vs allocating")
            assert_kai_close(got, ref, 1e-6, 1e-5, "no-alloc vs oracle")
    assert L.kai_gdn_hip_check_device_error() == 0


def test_noalloc_refuses_shapes_past_the_scratch(L):
    seq, ch = 4097, 8192  # 33 row tiles x 8192 channels > 262144 status words
    da = dev(np.ones(seq * ch, np.float32))
    out = dev(np.full(seq * ch, 7.0, np.float32))
    rc = L.kai_run_gdn_cumdecay_f32_noalloc_hip(P(da), P(out), seq, ch, stream())
    assert rc == HIP_ERROR_INVALID_VALUE
    assert np.all(host(out) == 7.0)
    # the entry point still works after a refusal
    a = gates(64, 33, 4)
    got = run(L, L.kai_run_gdn_cumdecay_f32_noalloc_hip, a, 64, 33)
    assert np.array_equal(bits(got), bits(orc.cumdecay_f32(a, 64, 33)))
