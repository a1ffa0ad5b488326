"""GPU parity of the register LU's two variants and of non-finite inputs.

The LU runs unmasked (multiplier 0 for the rows off the elimination) and
sends a system to the masked variant when its input holds -0 or a
non-finite entry, or when a final entry is non-finite. KVC_LU_MASKED=1 sends
every system to the masked variant, so both are checked against the oracle
on the same cases. Non-finite K / V entries reach the LU through the scores
and exercise the fallback itself; NaN results are compared by position (the
GPU and the x86 oracle may produce different NaN bit patterns), every other
value bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

from kvc_data import CASE_BY_NAME, beta_variant, make_case, nonfinite_variant, nonfinite_variant_names
from kvc_harness import case_params, kc, load_oracle, run_case

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def gpu():
    lib = kc.load_product()
    if not lib.dll.kv_compact_hip_available():
        pytest.fail("no usable GPU for the GPU test tier")
    return lib


@pytest.fixture(scope="module")
def orc():
    return load_oracle()


def same_nan(x, y, what):
    x = np.ascontiguousarray(x, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    nx, ny = np.isnan(x), np.isnan(y)
    assert np.array_equal(nx, ny), f"{what}: NaN positions differ"
    assert np.array_equal(bits(x[~nx]), bits(y[~ny])), f"{what}: values differ"


def same(a, b):
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    same_nan(a.beta, b.beta, "beta")
    same_nan(a.C_v, b.C_v, "C_v")
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        same_nan(np.float32(a.stats[k]), np.float32(b.stats[k]), k)


@pytest.mark.parametrize("name", ["cfg1_small", "cfg2_small_nodiv", "beta_clamped", "refine2_beta", "count",
                                  "tiny_T3", "dv_ne_dk", "prefix"])
def test_masked_variant_parity(gpu, orc, name, monkeypatch):
    monkeypatch.setenv("KVC_LU_MASKED", "1")
    c = CASE_BY_NAME[name]
    print(f"[case] masked {name}", flush=True)
    inp = make_case(c)
    same(run_case(gpu, c, inp), run_case(orc, c, inp))


def test_masked_variant_clamped_ls_chunks(gpu, orc, monkeypatch):
    """Clamped-LS beta (the LU also solves the mass fit) at 256 kept keys per chunk."""
    monkeypatch.setenv("KVC_LU_MASKED", "1")
    c, K, V, Q, nq = beta_variant("pgd_chunk")
    T, H, d = c["T"], c["H"], c["d"]
    print("[case] masked pgd_chunk", flush=True)
    a = gpu.compact(K, V, Q, T, nq, H, d, d, case_params(gpu, c, T))
    b = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T))
    same(a, b)


@pytest.mark.parametrize("pgd", [0, 1])
@pytest.mark.parametrize("name", nonfinite_variant_names())
def test_nonfinite_inputs(gpu, orc, name, pgd):
    c, K, V, Q, nq = nonfinite_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    extra = dict(skip_beta=0, nnls_method=1) if pgd else {}
    print(f"[case] nonfinite {name} pgd={pgd}", flush=True)
    a = gpu.compact(K, V, Q, T, nq, H, d, d, case_params(gpu, c, T, **extra))
    b = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T, **extra))
    same(a, b)
