"""GPU parity of diversity selection (api.cpp:175-233) against the oracle.

The GPU prunes each chunk's candidate keys by importance and certifies every
greedy pick against the largest pruned importance, widening the candidate
set when it cannot; the kept keys must therefore equal the reference's
exactly. The variants (tests/kvc_data.py) cover the default strength at the
Llama-3-8B-like chunk shape, strengths that disable pruning (s >= 1, s < 0),
near-duplicate keys (penalties near 1: the first pruning level fails and the
wider ones run), exact duplicate rows (ties in importance and cosine),
negative R-KV weights (pruning off, more candidates than the first level
holds), and shared prefixes up to and beyond the kept count.
"""
from __future__ import annotations

import numpy as np
import pytest

from kvc_data import diversity_variant, diversity_variant_names
from kvc_harness import case_params, kc, load_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    lib = kc.load_product()
    if not lib.dll.kv_compact_hip_available():
        pytest.fail("no usable GPU for the GPU test tier")
    return lib


@pytest.fixture(scope="module")
def orc():
    return load_oracle()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", diversity_variant_names())
def test_diversity_variant(gpu, orc, name):
    c, K, V, Q, nq = diversity_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    print(f"[div] {name} T={T} H={H} d={d} params={c['params']}", flush=True)
    a = gpu.compact(K, V, Q, T, nq, H, d, d, case_params(gpu, c, T))
    b = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T))
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    assert np.array_equal(bits(a.beta), bits(b.beta)), "beta"
    assert np.array_equal(bits(a.C_v), bits(b.C_v)), "C_v"
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k
