"""GPU parity of the refinement rounds (api.cpp:851-946) against the oracle.

Each round swaps a chunk's worst kept key (least compacted attention mass
over heads and queries) for its best unused key by importance, unless that
key's importance is at most half the worst one's, and refits beta and C_v.
The variants (tests/kvc_data.py) swap keys in every chunk, combine the
rounds with the clamped-LS and Lawson-Hanson beta fits, diversity and R-KV
weights, and include a call that keeps every key (no round applies).
"""
from __future__ import annotations

import numpy as np
import pytest

from kvc_data import refine_variant, refine_variant_names
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


@pytest.mark.parametrize("name", refine_variant_names())
def test_refine_variant(gpu, orc, name):
    c, K, V, Q, nq = refine_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    print(f"[refine] {name} T={T} H={H} d={d} params={c['params']}", flush=True)
    a = gpu.compact(K, V, Q, T, nq, H, d, d, case_params(gpu, c, T))
    b = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T))
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    assert np.array_equal(bits(a.beta), bits(b.beta)), "beta"
    assert np.array_equal(bits(a.C_v), bits(b.C_v)), "C_v"
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k
