"""GPU parity of the beta fit (api.cpp:812-831) against the oracle.

beta = logf(max(1e-12, w)) with w from the clamped unconstrained least
squares (nnls_method 1, math.h:683-757) or Lawson-Hanson NNLS (nnls_method 0,
math.h:283-452) on M = exp_scores[:, sel], b = row sums. beta then shifts the
compacted softmax, so C_v and the statistics depend on it too; everything
must match bit for bit. Lawson-Hanson on chunks keeping more than 256 keys
is refused (KV_COMPACT_E_UNSUPPORTED).
"""
from __future__ import annotations

import numpy as np
import pytest

from kvc_data import beta_variant, beta_variant_names
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


@pytest.mark.parametrize("name", beta_variant_names())
def test_beta_variant(gpu, orc, name):
    c, K, V, Q, nq = beta_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    print(f"[beta] {name} T={T} H={H} d={d} params={c['params']}", flush=True)
    if name == "lh_unchunked_big_t":
        rc, _ = gpu.compact_raw(K, V, Q, T, nq, H, d, d, case_params(gpu, c, T))
        assert rc == kc.E_UNSUPPORTED
        return
    a = gpu.compact(K, V, Q, T, nq, H, d, d, case_params(gpu, c, T))
    b = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T))
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    ba, bb = bits(a.beta), bits(b.beta)
    if not np.array_equal(ba, bb):
        bad = np.argwhere(ba != bb)
        raise AssertionError(f"beta differs at {len(bad)} of {ba.size}: first {bad[:3].tolist()}")
    assert np.array_equal(bits(a.C_v), bits(b.C_v)), "C_v"
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k
