"""GPU parity of the selection and fit options against the oracle, bit for bit.

- sensitivity weighting (math.h:579-618; api.cpp:651-666): per head, the
  largest per-key maximum over queries of the softmax weights over their mean;
  the global importance is the head-ordered sum of sens_h * imp_h[j];
- PGD iterations of the clamped least-squares beta fit (math.h:752-805);
- OMP key selection (math.h:832-950; api.cpp:690-711) on the exp scores and
  row sums summed over heads, with k_choice picks per step, refits every
  refit_interval steps and the PGD steps inside each refit.

Each case also runs the downstream beta fit, value refit and statistics, so
kept indices, beta, C_v and the three statistics must all match.
"""
from __future__ import annotations

import numpy as np
import pytest

from kvc_data import option_variant, option_variant_names
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


@pytest.mark.parametrize("name", option_variant_names())
def test_option_variant(gpu, orc, name):
    c, K, V, Q, nq = option_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    print(f"[option] {name} T={T} H={H} d={d} params={c['params']}", flush=True)
    a = gpu.compact(K, V, Q, T, nq, H, d, d, case_params(gpu, c, T))
    b = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T))
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    assert np.array_equal(bits(a.beta), bits(b.beta)), "beta"
    ca, cb = bits(a.C_v), bits(b.C_v)
    if not np.array_equal(ca, cb):
        bad = np.argwhere(ca != cb)
        raise AssertionError(f"C_v differs at {len(bad)} of {ca.size}: first {bad[:3].tolist()}")
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k


def test_options_on_device_batch(gpu, orc):
    """Sensitivity + OMP (k_choice 4, refit every 2nd step) + PGD beta through
    the multi-layer device entry: every layer equals its own oracle call."""
    import ctypes

    import hiprt
    c, K0, V0, Q0, nq = option_variant("omp_k4_r2_beta_pgd")
    T, H, d = c["T"], c["H"], c["d"]
    L = 2
    rng = np.random.default_rng(7)
    Ks = [K0, (K0 + 0.05 * rng.standard_normal(K0.shape)).astype(np.float32)]
    Vs = [V0, np.ascontiguousarray(V0[::-1])]
    Qs = [Q0, Q0]
    params = dict(c["params"], use_sensitivity=1)
    print(f"[option] device batch L={L} T={T} H={H} params={params}", flush=True)
    dll = kc.bind_device_api(gpu.dll)
    p = gpu.params(**params)
    t, _ = kc.plan(dll, T, nq, True, p)
    dK, dV, dQ = (hiprt.DevBuf(L * a[0].nbytes) for a in (Ks, Vs, Qs))
    for l in range(L):
        dK.upload(Ks[l], l * Ks[0].nbytes); dV.upload(Vs[l], l * Vs[0].nbytes); dQ.upload(Qs[l], l * Qs[0].nbytes)
    idx, beta, cv, st = (hiprt.DevBuf(n * 4) for n in (L * t, L * H * t, L * H * t * d, L * 3))
    out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)
    rc = dll.kvc_compact_layers_device(dK.value, dV.value, dQ.value, L, T, nq, H, d, d, T * H * d, T * H * d,
                                       nq * H * d, ctypes.byref(p), None, ctypes.byref(out), None)
    assert rc == 0
    gi = idx.download(np.int32, L * t).reshape(L, t)
    gb = beta.download(np.float32, L * H * t).reshape(L, H, t)
    gc = cv.download(np.float32, L * H * t * d).reshape(L, H, t, d)
    for l in range(L):
        b = orc.compact(Ks[l], Vs[l], Qs[l], T, nq, H, d, d, orc.params(**params))
        assert b.t == t
        assert np.array_equal(gi[l], b.indices), f"layer {l} indices"
        assert np.array_equal(bits(gb[l]), bits(b.beta)), f"layer {l} beta"
        assert np.array_equal(bits(gc[l]), bits(b.C_v)), f"layer {l} C_v"
