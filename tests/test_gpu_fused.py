"""The fused scoring kernel (KVC_FUSED=1: scores, chunk softmax, importance
and the refit target in one kernel whose scores stay in registers, the kept
keys' scores computed again for the compacted softmax) against the CPU
oracle, bit for bit, on the shapes it takes: d_v = 128, at most 32 reference
queries shared by every chunk, chunks of at most 1280 keys, fp32 K and V.

Each case first checks that the fused path ran (its call reports the chunk
softmax and refit-target stages as 0 ms) and then compares every output with
the oracle: ragged last chunks, 1 to 32 queries, the three score methods,
diversity on and off, a forced prefix, R-KV weights, the cheap global query
set, non-finite keys and values, a three-layer device batch, and one layer
of the 100,000-token headline workload.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from kvc_data import kv_cache, snapkv_queries, span_classifier_spec
from kvc_harness import kc, load_oracle

pytestmark = pytest.mark.gpu

STAGES = 11


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def gpu():
    lib = kc.load_product()
    if not lib.dll.kv_compact_hip_available():
        pytest.fail("no usable GPU for the GPU test tier")
    kc.bind_device_api(lib.dll)
    return lib


@pytest.fixture(scope="module")
def orc():
    return load_oracle()


@pytest.fixture
def fused():
    os.environ["KVC_FUSED"] = "1"
    yield
    os.environ.pop("KVC_FUSED", None)


def stage_times(gpu):
    buf = (ctypes.c_float * STAGES)()
    gpu.dll.kvc_stage_times(buf, STAGES)
    return list(buf)


def assert_fused_ran(gpu):
    st = stage_times(gpu)
    assert st[0] > 0.0 and st[1] == 0.0 and st[2] == 0.0, f"the fused path did not run: {st[:3]}"


def same_nan(x, y, what):
    """Equal bits, NaN positions equal (a NaN's payload may differ)."""
    x, y = np.asarray(x, np.float32), np.asarray(y, np.float32)
    nx, ny = np.isnan(x), np.isnan(y)
    assert np.array_equal(nx, ny), f"{what}: NaN positions differ"
    assert np.array_equal(bits(np.where(nx, 0, x)), bits(np.where(ny, 0, y))), what


def same(a, b):
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    same_nan(a.beta, b.beta, "beta")
    same_nan(a.C_v, b.C_v, "C_v")
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        same_nan(np.float32(a.stats[k]), np.float32(b.stats[k]), k)


CASES = [
    # name, T, H, n_q, params
    ("ragged_div", 3000, 2, 32, dict(target_ratio=0.2, use_diversity=1)),
    ("ragged_topk", 3000, 2, 32, dict(target_ratio=0.2)),
    ("max_method", 2600, 2, 32, dict(target_ratio=0.2, score_method=0)),
    ("mean_method", 2600, 2, 32, dict(target_ratio=0.2, score_method=2)),
    ("one_query", 1500, 3, 1, dict(target_ratio=0.5)),
    ("seven_queries", 1500, 1, 7, dict(target_ratio=0.5, use_diversity=1, diversity_strength=0.8)),
    ("prefix", 2000, 2, 24, dict(target_ratio=0.3, n_shared_prefix=40)),
    ("unchunked", 1100, 2, 16, dict(target_ratio=0.4, chunk_size=-1)),
    ("tiny", 3, 1, 2, dict(target_ratio=0.7)),
]


@pytest.mark.parametrize("name,T,H,nq,p", CASES, ids=[c[0] for c in CASES])
def test_fused_parity(gpu, orc, fused, name, T, H, nq, p):
    print(f"[fused] {name} T={T} H={H} nq={nq}", flush=True)
    d = 128
    K, V = kv_cache(T, H, d, 500 + T + nq, channel_scale=True)
    Q = snapkv_queries(K, nq, 500 + T)
    a = gpu.compact(K, V, Q, T, nq, H, d, d, gpu.params(**p))
    assert_fused_ran(gpu)
    same(a, orc.compact(K, V, Q, T, nq, H, d, d, orc.params(**p)))


def test_fused_cheap_global_queries(gpu, orc, fused):
    """Cheap reference queries over the whole call (rows of K at the
    reference's quadratic positions): T = 60 keys, 30 queries, unchunked."""
    T, H, d = 60, 2, 128
    K, V = kv_cache(T, H, d, 611)
    p = dict(target_ratio=0.5, use_cheap_qref=1)
    a = gpu.compact(K, V, None, T, 0, H, d, d, gpu.params(**p))
    assert_fused_ran(gpu)
    same(a, orc.compact(K, V, None, T, 0, H, d, d, orc.params(**p)))


def test_fused_rkv_weights(gpu, orc, fused):
    T, H, d, nq = 2800, 2, 128, 32
    K, V = kv_cache(T, H, d, 612, channel_scale=True)
    Q = snapkv_queries(K, nq, 612)
    s, e = span_classifier_spec(T, 612)

    def cls(pos, _data):
        return kc.KV_TOKEN_THINKING if s <= pos < e else (kc.KV_TOKEN_TRANSITION if pos == e else kc.KV_TOKEN_ANSWER)

    cb = kc.CLASSIFIER(cls)
    r = kc.Reasoning(cb, None, 0.3, 0.7, 0)
    pa = gpu.params(target_ratio=0.2, use_diversity=1)
    pa.reasoning = ctypes.pointer(r)
    pb = orc.params(target_ratio=0.2, use_diversity=1)
    pb.reasoning = ctypes.pointer(r)
    a = gpu.compact(K, V, Q, T, nq, H, d, d, pa)
    assert_fused_ran(gpu)
    same(a, orc.compact(K, V, Q, T, nq, H, d, d, pb))


@pytest.mark.parametrize("what", ["nan_k", "inf_k", "nan_v", "negzero_k", "nan_first_key"])
def test_fused_nonfinite(gpu, orc, fused, what):
    """NaN, inf and -0 reach the scores, maxima, exponentials and weighted
    sums the way the reference's arithmetic carries them."""
    T, H, d, nq = 1400, 2, 128, 16
    K, V = kv_cache(T, H, d, 613)
    Q = snapkv_queries(K, nq, 613)
    if what == "nan_k":
        K[700, 5] = np.nan
    elif what == "inf_k":
        K[1300, 200] = np.inf
    elif what == "nan_v":
        V[64, 130] = np.nan
    elif what == "negzero_k":
        K[11, :] = -0.0
    else:
        K[0, 3] = np.nan   # row[0] of every query row of head 0 is NaN: the maximum is NaN
    p = dict(target_ratio=0.3)
    print(f"[fused] nonfinite {what}", flush=True)
    a = gpu.compact(K, V, Q, T, nq, H, d, d, gpu.params(**p))
    assert_fused_ran(gpu)
    same(a, orc.compact(K, V, Q, T, nq, H, d, d, orc.params(**p)))


def test_fused_device_batch(gpu, orc, fused):
    """Three layers in one kvc_compact_layers_device call, diversity on."""
    import hiprt
    L, T, H, d, W = 3, 2700, 2, 128, 32
    Ks, Vs, Qs = [], [], []
    for l in range(L):
        K, V = kv_cache(T, H, d, 620 + l, channel_scale=True)
        Ks.append(K); Vs.append(V); Qs.append(snapkv_queries(K, W, 620 + l))
    dll = gpu.dll
    p = gpu.params(target_ratio=0.2, use_diversity=1)
    t, _ = kc.plan(dll, T, W, True, p)
    dK, dV, dQ = (hiprt.DevBuf(L * a[0].nbytes) for a in (Ks, Vs, Qs))
    for l in range(L):
        dK.upload(Ks[l], l * Ks[0].nbytes); dV.upload(Vs[l], l * Vs[0].nbytes); dQ.upload(Qs[l], l * Qs[0].nbytes)
    idx, beta, cv, st = (hiprt.DevBuf(n * 4) for n in (L * t, L * H * t, L * H * t * d, L * 3))
    out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)
    rc = dll.kvc_compact_layers_device(dK.value, dV.value, dQ.value, L, T, W, H, d, d, T * H * d, T * H * d,
                                       W * H * d, ctypes.byref(p), None, ctypes.byref(out), None)
    assert rc == 0
    assert_fused_ran(gpu)
    gi = idx.download(np.int32, L * t).reshape(L, t)
    gc = cv.download(np.float32, L * H * t * d).reshape(L, H, t, d)
    gs = st.download(np.float32, L * 3).reshape(L, 3)
    for l in range(L):
        b = orc.compact(Ks[l], Vs[l], Qs[l], T, W, H, d, d, orc.params(target_ratio=0.2, use_diversity=1))
        assert np.array_equal(gi[l], b.indices), l
        assert np.array_equal(bits(gc[l]), bits(b.C_v.reshape(H, t, d))), l
        assert bits(gs[l, 0]) == bits(np.float32(b.stats["avg_cosine_sim"])), l


def test_fused_headline_layer(gpu, orc, fused):
    """One layer of the headline workload (T = 100,000, 8 heads, d = 128,
    SnapKV W = 32, keep 0.2, diversity on), bit for bit."""
    T, H, d, W = 100000, 8, 128, 32
    print("[fused] headline layer T=100000 H=8 d=128", flush=True)
    K, V = kv_cache(T, H, d, 630, channel_scale=True)
    Q = snapkv_queries(K, W, 630)
    p = dict(target_ratio=0.2, use_diversity=1)
    a = gpu.compact(K, V, Q, T, W, H, d, d, gpu.params(**p))
    assert_fused_ran(gpu)
    same(a, orc.compact(K, V, Q, T, W, H, d, d, orc.params(**p)))


def test_default_path_is_unfused(gpu):
    """Without KVC_FUSED the separate kernels run (nonzero softmax stage)."""
    T, H, d, nq = 2600, 2, 128, 32
    K, V = kv_cache(T, H, d, 640)
    Q = snapkv_queries(K, nq, 640)
    os.environ.pop("KVC_FUSED", None)
    gpu.compact(K, V, Q, T, nq, H, d, d, gpu.params(target_ratio=0.2))
    assert stage_times(gpu)[1] > 0.0
