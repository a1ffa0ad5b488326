"""kvc_compact_layers_device_noalloc: the allocation-free entry point.

Its outputs equal kvc_compact_layers_device's bit for bit on two calls in a
row (the second smaller, so the fixed scratch still holds the first call's
data), free device memory does not change across its calls, and a call whose
workspace exceeds the fixed scratch returns KVC_E_SCRATCH before launching
anything.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from kvc_harness import kc

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def dev():
    lib = kc.load_product()
    if not lib.dll.kv_compact_hip_available():
        pytest.fail("no usable GPU for the GPU test tier")
    return lib, kc.bind_device_api(lib.dll)


def make(L, T, H, d, W, seed):
    r = np.random.default_rng(seed)
    E = H * d
    K = np.empty((L, T, E), np.float32)
    V = r.standard_normal((L, T, E), dtype=np.float32)
    Q = np.empty((L, W, E), np.float32)
    for l in range(L):
        scale = np.exp(r.normal(0.0, 0.5, size=E)).astype(np.float32)
        K[l] = r.standard_normal((T, E), dtype=np.float32) * scale
        Q[l] = K[l, -W:] + np.float32(0.1) * r.standard_normal((W, E), dtype=np.float32)
    return K, V, Q


def outputs(L, H, t, d):
    import hiprt
    return [hiprt.DevBuf(n * 4) for n in (L * t, L * H * t, L * H * t * d, L * 3)]


def run(fn, bufs, dK, dV, dQ, L, T, W, H, d, p, t, free_check=False):
    import hiprt
    idx, beta, cv, st = bufs
    out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)
    free0 = hiprt.mem_free() if free_check else 0
    rc = fn(dK.value, dV.value, dQ.value, L, T, W, H, d, d, T * H * d, T * H * d, W * H * d, ctypes.byref(p), None,
            ctypes.byref(out), None)
    if free_check:
        assert hiprt.mem_free() == free0, "device memory changed across the allocation-free call"
    res = (idx.download(np.int32, L * t), beta.download(np.float32, L * H * t),
           cv.download(np.float32, L * H * t * d), st.download(np.float32, L * 3)) if rc == 0 else None
    return rc, res


def test_noalloc_matches_arena_entry(dev):
    import hiprt
    lib, dll = dev
    cases = [
        # (L, T, H, d, W, seed, params): the second call is smaller
        (2, 4096, 4, 128, 32, 9101, dict(target_ratio=0.2, use_diversity=1)),
        (1, 2000, 2, 64, 16, 9102, dict(target_ratio=0.3)),
    ]
    for (L, T, H, d, W, seed, pk) in cases:
        print(f"[noalloc] L={L} T={T} H={H} d={d} W={W} {pk}", flush=True)
        K, V, Q = make(L, T, H, d, W, seed)
        dK, dV, dQ = hiprt.DevBuf(K.nbytes), hiprt.DevBuf(V.nbytes), hiprt.DevBuf(Q.nbytes)
        dK.upload(K); dV.upload(V); dQ.upload(Q)
        p = lib.params(**pk)
        t, _ = kc.plan(dll, T, W, True, p)
        bn, ba = outputs(L, H, t, d), outputs(L, H, t, d)
        rc_n, a = run(dll.kvc_compact_layers_device_noalloc, bn, dK, dV, dQ, L, T, W, H, d, p, t, free_check=True)
        assert rc_n == 0
        rc_a, b = run(dll.kvc_compact_layers_device, ba, dK, dV, dQ, L, T, W, H, d, p, t)
        assert rc_a == 0
        assert np.array_equal(a[0], b[0]), "indices"
        for k, (x, y) in enumerate(zip(a[1:], b[1:])):
            assert np.array_equal(bits(x), bits(y)), ("beta", "C_v", "stats")[k]


def test_noalloc_rejects_oversized(dev):
    import hiprt
    lib, dll = dev
    # a 32-layer, 100k-token call needs gigabytes of workspace: refused before
    # any launch (the inputs are never read, so small buffers stand in)
    small = hiprt.DevBuf(1 << 20)
    out = kc.DeviceOut(small.value, small.value, small.value, small.value)
    p = lib.params(target_ratio=0.2)
    free0 = hiprt.mem_free()
    rc = dll.kvc_compact_layers_device_noalloc(small.value, small.value, small.value, 32, 100000, 32, 8, 128, 128,
                                               100000 * 1024, 100000 * 1024, 32 * 1024, ctypes.byref(p), None,
                                               ctypes.byref(out), None)
    assert rc == kc.E_SCRATCH
    assert hiprt.mem_free() == free0
