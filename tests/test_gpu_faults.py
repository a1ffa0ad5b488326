"""Host-forced device faults surface as non-zero return codes, with no CPU
fallback, and the library recovers once the fault is cleared.

KVC_FAULT=alloc fails every workspace allocation; KVC_FAULT=launch stops a
compaction before its first kernel launch. Both are read at every call, so the
test sets and clears them inside one process; every kernel that does run exits
normally.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from kvc_data import STATE_CASE_BY_NAME, kv_cache, quantize_rows, snapkv_queries, state_blob
from kvc_harness import kc, load_oracle, state_case_params, state_t

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    lib = kc.load_product()
    if not lib.dll.kv_compact_hip_available():
        pytest.fail("no usable GPU for the GPU test tier")
    return lib


def calls(gpu):
    """(name, fn returning the call's return code, alloc-only) for each entry."""
    T, H, d = 1536, 2, 64
    K, V = kv_cache(T, H, d, 301, channel_scale=True)
    Q = snapkv_queries(K, 16, 301)
    p = gpu.params(target_ratio=0.2)
    Kq = quantize_rows(K, kc.KV_TYPE_Q8_0)
    Vq = quantize_rows(V, kc.KV_TYPE_Q8_0)
    c = STATE_CASE_BY_NAME["f16_basic"]
    blob = state_blob(c)

    def compact():
        return gpu.compact_raw(K, V, Q, T, 16, H, d, d, p)[0]

    def quantized():
        return gpu.quantized(Kq, Vq, None, kc.KV_TYPE_Q8_0, kc.KV_TYPE_Q8_0, Kq.shape[1], Vq.shape[1],
                             T, 0, H, d, d, gpu.params(target_ratio=0.2, use_cheap_qref=1))[0]

    def multi():
        return gpu.multi_round(K, V, Q, T, 16, H, d, d, gpu.params(target_ratio=0.5), 2)[0]

    def state():
        sp, keep = state_case_params(c)
        rc = kc.state_compact(gpu.dll, "kvc_", blob, sp, state_t(c))[0]
        del keep
        return rc

    def qrow():
        x = np.ones(64, np.float32)
        gpu._qrow.restype = ctypes.c_size_t
        out = np.zeros(64 * 4, np.uint8)
        return 0 if gpu._qrow(x.ctypes.data, kc.KV_TYPE_Q8_0, 64, out.ctypes.data) else -1

    return [("kv_compact", compact, False), ("kv_compact_quantized", quantized, False),
            ("kv_compact_multi_round", multi, False), ("kvc_state_compact", state, False),
            ("kv_quantize_row", qrow, True)]


@pytest.mark.parametrize("kind", ["alloc", "launch"])
def test_forced_fault_surfaces_and_clears(gpu, kind):
    orc = load_oracle()
    entries = calls(gpu)
    try:
        os.environ["KVC_FAULT"] = kind
        for name, fn, alloc_only in entries:
            if alloc_only and kind != "alloc":
                continue
            print(f"[fault] {kind} {name}", flush=True)
            rc = fn()
            assert rc != 0, f"{name} returned 0 under KVC_FAULT={kind}"
            if name != "kv_quantize_row":
                assert rc == kc.E_DEVICE, (name, rc)
    finally:
        os.environ.pop("KVC_FAULT", None)
    for name, fn, _ in entries:
        assert fn() == 0, f"{name} did not recover"
    # and the results after recovery are the oracle's
    T, H, d = 1536, 2, 64
    K, V = kv_cache(T, H, d, 301, channel_scale=True)
    Q = snapkv_queries(K, 16, 301)
    a = gpu.compact(K, V, Q, T, 16, H, d, d, gpu.params(target_ratio=0.2))
    b = orc.compact(K, V, Q, T, 16, H, d, d, orc.params(target_ratio=0.2))
    assert np.array_equal(a.indices, b.indices)
    assert np.array_equal(a.C_v.view(np.uint32), b.C_v.view(np.uint32))


def _live(gpu):
    gpu.dll.kvc_live_objects.restype = ctypes.c_int
    return gpu.dll.kvc_live_objects()


def test_pinned_ring_failure_frees_its_buffers(gpu):
    """KVC_FAULT=pin fails the pinned ring after its first buffer: the host
    call falls back to plain copies with the same results, the buffer made
    is freed, and once kvc_release_workspace clears the mark the ring is
    allocated again."""
    orc = load_oracle()
    T, H, d = 1536, 2, 64
    K, V = kv_cache(T, H, d, 302, channel_scale=True)
    Q = snapkv_queries(K, 16, 302)
    ref = orc.compact(K, V, Q, T, 16, H, d, d, orc.params(target_ratio=0.2))
    gpu.dll.kvc_release_workspace()
    base = _live(gpu)
    try:
        os.environ["KVC_PIN_BYTES"] = "4096"   # the inputs take many pieces
        os.environ["KVC_FAULT"] = "pin"
        for _ in range(3):
            print("[fault] pin kv_compact", flush=True)
            a = gpu.compact(K, V, Q, T, 16, H, d, d, gpu.params(target_ratio=0.2))
            assert np.array_equal(a.indices, ref.indices)
            assert np.array_equal(a.C_v.view(np.uint32), ref.C_v.view(np.uint32))
            assert _live(gpu) == base, "a failed ring set-up left objects behind"
        os.environ.pop("KVC_FAULT")
        gpu.dll.kvc_release_workspace()
        a = gpu.compact(K, V, Q, T, 16, H, d, d, gpu.params(target_ratio=0.2))
        assert np.array_equal(a.C_v.view(np.uint32), ref.C_v.view(np.uint32))
        assert _live(gpu) == base + 16, "the ring (8 buffers, 8 events) was not set up again"
    finally:
        os.environ.pop("KVC_FAULT", None)
        os.environ.pop("KVC_PIN_BYTES", None)


_INIT_CHILD = r"""
import ctypes, os, sys
sys.path.insert(0, sys.argv[1])
import kvcompact as kc
lib = kc.load_product()
lib.dll.kvc_live_objects.restype = ctypes.c_int
os.environ["KVC_FAULT"] = "init"
for i in range(5):
    assert lib.dll.kv_compact_hip_available() == 0, "set-up succeeded under KVC_FAULT=init"
    assert lib.dll.kvc_live_objects() == 0, ("objects left by a failed set-up", lib.dll.kvc_live_objects())
os.environ.pop("KVC_FAULT")
assert lib.dll.kv_compact_hip_available() == 1
n = lib.dll.kvc_live_objects()
assert n > 0
assert lib.dll.kv_compact_hip_available() == 1 and lib.dll.kvc_live_objects() == n
print("init-fault child ok", n, flush=True)
"""


def test_device_setup_failure_leaves_nothing(gpu):
    """KVC_FAULT=init fails the per-device set-up after its streams and first
    events are made: the call reports no device, every object it made is
    destroyed (the live count stays 0), and the set-up succeeds once the
    fault is cleared. The set-up happens once per process, so this runs in a
    child process of its own."""
    import subprocess
    import sys
    from pathlib import Path
    pkg = Path(kc.__file__).resolve().parent
    print("[fault] init child process", flush=True)
    r = subprocess.run([sys.executable, "-c", _INIT_CHILD, str(pkg)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-2000:])
    assert "init-fault child ok" in r.stdout
