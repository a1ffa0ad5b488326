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
