"""GPU parity of the host-pointer entries with the pinned transfer ring in
many pieces.

kv_compact, kv_compact_quantized and kvc_state_compact move their large
host buffers (K and V, the quantized rows, the state blob; C_v, the
requantized rows and the output blob on the way back) through a pinned ring
in pieces of at most 8 MB. The test switch KVC_PIN_BYTES shrinks the pieces
so that these moderate inputs take the ring in many pieces (the last one
partial, several per thread and buffer) and the results must still equal the
oracle's bit for bit.
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import numpy as np
import pytest

from kvc_data import T_F16, kv_cache, quantize_rows, snapkv_queries, state_blob
from kvc_harness import ORACLE_SO, kc, load_oracle, state_case_params, state_t

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


@contextlib.contextmanager
def pieces(n):
    old = os.environ.get("KVC_PIN_BYTES")
    os.environ["KVC_PIN_BYTES"] = str(n)
    try:
        yield
    finally:
        if old is None:
            os.environ.pop("KVC_PIN_BYTES", None)
        else:
            os.environ["KVC_PIN_BYTES"] = old


def same(a, b):
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    assert np.array_equal(bits(a.beta), bits(b.beta)), "beta"
    assert np.array_equal(bits(a.C_v), bits(b.C_v)), "C_v"
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k


@pytest.mark.parametrize("piece", [4100, 65540])
def test_host_compact_in_pieces(gpu, orc, piece):
    """H = 8, d = 128, T = 2560, SnapKV queries: K and V are 10.5 MB each."""
    T, H, d = 2560, 8, 128
    print(f"[transfer] kv_compact T={T} piece={piece}", flush=True)
    K, V = kv_cache(T, H, d, 301, channel_scale=True)
    Q = snapkv_queries(K, 32, 301)
    p = dict(target_ratio=0.2)
    with pieces(piece):
        a = gpu.compact(K, V, Q, T, 32, H, d, d, gpu.params(**p))
    b = orc.compact(K, V, Q, T, 32, H, d, d, orc.params(**p))
    same(a, b)


def test_release_between_calls(gpu, orc):
    """kvc_release_workspace frees the device workspace and the pinned ring;
    the next host-pointer call allocates both again and gives the same
    results."""
    T, H, d = 2560, 8, 128
    print("[transfer] release between calls", flush=True)
    K, V = kv_cache(T, H, d, 303)
    Q = snapkv_queries(K, 32, 303)
    p = dict(target_ratio=0.2)
    b = orc.compact(K, V, Q, T, 32, H, d, d, orc.params(**p))
    with pieces(65540):
        a1 = gpu.compact(K, V, Q, T, 32, H, d, d, gpu.params(**p))
        gpu.dll.kvc_release_workspace.restype = None
        gpu.dll.kvc_release_workspace()
        a2 = gpu.compact(K, V, Q, T, 32, H, d, d, gpu.params(**p))
    same(a1, b)
    same(a2, b)


def test_host_quantized_in_pieces(gpu, orc):
    """Q8_0 K, Q4_0 V, H = 8, d = 128, T = 2560, cheap queries: the rows go up
    and the requantized rows come back in pieces of 4100 bytes."""
    T, H, d = 2560, 8, 128
    print(f"[transfer] kv_compact_quantized T={T}", flush=True)
    K, V = kv_cache(T, H, d, 302)
    Kq, Vq = quantize_rows(K, 8), quantize_rows(V, 2)
    args = (Kq, Vq, None, 8, 2, Kq.shape[1], Vq.shape[1], T, 0, H, d, d)
    pk = dict(target_ratio=0.2, use_cheap_qref=1)
    with pieces(4100):
        ra, a = gpu.quantized(*args, gpu.params(**pk))
    rb, b = orc.quantized(*args, orc.params(**pk))
    assert ra == 0 and rb == 0
    same(a, b)
    assert np.array_equal(a.K_out, b.K_out) and np.array_equal(a.V_out, b.V_out)


def test_host_state_in_pieces(gpu, orc):
    """An F16 state blob of 2 layers x 4 heads x 128 and 2048 cells (4 MB)
    through kvc_state_compact, in pieces of 65540 bytes each way."""
    c = dict(name="pieces", T=2048, L=2, H=4, dk=128, dv=128, kt=T_F16, vt=T_F16, vtrans=0, seed=73, ratio=0.2)
    blob = state_blob(c)
    print(f"[transfer] state blob {len(blob)} bytes", flush=True)
    p, keep = state_case_params(c)
    with pieces(65540):
        rc, out, sel = kc.state_compact(gpu.dll, "kvc_", blob, p, state_t(c))
    rc_o, out_o, sel_o = kc.state_compact(ctypes.CDLL(str(ORACLE_SO)), "orc_", blob, p, state_t(c))
    del keep
    assert rc == 0 and rc_o == 0, (rc, rc_o)
    assert np.array_equal(sel, sel_o), "kept cells"
    assert out == out_o, "output blob"


@pytest.mark.parametrize("where", ["k_device", "v_device", "both_host"])
def test_host_device_mixes(gpu, orc, where):
    """kv_compact with K, V or neither already in device memory, diversity on:
    a host V uploads on its own stream while the kernels that read only K run
    (the diversity levels synchronise the call's stream meanwhile); results
    equal the oracle's bit for bit."""
    import hiprt
    T, H, d = 2560, 8, 128
    print(f"[transfer] mixed pointers {where}", flush=True)
    K, V = kv_cache(T, H, d, 304, channel_scale=True)
    Q = snapkv_queries(K, 32, 304)
    p = dict(target_ratio=0.2, use_diversity=1)
    dK = dV = None
    Ka, Va = K, V
    if where == "k_device":
        dK = hiprt.DevBuf(K.nbytes)
        dK.upload(K)
        Ka = dK.value
    elif where == "v_device":
        dV = hiprt.DevBuf(V.nbytes)
        dV.upload(V)
        Va = dV.value
    with pieces(65540):
        a = gpu.compact(Ka, Va, Q, T, 32, H, d, d, gpu.params(**p))
    b = orc.compact(K, V, Q, T, 32, H, d, d, orc.params(**p))
    same(a, b)
    del dK, dV


def test_failure_while_v_uploads(gpu, orc):
    """A call that stops while V is still being uploaded (KVC_FAULT=launch
    stops it before its first kernel; Lawson-Hanson beta on an unchunked call
    keeping more than 256 keys is refused with -5) returns its code with the
    result left empty (no arrays, t = 0), and the next call gives the oracle's
    results."""
    T, H, d = 2560, 8, 128
    print("[transfer] failure while V uploads", flush=True)
    K, V = kv_cache(T, H, d, 305)
    Q = snapkv_queries(K, 32, 305)
    cases = [("launch", dict(target_ratio=0.2), -6),
             (None, dict(target_ratio=0.2, chunk_size=-1, skip_beta=0, nnls_method=0), -5)]
    with pieces(65540):
        for fault, p, want in cases:
            if fault:
                os.environ["KVC_FAULT"] = fault
            try:
                rc, r = gpu.compact_raw(K, V, Q, T, 32, H, d, d, gpu.params(**p))
            finally:
                os.environ.pop("KVC_FAULT", None)
            assert rc == want, (fault, rc)
            assert r.t == 0 and r.n_head_kv == 0 and not r.selected_indices and not r.C_v and not r.beta
            gpu.free_result(r)
        a = gpu.compact(K, V, Q, T, 32, H, d, d, gpu.params(target_ratio=0.2))
    b = orc.compact(K, V, Q, T, 32, H, d, d, orc.params(target_ratio=0.2))
    same(a, b)
