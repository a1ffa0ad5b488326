"""GPU parity of the llama.cpp state blob compaction (kvc_state_compact and
kvc_state_compact_device) against the oracle, byte for byte.

The oracle's blob writer is itself byte-equal to the reference's own
parse/build on these cases (test_state.py), and the fixtures hold the
reference's output hashes, so the library's blob is checked against both.
"""
from __future__ import annotations

import ctypes
import hashlib
import struct
from pathlib import Path

import numpy as np
import pytest

from kvc_data import STATE_CASES, STATE_CASE_BY_NAME, T_F16, state_blob
from kvc_harness import ORACLE_SO, kc, state_case_params, state_t

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "state_cases.npz"


@pytest.fixture(scope="module")
def gpu():
    lib = kc.load_product()
    if not lib.dll.kv_compact_hip_available():
        pytest.fail("no usable GPU for the GPU test tier")
    return lib.dll


@pytest.fixture(scope="module")
def orc():
    return ctypes.CDLL(str(ORACLE_SO))


def run(dll, prefix, c, blob):
    p, keep = state_case_params(c)
    r = kc.state_compact(dll, prefix, blob, p, state_t(c))
    del keep
    return r


def first_diff(a: bytes, b: bytes):
    x, y = np.frombuffer(a, np.uint8), np.frombuffer(b, np.uint8)
    n = min(x.size, y.size)
    bad = np.nonzero(x[:n] != y[:n])[0]
    return f"sizes {x.size} / {y.size}, {bad.size} bytes differ, first at {bad[:5].tolist()}"


@pytest.mark.parametrize("name", [c["name"] for c in STATE_CASES])
def test_state_blob_parity(gpu, orc, name):
    c = STATE_CASE_BY_NAME[name]
    print(f"[state] {name} T={c['T']} L={c['L']} H={c['H']}", flush=True)
    blob = state_blob(c)
    rc, out, sel = run(gpu, "kvc_", c, blob)
    rc_o, out_o, sel_o = run(orc, "orc_", c, blob)
    assert rc == 0 and rc_o == 0, (rc, rc_o)
    assert np.array_equal(sel, sel_o), "kept cells"
    assert out == out_o, first_diff(out, out_o)
    g = np.load(GOLDEN)
    assert hashlib.sha256(out).hexdigest() == str(g[name + "_sha256"])


def test_state_device_entry(gpu, orc):
    """Device blob in, device blob out; a too-small output buffer reports the
    size it needs and writes nothing."""
    import hiprt
    c = STATE_CASE_BY_NAME["mixed_types_sens"]
    blob = state_blob(c)
    print(f"[state] device entry {c['name']}", flush=True)
    rc_o, out_o, sel_o = run(orc, "orc_", c, blob)
    assert rc_o == 0
    f = gpu.kvc_state_compact_device
    f.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(kc.StateParams), ctypes.c_void_p,
                  ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t), ctypes.c_void_p, ctypes.c_void_p]
    f.restype = ctypes.c_int
    src = hiprt.DevBuf(len(blob))
    src.upload(np.frombuffer(blob, np.uint8))
    dst = hiprt.DevBuf(len(blob))
    p, keep = state_case_params(c)
    n = ctypes.c_size_t(0)
    sel = np.full(state_t(c), -1, np.int32)
    rc = f(src.value, len(blob), ctypes.byref(p), dst.value, len(blob), ctypes.byref(n), sel.ctypes.data, None)
    assert rc == 0
    assert n.value == len(out_o)
    got = dst.download(np.uint8, n.value).tobytes()
    assert got == out_o, first_diff(got, out_o)
    assert np.array_equal(sel, sel_o)
    dst.zero()
    rc = f(src.value, len(blob), ctypes.byref(p), dst.value, 100, ctypes.byref(n), None, None)
    assert rc == kc.E_CAPACITY and n.value == len(out_o)
    assert not dst.download(np.uint8, 100).any()
    del keep


def test_state_parse_info_and_errors(gpu, orc):
    for c in STATE_CASES:
        blob = state_blob(c)
        rc, a = kc.state_info(gpu, "kvc_", blob, c.get("n_pos", 1))
        rc_o, b = kc.state_info(orc, "orc_", blob, c.get("n_pos", 1))
        assert rc == rc_o == 0
        for k, _ in kc.StateInfo._fields_:
            assert getattr(a, k) == getattr(b, k), (c["name"], k)
    c = STATE_CASE_BY_NAME["f16_basic"]
    blob = state_blob(c)
    for cut in (3, 40, len(blob) // 2, len(blob) - 1):
        assert run(gpu, "kvc_", c, blob[:cut])[0] == run(orc, "orc_", c, blob[:cut])[0] == -2, cut
    c2 = dict(c, name="x", n_stream=2, extra_cells=3)
    assert run(gpu, "kvc_", c2, state_blob(c2))[0] == kc.E_UNSUPPORTED
    b = bytearray(blob)
    i = blob.index(struct.pack("<iQ", T_F16, c["H"] * c["dk"] * 2))
    struct.pack_into("<i", b, i, 30)
    assert run(gpu, "kvc_", c, bytes(b))[0] == kc.E_UNSUPPORTED


def test_state_general_solver_shape(gpu, orc):
    """T = 2048, 4 heads of 128, 512 reference queries, 409 kept cells: the
    value systems exceed the register LU (general elimination) and the
    direction fits take 512 rows."""
    c = dict(name="big", T=2048, L=2, H=4, dk=128, dv=128, kt=T_F16, vt=T_F16, vtrans=0, seed=71, ratio=0.2)
    blob = state_blob(c)
    print(f"[state] general solver T={c['T']} H={c['H']} t={state_t(c)}", flush=True)
    rc, out, sel = run(gpu, "kvc_", c, blob)
    rc_o, out_o, sel_o = run(orc, "orc_", c, blob)
    assert rc == rc_o == 0
    assert np.array_equal(sel, sel_o)
    assert out == out_o, first_diff(out, out_o)
