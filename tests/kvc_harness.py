"""Run catalogue cases through any library exposing the kv-compact ABI."""
from __future__ import annotations

import ctypes
import os
import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(REPO / "kv-compact_amd"))
sys.path.insert(0, str(Path(__file__).resolve().parent))

import kvcompact as kc  # noqa: E402
from kvc_data import make_case, span_classifier_spec  # noqa: E402

ORACLE_SO = REPO / "oracle" / "liboracle.so"
REF_SO = REPO / "oracle" / "_ref" / "libkvref.so"
REF_HARNESS_SO = REPO / "oracle" / "_ref" / "libkvref_harness.so"

_keep = []  # keep ctypes callbacks alive


def make_reasoning(case, T):
    rk = case.get("rkv")
    if not rk:
        return None
    s, e = span_classifier_spec(T, case["seed"])

    def cls(pos, _data):
        if s <= pos < e:
            return kc.KV_TOKEN_THINKING
        if pos == e:
            return kc.KV_TOKEN_TRANSITION
        return kc.KV_TOKEN_ANSWER

    cb = kc.CLASSIFIER(cls)
    r = kc.Reasoning(cb, None, rk["thinking"], rk["transition"], 0)
    _keep.append((cb, r))
    return r


def case_params(lib, case, T, **extra):
    p = lib.params(**case["params"])
    for k, v in extra.items():
        setattr(p, k, v)
    r = make_reasoning(case, T)
    if r is not None:
        p.reasoning = ctypes.pointer(r)
    return p


def run_case(lib, case, inputs=None, **extra):
    K, V, Q, nq = inputs if inputs is not None else make_case(case)
    T, H, d = case["T"], case["H"], case["d"]
    dv = case.get("dv", d)
    p = case_params(lib, case, T, **extra)
    return lib.compact(K, V, Q, T, nq, H, d, dv, p)


def load_oracle():
    return kc.Lib(ORACLE_SO, prefix="orc_")


def load_ref():
    if not REF_SO.exists():
        return None
    return kc.Lib(REF_SO)


def state_case_params(c):
    """(StateParams, keepalive) for a state case dict."""
    return kc.state_params(c["ratio"], c["H"], n_ref=c.get("n_ref", 0), n_pos=c.get("n_pos", 1),
                           sens=c.get("sens", 0), layers=c.get("layers"))


def state_t(c):
    """Kept cells of a state case: max(1, (int)(T * ratio)) in float32."""
    return max(1, int(np.float32(c["T"]) * np.float32(c["ratio"])))


def ref_state_compact(blob: bytes, c):
    """The reference's own parse/build driven by the harness (CLI sequence)."""
    if not REF_HARNESS_SO.exists():
        return None
    dll = ctypes.CDLL(str(REF_HARNESS_SO))
    f = dll.ref_state_compact
    f.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_int, ctypes.c_float, ctypes.c_int,
                  ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_void_p),
                  ctypes.POINTER(ctypes.c_size_t), ctypes.c_void_p]
    f.restype = ctypes.c_int
    dll.ref_free.argtypes = [ctypes.c_void_p]
    b = np.frombuffer(blob, np.uint8)
    layers = c.get("layers")
    la = np.asarray(layers if layers is not None else [0], np.int32)
    out = ctypes.c_void_p()
    n = ctypes.c_size_t(0)
    t = state_t(c)
    sel = np.full(t, -1, np.int32)
    rc = f(b.ctypes.data, b.size, c.get("n_pos", 1), c["H"], c["ratio"], c.get("n_ref", 0), c.get("sens", 0),
           la.ctypes.data, len(layers) if layers is not None else -1, ctypes.byref(out), ctypes.byref(n),
           sel.ctypes.data)
    if rc != 0:
        return rc, None, None
    data = ctypes.string_at(out.value, n.value)
    dll.ref_free(out)
    return 0, data, sel
