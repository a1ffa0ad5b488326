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
