"""An external Python caller of libkv-compact, written against the C header
only, that drives the library the way the reference's ctypes wrapper does
(python/kv_compact/_bindings.py:167-255):

- the library is found through KV_COMPACT_LIB and loaded with ctypes.CDLL;
- inputs arrive head-major, (heads, tokens, dim), and are laid out as the
  C ABI's token-major [T x heads*dim] (queries likewise);
- parameters are kv_compact_params_default() with eight fields overridden
  (target_ratio, target_count, skip_beta, ridge, use_cheap_qref,
  score_method, chunk_size, n_threads);
- kv_compact() is called with float pointers; the kept indices and C_v are
  copied out element by element through the result's pointers, the kept keys
  are sliced from the head-major input, then kv_compact_result_free().

It declares its own ctypes structures from include/kv-compact-api.h, so an
ABI change in the library (field order, sizes, argument types) breaks it as
it would break the reference's wrapper.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np


class Stats(ctypes.Structure):
    _fields_ = [("avg_cosine_sim", ctypes.c_float), ("avg_mse", ctypes.c_float),
                ("avg_agreement", ctypes.c_float), ("elapsed_ms", ctypes.c_double),
                ("scoring_ms", ctypes.c_double), ("nnls_ms", ctypes.c_double)]


class Result(ctypes.Structure):
    _fields_ = [("t", ctypes.c_int), ("n_head_kv", ctypes.c_int),
                ("selected_indices", ctypes.POINTER(ctypes.c_int)),
                ("beta", ctypes.POINTER(ctypes.POINTER(ctypes.c_float))),
                ("C_v", ctypes.POINTER(ctypes.POINTER(ctypes.c_float))),
                ("stats", Stats)]


class Params(ctypes.Structure):
    _fields_ = [(n, ctypes.c_float if n in ("target_ratio", "ridge", "diversity_strength") else ctypes.c_int)
                for n in ("target_ratio", "target_count", "use_sensitivity", "ridge", "nnls_max_iter",
                          "refine_rounds", "use_diversity", "diversity_strength", "n_shared_prefix",
                          "use_cheap_qref", "skip_beta", "score_method", "use_omp", "omp_k_choice",
                          "omp_refit_interval", "nnls_method", "nnls_pgd_iters", "chunk_size", "n_threads")] + \
        [("layer_filter", ctypes.c_void_p), ("layer_filter_data", ctypes.c_void_p), ("reasoning", ctypes.c_void_p)]


# the wrapper's parameter set (its CompactParams defaults)
WRAPPER_DEFAULTS = dict(target_ratio=0.5, target_count=0, skip_beta=True, ridge=1e-6, use_cheap_qref=False,
                        score_method=1, chunk_size=0, n_threads=0)


def load(path=None):
    lib = ctypes.CDLL(path or os.environ["KV_COMPACT_LIB"])
    lib.kv_compact_params_default.restype = Params
    lib.kv_compact_params_default.argtypes = []
    fp = ctypes.POINTER(ctypes.c_float)
    lib.kv_compact.restype = ctypes.c_int
    lib.kv_compact.argtypes = [fp, fp, fp] + [ctypes.c_int] * 5 + [ctypes.POINTER(Params), ctypes.POINTER(Result)]
    lib.kv_compact_result_free.restype = None
    lib.kv_compact_result_free.argtypes = [ctypes.POINTER(Result)]
    return lib


def compact(lib, K, V, Q, **overrides):
    """K, V: (heads, T, dim); Q: (heads, n_q, dim) or None.
    Returns (indices, C_v (heads, t, d_v), K_selected, stats dict)."""
    prm = dict(WRAPPER_DEFAULTS, **overrides)
    H, T, dk = K.shape
    dv = V.shape[2]
    Kc = np.ascontiguousarray(K.transpose(1, 0, 2).reshape(T, H * dk), dtype=np.float32)
    Vc = np.ascontiguousarray(V.transpose(1, 0, 2).reshape(T, H * dv), dtype=np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    if Q is not None:
        nq = Q.shape[1]
        Qc = np.ascontiguousarray(Q.transpose(1, 0, 2).reshape(nq, H * dk), dtype=np.float32)
        qp = Qc.ctypes.data_as(fp)
    else:
        nq, qp = 0, None
    p = lib.kv_compact_params_default()
    p.target_ratio = prm["target_ratio"]
    p.target_count = prm["target_count"]
    p.skip_beta = 1 if prm["skip_beta"] else 0
    p.ridge = prm["ridge"]
    p.use_cheap_qref = 1 if prm["use_cheap_qref"] else 0
    p.score_method = prm["score_method"]
    p.chunk_size = prm["chunk_size"]
    p.n_threads = prm["n_threads"]
    r = Result()
    rc = lib.kv_compact(Kc.ctypes.data_as(fp), Vc.ctypes.data_as(fp), qp, T, nq, H, dk, dv,
                        ctypes.byref(p), ctypes.byref(r))
    if rc != 0:
        raise RuntimeError(f"kv_compact() returned error code {rc}")
    t = r.t
    idx = np.array([r.selected_indices[i] for i in range(t)], dtype=np.int32)
    cv = np.zeros((H, t, dv), np.float32)
    for h in range(H):
        row = r.C_v[h]
        for i in range(t * dv):
            cv[h, i // dv, i % dv] = row[i]
    ksel = K[:, idx, :]
    st = dict(avg_cosine_sim=r.stats.avg_cosine_sim, avg_mse=r.stats.avg_mse, avg_agreement=r.stats.avg_agreement)
    lib.kv_compact_result_free(ctypes.byref(r))
    return idx, cv, ksel, st


def replay_inputs(seed, H=2, T=700, d=32, nq=16):
    """Head-major inputs from the seeded generator."""
    from kvc_data import normal
    K = normal(seed, (H, T, d))
    V = normal(seed + 1, (H, T, d))
    Q = normal(seed + 2, (H, nq, d))
    return K, V, Q


REPLAY_CASES = [
    dict(name="wrapper_defaults", seed=91, q=True, kw={}),
    dict(name="beta_ridge", seed=92, q=True, kw=dict(skip_beta=False, ridge=1e-4, target_ratio=0.3)),
    dict(name="cheap_mean", seed=93, q=False, kw=dict(use_cheap_qref=True, score_method=2)),
    dict(name="count_chunked", seed=94, q=True, kw=dict(target_count=90, chunk_size=128, n_threads=2)),
]
