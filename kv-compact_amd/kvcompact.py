"""ctypes view of the kv-compact C ABI.

Mirrors the reference's Python binding (python/kv_compact/_bindings.py:28-74):
the same struct field order and C types, so a caller written against the
reference's ``libkv-compact.so`` works unchanged against this library.

``Lib`` wraps any shared object that exports the API, optionally with a
symbol prefix, so the same calling code drives:
  * the MI355X library        libkv-compact.so           (prefix "")
  * the test oracle           oracle/liboracle.so        (prefix "orc_", tests only)
  * the compiled reference    oracle/_ref/libkvref.so    (prefix "", tests only)
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent

KV_TYPE_F32, KV_TYPE_F16, KV_TYPE_Q4_0, KV_TYPE_Q4_1, KV_TYPE_Q8_0 = 0, 1, 2, 3, 8
KV_TYPE_BF16 = 30   # extension: bfloat16 rows (no reference counterpart)
KV_TOKEN_ANSWER, KV_TOKEN_THINKING, KV_TOKEN_TRANSITION = 0, 1, 2
E_UNSUPPORTED, E_DEVICE, E_SCRATCH, E_CAPACITY = -5, -6, -7, -8


class Stats(ctypes.Structure):
    _fields_ = [
        ("avg_cosine_sim", ctypes.c_float),
        ("avg_mse", ctypes.c_float),
        ("avg_agreement", ctypes.c_float),
        ("elapsed_ms", ctypes.c_double),
        ("scoring_ms", ctypes.c_double),
        ("nnls_ms", ctypes.c_double),
    ]


class Result(ctypes.Structure):
    _fields_ = [
        ("t", ctypes.c_int),
        ("n_head_kv", ctypes.c_int),
        ("selected_indices", ctypes.POINTER(ctypes.c_int)),
        ("beta", ctypes.POINTER(ctypes.POINTER(ctypes.c_float))),
        ("C_v", ctypes.POINTER(ctypes.POINTER(ctypes.c_float))),
        ("stats", Stats),
    ]


CLASSIFIER = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_int, ctypes.c_void_p)


class Reasoning(ctypes.Structure):
    _fields_ = [
        ("classifier", CLASSIFIER),
        ("classifier_data", ctypes.c_void_p),
        ("thinking_weight", ctypes.c_float),
        ("transition_weight", ctypes.c_float),
        ("token_offset", ctypes.c_int),
    ]


class Params(ctypes.Structure):
    _fields_ = [
        ("target_ratio", ctypes.c_float),
        ("target_count", ctypes.c_int),
        ("use_sensitivity", ctypes.c_int),
        ("ridge", ctypes.c_float),
        ("nnls_max_iter", ctypes.c_int),
        ("refine_rounds", ctypes.c_int),
        ("use_diversity", ctypes.c_int),
        ("diversity_strength", ctypes.c_float),
        ("n_shared_prefix", ctypes.c_int),
        ("use_cheap_qref", ctypes.c_int),
        ("skip_beta", ctypes.c_int),
        ("score_method", ctypes.c_int),
        ("use_omp", ctypes.c_int),
        ("omp_k_choice", ctypes.c_int),
        ("omp_refit_interval", ctypes.c_int),
        ("nnls_method", ctypes.c_int),
        ("nnls_pgd_iters", ctypes.c_int),
        ("chunk_size", ctypes.c_int),
        ("n_threads", ctypes.c_int),
        ("layer_filter", ctypes.c_void_p),
        ("layer_filter_data", ctypes.c_void_p),
        ("reasoning", ctypes.POINTER(Reasoning)),
    ]


class QuantResult(ctypes.Structure):
    _fields_ = [
        ("base", Result),
        ("k_type", ctypes.c_int),
        ("v_type", ctypes.c_int),
        ("K_out", ctypes.POINTER(ctypes.c_uint8)),
        ("V_out", ctypes.POINTER(ctypes.c_uint8)),
        ("k_row_bytes", ctypes.c_size_t),
        ("v_row_bytes", ctypes.c_size_t),
    ]


API_SYMBOLS = [
    "kv_compact_params_default", "kv_compact", "kv_compact_multi_round",
    "kv_compact_result_free", "kv_compact_quantized", "kv_compact_quant_result_free",
    "kv_dequantize_row", "kv_quantize_row", "kv_quant_row_elements", "kv_quant_row_bytes",
]
ACCEL_SYMBOLS = [
    "kv_compact_hip_available", "kv_compact_hip_mat_mul_ABt_scaled",
    "kv_compact_hip_score_all_heads", "kv_compact_hip_refit_target_all_heads",
    "kv_compact_hip_pool_free",
]

_vp = ctypes.c_void_p
_i = ctypes.c_int


def _ptr(a):
    """Host numpy array, torch tensor (host or device) or None -> void*."""
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return a.data_ptr()  # torch tensor


class Compacted:
    """Host copy of a kv_compact_result."""

    def __init__(self, res: Result, d_v: int):
        t, H = res.t, res.n_head_kv
        self.t = t
        self.n_head_kv = H
        self.indices = np.ctypeslib.as_array(res.selected_indices, (t,)).copy() if t else np.zeros(0, np.int32)
        self.beta = np.stack([np.ctypeslib.as_array(res.beta[h], (t,)).copy() for h in range(H)]) if t else np.zeros((H, 0), np.float32)
        self.C_v = np.stack([np.ctypeslib.as_array(res.C_v[h], (t * d_v,)).copy().reshape(t, d_v) for h in range(H)]) if t else np.zeros((H, 0, d_v), np.float32)
        s = res.stats
        self.stats = dict(avg_cosine_sim=s.avg_cosine_sim, avg_mse=s.avg_mse,
                          avg_agreement=s.avg_agreement, elapsed_ms=s.elapsed_ms,
                          scoring_ms=s.scoring_ms, nnls_ms=s.nnls_ms)


class Lib:
    def __init__(self, path, prefix: str = ""):
        self.path = str(path)
        # RTLD_LOCAL (ctypes' default) keeps same-named symbols of the
        # oracle, the reference and this library apart in one process.
        self.dll = ctypes.CDLL(self.path)
        self.prefix = prefix
        self._bind()

    def sym(self, name):
        if self.prefix and name.startswith("kv_compact_"):
            name = self.prefix + name[len("kv_compact_"):]
        elif self.prefix and name.startswith("kv_"):
            name = self.prefix + name[len("kv_"):]
        return getattr(self.dll, name)

    def _bind(self):
        d = self.prefix
        if d:
            names = dict(params_default=d + "params_default", compact=d + "kv_compact",
                         multi_round=d + "kv_compact_multi_round", result_free=d + "result_free",
                         quantized=d + "kv_compact_quantized", quant_result_free=d + "quant_result_free",
                         quantize_row=d + "quantize_row", dequantize_row=d + "dequantize_row",
                         row_elements=d + "quant_row_elements", row_bytes=d + "quant_row_bytes")
        else:
            names = dict(params_default="kv_compact_params_default", compact="kv_compact",
                         multi_round="kv_compact_multi_round", result_free="kv_compact_result_free",
                         quantized="kv_compact_quantized", quant_result_free="kv_compact_quant_result_free",
                         quantize_row="kv_quantize_row", dequantize_row="kv_dequantize_row",
                         row_elements="kv_quant_row_elements", row_bytes="kv_quant_row_bytes")
        g = lambda n: getattr(self.dll, names[n])
        self._params_default = g("params_default"); self._params_default.restype = Params; self._params_default.argtypes = []
        self._compact = g("compact")
        self._compact.argtypes = [_vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.POINTER(Params), ctypes.POINTER(Result)]
        self._compact.restype = _i
        self._multi = g("multi_round")
        self._multi.argtypes = [_vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.POINTER(Params), _i,
                                ctypes.POINTER(Result), ctypes.POINTER(Stats)]
        self._multi.restype = _i
        self._free = g("result_free"); self._free.argtypes = [ctypes.POINTER(Result)]; self._free.restype = None
        self._quant = g("quantized")
        self._quant.argtypes = [_vp, _vp, _vp, _i, _i, ctypes.c_size_t, ctypes.c_size_t, _i, _i, _i, _i, _i,
                                ctypes.POINTER(Params), ctypes.POINTER(QuantResult)]
        self._quant.restype = _i
        self._qfree = g("quant_result_free"); self._qfree.argtypes = [ctypes.POINTER(QuantResult)]; self._qfree.restype = None
        self._qrow = g("quantize_row"); self._qrow.argtypes = [_vp, _i, _i, _vp]; self._qrow.restype = ctypes.c_size_t
        self._dqrow = g("dequantize_row"); self._dqrow.argtypes = [_vp, _i, ctypes.c_size_t, _vp, _i]; self._dqrow.restype = _i
        self._rel = g("row_elements"); self._rel.argtypes = [_i, ctypes.c_size_t]; self._rel.restype = _i
        self._rb = g("row_bytes"); self._rb.argtypes = [_i, _i]; self._rb.restype = ctypes.c_size_t

    # -- API ------------------------------------------------------------
    def params(self, **kw) -> Params:
        p = self._params_default()
        for k, v in kw.items():
            if k == "reasoning":
                continue
            setattr(p, k, v)
        return p

    def compact_raw(self, K, V, Q, T, n_q, H, d_k, d_v, params=None):
        r = Result()
        rc = self._compact(_ptr(K), _ptr(V), _ptr(Q), T, n_q, H, d_k, d_v,
                           ctypes.byref(params) if params is not None else None, ctypes.byref(r))
        return rc, r

    def free_result(self, r):
        """kv_compact_result_free on a Result from compact_raw."""
        self._free(ctypes.byref(r))

    def compact(self, K, V, Q, T, n_q, H, d_k, d_v, params=None) -> Compacted:
        rc, r = self.compact_raw(K, V, Q, T, n_q, H, d_k, d_v, params)
        if rc != 0:
            self._free(ctypes.byref(r))
            raise RuntimeError(f"{self.path}: kv_compact returned {rc}")
        out = Compacted(r, d_v)
        self._free(ctypes.byref(r))
        return out

    def multi_round(self, K, V, Q, T, n_q, H, d_k, d_v, params, n_rounds):
        r = Result()
        per = (Stats * n_rounds)()
        rc = self._multi(_ptr(K), _ptr(V), _ptr(Q), T, n_q, H, d_k, d_v,
                         ctypes.byref(params) if params is not None else None, n_rounds,
                         ctypes.byref(r), per)
        if rc != 0:
            self._free(ctypes.byref(r))
            return rc, None, None
        out = Compacted(r, d_v)
        self._free(ctypes.byref(r))
        return 0, out, [per[i].avg_cosine_sim for i in range(n_rounds)]

    def quantized(self, Kq, Vq, Q, k_type, v_type, k_rb, v_rb, T, n_q, H, d_k, d_v, params=None):
        r = QuantResult()
        rc = self._quant(_ptr(Kq), _ptr(Vq), _ptr(Q), k_type, v_type, k_rb, v_rb, T, n_q, H, d_k, d_v,
                         ctypes.byref(params) if params is not None else None, ctypes.byref(r))
        if rc != 0:
            self._qfree(ctypes.byref(r))
            return rc, None
        base = Compacted(r.base, d_v)
        t = r.base.t
        base.K_out = np.ctypeslib.as_array(r.K_out, (t * k_rb,)).copy().reshape(t, k_rb) if t else None
        base.V_out = np.ctypeslib.as_array(r.V_out, (t * v_rb,)).copy().reshape(t, v_rb) if t else None
        base.k_row_bytes, base.v_row_bytes = r.k_row_bytes, r.v_row_bytes
        self._qfree(ctypes.byref(r))
        return 0, base

    def quantize_row(self, x: np.ndarray, typ: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        nb = self._rb(typ, x.size)
        out = np.zeros(max(nb, 1), np.uint8)
        n = self._qrow(x.ctypes.data, typ, x.size, out.ctypes.data)
        return out[:n]

    def dequantize_row(self, b: np.ndarray, typ: int, max_el: int) -> np.ndarray:
        b = np.ascontiguousarray(b, np.uint8)
        out = np.zeros(max_el, np.float32)
        n = self._dqrow(b.ctypes.data, typ, b.size, out.ctypes.data, max_el)
        return out[:n]

    def row_elements(self, typ, rb):
        return self._rel(typ, rb)

    def row_bytes(self, typ, n):
        return self._rb(typ, n)


class DeviceOut(ctypes.Structure):
    """kvc_device_out (include/kv-compact-device.h): device result buffers."""
    _fields_ = [
        ("indices", ctypes.c_void_p),
        ("beta", ctypes.c_void_p),
        ("C_v", ctypes.c_void_p),
        ("stats", ctypes.c_void_p),
    ]


def bind_device_api(dll):
    """Declare the additive device-resident entry points of libkv-compact.so."""
    dll.kvc_plan.argtypes = [_i, _i, _i, ctypes.POINTER(Params), ctypes.POINTER(_i), ctypes.POINTER(_i)]
    dll.kvc_plan.restype = _i
    dll.kvc_compact_layers_device.argtypes = [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i,
                                              ctypes.c_longlong, ctypes.c_longlong, ctypes.c_longlong,
                                              ctypes.POINTER(Params), _vp, ctypes.POINTER(DeviceOut), _vp]
    dll.kvc_compact_layers_device.restype = _i
    dll.kvc_compact_layers_device_noalloc.argtypes = dll.kvc_compact_layers_device.argtypes
    dll.kvc_compact_layers_device_noalloc.restype = _i
    dll.kvc_compact_quantized_layers_device.argtypes = [_vp, _vp, _vp, _i, _i, _i, ctypes.c_size_t, ctypes.c_size_t,
                                                        _i, _i, _i, _i, _i, ctypes.c_longlong, ctypes.c_longlong,
                                                        ctypes.c_longlong, ctypes.POINTER(Params),
                                                        ctypes.POINTER(DeviceOut), _vp, _vp, _vp]
    dll.kvc_compact_quantized_layers_device.restype = _i
    dll.kvc_compact_quantized_device.argtypes = [_vp, _vp, _vp, _i, _i, ctypes.c_size_t, ctypes.c_size_t,
                                                 _i, _i, _i, _i, _i, ctypes.POINTER(Params),
                                                 ctypes.POINTER(DeviceOut), _vp, _vp, _vp]
    dll.kvc_compact_quantized_device.restype = _i
    dll.kvc_stage_times.argtypes = [ctypes.POINTER(ctypes.c_float), _i]
    dll.kvc_stage_times.restype = _i
    dll.kv_compact_hip_available.restype = _i
    return dll


def plan(dll, T, n_q, q_given, params):
    t = _i(0)
    nc = _i(0)
    rc = dll.kvc_plan(T, n_q, 1 if q_given else 0, ctypes.byref(params), ctypes.byref(t), ctypes.byref(nc))
    if rc != 0:
        raise RuntimeError(f"kvc_plan returned {rc}")
    return t.value, nc.value


def product_lib_path() -> Path:
    return HERE / "libkv-compact.so"


def load_product() -> "Lib":
    p = Path(os.environ.get("KV_COMPACT_LIB", product_lib_path()))
    if not p.exists():
        raise FileNotFoundError(f"{p} not built: run __graft_entry__.build()")
    return Lib(p)


# -- llama.cpp state blob compaction (include/kvc-state.h) ---------------
LayerFilterFn = ctypes.CFUNCTYPE(_i, _i, _i, _vp)


class StateParams(ctypes.Structure):
    """kvc_state_params (include/kvc-state.h)."""
    _fields_ = [
        ("compact_ratio", ctypes.c_float),
        ("n_ref_queries", ctypes.c_int32),
        ("n_head_kv", ctypes.c_int32),
        ("n_pos_per_embd", ctypes.c_uint32),
        ("sensitivity_budget", ctypes.c_int32),
        ("layer_filter", LayerFilterFn),
        ("layer_filter_data", _vp),
    ]


class StateInfo(ctypes.Structure):
    """kvc_state_info (include/kvc-state.h)."""
    _fields_ = [
        ("n_stream", ctypes.c_uint32),
        ("cell_count", ctypes.c_uint32),
        ("v_trans", ctypes.c_uint32),
        ("n_layer", ctypes.c_uint32),
        ("n_embd_k", ctypes.c_int32),
        ("n_embd_v", ctypes.c_int32),
        ("kv_bytes", ctypes.c_uint64),
        ("trailing_bytes", ctypes.c_uint64),
    ]


def state_params(ratio, n_head_kv, n_ref=0, n_pos=1, sens=0, layers=None):
    """kvc_state_params; layers: explicit list of compacted layers (None: all).
    Returns (params, keepalive) - keep the second alive while the call runs."""
    p = StateParams()
    p.compact_ratio = ratio
    p.n_ref_queries = n_ref
    p.n_head_kv = n_head_kv
    p.n_pos_per_embd = n_pos
    p.sensitivity_budget = sens
    keep = None
    if layers is not None:
        allowed = set(int(x) for x in layers)
        keep = LayerFilterFn(lambda layer, n, data: 1 if layer in allowed else 0)
        p.layer_filter = keep
    return p, keep


def bind_state(dll, prefix):
    """prefix 'kvc_' (the library) or 'orc_' (the oracle): parse_info and compact."""
    info = getattr(dll, prefix + "state_parse_info")
    info.argtypes = [_vp, ctypes.c_size_t, ctypes.c_uint32, ctypes.POINTER(StateInfo)]
    info.restype = _i
    comp = getattr(dll, prefix + "state_compact")
    comp.argtypes = [_vp, ctypes.c_size_t, ctypes.POINTER(StateParams), ctypes.POINTER(_vp),
                     ctypes.POINTER(ctypes.c_size_t), _vp]
    comp.restype = _i
    free = getattr(dll, prefix + "state_free")
    free.argtypes = [_vp]
    free.restype = None
    return info, comp, free


def state_info(dll, prefix, blob: bytes, n_pos=1):
    info, _, _ = bind_state(dll, prefix)
    si = StateInfo()
    b = np.frombuffer(blob, np.uint8)
    rc = info(b.ctypes.data if b.size else None, b.size, n_pos, ctypes.byref(si))
    return rc, si


def state_compact(dll, prefix, blob: bytes, params: StateParams, t_max: int):
    """(rc, out bytes or None, selected int32[t] or None)."""
    _, comp, free = bind_state(dll, prefix)
    b = np.frombuffer(blob, np.uint8)
    out = _vp()
    n = ctypes.c_size_t(0)
    sel = np.full(max(t_max, 1), -1, np.int32)
    rc = comp(b.ctypes.data if b.size else None, b.size, ctypes.byref(params), ctypes.byref(out), ctypes.byref(n),
              sel.ctypes.data)
    if rc != 0:
        return rc, None, None
    data = ctypes.string_at(out.value, n.value) if n.value else b""
    free(out)
    return 0, data, sel
