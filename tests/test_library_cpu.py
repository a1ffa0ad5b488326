"""CPU-side checks of the MI355X library: it loads, exports every symbol the
headers declare, keeps the reference struct ABI, and refuses to run without a
GPU (no CPU fallback)."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import kvcompact as kc

REPO = Path(__file__).resolve().parent.parent
LIB = REPO / "kv-compact_amd" / "libkv-compact.so"


def declared_symbols():
    names = set()
    for h in (REPO / "include").glob("*.h"):
        txt = h.read_text()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        for m in re.finditer(r"^\s*(?:[A-Za-z_][\w\s\*]*?)\b((?:kv|kvc)_\w+)\s*\(", txt, flags=re.M):
            line_start = txt.rfind("\n", 0, m.start()) + 1
            if "static inline" in txt[line_start:m.end()]:
                continue
            names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.skip("library not built")
    return kc.Lib(LIB)


def test_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    decl = declared_symbols()
    assert set(kc.API_SYMBOLS) <= decl and set(kc.ACCEL_SYMBOLS) <= decl
    missing = decl - exported
    assert not missing, missing
    for s in decl:
        getattr(lib.dll, s)


def test_struct_abi_sizes():
    assert ctypes.sizeof(kc.Params) == 104
    assert ctypes.sizeof(kc.Reasoning) == 32
    assert ctypes.sizeof(kc.Stats) == 40
    assert ctypes.sizeof(kc.Result) == 72
    assert ctypes.sizeof(kc.QuantResult) == 112
    assert kc.Params.layer_filter.offset == 80 and kc.Params.reasoning.offset == 96
    assert kc.Result.stats.offset == 32 and kc.QuantResult.K_out.offset == 80


def test_defaults_match_reference(lib):
    p = lib.params()
    assert abs(p.target_ratio - 0.5) < 1e-7 and p.target_count == 0 and p.skip_beta == 1
    assert p.score_method == 1 and p.nnls_method == 1 and p.nnls_pgd_iters == 0
    assert abs(p.ridge - 1e-6) < 1e-12 and p.nnls_max_iter == 200 and abs(p.diversity_strength - 0.5) < 1e-7
    assert p.omp_k_choice == 1 and p.omp_refit_interval == 1 and p.chunk_size == 0 and p.n_threads == 0


def test_argument_errors_without_gpu(lib):
    """Validation precedes device use: the reference's codes come back here too."""
    rc, _ = lib.compact_raw(None, None, None, 0, 0, 0, 0, 0, None)
    assert rc == -1
    x = np.ones(4, np.float32)
    assert lib.compact_raw(x, x, x, 0, 1, 1, 1, 1, None)[0] == -2
    assert lib.compact_raw(x, x, x, 1, 0, 1, 1, 1, None)[0] == -2
    assert lib.row_elements(kc.KV_TYPE_Q8_0, 34 * 4) == 128
    assert lib.row_bytes(kc.KV_TYPE_Q4_0, 128) == 72


def test_no_cpu_fallback_without_gpu(lib):
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    K = np.ones((64, 32), np.float32)
    rc, _ = lib.compact_raw(K, K, None, 64, 0, 1, 32, 32, lib.params(use_cheap_qref=1))
    assert rc == kc.E_DEVICE
    dll = lib.dll
    dll.kv_compact_hip_available.restype = ctypes.c_int
    assert dll.kv_compact_hip_available() == 0
