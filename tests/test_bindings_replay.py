"""The reference wrapper's call sequence (python/kv_compact/_bindings.py:167-255)
replayed by an independent caller (tests/bindings_replay.py) against the
compiled reference (oracle/_ref, CPU tier) and the MI355X library (GPU tier);
both must reproduce the committed fixture tests/golden/bindings_replay.npz,
written from the reference by tests/golden/gen_golden.py."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import bindings_replay as br
from kvc_harness import REF_SO, kc

GOLDEN = Path(__file__).resolve().parent / "golden" / "bindings_replay.npz"


def check(out, g, name):
    idx, cv, ksel, st = out
    assert np.array_equal(idx, g[name + "_indices"])
    assert np.array_equal(cv.view(np.uint32), g[name + "_C_v"].view(np.uint32))
    assert np.array_equal(ksel, g[name + "_K_selected"])
    s = np.array([st["avg_cosine_sim"], st["avg_mse"], st["avg_agreement"]], np.float32)
    assert np.array_equal(s.view(np.uint32), g[name + "_stats"].view(np.uint32))


def run_all(lib):
    g = np.load(GOLDEN)
    for c in br.REPLAY_CASES:
        K, V, Q = br.replay_inputs(c["seed"])
        print(f"[replay] {c['name']}", flush=True)
        check(br.compact(lib, K, V, Q if c["q"] else None, **c["kw"]), g, c["name"])


def test_replay_against_reference():
    if not REF_SO.exists():
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    run_all(br.load(str(REF_SO)))


@pytest.mark.gpu
def test_replay_against_library():
    lib = br.load(str(kc.product_lib_path()))
    run_all(lib)
