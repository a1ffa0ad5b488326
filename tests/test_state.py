"""llama.cpp state blob compaction: the oracle against the reference.

The oracle's restatement of parsed_kv_state::parse (state.h:104-222), the
CLI's cross-layer selection and refit (kv-compact.cpp:380-690) and
build_compacted_state (state.h:645-810) must write the same bytes as the
reference's own parser and writer driven through oracle/_ref (where that is
built) and as the committed fixtures (tests/golden/state_cases.npz, written
from the reference by tests/golden/gen_golden.py). Cases cover every element
type, transposed V (including the flat-block decode of a block-coded
transposed V), M-RoPE cell extensions, trailing bytes, an explicit layer list
(rejected layers keep their values), sensitivity weighting, extra empty
streams, d_k != d_v and more than 256 reference queries.
"""
from __future__ import annotations

import hashlib
import struct
from pathlib import Path

import numpy as np
import pytest

from kvc_data import STATE_CASES, STATE_CASE_BY_NAME, T_F16, state_blob
from kvc_harness import ORACLE_SO, kc, ref_state_compact, state_case_params, state_t

GOLDEN = Path(__file__).resolve().parent / "golden" / "state_cases.npz"


@pytest.fixture(scope="module")
def orc():
    import ctypes
    return ctypes.CDLL(str(ORACLE_SO))


def run_oracle(orc, c, blob=None):
    blob = state_blob(c) if blob is None else blob
    p, keep = state_case_params(c)
    rc, out, sel = kc.state_compact(orc, "orc_", blob, p, state_t(c))
    del keep
    return rc, out, sel


@pytest.mark.parametrize("name", [c["name"] for c in STATE_CASES])
def test_oracle_state_matches_reference(orc, name):
    c = STATE_CASE_BY_NAME[name]
    blob = state_blob(c)
    r = ref_state_compact(blob, c)
    if r is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    rc_r, out_r, sel_r = r
    rc, out, sel = run_oracle(orc, c, blob)
    assert rc == 0 and rc_r == 0
    assert np.array_equal(sel, sel_r), "kept cells"
    assert len(out) == len(out_r), (len(out), len(out_r))
    if out != out_r:
        a, b = np.frombuffer(out, np.uint8), np.frombuffer(out_r, np.uint8)
        bad = np.nonzero(a != b)[0]
        raise AssertionError(f"{len(bad)} bytes differ, first at {bad[:5].tolist()}")


@pytest.mark.parametrize("name", [c["name"] for c in STATE_CASES])
def test_oracle_state_matches_fixture(orc, name):
    g = np.load(GOLDEN)
    c = STATE_CASE_BY_NAME[name]
    blob = state_blob(c)
    assert hashlib.sha256(blob).hexdigest() == str(g[name + "_input_sha256"]), "input generator drifted"
    rc, out, sel = run_oracle(orc, c, blob)
    assert rc == 0
    assert np.array_equal(sel, g[name + "_sel"])
    assert len(out) == int(g[name + "_size"])
    assert hashlib.sha256(out).hexdigest() == str(g[name + "_sha256"])


def test_state_layout_invariants(orc):
    """Closed-form layout of the compacted blob: header, t cells, per-layer
    sections of t rows, trailing bytes untouched; positions are the kept
    cells' positions in ascending order."""
    c = STATE_CASE_BY_NAME["imrope_q4_trailing"]
    blob = state_blob(c)
    rc, out, sel = run_oracle(orc, c, blob)
    assert rc == 0
    t = state_t(c)
    n_stream, tc = struct.unpack_from("<II", out, 0)
    assert (n_stream, tc) == (1, t)
    off = 8
    pos = []
    for _ in range(t):
        p, ns = struct.unpack_from("<iI", out, off)
        pos.append(p)
        off += 8 + 8 + 4 * ns   # n_pos_per_embd = 4: x, y
    assert pos == sorted(pos) and pos == list(sel)
    vt, nl = struct.unpack_from("<II", out, off)
    assert (vt, nl) == (0, c["L"])
    off += 8
    for _ in range(2 * c["L"]):
        typ, rb = struct.unpack_from("<iQ", out, off)
        off += 12 + t * rb
    assert out[off:] == c["trailing"]


def test_state_parse_info(orc):
    for c in STATE_CASES:
        blob = state_blob(c)
        rc, si = kc.state_info(orc, "orc_", blob, c.get("n_pos", 1))
        assert rc == 0
        assert (si.cell_count, si.n_layer, si.v_trans) == (c["T"], c["L"], c["vtrans"])
        assert (si.n_embd_k, si.n_embd_v) == (c["H"] * c["dk"], c["H"] * c["dv"])
        assert si.trailing_bytes == len(c.get("trailing", b""))
        assert si.kv_bytes + si.trailing_bytes == len(blob)


def test_state_errors(orc):
    c = STATE_CASE_BY_NAME["f16_basic"]
    blob = state_blob(c)
    p, keep = state_case_params(c)
    for cut in (3, 40, len(blob) // 2, len(blob) - len(c.get("trailing", b"")) - 1):
        assert kc.state_compact(orc, "orc_", blob[:cut], p, 64)[0] == -2, cut
    # a second stream holding cells is outside this build's scope
    c2 = dict(c, name="x", n_stream=2, extra_cells=3)
    assert run_oracle(orc, c2)[0] == kc.E_UNSUPPORTED
    # an element type outside F32/F16/Q4_0/Q4_1/Q8_0
    b = bytearray(blob)
    i = bytes(blob).index(struct.pack("<iQ", T_F16, c["H"] * c["dk"] * 2))
    struct.pack_into("<i", b, i, 30)
    assert kc.state_compact(orc, "orc_", bytes(b), p, 64)[0] == kc.E_UNSUPPORTED
    # kept count above the cell count
    p2, k2 = kc.state_params(1.5, c["H"])
    assert kc.state_compact(orc, "orc_", blob, p2, 1024)[0] == -2
    # n_head_kv that does not divide the row width
    p3, k3 = kc.state_params(0.2, 3)
    assert kc.state_compact(orc, "orc_", blob, p3, 64)[0] == -2
    del keep, k2, k3
