"""Pin the CPU oracle: golden fixtures from the compiled reference, the live
reference build where present, and closed-form / brute-force checks that a
plausible slip (dropped term, wrong index, transposed operand) would fail."""
from __future__ import annotations

import ctypes
import hashlib

import numpy as np
import pytest

from kvc_data import (CASES, CASE_BY_NAME, beta_variant, beta_variant_names, diversity_variant,
                      diversity_variant_names, kv_cache, make_case, nonfinite_variant, nonfinite_variant_names,
                      normal, option_variant, option_variant_names, refine_variant, refine_variant_names, uniform)
from kvc_harness import ORACLE_SO, REF_HARNESS_SO, REF_SO, case_params, kc, load_oracle, load_ref, run_case
from pathlib import Path

GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def orc():
    if not ORACLE_SO.exists():
        pytest.skip("oracle not built")
    return load_oracle()


def checksum(*arrs):
    m = hashlib.sha256()
    for a in arrs:
        if a is not None:
            m.update(np.ascontiguousarray(a).tobytes())
    return int.from_bytes(m.digest()[:8], "little")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", [c["name"] for c in CASES])
def test_oracle_matches_reference_fixture(orc, name):
    c = CASE_BY_NAME[name]
    g = np.load(GOLD / f"case_{name}.npz")
    inp = make_case(c)
    assert checksum(*inp[:3]) == int(g["input_checksum"]), "input generator drifted"
    r = run_case(orc, c, inp)
    assert np.array_equal(r.indices, g["indices"])
    assert np.array_equal(bits(r.beta), bits(g["beta"]))
    assert np.array_equal(bits(r.C_v), bits(g["C_v"]))
    st = np.array([r.stats["avg_cosine_sim"], r.stats["avg_mse"], r.stats["avg_agreement"]], np.float32)
    assert np.array_equal(bits(st), bits(g["stats"]))


@pytest.mark.parametrize("qc", ["quant_q8", "quant_q4", "quant_mixed", "quant_f16_q41"])
def test_oracle_quantized_fixture(orc, qc):
    g = np.load(GOLD / f"{qc}.npz")
    Kq, Vq = g["Kq"], g["Vq"]
    typ = {"quant_q8": (8, 8), "quant_q4": (2, 2), "quant_mixed": (8, 2), "quant_f16_q41": (1, 3)}[qc]
    H, d = 2, (32 if qc == "quant_f16_q41" else 64)
    T = Kq.shape[0]
    p = orc.params(target_ratio=0.2, use_cheap_qref=1)
    rc, r = orc.quantized(Kq, Vq, None, typ[0], typ[1], Kq.shape[1], Vq.shape[1], T, 0, H, d, d, p)
    assert rc == 0
    assert np.array_equal(r.indices, g["indices"])
    assert np.array_equal(r.K_out, g["K_out"])
    assert np.array_equal(r.V_out, g["V_out"])
    assert np.array_equal(bits(r.C_v), bits(g["C_v"]))
    # the stored quantized inputs are the reference codec of the generator output
    seed = {"quant_q8": 33, "quant_q4": 34, "quant_mixed": 35, "quant_f16_q41": 36}[qc]
    K, V = kv_cache(T, H, d, seed)
    Kq2 = np.stack([orc.quantize_row(K[i], typ[0]) for i in range(T)])
    assert np.array_equal(Kq2, Kq)


def test_oracle_multi_round_fixture(orc):
    g = np.load(GOLD / "multi_round.npz")
    c = CASE_BY_NAME["unchunked_r80"]
    K, V, Q, nq = make_case(c)
    rc, r, per = orc.multi_round(K, V, Q, c["T"], nq, c["H"], c["d"], c["d"], orc.params(target_ratio=0.7), 3)
    assert rc == 0
    assert np.array_equal(r.indices, g["indices"])
    assert np.array_equal(bits(r.C_v), bits(g["C_v"]))
    assert np.array_equal(bits(np.array(per, np.float32)), bits(g["per_round_cos"]))


def test_oracle_matches_live_reference_where_built(orc):
    ref = load_ref()
    if ref is None:
        pytest.skip("reference not compiled here (oracle/_ref)")
    for name in ("cfg2_small_div", "cfg5_small", "rkv_zero_ties"):
        c = CASE_BY_NAME[name]
        inp = make_case(c)
        a, b = run_case(orc, c, inp), run_case(ref, c, inp)
        assert np.array_equal(a.indices, b.indices)
        assert np.array_equal(bits(a.C_v), bits(b.C_v))


@pytest.mark.parametrize("name", diversity_variant_names())
def test_oracle_diversity_variants_match_live_reference(orc, name):
    """The diversity variants the GPU tests use, oracle vs the compiled reference."""
    ref = load_ref()
    if ref is None:
        pytest.skip("reference not compiled here (oracle/_ref)")
    c, K, V, Q, nq = diversity_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    a = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T))
    b = ref.compact(K, V, Q, T, nq, H, d, d, case_params(ref, c, T))
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices)
    assert np.array_equal(bits(a.C_v), bits(b.C_v))
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k


@pytest.mark.parametrize("name", beta_variant_names())
def test_oracle_beta_variants_match_live_reference(orc, name):
    """The beta-fit variants the GPU tests use, oracle vs the compiled reference."""
    ref = load_ref()
    if ref is None:
        pytest.skip("reference not compiled here (oracle/_ref)")
    c, K, V, Q, nq = beta_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    a = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T))
    b = ref.compact(K, V, Q, T, nq, H, d, d, case_params(ref, c, T))
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices)
    assert np.array_equal(bits(a.beta), bits(b.beta))
    assert np.array_equal(bits(a.C_v), bits(b.C_v))


@pytest.mark.parametrize("name", option_variant_names())
def test_oracle_option_variants_match_live_reference(orc, name):
    """Sensitivity weighting, PGD iterations and OMP selection: oracle vs the compiled reference."""
    ref = load_ref()
    if ref is None:
        pytest.skip("reference not compiled here (oracle/_ref)")
    c, K, V, Q, nq = option_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    a = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T))
    b = ref.compact(K, V, Q, T, nq, H, d, d, case_params(ref, c, T))
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices)
    assert np.array_equal(bits(a.beta), bits(b.beta))
    assert np.array_equal(bits(a.C_v), bits(b.C_v))
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k


@pytest.mark.parametrize("name", refine_variant_names())
def test_oracle_refine_variants_match_live_reference(orc, name):
    """The refinement variants the GPU tests use, oracle vs the compiled
    reference; each variant but the full-keep one changes the kept set."""
    ref = load_ref()
    if ref is None:
        pytest.skip("reference not compiled here (oracle/_ref)")
    c, K, V, Q, nq = refine_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    a = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T))
    b = ref.compact(K, V, Q, T, nq, H, d, d, case_params(ref, c, T))
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices)
    assert np.array_equal(bits(a.beta), bits(b.beta))
    assert np.array_equal(bits(a.C_v), bits(b.C_v))
    z = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T, refine_rounds=0))
    assert (name == "refine_full_keep") == np.array_equal(a.indices, z.indices)


@pytest.mark.parametrize("pgd", [0, 1])
@pytest.mark.parametrize("name", nonfinite_variant_names())
def test_oracle_nonfinite_inputs_match_live_reference(orc, name, pgd):
    """A NaN, inf or -0 in K or V: the oracle follows the compiled reference
    bit for bit, NaN patterns included (zero-beta and clamped-LS beta fits)."""
    ref = load_ref()
    if ref is None:
        pytest.skip("reference not compiled here (oracle/_ref)")
    c, K, V, Q, nq = nonfinite_variant(name)
    T, H, d = c["T"], c["H"], c["d"]
    extra = dict(skip_beta=0, nnls_method=1) if pgd else {}
    a = orc.compact(K, V, Q, T, nq, H, d, d, case_params(orc, c, T, **extra))
    b = ref.compact(K, V, Q, T, nq, H, d, d, case_params(ref, c, T, **extra))
    assert np.array_equal(a.indices, b.indices)
    assert np.array_equal(bits(a.beta), bits(b.beta))
    assert np.array_equal(bits(a.C_v), bits(b.C_v))
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k


# ---------------------------------------------------------------- blocks ---

def _o(name, *types, res=None):
    f = getattr(load_oracle().dll, name)
    f.argtypes = list(types)
    f.restype = res
    return f


fp, ci, cf = ctypes.c_void_p, ctypes.c_int, ctypes.c_float


def test_blocks_ls_nnls_softmax(orc):
    g = np.load(GOLD / "blocks.npz")
    A, B = g["ls_A"], g["ls_B"]
    X = np.zeros((40, 16), np.float32)
    _o("orc_ls_solve", fp, fp, fp, ci, ci, ci, cf)(A.ctypes.data, B.ctypes.data, X.ctypes.data, 24, 40, 16, 1e-6)
    assert np.array_equal(bits(X), bits(g["ls_X"]))
    M, b = g["nnls_M"], g["nnls_b"]
    w = np.zeros(30, np.float32)
    _o("orc_nnls_lh", fp, fp, fp, ci, ci, ci)(M.ctypes.data, b.ctypes.data, w.ctypes.data, 24, 30, 200)
    assert np.array_equal(bits(w), bits(g["nnls_lh_w"]))
    w2 = np.zeros(30, np.float32)
    _o("orc_nnls_clamped", fp, fp, fp, ci, ci, cf)(M.ctypes.data, b.ctypes.data, w2.ctypes.data, 24, 30, 1e-12)
    assert np.array_equal(bits(w2), bits(g["nnls_clamped_w"]))
    S = g["smi_S"]
    f = _o("orc_softmax_importance", fp, fp, fp, fp, fp, ci, ci, ci)
    for agg in (0, 1, 2):
        attn = np.zeros_like(S); imp = np.zeros(300, np.float32)
        f(S.ctypes.data, attn.ctypes.data, imp.ctypes.data, None, None, 16, 300, agg)
        assert np.array_equal(bits(attn), bits(g[f"smi_attn_{agg}"]))
        assert np.array_equal(bits(imp), bits(g[f"smi_imp_{agg}"]))


def test_blocks_codec(orc):
    g = np.load(GOLD / "blocks.npz")
    rows = g["codec_rows"]
    for name, typ in (("q8_0", 8), ("q4_0", 2), ("q4_1", 3), ("f16", 1)):
        enc = np.stack([orc.quantize_row(r, typ) for r in rows])
        assert np.array_equal(enc, g[f"codec_enc_{name}"]), name
        dec = np.stack([orc.dequantize_row(e, typ, 256) for e in enc])
        assert np.array_equal(bits(dec), bits(g[f"codec_dec_{name}"])), name
    f16 = _o("orc_f16_to_f32", ctypes.c_uint16, res=ctypes.c_float)
    allv = np.array([f16(i) for i in range(65536)], np.float32)
    assert np.array_equal(bits(allv), bits(g["f16_to_f32_all"]))
    f32 = _o("orc_f32_to_f16", ctypes.c_float, res=ctypes.c_uint16)
    out = np.array([f32(float(v)) for v in g["f32_to_f16_in"]], np.uint16)
    assert np.array_equal(out, g["f32_to_f16_out"])


# ------------------------------------------------- mathematics-fixed pins ---

def test_f16_decode_matches_ieee(orc):
    """Every finite half decodes to its IEEE value (numpy's float16)."""
    f16 = _o("orc_f16_to_f32", ctypes.c_uint16, res=ctypes.c_float)
    h = np.arange(65536, dtype=np.uint16)
    ieee = h.view(np.float16).astype(np.float32)
    mine = np.array([f16(int(i)) for i in h], np.float32)
    fin = np.isfinite(ieee)
    assert np.array_equal(bits(mine[fin]), bits(ieee[fin]))


def test_f32_to_f16_truncates(orc):
    """Encode truncates toward zero: |decode(encode(x))| <= |x| and within one half-ulp step."""
    f32 = _o("orc_f32_to_f16", ctypes.c_float, res=ctypes.c_uint16)
    x = (normal(77, (3000,)) * np.float32(50.0)).astype(np.float32)
    enc = np.array([f32(float(v)) for v in x], np.uint16).view(np.float16).astype(np.float32)
    assert np.all(np.abs(enc) <= np.abs(x))
    nxt = np.nextafter(np.abs(x).astype(np.float16), np.float16(np.inf)).astype(np.float32)
    assert np.all(np.abs(x) < nxt + 1e-30)


def test_bf16_extension_codec(orc):
    """KV_TYPE_BF16 (an extension, no reference counterpart): decode is the
    exact up-cast (upper 16 bits); encode rounds to nearest, ties to even,
    overflows to inf and keeps NaN a quiet NaN. Checked against known values,
    every one of the 65536 bf16 patterns, and a brute-force nearest search."""
    bf = kc.KV_TYPE_BF16
    assert orc.row_elements(bf, 512) == 256
    # every non-NaN bf16 pattern decodes to its float and re-encodes to itself
    pats = np.arange(65536, dtype=np.uint32)
    f = (pats << 16).view(np.float32)
    keep = ~np.isnan(f)
    enc = orc.quantize_row(f[keep], bf).view(np.uint16)
    assert np.array_equal(enc, pats[keep].astype(np.uint16))
    dec = orc.dequantize_row(pats[keep].astype(np.uint16).view(np.uint8), bf, int(keep.sum()))
    assert np.array_equal(dec.view(np.uint32), (pats[keep] << 16).astype(np.uint32))
    # known answers: ties to even, carries into the exponent, overflow, NaN
    cases = {0x3f808000: 0x3f80, 0x3f818000: 0x3f82, 0x3f808001: 0x3f81, 0x3f7fffff: 0x3f80,
             0x7f7fffff: 0x7f80, 0xff7fffff: 0xff80, 0x00008000: 0x0000, 0x00018000: 0x0002,
             0x7f800001: 0x7fc0, 0xffc00000: 0xffc0, 0x80000000: 0x8000}
    x = np.array(list(cases.keys()), np.uint32).view(np.float32)
    got = orc.quantize_row(x, bf).view(np.uint16)
    assert [int(v) for v in got] == list(cases.values())
    # random floats: the encoded value is a nearest bf16 (brute force over neighbours)
    r = (normal(91, (4000,)) * np.float32(1e3)).astype(np.float32)
    e = orc.quantize_row(r, bf).view(np.uint16).astype(np.uint32)
    dv = (e << 16).view(np.float32).astype(np.float64)
    lo = ((e - 1) << 16).view(np.float32).astype(np.float64)
    hi = ((e + 1) << 16).view(np.float32).astype(np.float64)
    err = np.abs(dv - r)
    assert np.all(err <= np.abs(lo - r)) and np.all(err <= np.abs(hi - r))


def test_codec_roundtrip_bounds(orc):
    """Q8_0 error <= amax/254 + f16 truncation of the scale; Q4_0 <= amax/14 + same
    (reference round-trip bounds, tests/test-kv-compact-math.cpp:1274-1345)."""
    x = normal(55, (64 * 32,))
    for typ, q in ((8, 127.0), (2, 7.0)):
        dec = orc.dequantize_row(orc.quantize_row(x, typ), typ, x.size)
        blk = np.abs(x.reshape(-1, 32)).max(axis=1, keepdims=True)
        err = np.abs(dec.reshape(-1, 32) - x.reshape(-1, 32))
        # half a step of the quantizer plus the scale truncation (rel 2^-10) times q steps
        bound = blk / (2 * q) + blk * (2.0 ** -10) * 1.01 + 1e-7
        if typ == 2:
            bound = blk / 7.0 + blk * (2.0 ** -10) * 9  # one-sided clamp at +7 levels
        assert np.all(err <= bound)


def test_expf_replica_bitexact_sample(orc):
    """The glibc-expf restatement used by the GPU kernels equals libm expf on
    the whole softmax domain; here a 2M-point sample (the exhaustive sweep over
    every float in [-104, 0] is run by the fixture author)."""
    rep = _o("orc_expf_replica", ctypes.c_float, res=ctypes.c_float)
    libm = ctypes.CDLL("libm.so.6").expf
    libm.argtypes = [ctypes.c_float]; libm.restype = ctypes.c_float
    u = splitmix_floats(2000)
    for v in u:
        a, b = rep(float(v)), libm(float(v))
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32), v
    # against the mathematical value: within one ulp
    xs = np.float32(u[:500])
    ex = np.exp(xs.astype(np.float64))
    got = np.array([rep(float(v)) for v in xs], np.float32)
    assert np.all(np.abs(got - ex) <= np.spacing(got.astype(np.float32)) * 1.0 + 1e-45)


def splitmix_floats(n):
    return (uniform(4242, n) * 52.0 - 52.0).astype(np.float32)


def test_softmax_importance_properties(orc):
    S = normal(5, (8, 100)) * np.float32(4.0)
    f = _o("orc_softmax_importance", fp, fp, fp, fp, fp, ci, ci, ci)
    res = {}
    for agg in (0, 1, 2):
        attn = np.zeros_like(S); imp = np.zeros(100, np.float32)
        f(S.ctypes.data, attn.ctypes.data, imp.ctypes.data, None, None, 8, 100, agg)
        res[agg] = (attn, imp)
    attn = res[1][0]
    ref = np.exp(S.astype(np.float64) - S.max(1, keepdims=True)); ref /= ref.sum(1, keepdims=True)
    assert np.allclose(attn, ref, rtol=1e-5, atol=1e-7)
    assert np.allclose(res[0][1], ref.max(0), rtol=1e-5)
    assert np.allclose(res[1][1], np.sqrt((ref ** 2).mean(0)), rtol=1e-5)
    assert np.allclose(res[2][1], ref.mean(0), rtol=1e-5)
    assert np.all(res[1][1] >= res[2][1] * (1 - 1e-6))   # RMS >= mean


def test_ls_exact_solution(orc):
    """Overdetermined, well-conditioned system: GE normal equations reach the
    fp64 least-squares solution (reference math tests 365-418)."""
    A = normal(8, (64, 12)); B = normal(9, (64, 5))
    X = np.zeros((12, 5), np.float32)
    _o("orc_ls_solve", fp, fp, fp, ci, ci, ci, cf)(A.ctypes.data, B.ctypes.data, X.ctypes.data, 64, 12, 5, 0.0)
    ex = np.linalg.lstsq(A.astype(np.float64), B.astype(np.float64), rcond=None)[0]
    assert np.allclose(X, ex, rtol=1e-3, atol=1e-4)


def test_nnls_kkt(orc):
    M = np.abs(normal(10, (20, 15))) + np.float32(0.1)
    b = normal(11, (20,)) + np.float32(2.0)
    w = np.zeros(15, np.float32)
    _o("orc_nnls_lh", fp, fp, fp, ci, ci, ci)(M.ctypes.data, b.ctypes.data, w.ctypes.data, 20, 15, 200)
    Md, bd, wd = M.astype(np.float64), b.astype(np.float64), w.astype(np.float64)
    grad = Md.T @ (Md @ wd - bd)
    assert np.all(w >= 1e-12 * 0.999)
    pos = w > 1e-6
    assert np.all(np.abs(grad[pos]) < 1e-2 * np.abs(Md.T @ bd).max())
    assert np.all(grad[~pos] > -1e-2 * np.abs(Md.T @ bd).max())


def test_topk_bruteforce_and_diversity_zero_strength(orc):
    imp = np.abs(normal(12, (300,)))
    out = np.zeros(40, np.int32)
    _o("orc_select_topk", fp, ci, ci, ci, fp, res=ci)(imp.ctypes.data, 300, 40, 0, out.ctypes.data)
    assert np.array_equal(out, np.sort(np.argsort(-imp, kind="stable")[:40]))
    K = normal(13, (300, 24))
    o2 = np.zeros(40, np.int32); order = np.zeros(40, np.int32)
    f = _o("orc_select_diverse", fp, fp, ci, ci, ci, cf, ci, fp, fp, res=ci)
    f(imp.ctypes.data, K.ctypes.data, 300, 40, 24, 0.0, 0, o2.ctypes.data, order.ctypes.data)
    assert np.array_equal(o2, out)
    assert np.array_equal(order, np.argsort(-imp, kind="stable")[:40])
    # with a penalty, an exact duplicate of the first pick is never chosen next
    K2 = K.copy(); top = int(np.argmax(imp)); nxt = int(np.argsort(-imp)[1])
    K2[nxt] = K2[top]
    f(imp.ctypes.data, K2.ctypes.data, 300, 40, 24, 1.0, 0, o2.ctypes.data, order.ctypes.data)
    assert order[0] == top and nxt not in set(order[:2].tolist())


def test_prefix_forced(orc):
    imp = np.abs(normal(14, (100,)))
    out = np.zeros(20, np.int32)
    _o("orc_select_topk", fp, ci, ci, ci, fp, res=ci)(imp.ctypes.data, 100, 20, 5, out.ctypes.data)
    assert set(range(5)) <= set(out.tolist())
    rest = np.sort(5 + np.argsort(-imp[5:], kind="stable")[:15])
    assert np.array_equal(out[5:], rest)


def test_chunk_plan_pins(orc):
    """Reference exact-count pins (tests/test-kv-compact-api.cpp:62-1119) and
    the configuration arithmetic of api.cpp:396-437."""
    plan = _o("orc_chunk_plan", fp, fp, ci)
    plan.argtypes = [ci, ctypes.POINTER(kc.Params), ctypes.POINTER(ci)]
    plan.restype = ci
    tc = _o("orc_target_count", ci, ctypes.POINTER(kc.Params), res=ci)

    def run(T, **kw):
        p = orc.params(**kw)
        cs = ci(0)
        n = plan(T, ctypes.byref(p), ctypes.byref(cs))
        return n, cs.value, tc(T, ctypes.byref(p))

    assert run(100000, target_ratio=0.2) == (79, 1280, 20000)
    assert run(16384, target_ratio=0.2) == (13, 1280, 3276)
    assert run(100000, target_ratio=0.5) == (196, 512, 50000)
    assert run(1048576, target_ratio=0.2) == (820, 1280, 209715)
    assert run(4096, target_ratio=0.5) == (8, 512, 2048)
    assert run(64, target_ratio=0.5)[2] == 32
    assert run(64, target_count=20)[2] == 20
    assert run(500, target_ratio=0.02)[2] == 10


def test_error_codes(orc):
    rc, _ = orc.compact_raw(None, None, None, 0, 0, 0, 0, 0, None)
    assert rc == -1
    x = np.ones(4, np.float32)
    assert orc.compact_raw(x, x, x, 0, 1, 1, 1, 1, None)[0] == -2
    assert orc.compact_raw(x, x, x, 1, 0, 1, 1, 1, None)[0] == -2


def test_numpy_quantizers_match_oracle(orc):
    """kvc_data.quantize_rows (used to build large Q8_0 / Q4_0 caches) equals the
    oracle's row quantizer byte for byte, zeros, -0 and tiny/huge scales included."""
    from kvc_data import normal, quantize_rows
    for typ in (8, 2):
        for s in range(4):
            x = (normal(500 + s, (48, 256)) * np.float32(10.0 ** (2 * s - 4))).astype(np.float32)
            x[3, :32] = 0.0
            x[5, 40] = -0.0
            x[7, 64:96] = np.float32(1e-30)
            a = quantize_rows(x, typ)
            b = np.stack([orc.quantize_row(x[i], typ) for i in range(x.shape[0])])
            assert np.array_equal(a, b), (typ, s)


def recode_identity_blocks(rows: np.ndarray, typ: int) -> np.ndarray:
    """The GPU's test for Q8_0 / Q4_0 blocks that decode-then-encode returns
    unchanged (k_recode_tile skips such rows): a positive normal f16 scale,
    Q8_0 codes with no -128 and a largest |q| of 127, Q4_0 codes with no 0 and
    a largest |q - 8| of 7. Per block of each row."""
    bb = 34 if typ == 8 else 18
    bl = rows.reshape(rows.shape[0], -1, bb)
    s = bl[..., 0].astype(np.uint32) | (bl[..., 1].astype(np.uint32) << 8)
    ok = (s >= 0x400) & (s <= 0x7BFF)
    c = bl[..., 2:]
    if typ == 8:
        return ok & ~(c == 0x80).any(-1) & ((c == 0x7F) | (c == 0x81)).any(-1)
    n = np.concatenate([c & 0xF, c >> 4], axis=-1)
    return ok & ~(n == 0).any(-1) & ((n == 1) | (n == 15)).any(-1)


@pytest.mark.parametrize("typ", [8, 2])
def test_recode_identity_blocks(orc, typ):
    """Every block that passes the GPU's identity test comes back byte for
    byte from the oracle's decode (state.h:355-375) and encode
    (state.h:528-567); the encoder's own blocks pass it, and blocks that fail
    it are re-encoded to other bytes often enough that the test has teeth.
    Scales cover the normal f16 range to its ends (0x0400, 0x7BFF)."""
    bb, n_el = (34 if typ == 8 else 18), 256
    nbk = n_el // 32
    rng = np.random.default_rng(77 + typ)
    rows = []
    for s in range(6):   # encoder output over many magnitudes
        x = (normal(900 + s, (64, n_el)) * np.float32(10.0 ** (2 * s - 6))).astype(np.float32)
        rows += [orc.quantize_row(x[i], typ) for i in range(x.shape[0])]
    # hand-made blocks: random codes, an extreme code forced in most of them,
    # scales drawn from both ends of the normal range and everywhere else
    ends = np.array([0x0001, 0x03FF, 0x0400, 0x0401, 0x7BFE, 0x7BFF, 0x7C00, 0x8400, 0x0000], np.uint16)
    for _ in range(384):
        bl = rng.integers(0, 256, size=(nbk, bb)).astype(np.uint8)
        sc = np.where(rng.random(nbk) < 0.5, rng.choice(ends, nbk), rng.integers(0x0400, 0x7C00, nbk)).astype(np.uint16)
        bl[:, 0], bl[:, 1] = sc & 0xFF, sc >> 8
        for k in range(nbk):
            if typ == 8:
                q = rng.integers(-127, 128, size=32).astype(np.int8)
                if rng.random() < 0.8:
                    q[rng.integers(32)] = rng.choice([127, -127])
                if rng.random() < 0.1:
                    q[rng.integers(32)] = -128
                bl[k, 2:] = q.view(np.uint8)
            else:
                n = rng.integers(1, 16, size=32).astype(np.uint8)
                if rng.random() < 0.8:
                    n[rng.integers(32)] = rng.choice([1, 15])
                else:
                    n = np.clip(n, 2, 14).astype(np.uint8)
                if rng.random() < 0.1:
                    n[rng.integers(32)] = 0
                bl[k, 2:] = n[0::2] | (n[1::2] << 4)
        rows.append(bl.reshape(-1))
    rows = np.stack(rows)
    ident = recode_identity_blocks(rows, typ)
    back = np.stack([orc.quantize_row(orc.dequantize_row(r, typ, n_el), typ) for r in rows])
    same = (back.reshape(rows.shape[0], nbk, bb) == rows.reshape(rows.shape[0], nbk, bb)).all(-1)
    assert same[ident].all(), "a block that passes the test changed on decode and encode"
    assert ident[128:384].all(), "the encoder's own blocks with normal f16 scales pass the test"
    assert not ident[:64].any(), "(scales of 1e-6 data are f16 subnormals or zero)"
    assert ident[384:].sum() > 500 and (~same[384:]).sum() > 500


def test_round_by_add_and_truncate():
    """The GPU row encoder's roundf: trunc(y + copysign(0.5 - 2^-25, y)) equals
    roundf (floor(|y| + 0.5) with y's sign) on every float with |y| < 2^23,
    exhaustively for y >= 0 and on every negative float below 2^-1 and from
    2^6 to 2^7 (the rounding of the sum is symmetric in the sign)."""
    c = np.float32(0.49999997)
    assert c == np.float32(0.5) - np.float32(2.0 ** -25)
    step = 1 << 24
    for b0 in range(0, 0x4B000000, step):
        y = np.arange(b0, b0 + step, dtype=np.uint32).view(np.float32)
        want = np.floor(y.astype(np.float64) + 0.5).astype(np.float32)
        assert np.array_equal(np.trunc(y + c), want), hex(b0)
    for lo, hi in ((0x80000000, 0xBF000000), (0xC2800000, 0xC3000000)):
        y = np.arange(lo, hi, 4093, dtype=np.uint32).view(np.float32)
        want = -np.floor(-y.astype(np.float64) + 0.5).astype(np.float32)
        got = np.trunc(y + np.copysign(c, y))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), hex(lo)


def test_accel_gemms_match_reference_fixture(orc):
    """The accelerator exports' CPU counterparts: orc_scores (one head) is the
    reference's mat_mul_ABt then the scale, orc_mat_mul_AB over a head's slice
    of V is its extract + mat_mul_AB, bit for bit with the fixture written by
    the compiled reference; and both are within fp32 rounding of an fp64
    product (a transposed operand or a dropped term fails that)."""
    g = np.load(GOLD / "matmul.npz")
    from kvc_data import matmul_inputs
    (A, B, scale), (W, Vall, H, dv) = matmul_inputs()
    assert int(g["in_checksum"]) == checksum(A, B, W, Vall)
    m, k = A.shape
    n = B.shape[0]
    C = np.zeros((m, n), np.float32)
    _o("orc_scores", fp, fp, fp, ci, ci, ci, ci, ci, cf)(A.ctypes.data, B.ctypes.data, C.ctypes.data, m, n, k, k, k,
                                                         float(np.float32(scale)))
    assert np.array_equal(bits(C), bits(g["abt_C"]))
    exact = (A.astype(np.float64) @ B.astype(np.float64).T) * np.float64(np.float32(scale))
    assert np.allclose(C, exact, rtol=0, atol=1e-4 * np.abs(exact).max())
    nq, T = W.shape[1], W.shape[2]
    f = _o("orc_mat_mul_AB", fp, fp, fp, ci, ci, ci, ci)
    for h in range(H):
        Y = np.zeros((nq, dv), np.float32)
        f(np.ascontiguousarray(W[h]).ctypes.data, Vall[:, h * dv:].ctypes.data, Y.ctypes.data, nq, T, dv, H * dv)
        assert np.array_equal(bits(Y), bits(g["ab_Y"][h])), h
        exact = W[h].astype(np.float64) @ Vall[:, h * dv:(h + 1) * dv].astype(np.float64)
        assert np.allclose(Y, exact, rtol=0, atol=1e-4 * np.abs(exact).max()), h
