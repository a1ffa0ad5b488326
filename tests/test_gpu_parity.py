"""GPU parity: the MI355X library against the CPU oracle, bit for bit.

Every output (kept indices, beta, C_v, the three quality statistics, the
requantized rows) must equal the oracle's exactly: the kernels keep the
reference's fp32 operation order.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from kvc_data import CASES, CASE_BY_NAME, kv_cache, make_case, snapkv_queries
from kvc_harness import kc, load_oracle, run_case

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


def same(a, b):
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    assert np.array_equal(bits(a.beta), bits(b.beta)), "beta"
    ca, cb = bits(a.C_v), bits(b.C_v)
    if not np.array_equal(ca, cb):
        bad = np.argwhere(ca != cb)
        raise AssertionError(f"C_v differs at {len(bad)} of {ca.size}: first {bad[:3].tolist()}")
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k


@pytest.mark.parametrize("name", [c["name"] for c in CASES])
def test_case_parity(gpu, orc, name):
    c = CASE_BY_NAME[name]
    print(f"[case] {name}", flush=True)
    inp = make_case(c)
    same(run_case(gpu, c, inp), run_case(orc, c, inp))


@pytest.mark.parametrize("ratio", [0.25, 0.3, 0.7])
def test_topk_boundary_ties(gpu, orc, ratio):
    """Top-t selection (no diversity) with every key row repeated four times:
    every importance appears four times, so the kept boundary usually splits
    a group of equal importances and the heap selection's tie order decides
    (0.25 keeps whole groups, 0.3 and 0.7 split one)."""
    T, H, d = 1024, 2, 32
    print(f"[case] topk_boundary_ties ratio={ratio}", flush=True)
    K0, _ = kv_cache(T // 4, H, d, 41)
    K = np.ascontiguousarray(np.repeat(K0, 4, axis=0))
    V, _ = kv_cache(T, H, d, 42)
    Q = np.ascontiguousarray(np.repeat(K0[-3:], 4, axis=0))
    p = dict(target_ratio=ratio)
    a = gpu.compact(K, V, Q, T, 12, H, d, d, gpu.params(**p))
    b = orc.compact(K, V, Q, T, 12, H, d, d, orc.params(**p))
    same(a, b)


def test_config1_shape(gpu, orc):
    """Single head, T=4096, d=128, 4 outlier channels x8, cheap Q_ref, 50%."""
    K, V = kv_cache(4096, 1, 128, 101, outliers=4)
    p = dict(target_ratio=0.5, use_cheap_qref=1)
    a = gpu.compact(K, V, None, 4096, 0, 1, 128, 128, gpu.params(**p))
    b = orc.compact(K, V, None, 4096, 0, 1, 128, 128, orc.params(**p))
    same(a, b)


def test_config2_slice(gpu, orc):
    """Llama-3-8B-shaped layer slice: H=8, d=128, T=2560, SnapKV W=32, 20%."""
    K, V = kv_cache(2560, 8, 128, 102, channel_scale=True)
    Q = snapkv_queries(K, 32, 102)
    p = dict(target_ratio=0.2)
    a = gpu.compact(K, V, Q, 2560, 32, 8, 128, 128, gpu.params(**p))
    b = orc.compact(K, V, Q, 2560, 32, 8, 128, 128, orc.params(**p))
    same(a, b)


@pytest.mark.parametrize("kt,vt", [(8, 8), (2, 2), (8, 2), (1, 3), (30, 30)])
def test_quantized_parity(gpu, orc, kt, vt):
    T, H, d = 700, 2, 64
    K, V = kv_cache(T, H, d, 60 + kt + vt)
    Kq = np.stack([orc.quantize_row(K[i], kt) for i in range(T)])
    Vq = np.stack([orc.quantize_row(V[i], vt) for i in range(T)])
    args = (Kq, Vq, None, kt, vt, Kq.shape[1], Vq.shape[1], T, 0, H, d, d)
    ra, a = gpu.quantized(*args, gpu.params(target_ratio=0.2, use_cheap_qref=1))
    rb, b = orc.quantized(*args, orc.params(target_ratio=0.2, use_cheap_qref=1))
    assert ra == 0 and rb == 0
    same(a, b)
    assert np.array_equal(a.K_out, b.K_out)
    assert np.array_equal(a.V_out, b.V_out)


def test_codec_rows(gpu, orc):
    from kvc_data import normal
    for typ in (0, 1, 2, 3, 8, 30):
        for s in range(3):
            x = (normal(300 + s, (256,)) * np.float32(10.0 ** (s - 1))).astype(np.float32)
            ea, eb = gpu.quantize_row(x, typ), orc.quantize_row(x, typ)
            assert np.array_equal(ea, eb), typ
            da, db = gpu.dequantize_row(ea, typ, 256), orc.dequantize_row(eb, typ, 256)
            assert np.array_equal(bits(da), bits(db)), typ


def test_multi_round(gpu, orc):
    c = CASE_BY_NAME["unchunked_r80"]
    K, V, Q, nq = make_case(c)
    ra, a, pa = gpu.multi_round(K, V, Q, c["T"], nq, c["H"], c["d"], c["d"], gpu.params(target_ratio=0.7), 3)
    rb, b, pb = orc.multi_round(K, V, Q, c["T"], nq, c["H"], c["d"], c["d"], orc.params(target_ratio=0.7), 3)
    assert ra == 0 and rb == 0
    same(a, b)
    assert np.array_equal(bits(np.array(pa, np.float32)), bits(np.array(pb, np.float32)))


def test_accel_plugin_scores(gpu, orc):
    """kv_compact_hip_score_all_heads equals the CPU scoring (mat_mul_ABt then scale)."""
    from kvc_data import normal
    nq, T, H, d = 16, 300, 3, 40
    Q = normal(7, (nq, H * d)); K = normal(8, (T, H * d))
    outs = [np.zeros(nq * T, np.float32) for _ in range(H)]
    arr = (ctypes.POINTER(ctypes.c_float) * H)(*[o.ctypes.data_as(ctypes.POINTER(ctypes.c_float)) for o in outs])
    f = gpu.dll.kv_compact_hip_score_all_heads
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                  ctypes.c_int, ctypes.c_float]
    scale = np.float32(1.0) / np.sqrt(np.float32(d))
    assert f(Q.ctypes.data, K.ctypes.data, ctypes.cast(arr, ctypes.c_void_p), nq, T, H, d, float(scale)) == 0
    sc = orc.dll.orc_scores
    sc.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 5 + [ctypes.c_float]
    for h in range(H):
        ref = np.zeros(nq * T, np.float32)
        sc(Q[:, h * d:].ctypes.data, K[:, h * d:].ctypes.data, ref.ctypes.data, nq, T, d, H * d, H * d, float(scale))
        assert np.array_equal(bits(outs[h]), bits(ref)), h


def _accel_fixture():
    from pathlib import Path
    from kvc_data import matmul_inputs
    return np.load(Path(__file__).resolve().parent / "golden" / "matmul.npz"), matmul_inputs()


def test_accel_plugin_mat_mul_ABt_scaled(gpu, orc):
    """kv_compact_hip_mat_mul_ABt_scaled (reference accel.h:24, hip:223-257)
    equals the CPU path's mat_mul_ABt followed by the scale, bit for bit: the
    reference's fixture and the oracle's sequential product."""
    g, ((A, B, scale), _) = _accel_fixture()
    m, k = A.shape
    n = B.shape[0]
    f = gpu.dll.kv_compact_hip_mat_mul_ABt_scaled
    f.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 3 + [ctypes.c_float]
    C = np.full((m, n), np.nan, np.float32)
    assert f(A.ctypes.data, B.ctypes.data, C.ctypes.data, m, n, k, float(np.float32(scale))) == 0
    assert np.array_equal(bits(C), bits(g["abt_C"]))
    # and an unscaled call at another shape against the oracle
    from kvc_data import normal
    A2, B2 = normal(905, (64, 130)), normal(906, (257, 130))
    C2 = np.zeros((64, 257), np.float32)
    assert f(A2.ctypes.data, B2.ctypes.data, C2.ctypes.data, 64, 257, 130, 1.0) == 0
    R2 = np.zeros_like(C2)
    sc = orc.dll.orc_scores
    sc.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 5 + [ctypes.c_float]
    sc(A2.ctypes.data, B2.ctypes.data, R2.ctypes.data, 64, 257, 130, 130, 130, 1.0)
    assert np.array_equal(bits(C2), bits(R2))


def test_accel_plugin_refit_target(gpu, orc):
    """kv_compact_hip_refit_target_all_heads (reference accel.h:50,
    hip:372-462; called by api.cpp:762-775) equals the CPU path's per-head
    mat_mul_AB over V's head slice, bit for bit: the reference's fixture and
    the oracle's sequential product."""
    g, (_, (W, Vall, H, dv)) = _accel_fixture()
    nq, T = W.shape[1], W.shape[2]
    Ws = [np.ascontiguousarray(W[h]) for h in range(H)]
    Ys = [np.full((nq, dv), np.nan, np.float32) for _ in range(H)]
    P = ctypes.POINTER(ctypes.c_float)
    wa = (P * H)(*[w.ctypes.data_as(P) for w in Ws])
    ya = (P * H)(*[y.ctypes.data_as(P) for y in Ys])
    f = gpu.dll.kv_compact_hip_refit_target_all_heads
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int] * 4
    assert f(ctypes.cast(wa, ctypes.c_void_p), Vall.ctypes.data, ctypes.cast(ya, ctypes.c_void_p), nq, T, H, dv) == 0
    mm = orc.dll.orc_mat_mul_AB
    mm.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] * 4
    for h in range(H):
        assert np.array_equal(bits(Ys[h]), bits(g["ab_Y"][h])), h
        R = np.zeros((nq, dv), np.float32)
        mm(Ws[h].ctypes.data, Vall[:, h * dv:].ctypes.data, R.ctypes.data, nq, T, dv, H * dv)
        assert np.array_equal(bits(Ys[h]), bits(R)), h


def test_device_batch_api(gpu, orc):
    """Three layers in one device-resident call equal three oracle calls."""
    import hiprt
    L, T, H, d = 3, 1536, 2, 64
    Ks, Vs, Qs = [], [], []
    for l in range(L):
        K, V = kv_cache(T, H, d, 200 + l, channel_scale=True)
        Ks.append(K); Vs.append(V); Qs.append(snapkv_queries(K, 32, 200 + l))
    dll = kc.bind_device_api(gpu.dll)
    p = gpu.params(target_ratio=0.2)
    t, _ = kc.plan(dll, T, 32, True, p)
    dK, dV, dQ = (hiprt.DevBuf(L * a[0].nbytes) for a in (Ks, Vs, Qs))
    for l in range(L):
        dK.upload(Ks[l], l * Ks[0].nbytes); dV.upload(Vs[l], l * Vs[0].nbytes); dQ.upload(Qs[l], l * Qs[0].nbytes)
    idx, beta, cv, st = (hiprt.DevBuf(n * 4) for n in (L * t, L * H * t, L * H * t * d, L * 3))
    out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)
    rc = dll.kvc_compact_layers_device(dK.value, dV.value, dQ.value, L, T, 32, H, d, d, T * H * d, T * H * d,
                                       32 * H * d, ctypes.byref(p), None, ctypes.byref(out), None)
    assert rc == 0
    gi = idx.download(np.int32, L * t).reshape(L, t)
    gc = cv.download(np.float32, L * H * t * d).reshape(L, H, t, d)
    gs = st.download(np.float32, L * 3).reshape(L, 3)
    for l in range(L):
        b = orc.compact(Ks[l], Vs[l], Qs[l], T, 32, H, d, d, orc.params(target_ratio=0.2))
        assert np.array_equal(gi[l], b.indices)
        assert np.array_equal(bits(gc[l]), bits(b.C_v))
        assert np.float32(gs[l, 0]).view(np.uint32) == np.float32(b.stats["avg_cosine_sim"]).view(np.uint32)


def test_mixed_chunk_sizes(gpu, orc):
    """A shared prefix of 400 makes chunk 0 keep 400 keys (general elimination)
    while the other chunks keep <= 256 (register LU): both solvers in one call."""
    from kvc_harness import case_params
    c = dict(name="mixed_chunks", T=2000, H=2, d=32, seed=40,
             params=dict(target_ratio=0.2, n_shared_prefix=400))
    K, V = kv_cache(2000, 2, 32, 40)
    Q = snapkv_queries(K, 16, 40)
    print("[case] mixed_chunks", flush=True)
    a = gpu.compact(K, V, Q, 2000, 16, 2, 32, 32, case_params(gpu, c, 2000))
    b = orc.compact(K, V, Q, 2000, 16, 2, 32, 32, case_params(orc, c, 2000))
    same(a, b)


@pytest.mark.parametrize("T,H,d,nq", [(1000, 2, 64, 12), (1300, 3, 128, 20)])
def test_stats_partial_query_groups(gpu, orc, T, H, d, nq):
    """The original-attention statistics' sums that run beside the
    factorization (d_v a multiple of 64, T a multiple of 4), with query
    counts that fill only part of a wave's eight sums (12: the second wave
    half used; 20: the third) and a last key tile of 40 or 20 keys; three
    heads leave one of the four statistics heads unused."""
    K, V = kv_cache(T, H, d, 45 + H)
    Q = snapkv_queries(K, nq, 45 + H)
    p = dict(target_ratio=0.2)
    print(f"[case] stats_partial T={T} H={H} d={d} nq={nq}", flush=True)
    a = gpu.compact(K, V, Q, T, nq, H, d, d, gpu.params(**p))
    b = orc.compact(K, V, Q, T, nq, H, d, d, orc.params(**p))
    same(a, b)


def test_config3_bf16_slice(gpu, orc):
    """Long-context shape: 4 KV heads x d=256 with bf16 storage (K/V rows
    rounded to bf16, passed as KV_TYPE_BF16), two 1280-token chunks, keep 0.5
    and 0.2 with SnapKV queries; the compaction runs on the exact fp32
    up-cast, the kept K rows and C_v rows come back as bf16."""
    from kvc_harness import kc as _kc
    T, H, d = 2560, 4, 256
    K, V = kv_cache(T, H, d, 70, channel_scale=True)
    Kb = np.stack([orc.quantize_row(K[i], _kc.KV_TYPE_BF16) for i in range(T)])
    Vb = np.stack([orc.quantize_row(V[i], _kc.KV_TYPE_BF16) for i in range(T)])
    Kf = np.stack([orc.dequantize_row(Kb[i], _kc.KV_TYPE_BF16, H * d) for i in range(T)]).astype(np.float32)
    Q = snapkv_queries(np.ascontiguousarray(Kf), 32, 70)
    for ratio in (0.5, 0.2):
        print(f"[case] config3_bf16 ratio={ratio}", flush=True)
        args = (Kb, Vb, Q, 30, 30, Kb.shape[1], Vb.shape[1], T, 32, H, d, d)
        ra, a = gpu.quantized(*args, gpu.params(target_ratio=ratio))
        rb, b = orc.quantized(*args, orc.params(target_ratio=ratio))
        assert ra == 0 and rb == 0
        same(a, b)
        assert np.array_equal(a.K_out, b.K_out)
        assert np.array_equal(a.V_out, b.V_out)


def test_many_reference_queries(gpu, orc):
    """300 query rows (beyond one LDS row-sum slot per thread of a 256-thread
    block): chunked and unchunked calls equal the oracle."""
    K, V = kv_cache(3000, 2, 64, 81, channel_scale=True)
    Q = snapkv_queries(K, 300, 81)
    for kw in (dict(target_ratio=0.2), dict(target_ratio=0.1, chunk_size=-1, skip_beta=0)):
        print(f"[case] n_q=300 {kw}", flush=True)
        a = gpu.compact(K, V, Q, 3000, 300, 2, 64, 64, gpu.params(**kw))
        b = orc.compact(K, V, Q, 3000, 300, 2, 64, 64, orc.params(**kw))
        same(a, b)
