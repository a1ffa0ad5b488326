"""Parity and invariants at the full sizes of the measured configurations.

* One layer of the headline workload (T = 100,000, 8 KV heads, d = 128,
  SnapKV W = 32, keep 0.2, diversity on): every output equal to the oracle's.
* One layer of the Llama-3-8B-shaped configuration (T = 16,384, its 1,024-key
  tail chunk included) and one of the long-context configuration (T =
  100,000, 4 KV heads, d = 256, bf16 storage, keep 0.5 and 0.2): every
  output equal to the oracle's.
* One layer with the 1M-token configuration's options (Lawson-Hanson beta,
  diversity, one refinement round, R-KV span weights) at T = 100,000 and
  4 KV heads: every output equal to the oracle's.
* The 1M-token configuration itself (10 layers x 4 KV heads x d = 128,
  T = 1,048,576) in one device-resident call, where the oracle would take
  minutes per layer: size-independent invariants (kept count from the chunk
  plan, ascending in-range positions, exact per-chunk counts, finite beta >=
  log(1e-12) and C_v, statistics in range) and the batch's layer 0 equal bit
  for bit to a one-layer call on the same data.
* The Llama-3-8B-shaped configuration as one 32-layer device call (layer 0
  equal to the oracle, layers 15 and 31 equal to one-layer calls) and the
  long-context bf16 configuration as one 10-layer device call (layers 0, 4
  and 9 equal to one-layer calls).
Inputs come from numpy's seeded generator (the data is made here, not read).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from kvc_harness import case_params, kc, load_oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    lib = kc.load_product()
    if not lib.dll.kv_compact_hip_available():
        pytest.fail("no usable GPU for the GPU test tier")
    return lib


@pytest.fixture(scope="module")
def orc():
    return load_oracle()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def layer(T, H, d, seed, W=32):
    r = np.random.default_rng(seed)
    scale = np.exp(r.normal(0.0, 0.5, size=H * d)).astype(np.float32)
    K = (r.standard_normal((T, H * d), dtype=np.float32) * scale).astype(np.float32)
    V = r.standard_normal((T, H * d), dtype=np.float32)
    Q = (K[-W:] + np.float32(0.1) * r.standard_normal((W, H * d), dtype=np.float32)).astype(np.float32)
    return np.ascontiguousarray(K), V, np.ascontiguousarray(Q)


def span(T, seed, frac=0.3):
    r = np.random.default_rng(seed)
    s = int(r.integers(0, T - int(frac * T)))
    return s, s + int(frac * T)


def same(a, b):
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    assert np.array_equal(bits(a.beta), bits(b.beta)), "beta"
    assert np.array_equal(bits(a.C_v), bits(b.C_v)), "C_v"
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k


def test_headline_layer_exact(gpu, orc):
    T, H, d = 100000, 8, 128
    K, V, Q = layer(T, H, d, 7001)
    print("[full] headline layer T=100000 H=8 d=128 diversity", flush=True)
    a = gpu.compact(K, V, Q, T, 32, H, d, d, gpu.params(target_ratio=0.2, use_diversity=1))
    b = orc.compact(K, V, Q, T, 32, H, d, d, orc.params(target_ratio=0.2, use_diversity=1))
    assert a.t == 20000
    same(a, b)


def test_config2_layer_exact(gpu, orc):
    """One layer of the Llama-3-8B-shaped configuration: T = 16,384, 8 KV
    heads, d = 128, SnapKV W = 32, keep 0.2, diversity on; the plan ends in a
    1,024-key tail chunk."""
    T, H, d = 16384, 8, 128
    K, V, Q = layer(T, H, d, 7004)
    print("[full] config-2 layer T=16384 H=8 d=128 diversity", flush=True)
    a = gpu.compact(K, V, Q, T, 32, H, d, d, gpu.params(target_ratio=0.2, use_diversity=1))
    b = orc.compact(K, V, Q, T, 32, H, d, d, orc.params(target_ratio=0.2, use_diversity=1))
    same(a, b)


@pytest.mark.parametrize("ratio", [0.5, 0.2])
def test_config3_layer_exact_bf16(gpu, orc, ratio):
    """One layer of the long-context configuration: T = 100,000, 4 KV heads,
    d = 256, K and V stored as bf16 (fp32 arithmetic), SnapKV W = 32, keep
    0.5 and 0.2 with auto-chunking; the kept K rows and C_v rows come back as
    bf16."""
    T, H, d = 100000, 4, 256
    K, V, Q = layer(T, H, d, 7005)
    print(f"[full] config-3 layer T=100000 H=4 d=256 bf16 ratio={ratio}", flush=True)
    Kb = np.stack([orc.quantize_row(K[i], kc.KV_TYPE_BF16) for i in range(T)])
    Vb = np.stack([orc.quantize_row(V[i], kc.KV_TYPE_BF16) for i in range(T)])
    del K, V
    args = (Kb, Vb, Q, kc.KV_TYPE_BF16, kc.KV_TYPE_BF16, Kb.shape[1], Vb.shape[1], T, 32, H, d, d)
    ra, a = gpu.quantized(*args, gpu.params(target_ratio=ratio))
    rb, b = orc.quantized(*args, orc.params(target_ratio=ratio))
    assert ra == 0 and rb == 0
    same(a, b)
    assert np.array_equal(a.K_out, b.K_out) and np.array_equal(a.V_out, b.V_out)


def c5_params(lib, T, s):
    c = dict(name="c5", T=T, H=4, d=128, seed=0, params=dict(target_ratio=0.2, skip_beta=0, nnls_method=0,
                                                            use_diversity=1, refine_rounds=1))
    p = case_params(lib, c, T)
    cls = kc.CLASSIFIER(lambda pos, _d: kc.KV_TOKEN_THINKING if s[0] <= pos < s[1] else
                        (kc.KV_TOKEN_TRANSITION if pos == s[1] else kc.KV_TOKEN_ANSWER))
    r = kc.Reasoning(cls, None, 0.3, 0.7, 0)
    p.reasoning = ctypes.pointer(r)
    return p, (cls, r)


def test_config5_options_layer_exact(gpu, orc):
    T, H, d = 100000, 4, 128
    K, V, Q = layer(T, H, d, 7002)
    s = span(T, 7002)
    print("[full] 1M-config options on one 100k layer", flush=True)
    pg, keep_g = c5_params(gpu, T, s)
    po, keep_o = c5_params(orc, T, s)
    a = gpu.compact(K, V, Q, T, 32, H, d, d, pg)
    b = orc.compact(K, V, Q, T, 32, H, d, d, po)
    same(a, b)


def test_config5_full_size_invariants(gpu):
    import hiprt
    L, T, H, d, W = 10, 1048576, 4, 128, 32
    E = H * d
    print("[full] 1M-token configuration, 10 layers, device batch", flush=True)
    dll = kc.bind_device_api(gpu.dll)
    p = gpu.params(target_ratio=0.2, skip_beta=0, nnls_method=0, use_diversity=1, refine_rounds=1)
    t, n_chunks = kc.plan(dll, T, W, True, p)
    assert (t, n_chunks) == (819 * 256 + 51, 820)
    r = np.random.default_rng(7003)
    pool = r.standard_normal(T * E + 8192 * E, dtype=np.float32)
    dK, dV, dQ = hiprt.DevBuf(L * T * E * 4), hiprt.DevBuf(L * T * E * 4), hiprt.DevBuf(L * W * E * 4)
    layers = []
    for l in range(L):
        o1, o2 = (int(x) * E for x in r.integers(0, 8192, size=2))
        scale = np.exp(r.normal(0.0, 0.5, size=E)).astype(np.float32)
        K = (pool[o1:o1 + T * E].reshape(T, E) * scale).astype(np.float32)
        V = pool[o2:o2 + T * E].reshape(T, E)
        Q = (K[-W:] + np.float32(0.1) * r.standard_normal((W, E), dtype=np.float32)).astype(np.float32)
        dK.upload(K, l * T * E * 4)
        dV.upload(V, l * T * E * 4)
        dQ.upload(Q, l * W * E * 4)
        del K
    s0, s1 = span(T, 7003)
    wts = np.ones(T, np.float32)
    wts[s0:s1] = 0.3
    wts[s1] = 0.7
    dW = hiprt.DevBuf(T * 4)
    dW.upload(wts)

    def run(nl, k_off, v_off, q_off):
        idx, beta, cv, st = (hiprt.DevBuf(n * 4) for n in (nl * t, nl * H * t, nl * H * t * d, nl * 3))
        out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)
        rc = dll.kvc_compact_layers_device(dK.value + k_off, dV.value + v_off, dQ.value + q_off, nl, T, W, H, d, d,
                                           T * E, T * E, W * E, ctypes.byref(p), dW.value, ctypes.byref(out), None)
        assert rc == 0
        return (idx.download(np.int32, nl * t).reshape(nl, t), beta.download(np.float32, nl * H * t),
                cv.download(np.float32, nl * H * t * d), st.download(np.float32, nl * 3).reshape(nl, 3))

    gi, gb, gc, gs = run(L, 0, 0, 0)
    per_chunk = np.full(n_chunks, 256)
    per_chunk[-1] = 51
    for l in range(L):
        ix = gi[l]
        assert np.all(np.diff(ix) > 0) and ix[0] >= 0 and ix[-1] < T
        assert np.array_equal(np.bincount(ix // 1280, minlength=n_chunks), per_chunk)
        assert 0.0 < gs[l, 0] <= 1.0 + 1e-6 and gs[l, 1] >= 0.0 and 0.0 <= gs[l, 2] <= 1.0
    assert np.all(np.isfinite(gb)) and gb.min() >= np.float32(np.log(np.float32(1e-12))) - 1e-3
    assert np.all(np.isfinite(gc))
    i0, b0, c0, s0_ = run(1, 0, 0, 0)
    assert np.array_equal(i0[0], gi[0])
    assert np.array_equal(bits(b0), bits(gb[:H * t]))
    assert np.array_equal(bits(c0), bits(gc[:H * t * d]))
    assert np.array_equal(bits(s0_[0]), bits(gs[0]))


def device_layers(dll, dK, dV, dQ, nl, T, W, H, d, t, p, k_off=0, v_off=0, q_off=0):
    """kvc_compact_layers_device on nl layers at the given byte offsets; the
    outputs per layer."""
    import hiprt
    E = H * d
    idx, beta, cv, st = (hiprt.DevBuf(n * 4) for n in (nl * t, nl * H * t, nl * H * t * d, nl * 3))
    out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)
    rc = dll.kvc_compact_layers_device(dK.value + k_off, dV.value + v_off, dQ.value + q_off, nl, T, W, H, d, d,
                                       T * E, T * E, W * E, ctypes.byref(p), None, ctypes.byref(out), None)
    assert rc == 0
    return (idx.download(np.int32, nl * t).reshape(nl, t), beta.download(np.float32, nl * H * t).reshape(nl, -1),
            cv.download(np.float32, nl * H * t * d).reshape(nl, -1), st.download(np.float32, nl * 3).reshape(nl, 3))


def test_config2_full_batch(gpu, orc):
    """The Llama-3-8B-shaped configuration as one device call over all 32
    layers (T = 16,384, 8 KV heads, d = 128, SnapKV W = 32, keep 0.2,
    diversity on): layer 0 (the data of test_config2_layer_exact) equal to
    the oracle's outputs, layers 15 and 31 equal bit for bit to one-layer
    calls on the same data, and the chunk plan's counts in every layer."""
    import hiprt
    L, T, H, d, W = 32, 16384, 8, 128, 32
    E = H * d
    print("[full] config-2 batch: 32 layers x T=16384 x 8 heads, diversity", flush=True)
    dll = kc.bind_device_api(gpu.dll)
    p = gpu.params(target_ratio=0.2, use_diversity=1)
    t, n_chunks = kc.plan(dll, T, W, True, p)
    dK, dV, dQ = hiprt.DevBuf(L * T * E * 4), hiprt.DevBuf(L * T * E * 4), hiprt.DevBuf(L * W * E * 4)
    K0, V0, Q0 = layer(T, H, d, 7004)
    dK.upload(K0)
    dV.upload(V0)
    dQ.upload(Q0)
    r = np.random.default_rng(7006)
    pool = r.standard_normal(T * E + 4096 * E, dtype=np.float32)
    for l in range(1, L):
        o1, o2 = (int(x) * E for x in r.integers(0, 4096, size=2))
        scale = np.exp(r.normal(0.0, 0.5, size=E)).astype(np.float32)
        K = (pool[o1:o1 + T * E].reshape(T, E) * scale).astype(np.float32)
        Q = (K[-W:] + np.float32(0.1) * r.standard_normal((W, E), dtype=np.float32)).astype(np.float32)
        dK.upload(K, l * T * E * 4)
        dV.upload(pool[o2:o2 + T * E], l * T * E * 4)
        dQ.upload(Q, l * W * E * 4)
        del K
    gi, gb, gc, gs = device_layers(dll, dK, dV, dQ, L, T, W, H, d, t, p)
    for l in range(L):
        ix = gi[l]
        assert np.all(np.diff(ix) > 0) and ix[0] >= 0 and ix[-1] < T
        assert np.all(np.isfinite(gc[l])) and 0.0 < gs[l, 0] <= 1.0 + 1e-6
    b = orc.compact(K0, V0, Q0, T, W, H, d, d, orc.params(target_ratio=0.2, use_diversity=1))
    assert b.t == t
    assert np.array_equal(gi[0], b.indices), "layer 0 indices"
    assert np.array_equal(bits(gb[0]), bits(np.asarray(b.beta).reshape(-1))), "layer 0 beta"
    assert np.array_equal(bits(gc[0]), bits(np.asarray(b.C_v).reshape(-1))), "layer 0 C_v"
    st = np.array([b.stats["avg_cosine_sim"], b.stats["avg_mse"], b.stats["avg_agreement"]], np.float32)
    assert np.array_equal(bits(gs[0]), bits(st)), "layer 0 stats"
    for l in (15, 31):
        i1, b1, c1, s1 = device_layers(dll, dK, dV, dQ, 1, T, W, H, d, t, p, l * T * E * 4, l * T * E * 4,
                                       l * W * E * 4)
        assert np.array_equal(i1[0], gi[l]), f"layer {l} indices"
        assert np.array_equal(bits(b1[0]), bits(gb[l])), f"layer {l} beta"
        assert np.array_equal(bits(c1[0]), bits(gc[l])), f"layer {l} C_v"
        assert np.array_equal(bits(s1[0]), bits(gs[l])), f"layer {l} stats"


def to_bf16(x):
    """fp32 -> bf16 bits (round to nearest even; the inputs have no NaN)"""
    u = x.view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def test_config3_full_batch_bf16(gpu):
    """The long-context configuration as one device call over all 10 layers
    (T = 100,000, 4 KV heads, d = 256, bf16 K and V, SnapKV W = 32, keep
    0.2): layers 0, 4 and 9 equal bit for bit (indices, beta, C_v, statistics
    and the bf16 output rows) to one-layer calls on the same data; the
    one-layer bf16 path is compared with the oracle in
    test_config3_layer_exact_bf16. Every layer's rows are distinct rotations
    of one bf16 cache with its own queries."""
    import hiprt
    L, T, H, d, W = 10, 100000, 4, 256, 32
    E = H * d
    print("[full] config-3 batch: 10 layers x T=100000 x 4 heads x d=256, bf16", flush=True)
    dll = kc.bind_device_api(gpu.dll)
    p = gpu.params(target_ratio=0.2)
    t, _ = kc.plan(dll, T, W, True, p)
    K, V, _ = layer(T, H, d, 7007)
    Kb, Vb = to_bf16(K), to_bf16(V)
    del K, V
    rb = E * 2
    dKq, dVq, dQ = hiprt.DevBuf(L * T * rb), hiprt.DevBuf(L * T * rb), hiprt.DevBuf(L * W * E * 4)
    r = np.random.default_rng(7008)
    for l in range(L):
        sh = 9973 * l
        Kl = np.ascontiguousarray(np.roll(Kb, sh, axis=0))
        dKq.upload(Kl, l * T * rb)
        dVq.upload(np.ascontiguousarray(np.roll(Vb, 3 * sh, axis=0)), l * T * rb)
        Kf = (Kl[-W:].astype(np.uint32) << np.uint32(16)).view(np.float32)
        Q = (Kf + np.float32(0.1) * r.standard_normal((W, E), dtype=np.float32)).astype(np.float32)
        dQ.upload(np.ascontiguousarray(Q), l * W * E * 4)
    bf = kc.KV_TYPE_BF16

    def run(nl, l0):
        idx, beta, cv, st = (hiprt.DevBuf(n * 4) for n in (nl * t, nl * H * t, nl * H * t * d, nl * 3))
        ko, vo = hiprt.DevBuf(nl * t * rb), hiprt.DevBuf(nl * t * rb)
        out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)
        rc = dll.kvc_compact_quantized_layers_device(dKq.value + l0 * T * rb, dVq.value + l0 * T * rb,
                                                     dQ.value + l0 * W * E * 4, nl, bf, bf, rb, rb, T, W, H, d, d,
                                                     T * rb, T * rb, W * E, ctypes.byref(p), ctypes.byref(out),
                                                     ko.value, vo.value, None)
        assert rc == 0
        return (idx.download(np.int32, nl * t).reshape(nl, t), beta.download(np.float32, nl * H * t).reshape(nl, -1),
                cv.download(np.float32, nl * H * t * d).reshape(nl, -1), st.download(np.float32, nl * 3).reshape(nl, 3),
                ko.download(np.uint8, nl * t * rb).reshape(nl, -1), vo.download(np.uint8, nl * t * rb).reshape(nl, -1))

    full = run(L, 0)
    for l in range(L):
        assert np.all(np.diff(full[0][l]) > 0) and np.all(np.isfinite(full[2][l]))
    for l in (0, 4, 9):
        one = run(1, l)
        for name, a, b in zip(("indices", "beta", "C_v", "stats", "K_out", "V_out"), one, full):
            x, y = a[0], b[l]
            if x.dtype == np.float32:
                x, y = bits(x), bits(y)
            assert np.array_equal(x, y), f"layer {l} {name}"
