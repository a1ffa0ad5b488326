"""GPU parity of the quantized pipeline (dequantize -> compact -> requantize,
reference api.cpp:1182-1257) at the Q8_0 / Q4_0 configuration's shape:
8 KV heads x d = 128, cheap reference queries, keep 0.2, chunked (1280-token
chunks). Every output, the requantized K and V rows included, must equal the
oracle's bit for bit, through the host entry (kv_compact_quantized), the
one-layer device entry and the multi-layer device entry. At the full
configuration (32 layers x T = 32,768) the multi-layer call is checked by
size-independent properties, against a one-layer call on the same data, and
row by row against the reference codec applied to its own outputs.
Inputs are quantized here from seeded N(0,1) data (kvc_data.quantize_rows,
which test_oracle.py pins against the oracle's row quantizer).
"""
from __future__ import annotations

import contextlib
import ctypes
import os

import numpy as np
import pytest

from kvc_data import kv_cache, quantize_rows
from kvc_harness import kc, load_oracle

pytestmark = pytest.mark.gpu

ROW_BYTES = {8: 34, 2: 18}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def gpu():
    lib = kc.load_product()
    if not lib.dll.kv_compact_hip_available():
        pytest.fail("no usable GPU for the GPU test tier")
    kc.bind_device_api(lib.dll)
    return lib


@pytest.fixture(scope="module")
def orc():
    return load_oracle()


def same(a, b):
    assert a.t == b.t
    assert np.array_equal(a.indices, b.indices), "indices"
    assert np.array_equal(bits(a.beta), bits(b.beta)), "beta"
    assert np.array_equal(bits(a.C_v), bits(b.C_v)), "C_v"
    for k in ("avg_cosine_sim", "avg_mse", "avg_agreement"):
        assert np.float32(a.stats[k]).view(np.uint32) == np.float32(b.stats[k]).view(np.uint32), k


def dequant_q(rows, typ):
    """Reference codec decode (state.h:355-375) of Q8_0 / Q4_0 rows, numpy."""
    nb = rows.shape[1] // ROW_BYTES[typ]
    bl = rows.reshape(rows.shape[0], nb, ROW_BYTES[typ])
    d = bl[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    if typ == 8:
        q = bl[:, :, 2:].view(np.int8).astype(np.float32)
    else:
        by = bl[:, :, 2:]
        q = np.empty((rows.shape[0], nb, 32), np.float32)
        q[:, :, 0::2] = (by & 0xF).astype(np.float32) - np.float32(8.0)
        q[:, :, 1::2] = (by >> 4).astype(np.float32) - np.float32(8.0)
    return (d * q).astype(np.float32).reshape(rows.shape[0], -1)


def device_call(gpu, Kq, Vq, kt, vt, L, T, H, d, p):
    """kvc_compact_quantized_layers_device on L layers (Kq/Vq [L][T][row bytes])."""
    import hiprt
    dll = gpu.dll
    t, _ = kc.plan(dll, T, 0, False, p)
    krb, vrb = Kq.shape[-1], Vq.shape[-1]
    dKq, dVq = hiprt.DevBuf(Kq.nbytes), hiprt.DevBuf(Vq.nbytes)
    dKq.upload(Kq)
    dVq.upload(Vq)
    idx, beta, cv, st = (hiprt.DevBuf(n * 4) for n in (L * t, L * H * t, L * H * t * d, L * 3))
    ko, vo = hiprt.DevBuf(L * t * krb), hiprt.DevBuf(L * t * vrb)
    out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)
    if L == 1:
        rc = dll.kvc_compact_quantized_device(dKq.value, dVq.value, None, kt, vt, krb, vrb, T, 0, H, d, d,
                                              ctypes.byref(p), ctypes.byref(out), ko.value, vo.value, None)
    else:
        rc = dll.kvc_compact_quantized_layers_device(dKq.value, dVq.value, None, L, kt, vt, krb, vrb, T, 0, H, d, d,
                                                     T * krb, T * vrb, 0, ctypes.byref(p), ctypes.byref(out),
                                                     ko.value, vo.value, None)
    assert rc == 0
    return dict(t=t, indices=idx.download(np.int32, L * t).reshape(L, t),
                beta=beta.download(np.float32, L * H * t).reshape(L, H, t),
                C_v=cv.download(np.float32, L * H * t * d).reshape(L, H, t, d),
                stats=st.download(np.float32, L * 3).reshape(L, 3),
                K_out=ko.download(np.uint8, L * t * krb).reshape(L, t, krb),
                V_out=vo.download(np.uint8, L * t * vrb).reshape(L, t, vrb))


def same_device(dv, l, ref, H, d):
    t = ref.t
    assert dv["t"] == t
    assert np.array_equal(dv["indices"][l], ref.indices), "indices"
    assert np.array_equal(bits(dv["beta"][l]), bits(np.asarray(ref.beta).reshape(H, t))), "beta"
    assert np.array_equal(bits(dv["C_v"][l]), bits(np.asarray(ref.C_v).reshape(H, t, d))), "C_v"
    st = np.array([ref.stats["avg_cosine_sim"], ref.stats["avg_mse"], ref.stats["avg_agreement"]], np.float32)
    assert np.array_equal(bits(dv["stats"][l]), bits(st)), "stats"
    assert np.array_equal(dv["K_out"][l], ref.K_out), "K_out"
    assert np.array_equal(dv["V_out"][l], ref.V_out), "V_out"


@contextlib.contextmanager
def inplace(flag):
    """KVC_INPLACE=0 sends Q8_0 / Q4_0 caches through the whole-cache decode
    instead of the kernels' in-register decode; both must give the oracle's
    outputs."""
    old = os.environ.get("KVC_INPLACE")
    os.environ["KVC_INPLACE"] = flag
    try:
        yield
    finally:
        if old is None:
            os.environ.pop("KVC_INPLACE", None)
        else:
            os.environ["KVC_INPLACE"] = old


@pytest.mark.parametrize("mode", ["1", "0"])
@pytest.mark.parametrize("kt,vt", [(8, 8), (2, 2), (2, 8)])
def test_config4_chunked(gpu, orc, kt, vt, mode):
    """8 heads x d = 128, T = 2560 (two 1280-token chunks), both device entries and the host entry,
    with K and V decoded in the kernels (mode 1) and by the whole-cache pass (mode 0)."""
    T, H, d = 2560, 8, 128
    print(f"[quant] config-4 shape T={T} k_type={kt} v_type={vt} inplace={mode}", flush=True)
    K, V = kv_cache(T, H, d, 4000 + kt * 10 + vt)
    Kq, Vq = quantize_rows(K, kt), quantize_rows(V, vt)
    pk = dict(target_ratio=0.2, use_cheap_qref=1)
    args = (Kq, Vq, None, kt, vt, Kq.shape[1], Vq.shape[1], T, 0, H, d, d)
    rb, b = orc.quantized(*args, orc.params(**pk))
    with inplace(mode):
        ra, a = gpu.quantized(*args, gpu.params(**pk))
        dv = device_call(gpu, Kq[None], Vq[None], kt, vt, 1, T, H, d, gpu.params(**pk))
    assert ra == 0 and rb == 0
    same(a, b)
    assert np.array_equal(a.K_out, b.K_out) and np.array_equal(a.V_out, b.V_out)
    same_device(dv, 0, b, H, d)


@pytest.mark.parametrize("case", ["given_q_beta", "diversity", "d96"])
def test_quantized_options(gpu, orc, case):
    """In-register decode on the other readers of K and V: provided reference
    queries with the beta fit (scores of a quantized K against fp32 queries),
    the diversity Gram of quantized key rows, and d = 96 (the general refit
    tiles and statistics columns past d_v)."""
    T, H, d = 2560, 8, 128
    kt, vt = 8, 2
    pk = dict(target_ratio=0.2)
    if case == "d96":
        H, d, kt, vt = 4, 96, 2, 8
    K, V = kv_cache(T, H, d, 4300 + len(case))
    Kq, Vq = quantize_rows(K, kt), quantize_rows(V, vt)
    Q, nq = None, 0
    if case == "given_q_beta":
        Kd = dequant_q(Kq, kt)
        Q = np.ascontiguousarray(Kd[-32:] + np.float32(0.1) * np.random.default_rng(43).standard_normal(
            (32, H * d), dtype=np.float32), np.float32)
        nq = 32
        pk.update(skip_beta=0)
    else:
        pk.update(use_cheap_qref=1)
    if case == "diversity":
        pk.update(use_diversity=1, diversity_strength=0.5)
    print(f"[quant] options {case} T={T} H={H} d={d}", flush=True)
    args = (Kq, Vq, Q, kt, vt, Kq.shape[1], Vq.shape[1], T, nq, H, d, d)
    rb, b = orc.quantized(*args, orc.params(**pk))
    ra, a = gpu.quantized(*args, gpu.params(**pk))
    assert ra == 0 and rb == 0
    same(a, b)
    assert np.array_equal(a.K_out, b.K_out) and np.array_equal(a.V_out, b.V_out)


def test_quantized_layers_device(gpu, orc):
    """Three layers (Q4_0 keys, Q8_0 values) in one call: each layer equals the oracle's one-layer result."""
    L, T, H, d, kt, vt = 3, 2560, 8, 128, 2, 8
    print(f"[quant] layers L={L} T={T}", flush=True)
    Kq = np.empty((L, T, H * d // 32 * ROW_BYTES[kt]), np.uint8)
    Vq = np.empty((L, T, H * d // 32 * ROW_BYTES[vt]), np.uint8)
    for l in range(L):
        K, V = kv_cache(T, H, d, 4100 + l)
        Kq[l], Vq[l] = quantize_rows(K, kt), quantize_rows(V, vt)
    pk = dict(target_ratio=0.2, use_cheap_qref=1)
    dv = device_call(gpu, Kq, Vq, kt, vt, L, T, H, d, gpu.params(**pk))
    for l in range(L):
        rb, b = orc.quantized(Kq[l], Vq[l], None, kt, vt, Kq.shape[2], Vq.shape[2], T, 0, H, d, d, orc.params(**pk))
        assert rb == 0
        same_device(dv, l, b, H, d)


@pytest.mark.parametrize("kt", [8, 2])
def test_recode_noncanonical_blocks(gpu, orc, kt):
    """K blocks the encoder never writes, spread over the cache beside ordinary
    ones: negative, zero and subnormal scales; Q8_0 codes of -128 or with a
    largest |q| under 127; Q4_0 codes of 0 or with a largest |q - 8| under 7.
    The kept K rows are decoded and encoded again in place on the GPU, where
    rows whose blocks all come back unchanged are left as they are; every
    output must still equal the oracle's decode and encode (state.h:355-375,
    state.h:528-567) bit for bit."""
    L, T, H, d, vt = 2, 2560, 8, 128, 8
    bb = ROW_BYTES[kt]
    nb = H * d // 32
    rng = np.random.default_rng(4300 + kt)
    Kq = np.empty((L, T, nb * bb), np.uint8)
    Vq = np.empty((L, T, nb * ROW_BYTES[vt]), np.uint8)
    for l in range(L):
        K, V = kv_cache(T, H, d, 4310 + l)
        Kq[l], Vq[l] = quantize_rows(K, kt), quantize_rows(V, vt)
    blk = Kq.reshape(L, T, nb, bb)
    kind = rng.integers(0, 10, size=(L, T, nb))          # 0-4 the odd blocks, 5-9 left as written
    scale = blk[..., 0].astype(np.uint16) | (blk[..., 1].astype(np.uint16) << 8)
    scale = np.where(kind == 0, scale | 0x8000, scale)
    scale = np.where(kind == 1, 0, scale)
    scale = np.where(kind == 2, rng.integers(1, 0x400, size=scale.shape), scale).astype(np.uint16)
    blk[..., 0] = scale & 0xFF
    blk[..., 1] = scale >> 8
    codes = blk[..., 2:]
    pos = rng.integers(0, bb - 2, size=(L, T, nb))
    if kt == 8:
        q = codes.view(np.int8)
        hit = (kind == 3)[..., None] & (np.arange(bb - 2) == pos[..., None])
        q[...] = np.where(hit, np.int8(-128), q)
        q[...] = np.where((kind == 4)[..., None], q >> 1, q)
    else:
        lo, hi = codes & 0xF, codes >> 4
        hit = (kind == 3)[..., None] & (np.arange(bb - 2) == pos[..., None])
        lo = np.where(hit, 0, lo)
        shrink = (kind == 4)[..., None]
        lo = np.where(shrink, 8 + ((lo.astype(np.int16) - 8) >> 1), lo)
        hi = np.where(shrink, 8 + ((hi.astype(np.int16) - 8) >> 1), hi)
        codes[...] = (lo | (hi << 4)).astype(np.uint8)
    print(f"[quant] non-canonical K blocks kt={kt} L={L} T={T}", flush=True)
    pk = dict(target_ratio=0.2, use_cheap_qref=1)
    dv = device_call(gpu, Kq, Vq, kt, vt, L, T, H, d, gpu.params(**pk))
    for l in range(L):
        kept = kind[l][dv["indices"][l]]
        assert all((kept == k).any() for k in range(10)), "every kind of block among the kept rows"
        rb, b = orc.quantized(Kq[l], Vq[l], None, kt, vt, Kq.shape[2], Vq.shape[2], T, 0, H, d, d, orc.params(**pk))
        assert rb == 0
        same_device(dv, l, b, H, d)


@pytest.mark.parametrize("typ", [8, 2])
def test_config4_full_size(gpu, typ):
    """32 layers x 8 heads x d = 128, T = 32,768 in one device call (Q8_0 or Q4_0 keys and values)."""
    L, T, H, d = 32, 32768, 8, 128
    E = H * d
    print(f"[quant] full configuration L={L} T={T} type={typ}", flush=True)
    r = np.random.default_rng(4200 + typ)
    pool = quantize_rows(r.standard_normal((T + 4096, E), dtype=np.float32), typ)
    rb = pool.shape[1]
    Kq = np.empty((L, T, rb), np.uint8)
    Vq = np.empty((L, T, rb), np.uint8)
    for l in range(L):
        o1, o2 = (int(x) for x in r.integers(0, 4096, size=2))
        Kq[l] = pool[o1:o1 + T]
        Vq[l] = pool[o2:o2 + T]
    p = gpu.params(target_ratio=0.2, use_cheap_qref=1)
    dv = device_call(gpu, Kq, Vq, typ, typ, L, T, H, d, p)
    t = dv["t"]
    assert t == 25 * 256 + 153
    per_chunk = np.full(26, 256)
    per_chunk[-1] = 153
    for l in range(L):
        ix = dv["indices"][l]
        assert np.all(np.diff(ix) > 0) and ix[0] >= 0 and ix[-1] < T
        assert np.array_equal(np.bincount(ix // 1280, minlength=26), per_chunk)
        s = dv["stats"][l]
        assert 0.0 < s[0] <= 1.0 + 1e-6 and s[1] >= 0.0 and 0.0 <= s[2] <= 1.0
    assert np.all(dv["beta"] == 0.0) and np.all(np.isfinite(dv["C_v"]))
    # layer 0 alone gives the same outputs
    d1 = device_call(gpu, Kq[:1], Vq[:1], typ, typ, 1, T, H, d, p)
    for k in ("indices", "K_out", "V_out"):
        assert np.array_equal(d1[k][0], dv[k][0]), k
    for k in ("beta", "C_v", "stats"):
        assert np.array_equal(bits(d1[k][0]), bits(dv[k][0])), k
    # requantized rows: the reference codec of the kept dequantized K rows and
    # of the refitted value rows (sampled rows of two layers)
    for l in (0, L - 1):
        j = np.unique(r.integers(0, t, size=64))
        kept = dequant_q(Kq[l][dv["indices"][l][j]], typ)
        assert np.array_equal(quantize_rows(kept, typ), dv["K_out"][l][j])
        vrows = dv["C_v"][l][:, j, :].transpose(1, 0, 2).reshape(len(j), E)
        assert np.array_equal(quantize_rows(vrows, typ), dv["V_out"][l][j])


def test_quantized_odd_layout(gpu, orc):
    """Odd layer strides and odd output addresses (caller layouts the 2-byte
    codec accesses cannot take): K and V go through the byte-wise decode and
    the kept rows through the byte-wise encode; outputs equal the oracle's."""
    import hiprt
    L, T, H, d, kt, vt = 2, 1536, 4, 64, 8, 2
    print(f"[quant] odd layout L={L} T={T} H={H} d={d}", flush=True)
    krb, vrb = H * d // 32 * ROW_BYTES[kt], H * d // 32 * ROW_BYTES[vt]
    lsk, lsv = T * krb + 1, T * vrb + 3
    Kq = np.zeros(L * lsk, np.uint8)
    Vq = np.zeros(L * lsv, np.uint8)
    per = []
    for l in range(L):
        K, V = kv_cache(T, H, d, 4400 + l)
        kq, vq = quantize_rows(K, kt), quantize_rows(V, vt)
        Kq[l * lsk:l * lsk + T * krb] = kq.reshape(-1)
        Vq[l * lsv:l * lsv + T * vrb] = vq.reshape(-1)
        per.append((kq, vq))
    p = gpu.params(target_ratio=0.2, use_cheap_qref=1)
    dll = gpu.dll
    t, _ = kc.plan(dll, T, 0, False, p)
    dKq, dVq = hiprt.DevBuf(Kq.nbytes), hiprt.DevBuf(Vq.nbytes)
    dKq.upload(Kq)
    dVq.upload(Vq)
    idx, beta, cv, st = (hiprt.DevBuf(n * 4) for n in (L * t, L * H * t, L * H * t * d, L * 3))
    ko, vo = hiprt.DevBuf(L * t * krb + 16), hiprt.DevBuf(L * t * vrb + 16)
    out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)
    rc = dll.kvc_compact_quantized_layers_device(dKq.value, dVq.value, None, L, kt, vt, krb, vrb, T, 0, H, d, d,
                                                 lsk, lsv, 0, ctypes.byref(p), ctypes.byref(out),
                                                 ko.value + 1, vo.value + 3, None)
    assert rc == 0
    dv = dict(t=t, indices=idx.download(np.int32, L * t).reshape(L, t),
              beta=beta.download(np.float32, L * H * t).reshape(L, H, t),
              C_v=cv.download(np.float32, L * H * t * d).reshape(L, H, t, d),
              stats=st.download(np.float32, L * 3).reshape(L, 3),
              K_out=ko.download(np.uint8, L * t * krb + 16)[1:1 + L * t * krb].reshape(L, t, krb),
              V_out=vo.download(np.uint8, L * t * vrb + 16)[3:3 + L * t * vrb].reshape(L, t, vrb))
    for l in range(L):
        kq, vq = per[l]
        rb, b = orc.quantized(kq, vq, None, kt, vt, krb, vrb, T, 0, H, d, d, orc.params(target_ratio=0.2,
                                                                                     use_cheap_qref=1))
        assert rb == 0
        same_device(dv, l, b, H, d)
