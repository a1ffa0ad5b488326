"""Deterministic synthetic KV caches for fixtures and parity tests.

Integer-only SplitMix64 stream -> uniforms with 24-bit mantissas -> an
Irwin-Hall sum of four (approximately normal). Every step is exact IEEE
arithmetic, so the same seed yields the same float32 bytes on any machine,
which lets the golden fixtures store outputs only and regenerate inputs.
"""
from __future__ import annotations

import numpy as np

_M = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(seed: int, n: int) -> np.ndarray:
    """Uniform in [-1, 1) with 24-bit resolution (exact float32 values)."""
    z = splitmix64(seed, n) >> np.uint64(40)          # 24 bits
    return (z.astype(np.float64) - 8388608.0) / 8388608.0


def normal(seed: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    u = uniform(seed, 4 * n).reshape(4, n)
    s = ((u[0] + u[1]) + u[2]) + u[3]                # exact in float64
    return (s * 0.8660254037844386).astype(np.float32).reshape(shape)


# Inputs of the accelerator GEMM fixtures (tests/golden/matmul.npz): the
# reference's scores product mat_mul_ABt then the scale, and its refit target
# mat_mul_AB over each head's slice of V. Shapes no tile divides.
MATMUL_ABT = (37, 301, 72, 0.117851130)        # m, n, k, scale
MATMUL_AB = (29, 333, 3, 40)                    # n_q, T, H, d_v


def matmul_inputs():
    """((A, B, scale), (W [H][n_q][T], V_all [T][H*d_v], H, d_v))."""
    m, n, k, scale = MATMUL_ABT
    A = normal(901, (m, k)); B = normal(902, (n, k))
    nq, T, H, dv = MATMUL_AB
    W = np.abs(normal(903, (H, nq, T))).astype(np.float32)
    Vall = normal(904, (T, H * dv))
    return (A, B, scale), (W, Vall, H, dv)


def kv_cache(T: int, H: int, d: int, seed: int, outliers: int = 0, channel_scale: bool = False):
    """K, V [T x H*d] float32. outliers: that many key/value channels x8.
    channel_scale: per-channel key scale in [0.25, 4) (log-uniform-like)."""
    K = normal(seed * 7 + 1, (T, H * d))
    V = normal(seed * 7 + 2, (T, H * d))
    if channel_scale:
        u = uniform(seed * 7 + 3, H * d)
        scale = np.exp2(np.round(u * 8.0) / 4.0).astype(np.float32)   # 2^(k/4), k in [-8, 8]
        K = (K * scale).astype(np.float32)
    if outliers:
        ch = (splitmix64(seed * 7 + 4, outliers) % np.uint64(H * d)).astype(np.int64)
        K[:, ch] *= np.float32(8.0)
        V[:, ch] *= np.float32(8.0)
    return np.ascontiguousarray(K), np.ascontiguousarray(V)


def snapkv_queries(K: np.ndarray, W: int, seed: int, noise: float = 0.1) -> np.ndarray:
    """SnapKV window: the last W key rows plus N(0, noise^2) noise."""
    Q = K[-W:].astype(np.float32) + (normal(seed * 7 + 5, (W, K.shape[1])) * np.float32(noise))
    return np.ascontiguousarray(Q.astype(np.float32))


def gen_data(n: int, seed: int) -> np.ndarray:
    """Smooth deterministic pattern in the spirit of the reference tests'
    sin/cos generator (tests/test-kv-compact-api.cpp:16-21), built from
    integer arithmetic only."""
    i = np.arange(n, dtype=np.int64)
    a = ((i * 7 + seed) % 97).astype(np.float64) / 48.0 - 1.0
    b = ((i * 3 + seed + 17) % 61).astype(np.float64) / 30.0 - 1.0
    return (a + 0.3 * b).astype(np.float32)


# --------------------------------------------------------------------------
# Case catalogue shared by the fixture generator, the oracle tests and the
# GPU parity tests. Each case: shape, data recipe and parameter overrides.
# --------------------------------------------------------------------------

def make_case(c: dict):
    """Return (K, V, Q or None, n_q) for a case dict."""
    T, H, d = c["T"], c["H"], c["d"]
    dv = c.get("dv", d)
    if c.get("data") == "pattern":
        K = gen_data(T * H * d, c["seed"]).reshape(T, H * d)
        V = gen_data(T * H * dv, c["seed"] + 500).reshape(T, H * dv)
        nq = c.get("n_q", 0)
        Q = gen_data(nq * H * d, c["seed"] + 900).reshape(nq, H * d) if nq else None
        return np.ascontiguousarray(K), np.ascontiguousarray(V), Q, nq
    K, V = kv_cache(T, H, d, c["seed"], outliers=c.get("outliers", 0),
                    channel_scale=c.get("channel_scale", False))
    if dv != d:
        V = normal(c["seed"] * 7 + 9, (T, H * dv))
    q = c.get("qref", "cheap")
    if q == "snapkv":
        Q = snapkv_queries(K, c.get("W", 32), c["seed"])
        return K, V, Q, Q.shape[0]
    if q == "random":
        nq = c["n_q"]
        return K, V, normal(c["seed"] * 7 + 6, (nq, H * d)), nq
    return K, V, None, 0


def span_classifier_spec(T: int, seed: int, frac: float = 0.3):
    """Contiguous THINKING span [s, s + frac*T), ANSWER elsewhere."""
    L = int(frac * T)
    s = int(splitmix64(seed * 7 + 8, 1)[0] % np.uint64(max(T - L, 1)))
    return s, s + L


CASES = [
    # name, shape, data, params
    dict(name="cfg1_small", T=1024, H=1, d=64, seed=1, outliers=4, qref="cheap",
         params=dict(target_ratio=0.5, use_cheap_qref=1)),
    dict(name="cfg1_shape", T=4096, H=1, d=128, seed=2, outliers=4, qref="cheap",
         params=dict(target_ratio=0.5, use_cheap_qref=1)),
    dict(name="cfg2_small_div", T=1536, H=2, d=64, seed=3, channel_scale=True, qref="snapkv",
         params=dict(target_ratio=0.2, use_diversity=1)),
    dict(name="cfg2_small_nodiv", T=1536, H=2, d=64, seed=4, channel_scale=True, qref="snapkv",
         params=dict(target_ratio=0.2)),
    dict(name="unchunked_r20", T=128, H=4, d=32, seed=5, qref="random", n_q=64,
         params=dict(target_ratio=0.2)),
    dict(name="unchunked_r80", T=128, H=4, d=32, seed=5, qref="random", n_q=64,
         params=dict(target_ratio=0.8)),
    dict(name="pattern_basic", T=64, H=4, d=32, seed=1, data="pattern", n_q=32,
         params=dict(target_ratio=0.5)),
    dict(name="score_max", T=256, H=2, d=32, seed=6, qref="random", n_q=16,
         params=dict(target_ratio=0.25, score_method=0)),
    dict(name="score_mean", T=256, H=2, d=32, seed=6, qref="random", n_q=16,
         params=dict(target_ratio=0.25, score_method=2)),
    dict(name="prefix", T=200, H=2, d=16, seed=7, qref="random", n_q=8,
         params=dict(target_ratio=0.3, n_shared_prefix=10)),
    dict(name="prefix_div", T=200, H=2, d=16, seed=7, qref="random", n_q=8,
         params=dict(target_ratio=0.3, n_shared_prefix=10, use_diversity=1)),
    dict(name="count", T=300, H=2, d=16, seed=8, qref="random", n_q=16,
         params=dict(target_count=40)),
    dict(name="count_all", T=48, H=2, d=8, seed=9, qref="random", n_q=8,
         params=dict(target_count=48)),
    dict(name="beta_clamped", T=160, H=2, d=16, seed=10, qref="random", n_q=24,
         params=dict(target_ratio=0.25, skip_beta=0, nnls_method=1)),
    dict(name="beta_lh", T=160, H=2, d=16, seed=10, qref="random", n_q=24,
         params=dict(target_ratio=0.25, skip_beta=0, nnls_method=0)),
    dict(name="refine1", T=160, H=2, d=16, seed=11, qref="random", n_q=24,
         params=dict(target_ratio=0.25, refine_rounds=1)),
    dict(name="refine2_beta", T=160, H=2, d=16, seed=11, qref="random", n_q=24,
         params=dict(target_ratio=0.25, refine_rounds=2, skip_beta=0, nnls_method=0)),
    dict(name="chunk_explicit", T=500, H=2, d=16, seed=12, qref="random", n_q=16,
         params=dict(target_ratio=0.5, chunk_size=200)),
    dict(name="chunk_prefix_cheap", T=700, H=2, d=16, seed=13, qref="cheap",
         params=dict(target_ratio=0.5, chunk_size=256, n_shared_prefix=20, use_cheap_qref=1)),
    dict(name="rkv_span", T=640, H=2, d=32, seed=14, qref="snapkv", W=16,
         rkv=dict(thinking=0.3, transition=0.7),
         params=dict(target_ratio=0.5, chunk_size=256)),
    dict(name="rkv_zero_ties", T=256, H=2, d=16, seed=15, qref="random", n_q=16,
         rkv=dict(thinking=0.0, transition=0.0),
         params=dict(target_ratio=0.8)),
    dict(name="cfg5_small", T=2560, H=2, d=32, seed=16, channel_scale=True, qref="snapkv",
         rkv=dict(thinking=0.3, transition=0.7),
         params=dict(target_ratio=0.2, skip_beta=0, nnls_method=0, use_diversity=1, refine_rounds=1)),
    dict(name="tiny_T1", T=1, H=1, d=4, seed=17, qref="random", n_q=2, params=dict()),
    dict(name="tiny_T3", T=3, H=2, d=4, seed=18, qref="random", n_q=2, params=dict(target_ratio=0.9)),
    dict(name="dv_ne_dk", T=96, H=2, d=16, dv=24, seed=19, qref="random", n_q=8,
         params=dict(target_ratio=0.5)),
    dict(name="unchunked_big_t", T=700, H=1, d=32, seed=20, qref="random", n_q=16,
         params=dict(target_ratio=0.5, chunk_size=-1)),
    # t = 600: the general elimination's panels narrower than 32 columns
    dict(name="unchunked_t600", T=1200, H=2, d=16, seed=21, qref="random", n_q=24,
         params=dict(target_ratio=0.5, chunk_size=-1)),
    # t = 600, d_v = 128: the general elimination's back substitution in three
    # passes of right-hand-side columns (43, 43, 42)
    dict(name="unchunked_t600_d128", T=1200, H=1, d=128, seed=22, qref="random", n_q=24,
         params=dict(target_ratio=0.5, chunk_size=-1)),
]

CASE_BY_NAME = {c["name"]: c for c in CASES}


# --------------------------------------------------------------------------
# Diversity-selection variants (api.cpp:175-233): shapes and data that push
# the GPU's candidate pruning through each of its levels.
# --------------------------------------------------------------------------

def diversity_variant_names():
    return (["llama_chunk"] + [f"strength_{s}" for s in (0.0, 0.2, 0.8, 0.999, 1.0, 1.7, -0.5)] +
            ["near_dup", "dup_rows", "rkv_negative", "rkv_span_div"] +
            [f"prefix_{p}" for p in (100, 256, 400)] + ["cheap_unchunked"])


def diversity_variant(name: str):
    """Return (case, K, V, Q or None, n_q) for a diversity variant."""
    if name == "llama_chunk":   # H=8, d=128: 1024-wide key rows, chunks of 1280 keeping 256
        c = dict(name=name, T=4096, H=8, d=128, seed=31, params=dict(target_ratio=0.2, use_diversity=1))
        K, V = kv_cache(4096, 8, 128, 31, channel_scale=True)
        return c, K, V, snapkv_queries(K, 32, 31), 32
    if name.startswith("strength_"):   # s >= 1 and s < 0 disable pruning
        s = float(name.split("_", 1)[1])
        c = dict(name=name, T=1536, H=2, d=64, seed=32,
                 params=dict(target_ratio=0.2, use_diversity=1, diversity_strength=s))
        K, V = kv_cache(1536, 2, 64, 32, channel_scale=True)
        return c, K, V, snapkv_queries(K, 32, 32), 32
    if name == "near_dup":   # one shared row + 1% noise: cosines near 1
        T, H, d = 1280, 2, 64
        base = normal(3301, (1, H * d))
        K = np.ascontiguousarray((base + np.float32(0.01) * normal(3302, (T, H * d))).astype(np.float32))
        V = normal(3303, (T, H * d))
        Q = np.ascontiguousarray((K[-16:] + np.float32(0.5) * normal(3304, (16, H * d))).astype(np.float32))
        c = dict(name=name, T=T, H=H, d=d, seed=33, params=dict(target_ratio=0.2, use_diversity=1))
        return c, K, V, Q, 16
    if name == "dup_rows":   # every key row four times: importance and cosine ties
        T, H, d = 1024, 2, 32
        K0, _ = kv_cache(T // 4, H, d, 34)
        K = np.ascontiguousarray(np.repeat(K0, 4, axis=0))
        V, _ = kv_cache(T, H, d, 35)
        c = dict(name=name, T=T, H=H, d=d, seed=34, params=dict(target_ratio=0.25, use_diversity=1))
        return c, K, V, normal(3401, (12, H * d)), 12
    if name in ("rkv_negative", "rkv_span_div"):   # negative weights disable pruning
        w = -0.5 if name == "rkv_negative" else 0.3
        seed = 36 if name == "rkv_negative" else 37
        c = dict(name=name, T=2560, H=2, d=32, seed=seed, rkv=dict(thinking=w, transition=0.7),
                 params=dict(target_ratio=0.2, use_diversity=1))
        K, V = kv_cache(2560, 2, 32, seed, channel_scale=True)
        return c, K, V, snapkv_queries(K, 16, seed), 16
    if name.startswith("prefix_"):   # prefix below, at and above chunk 0's kept count
        p = int(name.split("_", 1)[1])
        c = dict(name=name, T=2000, H=2, d=32, seed=38,
                 params=dict(target_ratio=0.2, use_diversity=1, n_shared_prefix=p))
        K, V = kv_cache(2000, 2, 32, 38)
        return c, K, V, snapkv_queries(K, 16, 38), 16
    if name == "cheap_unchunked":
        c = dict(name=name, T=900, H=2, d=32, seed=39,
                 params=dict(target_ratio=0.3, use_diversity=1, use_cheap_qref=1, chunk_size=-1))
        K, V = kv_cache(900, 2, 32, 39)
        return c, K, V, None, 0
    raise KeyError(name)


# --------------------------------------------------------------------------
# Beta-fit variants (api.cpp:812-831): clamped LS (nnls_method 1) and
# Lawson-Hanson (nnls_method 0) at chunked shapes.
# --------------------------------------------------------------------------

def beta_variant_names():
    return ["pgd_chunk", "lh_chunk", "lh_div_rkv", "lh_cheap", "pgd_unchunked_big_t", "lh_unchunked_big_t",
            "lh_iter_cap"]


def beta_variant(name: str):
    """Return (case, K, V, Q or None, n_q)."""
    if name in ("pgd_chunk", "lh_chunk", "lh_iter_cap"):
        m = 1 if name == "pgd_chunk" else 0
        extra = dict(nnls_max_iter=3) if name == "lh_iter_cap" else {}
        c = dict(name=name, T=2560, H=2, d=64, seed=41,
                 params=dict(target_ratio=0.2, skip_beta=0, nnls_method=m, **extra))
        K, V = kv_cache(2560, 2, 64, 41, channel_scale=True)
        return c, K, V, snapkv_queries(K, 32, 41), 32
    if name == "lh_div_rkv":   # the 1M-token configuration's options, without refinement
        c = dict(name=name, T=2560, H=4, d=32, seed=42, rkv=dict(thinking=0.3, transition=0.7),
                 params=dict(target_ratio=0.2, skip_beta=0, nnls_method=0, use_diversity=1))
        K, V = kv_cache(2560, 4, 32, 42, channel_scale=True)
        return c, K, V, snapkv_queries(K, 32, 42), 32
    if name == "lh_cheap":   # 64 cheap queries per chunk
        c = dict(name=name, T=3000, H=2, d=32, seed=43,
                 params=dict(target_ratio=0.2, skip_beta=0, nnls_method=0, use_cheap_qref=1))
        K, V = kv_cache(3000, 2, 32, 43)
        return c, K, V, None, 0
    if name in ("pgd_unchunked_big_t", "lh_unchunked_big_t"):   # t = 350 > 256
        m = 1 if name.startswith("pgd") else 0
        c = dict(name=name, T=700, H=1, d=32, seed=44,
                 params=dict(target_ratio=0.5, chunk_size=-1, skip_beta=0, nnls_method=m))
        K, V = kv_cache(700, 1, 32, 44)
        return c, K, V, normal(4401, (16, 32)), 16
    raise KeyError(name)


# --------------------------------------------------------------------------
# Refinement-round variants (api.cpp:851-946) at chunked shapes.
# --------------------------------------------------------------------------

def refine_variant_names():
    return ["refine3_pgd", "refine2_skipbeta_div", "cfg5_chunked", "refine_full_keep", "refine_unchunked"]


def refine_variant(name: str):
    """Return (case, K, V, Q or None, n_q)."""
    if name == "refine3_pgd":
        c = dict(name=name, T=2560, H=2, d=32, seed=51,
                 params=dict(target_ratio=0.2, skip_beta=0, nnls_method=1, refine_rounds=3))
        K, V = kv_cache(2560, 2, 32, 51, channel_scale=True)
        return c, K, V, snapkv_queries(K, 16, 51), 16
    if name == "refine2_skipbeta_div":
        c = dict(name=name, T=2560, H=2, d=32, seed=52, params=dict(target_ratio=0.2, use_diversity=1, refine_rounds=2))
        K, V = kv_cache(2560, 2, 32, 52, channel_scale=True)
        return c, K, V, snapkv_queries(K, 16, 52), 16
    if name == "cfg5_chunked":   # the 1M-token configuration's options on 4 chunks of 1280
        c = dict(name=name, T=5120, H=4, d=32, seed=53, rkv=dict(thinking=0.3, transition=0.7),
                 params=dict(target_ratio=0.2, skip_beta=0, nnls_method=0, use_diversity=1, refine_rounds=1))
        K, V = kv_cache(5120, 4, 32, 53, channel_scale=True)
        return c, K, V, snapkv_queries(K, 32, 53), 32
    if name == "refine_full_keep":   # t == T: the rounds do nothing
        c = dict(name=name, T=200, H=2, d=16, seed=54, params=dict(target_count=200, refine_rounds=2))
        K, V = kv_cache(200, 2, 16, 54)
        return c, K, V, normal(5401, (8, 32)), 8
    if name == "refine_unchunked":
        c = dict(name=name, T=600, H=2, d=16, seed=55,
                 params=dict(target_ratio=0.3, chunk_size=-1, refine_rounds=4, skip_beta=0, nnls_method=0))
        K, V = kv_cache(600, 2, 16, 55)
        return c, K, V, normal(5501, (12, 32)), 12
    raise KeyError(name)


def nonfinite_variant_names():
    return ["nan_k", "inf_k", "nan_v", "negzero_k_row"]


def nonfinite_variant(name: str):
    """Return (case, K, V, Q, n_q): one NaN / inf / -0 planted in an otherwise
    ordinary cache (the reference's arithmetic carries them through)."""
    T, H, d = 600, 2, 32
    K, V = kv_cache(T, H, d, 77)
    Q = snapkv_queries(K, 16, 77)
    if name == "nan_k":
        K[123, 5] = np.nan
    elif name == "inf_k":
        K[321, 40] = np.inf
    elif name == "nan_v":
        V[50, 3] = np.nan
    elif name == "negzero_k_row":
        K[10, :] = -0.0
    c = dict(name=name, T=T, H=H, d=d, seed=77, params=dict(target_ratio=0.3))
    return c, K, V, Q, 16


# ---------------------------------------------------------------------------
# Vectorized reference-codec quantizers (state.h:508-567) for building large
# synthetic Q8_0 / Q4_0 caches quickly. test_oracle.py pins them byte for byte
# against the oracle's row quantizer.
# ---------------------------------------------------------------------------
def f32_to_f16_trunc(x: np.ndarray) -> np.ndarray:
    """The reference's f32 -> f16: mantissa truncated, NaN -> Inf (state.h:508-525)."""
    f = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.int64)
    sign = (f >> 16) & 0x8000
    e = ((f >> 23) & 0xFF) - 127 + 15
    m = (f >> 13) & 0x3FF
    sub = np.where(e < -10, 0, ((m | 0x400) >> np.clip(1 - e, 0, 31)))
    out = np.where(e <= 0, sign | sub, np.where(e >= 31, sign | 0x7C00, sign | (np.clip(e, 0, 31) << 10) | m))
    return out.astype(np.uint16)


def roundf(v: np.ndarray) -> np.ndarray:
    """C roundf (half away from zero) for float32 values."""
    r = np.trunc(v)
    frac = np.abs(v - r)   # exact for |v| < 2^23
    return (r + np.where(frac >= np.float32(0.5), np.sign(v), 0)).astype(np.float32)


def quantize_rows(x: np.ndarray, typ: int) -> np.ndarray:
    """Rows of float32 (n a multiple of 32) -> reference Q8_0 (typ 8) or Q4_0 (typ 2) bytes."""
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    b = x.reshape(rows, n // 32, 32)
    amax = np.max(np.abs(b), axis=2)   # the blocks here hold no NaN
    if typ == 8:
        d = (amax / np.float32(127.0)).astype(np.float32)
        with np.errstate(divide="ignore"):
            idv = np.where(d != 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
        v = (b * idv[:, :, None]).astype(np.float32)
        q = roundf(np.maximum(np.float32(-128.0), np.minimum(np.float32(127.0), v))).astype(np.int8)
        out = np.empty((rows, n // 32, 34), np.uint8)
        out[:, :, 0:2] = f32_to_f16_trunc(d).view(np.uint8).reshape(rows, n // 32, 2)
        out[:, :, 2:] = q.view(np.uint8)
    elif typ == 2:
        d = (amax / np.float32(7.0)).astype(np.float32)
        with np.errstate(divide="ignore"):
            idv = np.where(d != 0, np.float32(7.0) / amax, np.float32(0.0)).astype(np.float32)
        v = ((b * idv[:, :, None]).astype(np.float32) + np.float32(8.0)).astype(np.float32)
        q = np.maximum(np.float32(0.0), np.minimum(np.float32(15.0), roundf(v))).astype(np.uint8)
        out = np.empty((rows, n // 32, 18), np.uint8)
        out[:, :, 0:2] = f32_to_f16_trunc(d).view(np.uint8).reshape(rows, n // 32, 2)
        out[:, :, 2:] = q[:, :, 0::2] | (q[:, :, 1::2] << 4)
    else:
        raise ValueError(typ)
    return out.reshape(rows, -1)


# --------------------------------------------------------------------------
# Options past the defaults: sensitivity weighting (math.h:579-618,
# api.cpp:651-666), projected-gradient NNLS iterations (math.h:752-805) and
# OMP key selection (math.h:832-950, api.cpp:690-711).
# --------------------------------------------------------------------------

def option_variant_names():
    return ["sens_chunk", "sens_max_div", "sens_mean_cheap", "pgd_iters_chunk", "pgd_iters_unchunked",
            "omp_k1", "omp_k4_r2_beta_pgd", "omp_lh_beta", "omp_refine", "omp_cheap_chunk"]


def option_variant(name: str):
    """Return (case, K, V, Q or None, n_q)."""
    def snap(T, H, d, seed, **params):
        c = dict(name=name, T=T, H=H, d=d, seed=seed, params=params)
        K, V = kv_cache(T, H, d, seed, channel_scale=True)
        return c, K, V, snapkv_queries(K, 32, seed), 32

    def cheap(T, H, d, seed, **params):
        c = dict(name=name, T=T, H=H, d=d, seed=seed, params=dict(use_cheap_qref=1, **params))
        K, V = kv_cache(T, H, d, seed)
        return c, K, V, None, 0

    if name == "sens_chunk":
        return snap(2560, 4, 64, 51, target_ratio=0.2, use_sensitivity=1)
    if name == "sens_max_div":
        return snap(2000, 3, 32, 52, target_ratio=0.2, use_sensitivity=1, score_method=0, use_diversity=1)
    if name == "sens_mean_cheap":
        return cheap(3000, 2, 32, 53, target_ratio=0.2, use_sensitivity=1, score_method=2)
    if name == "pgd_iters_chunk":
        return snap(2560, 2, 64, 54, target_ratio=0.2, skip_beta=0, nnls_method=1, nnls_pgd_iters=20)
    if name == "pgd_iters_unchunked":
        return snap(700, 1, 32, 55, target_ratio=0.3, chunk_size=-1, skip_beta=0, nnls_method=1, nnls_pgd_iters=5)
    if name == "omp_k1":
        return snap(1000, 2, 32, 56, target_ratio=0.2, use_omp=1)
    if name == "omp_k4_r2_beta_pgd":
        return snap(2560, 2, 32, 57, target_ratio=0.2, use_omp=1, omp_k_choice=4, omp_refit_interval=2,
                    skip_beta=0, nnls_method=1, nnls_pgd_iters=3)
    if name == "omp_lh_beta":
        return snap(1500, 2, 32, 58, target_ratio=0.15, use_omp=1, omp_k_choice=2, skip_beta=0, nnls_method=0)
    if name == "omp_refine":
        return snap(1200, 2, 32, 59, target_ratio=0.2, use_omp=1, refine_rounds=1, skip_beta=0)
    if name == "omp_cheap_chunk":
        return cheap(1800, 2, 32, 60, target_ratio=0.2, use_omp=1, omp_k_choice=3, use_sensitivity=1)
    raise KeyError(name)


# -- llama.cpp state blobs (include/kv-compact-state.h layout) -------------------
# Synthetic blobs in the format llama_state_seq_get_data writes, built from the
# seeded generator: encoded payloads are drawn directly (random int8 / nibbles
# with positive f16 scales for the block codecs, f16 / f32 of normal values
# with some exact -0 and +0 entries), so every decode path is exercised.
T_F32, T_F16, T_Q4_0, T_Q4_1, T_Q8_0 = 0, 1, 2, 3, 8
_BLOCK = {T_Q8_0: 34, T_Q4_0: 18, T_Q4_1: 20}


def _u8(seed, n):
    return (splitmix64(seed, n) & 0xFF).astype(np.uint8)


def _payload(typ: int, n_el: int, rows: int, seed: int) -> bytes:
    """rows x n_el values of `typ`, row-major bytes."""
    if typ in (T_F32, T_F16):
        x = normal(seed, (rows, n_el))
        z = _u8(seed + 1, rows * n_el).reshape(rows, n_el)
        x = np.where(z < 6, np.float32(-0.0), np.where(z < 9, np.float32(0.0), x)).astype(np.float32)
        return (x if typ == T_F32 else x.astype(np.float16)).tobytes()
    nb = n_el // 32
    bb = _BLOCK[typ]
    raw = _u8(seed, rows * nb * bb).reshape(rows * nb, bb)
    d = (np.abs(normal(seed + 2, (rows * nb,))) * 0.05 + 0.01).astype(np.float16)
    raw[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    if typ == T_Q4_1:
        m = (normal(seed + 3, (rows * nb,)) * 0.3).astype(np.float16)
        raw[:, 2:4] = m.view(np.uint8).reshape(-1, 2)
    return raw.tobytes()


def state_blob(c: dict) -> bytes:
    """Blob for a state case dict: T, L, H, dk, dv, kt, vt, vtrans, n_pos, seed,
    optional n_stream (extra streams empty unless extra_cells), trailing."""
    import struct
    T, L, H, dk, dv = c["T"], c["L"], c["H"], c["dk"], c["dv"]
    seed, n_pos = c["seed"], c.get("n_pos", 1)
    nk, nv = H * dk, H * dv
    out = bytearray()
    n_stream = c.get("n_stream", 1)
    out += struct.pack("<I", n_stream)
    out += struct.pack("<I", T)
    z = splitmix64(seed * 7 + 1, 4 * T)
    for i in range(T):
        ns = 1 + int(z[i] % 3)
        out += struct.pack("<iI", i + int(c.get("pos0", 0)), ns)
        if n_pos > 1:
            out += struct.pack("<ii", int(z[T + i] % 64), int(z[2 * T + i] % 64))
        for k in range(ns):
            out += struct.pack("<i", int((z[3 * T + i] >> (8 * k)) % 8))
    out += struct.pack("<II", int(c["vtrans"]), L)
    for l in range(L):
        kt = c["kt"][l] if isinstance(c["kt"], (list, tuple)) else c["kt"]
        rb = nk * 4 if kt == T_F32 else nk * 2 if kt == T_F16 else nk // 32 * _BLOCK[kt]
        out += struct.pack("<iQ", kt, rb)
        out += _payload(kt, nk, T, seed * 101 + l)
    for l in range(L):
        vt = c["vt"][l] if isinstance(c["vt"], (list, tuple)) else c["vt"]
        if not c["vtrans"]:
            rb = nv * 4 if vt == T_F32 else nv * 2 if vt == T_F16 else nv // 32 * _BLOCK[vt]
            out += struct.pack("<iQ", vt, rb)
            out += _payload(vt, nv, T, seed * 211 + l)
        else:
            # [embd][cell]: v_size_el is the element size (f32 / f16) or, for
            # block codecs, the block size (as llama.cpp's ggml_type_size)
            el = 4 if vt == T_F32 else 2 if vt == T_F16 else _BLOCK[vt]
            out += struct.pack("<iII", vt, el, nv)
            if vt in (T_F32, T_F16):
                out += _payload(vt, T, nv, seed * 307 + l)
            else:
                body = bytearray(nv * T * el)
                enc = _payload(vt, nv * T // 32 * 32, 1, seed * 307 + l) if nv * T >= 32 else b""
                body[:len(enc)] = enc
                out += bytes(body)
    for s in range(1, n_stream):
        ec = c.get("extra_cells", 0) if s == 1 else 0
        out += struct.pack("<I", ec)
        if ec:
            for i in range(ec):
                out += struct.pack("<iIi", i, 1, 0)
            out += struct.pack("<II", 0, 0)
    out += bytes(c.get("trailing", b""))
    return bytes(out)


STATE_CASES = [
    dict(name="f16_basic", T=300, L=3, H=2, dk=32, dv=32, kt=T_F16, vt=T_F16, vtrans=0, seed=61, ratio=0.2),
    dict(name="q8_vtrans_f16", T=257, L=2, H=2, dk=64, dv=64, kt=T_Q8_0, vt=T_F16, vtrans=1, seed=62, ratio=0.3),
    dict(name="imrope_q4_trailing", T=200, L=2, H=4, dk=32, dv=32, kt=T_Q4_0, vt=T_Q4_1, vtrans=0, n_pos=4,
         seed=63, ratio=0.25, trailing=bytes(range(37))),
    dict(name="f32_sens_nref", T=240, L=3, H=2, dk=32, dv=32, kt=T_F32, vt=T_F32, vtrans=0, seed=64, ratio=0.2,
         sens=1, n_ref=40),
    dict(name="q8_filter", T=220, L=3, H=2, dk=64, dv=64, kt=T_Q8_0, vt=T_Q8_0, vtrans=0, seed=65, ratio=0.2,
         layers=[0, 2]),
    dict(name="vtrans_q8_flat", T=160, L=2, H=1, dk=32, dv=32, kt=T_F16, vt=T_Q8_0, vtrans=1, seed=66, ratio=0.3),
    dict(name="two_streams_dk_ne_dv", T=180, L=2, H=2, dk=64, dv=32, kt=T_F16, vt=T_F32, vtrans=1, seed=67,
         ratio=0.2, n_stream=2),
    dict(name="mixed_types_sens", T=260, L=4, H=2, dk=32, dv=32, kt=[T_F16, T_Q8_0, T_Q4_1, T_F32],
         vt=[T_Q4_0, T_F16, T_Q8_0, T_F32], vtrans=0, seed=68, ratio=0.15, sens=1),
    dict(name="t1_small", T=20, L=1, H=1, dk=32, dv=32, kt=T_F16, vt=T_F16, vtrans=1, seed=69, ratio=0.01),
    dict(name="large_nref", T=1200, L=2, H=2, dk=64, dv=64, kt=T_F16, vt=T_F16, vtrans=0, seed=70, ratio=0.1,
         n_ref=300),
]
STATE_CASE_BY_NAME = {c["name"]: c for c in STATE_CASES}
