"""Write golden fixtures from the compiled reference.

Run in the container that holds the reference checkout, after
`make -C oracle ref` has compiled it into oracle/_ref/:

    python tests/golden/gen_golden.py          (everything)
    python tests/golden/gen_golden.py state    (the state blob cases only)
    python tests/golden/gen_golden.py replay   (the wrapper call-sequence replay only)
    python tests/golden/gen_golden.py matmul   (the accelerator GEMMs only)
    python tests/golden/gen_golden.py case NAME   (one case of the catalogue)

Inputs are regenerated from seeds by tests/kvc_data.py (integer-only
generator), so each fixture stores only the reference's outputs plus an
input checksum: indices, beta, C_v and the three quality statistics for the
case catalogue; quantized and multi-round runs; and known-answer vectors for
the reference's building blocks (least squares, NNLS, softmax-importance,
codec, f16 conversions).
"""
from __future__ import annotations

import ctypes
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from kvc_data import CASES, kv_cache, make_case, matmul_inputs, normal, uniform  # noqa: E402
from kvc_harness import REF_HARNESS_SO, kc, load_ref, run_case  # noqa: E402


def checksum(*arrs):
    """First 8 bytes of the SHA-256 of the concatenated input bytes."""
    import hashlib
    m = hashlib.sha256()
    for a in arrs:
        if a is not None:
            m.update(np.ascontiguousarray(a).tobytes())
    return int.from_bytes(m.digest()[:8], "little")


def stats_arr(st):
    return np.array([st["avg_cosine_sim"], st["avg_mse"], st["avg_agreement"]], np.float32)


QUANT_CASES = [
    dict(name="quant_q8", T=600, H=2, d=64, seed=33, k=kc.KV_TYPE_Q8_0, v=kc.KV_TYPE_Q8_0),
    dict(name="quant_q4", T=600, H=2, d=64, seed=34, k=kc.KV_TYPE_Q4_0, v=kc.KV_TYPE_Q4_0),
    dict(name="quant_mixed", T=600, H=2, d=64, seed=35, k=kc.KV_TYPE_Q8_0, v=kc.KV_TYPE_Q4_0),
    dict(name="quant_f16_q41", T=300, H=2, d=32, seed=36, k=kc.KV_TYPE_F16, v=kc.KV_TYPE_Q4_1),
]


def quant_inputs(ref, c):
    K, V = kv_cache(c["T"], c["H"], c["d"], c["seed"])
    Kq = np.stack([ref.quantize_row(K[i], c["k"]) for i in range(c["T"])])
    Vq = np.stack([ref.quantize_row(V[i], c["v"]) for i in range(c["T"])])
    return K, V, np.ascontiguousarray(Kq), np.ascontiguousarray(Vq)


def codec_vectors():
    """Rows exercising zeros, tiny/huge magnitudes, signs and half-way values."""
    rows = [
        normal(901, (256,)),
        normal(902, (256,)) * np.float32(1e-6),
        normal(903, (256,)) * np.float32(3e4),
        np.zeros(256, np.float32),
        np.tile(np.array([0.5, -0.5, 1.5, -1.5, 2.5, 127.0, -128.0, 7.0], np.float32), 32),
        (uniform(904, 256) * 1e-7).astype(np.float32),
    ]
    return np.stack(rows).astype(np.float32)


def write_state_fixtures():
    """llama.cpp state blob cases through the reference's own parse/build
    (oracle/_ref harness, the CLI's call sequence): kept cells, output size and
    SHA-256 of the compacted blob (the inputs regenerate from their seeds)."""
    import hashlib

    from kvc_data import STATE_CASES, state_blob
    from kvc_harness import ref_state_compact
    out = {}
    for c in STATE_CASES:
        blob = state_blob(c)
        rc, data, sel = ref_state_compact(blob, c)
        assert rc == 0, c["name"]
        out[c["name"] + "_sel"] = sel.astype(np.int32)
        out[c["name"] + "_size"] = np.int64(len(data))
        out[c["name"] + "_sha256"] = np.array(hashlib.sha256(data).hexdigest())
        out[c["name"] + "_input_sha256"] = np.array(hashlib.sha256(blob).hexdigest())
    np.savez_compressed(HERE / "state_cases.npz", **out)
    print("wrote", len(STATE_CASES), "state cases")


def write_replay_fixtures():
    """The reference wrapper's call sequence replayed against the compiled
    reference (tests/bindings_replay.py)."""
    import bindings_replay as br
    from kvc_harness import REF_SO
    lib = br.load(str(REF_SO))
    out = {}
    for c in br.REPLAY_CASES:
        K, V, Q = br.replay_inputs(c["seed"])
        idx, cv, ksel, st = br.compact(lib, K, V, Q if c["q"] else None, **c["kw"])
        out[c["name"] + "_indices"] = idx
        out[c["name"] + "_C_v"] = cv
        out[c["name"] + "_K_selected"] = ksel
        out[c["name"] + "_stats"] = np.array([st["avg_cosine_sim"], st["avg_mse"], st["avg_agreement"]], np.float32)
    np.savez_compressed(HERE / "bindings_replay.npz", **out)
    print("wrote", len(br.REPLAY_CASES), "replay cases")


# The reference's two accelerator GEMMs, computed by its CPU path: the
# scores mat_mul_ABt followed by the scale (api.cpp:619-627) for
# kv_compact_hip_mat_mul_ABt_scaled, and the refit target's per-head slice of
# V followed by mat_mul_AB (api.cpp:776-781) for
# kv_compact_hip_refit_target_all_heads (inputs: kvc_data.matmul_inputs).
def write_matmul_fixtures():
    h = ctypes.CDLL(str(REF_HARNESS_SO))
    fp, ci = ctypes.c_void_p, ctypes.c_int
    h.ref_mat_mul_ABt.argtypes = [fp, fp, fp, ci, ci, ci]
    h.ref_mat_mul_AB.argtypes = [fp, fp, fp, ci, ci, ci]
    (A, B, scale), (W, Vall, H, dv) = matmul_inputs()
    m, k = A.shape
    n = B.shape[0]
    C = np.zeros((m, n), np.float32)
    h.ref_mat_mul_ABt(A.ctypes.data, B.ctypes.data, C.ctypes.data, m, n, k)
    C = (C * np.float32(scale)).astype(np.float32)
    nq, T = W.shape[1], W.shape[2]
    Y = np.zeros((H, nq, dv), np.float32)
    for hh in range(H):
        vh = np.ascontiguousarray(Vall[:, hh * dv:(hh + 1) * dv])
        W_h = np.ascontiguousarray(W[hh])
        h.ref_mat_mul_AB(W_h.ctypes.data, vh.ctypes.data, Y[hh].ctypes.data, nq, T, dv)
    np.savez_compressed(HERE / "matmul.npz", abt_C=C, ab_Y=Y,
                        in_checksum=np.uint64(checksum(A, B, W, Vall)))


def main():
    if len(sys.argv) > 1 and sys.argv[1] in ("state", "replay", "matmul"):
        {"state": write_state_fixtures, "replay": write_replay_fixtures,
         "matmul": write_matmul_fixtures}[sys.argv[1]]()
        return
    ref = load_ref()
    if ref is None:
        raise SystemExit("oracle/_ref/libkvref.so missing: run `make -C oracle ref` first")
    one = sys.argv[2] if len(sys.argv) > 2 and sys.argv[1] == "case" else None
    out = {}
    for c in CASES:
        if one is not None and c["name"] != one:
            continue
        inp = make_case(c)
        r = run_case(ref, c, inp)
        np.savez_compressed(HERE / f"case_{c['name']}.npz", indices=r.indices.astype(np.int32),
                            beta=r.beta, C_v=r.C_v, stats=stats_arr(r.stats),
                            input_checksum=np.uint64(checksum(*inp[:3])))
        out[c["name"]] = r.t
    if one is not None:
        return
    for c in QUANT_CASES:
        K, V, Kq, Vq = quant_inputs(ref, c)
        kr, vr = Kq.shape[1], Vq.shape[1]
        p = ref.params(target_ratio=0.2, use_cheap_qref=1)
        rc, r = ref.quantized(Kq, Vq, None, c["k"], c["v"], kr, vr, c["T"], 0, c["H"], c["d"], c["d"], p)
        assert rc == 0
        np.savez_compressed(HERE / f"{c['name']}.npz", Kq=Kq, Vq=Vq, indices=r.indices.astype(np.int32),
                            C_v=r.C_v, K_out=r.K_out, V_out=r.V_out, stats=stats_arr(r.stats),
                            input_checksum=np.uint64(checksum(K, V)))
    # multi-round
    from kvc_data import CASE_BY_NAME
    c = CASE_BY_NAME["unchunked_r80"]
    K, V, Q, nq = make_case(c)
    rc, r, per = ref.multi_round(K, V, Q, c["T"], nq, c["H"], c["d"], c["d"], ref.params(target_ratio=0.7), 3)
    np.savez_compressed(HERE / "multi_round.npz", indices=r.indices.astype(np.int32), beta=r.beta, C_v=r.C_v,
                        stats=stats_arr(r.stats), per_round_cos=np.array(per, np.float32))

    # building blocks through the harness
    h = ctypes.CDLL(str(REF_HARNESS_SO))
    fp = ctypes.c_void_p
    blocks = {}
    A = normal(1001, (24, 40)); A = np.abs(A) / np.float32(10.0); A = A.astype(np.float32)
    B = normal(1002, (24, 16))
    X = np.zeros((40, 16), np.float32)
    h.ref_least_squares_solve.argtypes = [fp, fp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float]
    h.ref_least_squares_solve(A.ctypes.data, B.ctypes.data, X.ctypes.data, 24, 40, 16, ctypes.c_float(1e-6))
    blocks.update(ls_A=A, ls_B=B, ls_X=X)
    M = (np.exp(normal(1003, (24, 30)).astype(np.float64)).astype(np.float32))
    b = M[:, :12].sum(axis=1).astype(np.float32) * np.float32(0.7)
    W = np.zeros(30, np.float32)
    h.ref_nnls_solve.argtypes = [fp, fp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    h.ref_nnls_solve(M.ctypes.data, b.ctypes.data, W.ctypes.data, 24, 30, 200)
    W2 = np.zeros(30, np.float32)
    h.ref_nnls_pgd_solve.argtypes = [fp, fp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int]
    h.ref_nnls_pgd_solve(M.ctypes.data, b.ctypes.data, W2.ctypes.data, 24, 30, ctypes.c_float(1e-12), 0)
    blocks.update(nnls_M=M, nnls_b=b, nnls_lh_w=W, nnls_clamped_w=W2)
    S = normal(1004, (16, 300)) * np.float32(3.0)
    for agg in (0, 1, 2):
        attn = np.zeros_like(S); imp = np.zeros(300, np.float32)
        h.ref_softmax_importance.argtypes = [fp, fp, fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        h.ref_softmax_importance(S.ctypes.data, attn.ctypes.data, imp.ctypes.data, 16, 300, agg)
        blocks[f"smi_attn_{agg}"] = attn
        blocks[f"smi_imp_{agg}"] = imp
    blocks["smi_S"] = S
    rows = codec_vectors()
    blocks["codec_rows"] = rows
    h.ref_convert_from_f32.argtypes = [fp, ctypes.c_int, fp, ctypes.c_int]
    h.ref_convert_from_f32.restype = ctypes.c_size_t
    h.ref_convert_to_f32.argtypes = [fp, ctypes.c_int, fp, ctypes.c_size_t]
    for name, typ, bb in (("q8_0", 8, 34), ("q4_0", 2, 18), ("q4_1", 3, 20), ("f16", 1, 64)):
        enc = np.zeros((rows.shape[0], 8 * bb if typ != 1 else 512), np.uint8)
        dec = np.zeros_like(rows)
        for i in range(rows.shape[0]):
            n = h.ref_convert_from_f32(rows[i].ctypes.data, typ, enc[i].ctypes.data, 256)
            assert n == enc.shape[1]
            h.ref_convert_to_f32(enc[i].ctypes.data, typ, dec[i].ctypes.data, 256)
        blocks[f"codec_enc_{name}"] = enc
        blocks[f"codec_dec_{name}"] = dec
    h.ref_f16_to_f32.argtypes = [ctypes.c_uint16]; h.ref_f16_to_f32.restype = ctypes.c_float
    blocks["f16_to_f32_all"] = np.array([h.ref_f16_to_f32(i) for i in range(65536)], np.float32)
    h.ref_f32_to_f16.argtypes = [ctypes.c_float]; h.ref_f32_to_f16.restype = ctypes.c_uint16
    probe = np.concatenate([normal(1005, (4000,)) * np.float32(100.0), normal(1006, (1000,)) * np.float32(1e-5),
                            np.array([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 6e-8, 3e-8, np.inf, -np.inf, np.nan], np.float32)]).astype(np.float32)
    blocks["f32_to_f16_in"] = probe
    blocks["f32_to_f16_out"] = np.array([h.ref_f32_to_f16(float(v)) for v in probe], np.uint16)
    np.savez_compressed(HERE / "blocks.npz", **blocks)
    write_state_fixtures()
    write_replay_fixtures()
    write_matmul_fixtures()
    print("wrote", len(out), "cases,", len(QUANT_CASES), "quantized cases, multi-round and blocks")


if __name__ == "__main__":
    main()
