#!/usr/bin/env python3
"""Compaction throughput on one MI355X.

Workload (the headline configuration): a Llama-3-8B-shaped KV cache of
32 layers x 8 KV heads x head_dim 128 at T = 100,000 tokens, fp32, compacted
to 20% retention (t = 20,000 kept per layer) with diversity selection on
(strength 0.5) and otherwise default parameters (RMS importance,
skip_beta = 1, auto chunking: 79 chunks of 1280 tokens, 256 kept per chunk).
The same data is also timed with diversity off ("other_mode"). Keys ~ N(0,1) times a per-(layer, channel) scale drawn
from LogNormal(0, 0.5); values ~ N(0,1); SnapKV reference queries = the last
32 keys + N(0, 0.1^2) noise. Synthetic data, generated once on the host and
resident in HBM before the timed region.

One step = one device-resident call compacting all 32 layers (scoring,
selection, value refit and the quality statistics the reference computes in
every call). metric = T / step time (tokens of context compacted per second
across all layers, the reference benches' definition).

Prints one JSON line (driver contract) with a "roofline" object for the
dominant kernel (from HIP events recorded by the library on its stream) and a
"cpu_baseline" object: the reference's own CPU path compiled from its sources
(oracle/_ref/libkvref.so, OpenMP over every host core) timed on a bounded
sample of the same data, or the oracle port when the reference build is
absent.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "kv-compact_amd"))

import kvcompact as kc  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
FP32_PEAK_TFLOPS = 157.3       # MI355X fp32 (published)
# fp32 multiply and add issued separately on the vector ALUs (the reference's
# rounding: no FMA, no packed fp32), two or more waves per SIMD: 256 CUs x 4
# SIMDs x 32 lanes x 2.4 GHz, measured with s_memtime microbenchmarks
VALU_CEILING_TOPS = 78.6
STAGES = ["scores", "chunk_softmax_importance", "refit_target", "selection", "beta_fit", "compacted_softmax",
          "normal_equations", "lu_factorization", "substitution", "refinement", "quality_stats"]
QSTAGES = STAGES + ["dequantize", "requantize"]
STAGE_KERNELS = {"scores": "k_scores", "chunk_softmax_importance": "k_softmax_importance",
                 "refit_target": "k_refit_target",
                 "selection": "k_global_importance + k_select_topk (or k_div_candidates + k_div_gram + k_div_greedy)",
                 "beta_fit": "k_gather_exp + k_ls_build + k_ge_lu + k_ge_solve (or k_nnls_lh) + k_beta_log",
                 "compacted_softmax": "k_ls_softmax", "normal_equations": "k_ls_build",
                 "lu_factorization": "k_ge_lu<false, true> (steps 0-127) + k_ge_lu_tail (the rest)",
                 "substitution": "k_ge_subst",
                 "refinement": "k_refine_step + the beta and C_v refit per round",
                 "quality_stats": "k_scores + k_row_softmax + k_stats_sum + k_stats_final"}


def gen_layers(L, T, H, d, W, seed):
    """Yield (K, V, Q) float32 host arrays per layer. One pool of normals is
    drawn once; each layer takes its own windows of it and its own channel
    scales, so layers differ without drawing 26 GB of normals."""
    E = H * d
    rng = np.random.default_rng(seed)
    pool = rng.standard_normal(3 * T * E + 4096, dtype=np.float32)
    for l in range(L):
        r = np.random.default_rng(seed * 1000 + l)
        o1, o2 = (int(x) for x in r.integers(0, pool.size - T * E, size=2))
        scale = np.exp(r.normal(0.0, 0.5, size=E)).astype(np.float32)
        K = (pool[o1:o1 + T * E].reshape(T, E) * scale).astype(np.float32)
        V = pool[o2:o2 + T * E].reshape(T, E)
        Q = (K[-W:] + r.normal(0.0, 0.1, size=(W, E)).astype(np.float32)).astype(np.float32)
        yield np.ascontiguousarray(K), np.ascontiguousarray(V), np.ascontiguousarray(Q)


def stage_model(L, T, H, d, nq, t, n_chunks, tc):
    """Algorithmic bytes and flops of each stage for one call (all layers).
    Per (token, layer, head): scoring reads one key row (4d B) and does 2*nq*d
    flops; the refit target reads one value row and does 2*nq*d flops."""
    E = H * d
    units = L * H * n_chunks
    n, p = tc, d
    # LU of the n x n Gram matrix: step c divides n-1-c multipliers and
    # updates (n-1-c) x (n-1-c) entries with one multiply and one subtract
    lu = sum(2 * (n - 1 - c) * (n - 1 - c) + (n - 1 - c) for c in range(n))
    # forward + back substitution over p right-hand sides (one multiply and
    # one subtract per L / U entry and column, one divide per row and column)
    subst = p * (2 * n * (n - 1) + n)
    m = {
        "scores": dict(bytes=4 * L * T * E + 4 * L * H * nq * T, flops=2 * L * H * nq * T * d),
        "chunk_softmax_importance": dict(bytes=4 * L * H * nq * T * 2 + 4 * L * H * T, flops=0),
        "refit_target": dict(bytes=4 * L * H * nq * T + 4 * L * T * E, flops=2 * L * H * nq * T * d),
        "selection": dict(bytes=4 * L * H * T + 4 * L * t, flops=0),
        "beta_fit": dict(bytes=0, flops=0),
        "refinement": dict(bytes=0, flops=0),
        "compacted_softmax": dict(bytes=4 * L * H * nq * t * 2, flops=0),
        # the normal equations write B = X^T Y only; the register LU forms
        # M = X^T X (one triangle's worth of sums) from X, then factors it
        "normal_equations": dict(bytes=4 * units * (nq * (n + p) + n * p), flops=2 * nq * units * n * p),
        "lu_factorization": dict(bytes=4 * units * (nq * n + n * n),
                                 flops=units * (lu + nq * n * (n + 1))),
        "substitution": dict(bytes=4 * units * (n * n + 3 * n * p), flops=units * subst),
        "quality_stats": dict(bytes=4 * L * min(H, 4) * T * 2 * d, flops=2 * L * min(H, 4) * min(nq, 32) * T * 2 * d),
    }
    return m


def roofline(name, model, ms):
    b, f = model[name]["bytes"], model[name]["flops"]
    t_hbm = b / (HBM_PEAK_GBS * 1e9)
    t_cmp = f / (FP32_PEAK_TFLOPS * 1e12)
    s = ms / 1e3
    if t_cmp > t_hbm:
        # fp32 arithmetic on the vector ALUs in the reference's operation
        # order (no MFMA: a reordered or fused sum would change the results)
        ach = f / s / 1e12
        return dict(kernel=STAGE_KERNELS[name], stage=name, bound="valu", achieved=round(ach, 3), peak=FP32_PEAK_TFLOPS,
                    unit="TFLOP/s", frac=round(ach / FP32_PEAK_TFLOPS, 4), traffic=None, ms=round(ms, 3),
                    valu_ceiling=VALU_CEILING_TOPS, frac_of_valu_ceiling=round(ach / VALU_CEILING_TOPS, 4),
                    algorithmic_flops=f, algorithmic_bytes=b)
    ach = b / s / 1e9
    return dict(kernel=STAGE_KERNELS[name], stage=name, bound="hbm", achieved=round(ach, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                frac=round(ach / HBM_PEAK_GBS, 4), traffic=None, ms=round(ms, 3),
                algorithmic_flops=f, algorithmic_bytes=b)


def host_info() -> dict:
    """Device and host descriptions for the record, read from sysfs and /proc
    (no other program is started: this process may already hold the GPU)."""
    arch, model, product = "", "", ""
    try:
        for node in sorted(Path("/sys/class/kfd/kfd/topology/nodes").iterdir()):
            name = (node / "name").read_text().strip() if (node / "name").exists() else ""
            if name.startswith("gfx"):
                arch = name
                for line in (node / "properties").read_text().splitlines():
                    k, _, v = line.partition(" ")
                    if k == "device_id" and v.strip().isdigit():
                        model = f"0x{int(v):04x}"
                break
    except OSError:
        pass
    try:
        for card in sorted(Path("/sys/class/drm").glob("card*/device/product_name")):
            product = card.read_text().strip()
            if product:
                break
    except OSError:
        pass
    cpu = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    dev = product or f"AMD Instinct {arch}"
    if model:
        dev += f" ({arch}, PCI device {model})" if product else f" (PCI device {model})"
    return {"device": dev, "cpu_model": cpu, "host_cpus": os.cpu_count(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS", "")}


def cpu_baseline(K, V, Q, T, H, d, ratio, L_total, diversity):
    """The reference CPU path (compiled from its sources) on layer 0 at full T,
    scaled to all layers; falls back to the oracle port."""
    ref = REPO / "oracle" / "_ref" / "libkvref.so"
    if ref.exists():
        lib, kind = kc.Lib(ref), "reference"
    else:
        lib, kind = kc.Lib(REPO / "oracle" / "liboracle.so", prefix="orc_"), "port"
    p = lib.params(target_ratio=ratio, use_diversity=diversity)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
    t0 = time.perf_counter()
    r = lib.compact(K, V, Q, T, Q.shape[0], H, d, d, p)
    dt = time.perf_counter() - t0
    per_layer = dt
    if r is None:
        raise RuntimeError("CPU baseline call failed")
    return dict(value=round(T / (per_layer * L_total), 2), unit="tok/s", cores=threads, kind=kind,
                sample=f"layer 0 of {L_total} at full T={T} ({dt:.1f} s, all-layer rate = T/(time*{L_total}))",
                seconds=round(dt, 2), kept=r.t, cos=r.stats["avg_cosine_sim"])


def _pmc_per_dispatch(path: Path) -> dict:
    """kernel -> (dispatches, {counter: mean value per dispatch}, mean ms per
    dispatch) from a rocprofv3 --pmc csv"""
    import csv
    tot, disp, dur = {}, {}, {}
    with open(path) as f:
        for r in csv.DictReader(f):
            k = r["Kernel_Name"].split("(")[0].replace("void ", "")
            c = tot.setdefault(k, {})
            c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            disp.setdefault(k, set()).add(r["Dispatch_Id"])
            dur.setdefault(k, {})[r["Dispatch_Id"]] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6
    return {k: (len(disp[k]), {c: v / len(disp[k]) for c, v in tot[k].items()},
                sum(dur[k].values()) / len(dur[k])) for k in tot}


# The counter passes of one bench step (each its own rocprofv3 run; at most 4
# TCC and 8 SQ counters per pass on this GPU):
PMC_PASSES = {
    "rd": "TCC_EA0_RDREQ_128B_sum TCC_EA0_RDREQ_64B_sum TCC_EA0_RDREQ_32B_sum TCC_EA0_RDREQ_sum",
    "wr": "TCC_EA0_WRREQ_sum TCC_EA0_WRREQ_64B_sum GRBM_GUI_ACTIVE",
    "v1": "SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_THREAD_CYCLES_VALU SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_INSTS_LDS "
          "SQ_ACTIVE_INST_LDS SQ_LDS_BANK_CONFLICT GRBM_GUI_ACTIVE",
    "v2": "SQ_WAIT_INST_ANY SQ_WAIT_ANY SQ_ACTIVE_INST_ANY SQ_INSTS_SALU SQ_ACTIVE_INST_SCA SQ_INSTS_SMEM SQ_WAVES "
          "SQ_INSTS_VMEM_RD GRBM_GUI_ACTIVE",
}
N_XCD, N_SIMD = 8, 1024   # MI355X: GRBM_GUI_ACTIVE sums the 8 XCDs' clocks; 256 CUs x 4 SIMDs


def _read_bytes(c: dict) -> float:
    # L2 -> fabric read requests resolved by size (the FETCH_SIZE expression
    # counts a 128-byte request as 64 bytes on this GPU)
    return (c.get("TCC_EA0_RDREQ_128B_sum", 0.0) * 128 + c.get("TCC_EA0_RDREQ_64B_sum", 0.0) * 64 +
            c.get("TCC_EA0_RDREQ_32B_sum", 0.0) * 32)


def _write_bytes(c: dict) -> float:
    w64 = c.get("TCC_EA0_WRREQ_64B_sum", 0.0)
    return (c.get("TCC_EA0_WRREQ_sum", 0.0) - w64) * 32 + w64 * 64


def summarize_pmc(d: Path) -> dict:
    """Per-kernel HBM bytes and instruction counters of one bench step, from
    the counter passes PMC_PASSES under d/<pass>/, with the byte formulas
    checked on the runtime's copy kernel moving a known number of bytes
    (d/crd, d/cwr; the size in d/crd.log)."""
    calib = None
    for line in (d / "crd.log").read_text().splitlines() if (d / "crd.log").exists() else []:
        if line.startswith("{") and "copy_calibration_bytes" in line:
            calib = json.loads(line)["copy_calibration_bytes"]
    out = {"passes": PMC_PASSES, "kernels": {}}
    if calib:
        cr = _pmc_per_dispatch(d / "crd" / "run_counter_collection.csv")["__amd_rocclr_copyBuffer"][1]
        cw = _pmc_per_dispatch(d / "cwr" / "run_counter_collection.csv")["__amd_rocclr_copyBuffer"][1]
        out["copy_check"] = {"bytes": calib, "read_bytes_counted": _read_bytes(cr),
                             "write_bytes_counted": _write_bytes(cw)}
    # (passes that were not run are left out: bytes alone need rd and wr)
    P = {n: _pmc_per_dispatch(d / n / "run_counter_collection.csv") for n in PMC_PASSES
         if (d / n / "run_counter_collection.csv").exists()}
    for k, (n, c, ms) in P["rd"].items():
        w = P.get("wr", {}).get(k, (0, {}, 0.0))[1]
        v1 = P.get("v1", {}).get(k, (0, {}, 0.0))[1]
        v2 = P.get("v2", {}).get(k, (0, {}, 0.0))[1]
        rb, wb = _read_bytes(c), _write_bytes(w)
        cyc = v1.get("GRBM_GUI_ACTIVE", 0.0) / N_XCD   # the dispatch's clocks
        e = {"dispatches": n, "ms": round(ms, 4), "read_bytes": int(rb), "write_bytes": int(wb),
             "hbm_bytes": int(rb + wb), "hbm_gbs": round((rb + wb) / (ms * 1e6), 1) if ms else None}
        if cyc and v1:
            e["valu_insts"] = int(v1.get("SQ_INSTS_VALU", 0.0))
            # wave64 VALU instructions issued per SIMD per clock (two issue
            # per four clocks from different waves at most for fp32 work)
            e["valu_issue_per_simd_clock"] = round(v1.get("SQ_INSTS_VALU", 0.0) / (N_SIMD * cyc), 4)
            e["valu_lane_util"] = round(v1.get("SQ_THREAD_CYCLES_VALU", 0.0) /
                                        max(1.0, 64 * v1.get("SQ_ACTIVE_INST_VALU", 0.0)), 3)
            e["lds_insts"] = int(v1.get("SQ_INSTS_LDS", 0.0))
            e["lds_bank_conflict_frac"] = round(v1.get("SQ_LDS_BANK_CONFLICT", 0.0) /
                                                max(1.0, v1.get("SQ_ACTIVE_INST_LDS", 0.0)), 4)
        if v2:
            wc = max(1.0, v2.get("SQ_WAVE_CYCLES", v1.get("SQ_WAVE_CYCLES", 1.0)))
            e["salu_insts"] = int(v2.get("SQ_INSTS_SALU", 0.0))
            e["wave_wait_frac"] = round(v2.get("SQ_WAIT_ANY", 0.0) / wc, 3)
            e["wave_issue_wait_frac"] = round(v2.get("SQ_WAIT_INST_ANY", 0.0) / wc, 3)
        out["kernels"][k] = e
    return out


def config1_point(lib, seed):
    """The single-head configuration (T = 4096, d = 128, four outlier channels
    x8, cheap reference queries, keep 0.5): the GPU library through the host
    entry point, and the reference CPU path on one thread and on every core."""
    sys.path.insert(0, str(REPO / "tests"))
    from kvc_data import kv_cache
    T, H, d = 4096, 1, 128
    K, V = kv_cache(T, H, d, seed, outliers=4)
    out = {"workload": "1 layer x 1 KV head x d=128, T=4096, fp32, 4 outlier channels x8, cheap Q_ref, keep 0.5"}
    p = lib.params(target_ratio=0.5, use_cheap_qref=1)
    lib.compact(K, V, None, T, 0, H, d, d, p)   # warm
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        lib.compact(K, V, None, T, 0, H, d, d, p)
        ts.append(time.perf_counter() - t0)
    out["gpu_host_entry_tok_s"] = round(T / float(np.median(ts)), 1)
    ref = REPO / "oracle" / "_ref" / "libkvref.so"
    if ref.exists():
        rl = kc.Lib(ref)
        for threads in (1, 0):
            pr = rl.params(target_ratio=0.5, use_cheap_qref=1, n_threads=threads)
            ts = []
            for _ in range(3):
                t0 = time.perf_counter()
                rl.compact(K, V, None, T, 0, H, d, d, pr)
                ts.append(time.perf_counter() - t0)
            key = "cpu_reference_1_thread_tok_s" if threads == 1 else "cpu_reference_all_threads_tok_s"
            out[key] = round(T / float(np.median(ts)), 1)
    return out


def drop_in_mode(lib, L, T, H, d, W, ratio, diversity, seed):
    """Drop-in mode: the reference's own host-pointer kv_compact() once per
    layer (host buffers in, malloc'd results out), every layer of the
    workload; the time counts the C calls only, kv_compact and
    kv_compact_result_free (data generation and this wrapper's copy of the
    results into numpy excluded)."""
    p = lib.params(target_ratio=ratio, use_diversity=diversity)
    total = 0.0
    for l, (K, V, Q) in enumerate(gen_layers(L, T, H, d, W, seed)):
        if l == 0:   # untimed warm-up call (the library's pinned transfer ring is allocated on first use)
            rc, r = lib.compact_raw(K, V, Q, T, W, H, d, d, p)
            lib.free_result(r)
        t0 = time.perf_counter()
        rc, r = lib.compact_raw(K, V, Q, T, W, H, d, d, p)
        lib.free_result(r)
        total += time.perf_counter() - t0
        if rc != 0:
            raise RuntimeError(f"kv_compact returned {rc}")
    bytes_in = 2 * L * T * H * d * 4
    return {"value": round(T / total, 1), "unit": "tok/s", "seconds": round(total, 3),
            "host_to_device_gb": round(bytes_in / 1e9, 2),
            "host_link_bound_tok_s": round(T / (bytes_in / 64e9), 1),
            "note": f"{L} kv_compact calls with pageable host buffers (one layer each), results copied back "
                    "into malloc'd arrays, each call's kv_compact_result_free included; one untimed warm-up call"}


def quantized_mode(dll, lib, hiprt, L, T, H, d, ratio, steps, warmup, seed):
    """Q8_0 and Q4_0 caches of N(0,1) data: the multi-layer quantized device
    entry (compact, requantize) on all layers, inputs resident; the kernels
    decode K and V blocks in registers as they load them. The same call with
    KVC_INPLACE=0 (a whole-cache decode to fp32 first) is reported beside it."""
    sys.path.insert(0, str(REPO / "tests"))
    from kvc_data import quantize_rows
    E = H * d
    p = lib.params(target_ratio=ratio, use_cheap_qref=1)
    t, n_chunks = kc.plan(dll, T, 0, False, p)
    res = {"workload": f"{L} layers x {H} KV heads x d={d}, T={T}, keep {ratio:g} (t={t}/layer, {n_chunks} chunks), "
                       f"cheap Q_ref, K and V in the codec"}
    rng = np.random.default_rng(seed)
    for typ, name in ((8, "q8_0"), (2, "q4_0")):
        pool = quantize_rows(rng.standard_normal((T + 4096, E), dtype=np.float32), typ)
        rb = pool.shape[1]
        dKq, dVq = hiprt.DevBuf(L * T * rb), hiprt.DevBuf(L * T * rb)
        for l in range(L):
            o1, o2 = (int(x) for x in rng.integers(0, 4096, size=2))
            dKq.upload(pool[o1:o1 + T], l * T * rb)
            dVq.upload(pool[o2:o2 + T], l * T * rb)
        bufs = [hiprt.DevBuf(n * 4) for n in (L * t, L * H * t, L * H * t * d, L * 3)]
        ko, vo = hiprt.DevBuf(L * t * rb), hiprt.DevBuf(L * t * rb)
        out = kc.DeviceOut(*(b.value for b in bufs))

        def step():
            rc = dll.kvc_compact_quantized_layers_device(dKq.value, dVq.value, None, L, typ, typ, rb, rb, T, 0, H, d,
                                                         d, T * rb, T * rb, 0, ctypes.byref(p), ctypes.byref(out),
                                                         ko.value, vo.value, None)
            if rc != 0:
                raise RuntimeError(f"kvc_compact_quantized_layers_device returned {rc}")

        for mode in ("1", "0"):
            old_env = os.environ.get("KVC_INPLACE")
            os.environ["KVC_INPLACE"] = mode
            try:
                for _ in range(warmup):
                    step()
                hiprt.synchronize()
                acc = np.zeros(len(QSTAGES))
                buf = (ctypes.c_float * len(QSTAGES))()
                t0 = time.perf_counter()
                for _ in range(steps):
                    step()
                    dll.kvc_stage_times(buf, len(QSTAGES))
                    acc += np.array(buf[:])
                hiprt.synchronize()
                ms = (time.perf_counter() - t0) / steps * 1e3
            finally:
                if old_env is None:
                    os.environ.pop("KVC_INPLACE", None)
                else:
                    os.environ["KVC_INPLACE"] = old_env
            acc /= steps
            st = dict(zip(QSTAGES, acc))
            if mode == "1":
                # kept K rows decoded and re-encoded (read and write the rows),
                # C_v read and its rows written
                rq_bytes = L * t * (2 * rb + E * 4 + rb)
                r = {"decode": "in the kernels' loads (no fp32 copy of the cache)",
                     "value": round(T / (ms / 1e3), 1), "unit": "tok/s", "ms_per_step": round(ms, 3),
                     "row_bytes": rb, "stage_ms": {k: round(float(v), 3) for k, v in st.items()}}
            else:
                dq_bytes = 2 * L * T * (rb + E * 4)             # read the rows, write fp32
                rq_bytes = 2 * L * t * (E * 4 + rb)             # read kept K rows and C_v, write the rows
                r = {"decode": "whole-cache pass to fp32 first (KVC_INPLACE=0)",
                     "value": round(T / (ms / 1e3), 1), "unit": "tok/s", "ms_per_step": round(ms, 3),
                     "stage_ms": {k: round(float(v), 3) for k, v in st.items()},
                     "dequantize_gb_s": round(dq_bytes / (st["dequantize"] / 1e3) / 1e9, 1)
                     if st["dequantize"] else None,
                     "dequantize_frac_hbm": round(dq_bytes / (st["dequantize"] / 1e3) / 1e9 / HBM_PEAK_GBS, 4)
                     if st["dequantize"] else None,
                     "dequantize_bytes": dq_bytes}
            r["requantize_gb_s"] = round(rq_bytes / (st["requantize"] / 1e3) / 1e9, 1) if st["requantize"] else None
            r["requantize_frac_hbm"] = (round(rq_bytes / (st["requantize"] / 1e3) / 1e9 / HBM_PEAK_GBS, 4)
                                        if st["requantize"] else None)
            r["requantize_bytes"] = rq_bytes
            res[name if mode == "1" else name + "_whole_cache"] = r
            print(f"[bench] quantized {name} inplace={mode}: {ms:.1f} ms per step, dequantize "
                  f"{st['dequantize']:.2f} ms, requantize {st['requantize']:.2f} ms", file=sys.stderr, flush=True)
        del dKq, dVq, bufs, ko, vo
    return res


def state_mode(dll, hiprt, L, T, H, d, ratio, steps, warmup, seed):
    """A llama.cpp sequence state blob (F16 K and V rows, L layers x H heads x
    d) compacted by kvc_state_compact_device: parse, score every layer with the
    default reference queries (the last max(16, T/4) keys), one top-t across
    layers and heads, per-head value refit and beta directions, blob written
    back; device blob in, device blob out."""
    sys.path.insert(0, str(REPO / "tests"))
    from kvc_data import T_F16, state_blob
    c = dict(T=T, L=L, H=H, dk=d, dv=d, kt=T_F16, vt=T_F16, vtrans=0, seed=seed, ratio=ratio)
    blob = state_blob(c)
    p, keep = kc.state_params(ratio, H)
    f = dll.kvc_state_compact_device
    f.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(kc.StateParams), ctypes.c_void_p,
                  ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t), ctypes.c_void_p, ctypes.c_void_p]
    f.restype = ctypes.c_int
    src, dst = hiprt.DevBuf(len(blob)), hiprt.DevBuf(len(blob))
    src.upload(np.frombuffer(blob, np.uint8))
    n = ctypes.c_size_t(0)

    def step():
        rc = f(src.value, len(blob), ctypes.byref(p), dst.value, len(blob), ctypes.byref(n), None, None)
        if rc != 0:
            raise RuntimeError(f"kvc_state_compact_device returned {rc}")
    for _ in range(warmup):
        step()
    hiprt.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    hiprt.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    t = max(1, int(np.float32(T) * np.float32(ratio)))
    del keep
    return {"workload": f"{L} layers x {H} KV heads x d={d}, {T} cells, F16 rows, keep {ratio:g} "
                        f"({t} cells, one set for all layers), default reference queries ({max(16, T // 4)})",
            "ms_per_call": round(ms, 3), "cells_per_s": round(T / (ms / 1e3), 1),
            "blob_bytes_in": len(blob), "blob_bytes_out": int(n.value)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--T", type=int, default=100000)
    ap.add_argument("--heads", type=int, default=8)
    ap.add_argument("--dim", type=int, default=128)
    ap.add_argument("--ratio", type=float, default=0.2)
    ap.add_argument("--window", type=int, default=32)
    ap.add_argument("--diversity", type=int, default=1,
                    help="1 (default): diversity selection on, the headline mode; the other mode is "
                         "timed after it and reported under 'other_mode'")
    ap.add_argument("--one-mode", action="store_true", help="time only the --diversity mode")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the extra records (config-1 point, drop-in mode, quantized caches)")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--summarize-pmc", metavar="DIR", default="",
                    help="summarise rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE csv runs under DIR "
                         "(cf/, cw/: copy calibration; bf/, bw/: one bench step) into per-kernel HBM "
                         "bytes per dispatch, printed as JSON, and exit")
    ap.add_argument("--quantized-only", action="store_true",
                    help="only time the quantized-cache record (32 layers, T=32768, Q8_0 and Q4_0, "
                         "decoded in the kernels' loads and by a whole-cache pass), print it as JSON and exit")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only copy BYTES device-to-device once (the reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and exit")
    a = ap.parse_args()
    if a.summarize_pmc:
        print(json.dumps(summarize_pmc(Path(a.summarize_pmc)), indent=1))
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for {max(a.gpus, world)}); "
              "the compaction path shards by layer or chunk with no exchange, which this build does not run",
              file=sys.stderr)
        sys.exit(2)

    import hiprt
    if a.copy_calibration:
        src, dst = hiprt.DevBuf(a.copy_calibration), hiprt.DevBuf(a.copy_calibration)
        src.zero()
        hiprt.synchronize()
        hiprt.check(hiprt.hip().hipMemcpy(dst.value, src.value, a.copy_calibration, hiprt.D2D), "hipMemcpy D2D")
        hiprt.synchronize()
        # the same copy timed (10 back to back): the rate a plain device copy
        # reaches on this GPU, reading and writing BYTES each
        e0, e1 = hiprt.Event(), hiprt.Event()
        e0.record()
        for _ in range(10):
            hiprt.check(hiprt.hip().hipMemcpyAsync(dst.value, src.value, a.copy_calibration, hiprt.D2D, None),
                        "hipMemcpyAsync D2D")
        e1.record()
        ms = e0.elapsed_ms(e1) / 10
        print(json.dumps({"copy_calibration_bytes": a.copy_calibration, "copy_ms": round(ms, 4),
                          "copy_gb_s": round(2 * a.copy_calibration / (ms * 1e6), 1)}), flush=True)
        return
    lib = kc.load_product()
    dll = kc.bind_device_api(lib.dll)
    if not dll.kv_compact_hip_available():
        raise SystemExit("no usable GPU")
    if a.quantized_only:
        print(json.dumps({"quantized": quantized_mode(dll, lib, hiprt, 32, 32768, a.heads, a.dim, a.ratio, a.steps,
                                                      a.warmup, a.seed + 7)}), flush=True)
        return
    L, T, H, d, W = a.layers, a.T, a.heads, a.dim, a.window
    E = H * d
    p = lib.params(target_ratio=a.ratio, use_diversity=a.diversity)
    t, n_chunks = kc.plan(dll, T, W, True, p)

    dK = hiprt.DevBuf(L * T * E * 4)
    dV = hiprt.DevBuf(L * T * E * 4)
    dQ = hiprt.DevBuf(L * W * E * 4)
    first = None
    t0 = time.perf_counter()
    for l, (K, V, Q) in enumerate(gen_layers(L, T, H, d, W, a.seed)):
        dK.upload(K, l * T * E * 4)
        dV.upload(V, l * T * E * 4)
        dQ.upload(Q, l * W * E * 4)
        if l == 0:
            first = (K.copy(), V.copy(), Q.copy())
    print(f"[bench] data ready: {L} layers x T={T} x {H}x{d} ({2 * L * T * E * 4 / 1e9:.1f} GB) in "
          f"{time.perf_counter() - t0:.1f} s; t={t} per layer, {n_chunks} chunks", file=sys.stderr, flush=True)
    idx = hiprt.DevBuf(L * t * 4)
    beta = hiprt.DevBuf(L * H * t * 4)
    cv = hiprt.DevBuf(L * H * t * d * 4)
    st = hiprt.DevBuf(L * 3 * 4)
    out = kc.DeviceOut(idx.value, beta.value, cv.value, st.value)

    def timed(params, tag):
        """warmup, then exactly a.steps timed calls bracketed by device syncs"""
        def step():
            rc = dll.kvc_compact_layers_device(dK.value, dV.value, dQ.value, L, T, W, H, d, d, T * E, T * E,
                                               W * E, ctypes.byref(params), None, ctypes.byref(out), None)
            if rc != 0:
                raise RuntimeError(f"kvc_compact_layers_device returned {rc}")

        acc = np.zeros(len(STAGES))
        buf = (ctypes.c_float * len(STAGES))()
        for i in range(a.warmup):
            ts = time.perf_counter()
            step()
            print(f"[bench] {tag} warmup {i}: {(time.perf_counter() - ts) * 1e3:.1f} ms", file=sys.stderr, flush=True)
        hiprt.synchronize()
        t_start = time.perf_counter()
        for i in range(a.steps):
            ts = time.perf_counter()
            step()
            dll.kvc_stage_times(buf, len(STAGES))
            acc += np.array(buf[:])
            print(f"[bench] {tag} step {i}: {(time.perf_counter() - ts) * 1e3:.1f} ms", file=sys.stderr, flush=True)
        hiprt.synchronize()
        return (time.perf_counter() - t_start) / a.steps * 1e3, acc / a.steps

    other = None
    if not a.one_mode:
        p_other = lib.params(target_ratio=a.ratio, use_diversity=0 if a.diversity else 1)
        ms_o, stage_o = timed(p_other, "diversity " + ("off" if a.diversity else "on"))
        other = {"diversity": "off" if a.diversity else "on", "value": round(T / (ms_o / 1e3), 1),
                 "ms_per_step": round(ms_o, 3),
                 "stage_ms": {k: round(float(v), 3) for k, v in zip(STAGES, stage_o)}}
    ms, stage_ms = timed(p, "diversity " + ("on" if a.diversity else "off"))
    model = stage_model(L, T, H, d, W, t, n_chunks, 256 if n_chunks > 1 else t)
    dom = STAGES[int(np.argmax(stage_ms))]
    roof = roofline(dom, model, float(stage_ms[int(np.argmax(stage_ms))]))
    # HBM bytes per launch of the dominant kernel from the committed rocprofv3
    # FETCH_SIZE / WRITE_SIZE summary of this exact workload (copy-calibrated)
    prof = REPO / "profiles" / "hbm_traffic_100k_32layer_pmc.json"
    headline = (L, T, H, d, W, a.ratio, a.diversity) == (32, 100000, 8, 128, 32, 0.2, 1)
    # the profiler's names of the stage's kernels (the LU: the whole-matrix
    # kernel's split instance for steps 0-127, then the trailing-matrix
    # kernel; every system of this workload runs these two)
    knames = {"lu_factorization": ["kvc::k_ge_lu<false, true>", "kvc::k_ge_lu_tail"]}.get(
        dom, ["kvc::" + STAGE_KERNELS[dom]])
    if headline and prof.exists():
        kern = json.loads(prof.read_text())["kernels"]
        if all(k in kern for k in knames):
            roof["traffic"] = sum(kern[k]["hbm_bytes"] for k in knames)
            roof["traffic_source"] = str(prof.relative_to(REPO))
    stats = st.download(np.float32, L * 3).reshape(L, 3)
    del dK, dV, dQ, idx, beta, cv, st

    extras = {}
    if not a.no_extras:
        extras["quantized"] = quantized_mode(dll, lib, hiprt, 32, 32768, H, d, a.ratio, a.steps, a.warmup, a.seed + 7)
        extras["state_blob"] = state_mode(dll, hiprt, 32, 2048, H, d, a.ratio, 3, 1, a.seed + 11)
        print(f"[bench] state blob: {extras['state_blob']}", file=sys.stderr, flush=True)
        extras["drop_in_host_pointers"] = drop_in_mode(lib, L, T, H, d, W, a.ratio, a.diversity, a.seed)
        print(f"[bench] drop-in mode: {extras['drop_in_host_pointers']}", file=sys.stderr, flush=True)
        extras["config1"] = config1_point(lib, 101)
        print(f"[bench] config 1: {extras['config1']}", file=sys.stderr, flush=True)

    cpu = None
    if not a.no_cpu:
        K0, V0, Q0 = first
        cpu = cpu_baseline(K0, V0, Q0, T, H, d, a.ratio, L, a.diversity)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)

    line = {
        "metric": "compacted tok/s @100k ctx, 20% keep (32L×8H, d=128); % of MFMA/HBM peak",
        "value": round(T / (ms / 1e3), 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{L} layers x {H} KV heads x d={d}, T={T}, fp32, keep {a.ratio:g} "
                        f"(t={t}/layer, {n_chunks} chunks), SnapKV W={W}, RMS, skip_beta=1, "
                        f"diversity={'on' if a.diversity else 'off'}",
            "layers": L, "T": T, "kv_heads": H, "head_dim": d, "keep_ratio": a.ratio, "kept_per_layer": t,
            "parallelism": "single GPU", **host_info(),
        },
        "stage_ms": {k: round(float(v), 3) for k, v in zip(STAGES, stage_ms)},
        "other_mode": other,
        "roofline": roof,
        "cpu_baseline": cpu,
        "speedup_vs_cpu": round((T / (ms / 1e3)) / cpu["value"], 1) if cpu else None,
        "quality": {"avg_cosine_sim_layer0": float(stats[0, 0]), "avg_cosine_sim_min": float(stats[:, 0].min())},
        **extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
