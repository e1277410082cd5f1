#!/usr/bin/env python3
"""Benchmark of the MI355X bf16 flash-attention forward (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

One step = one attn_flash call (one fused kernel launch) over the headline workload,
Benchmark configuration c3 at 4k: GQA prefill B=4, Hq=32, Hkv=8, D=128, Sq=Sk=4096, non-causal,
bf16 Q/K/V ~ N(0,1) (synthetic, seeded), fp32 O. Inputs are resident in HBM before timing;
each timed call rotates through a pool of input copies larger than 2x the 256 MiB Infinity
Cache, so every call streams from HBM (the reference's DDR-cold rule, flash.c:982-991).

Prints ONE JSON line on stdout (diagnostics go to stderr). `value` is TFLOP/s of useful
work 4*B*Hq*Sq*Sk*D per step over the wall-clock of the timed steps; `roofline.achieved`
is the same work over the kernel's average duration from HIP events on its stream. The
other benchmark configurations (decode GB/s, 1k/2k prefill, MQA, ragged) are reported
under "extra". The CPU baseline is the oracle (the reference's scalar fp32 attn_ref,
restated in C) timed on a bounded spread-row sample of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 (published)
HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E (published)
SEED0 = 0x12345678
INFINITY_CACHE = 256 << 20

# VALU-issue floor of the online softmax, per score and SIMD: one v_fma_f32 (s*c - m*c), one
# v_exp_f32, one v_add_f32 (the row sum of the fp32 p) and half a v_cvt_pk_bf16_f32 (P to bf16),
# with packed FP32 off. A wave64 VALU instruction takes 4 cycles on a 16-lane SIMD; v_exp_f32
# about twice that (roofline_bench valu: 4.4 cycles per fma, 11.8 per exp + add step). That is
# 18 cycles per 64 scores. 1024 SIMDs at the 2.4 GHz rating.
VALU_CYCLES_PER_SCORE = (4 + 8 + 4 + 2) / 64.0
SIMDS, CLOCK_HZ = 1024, 2.4e9


def bounds(flops, scores, kernel_ms):
    """The MFMA and VALU-issue floors of a prefill (ms) and the kernel's fraction of the higher
    one, the roofline that binds: D = 64 has half the MFMA work per score of D = 128 and the same
    softmax, so its VALU floor passes its MFMA floor."""
    mfma_ms = flops / (MFMA_BF16_PEAK_TFLOPS * 1e12) * 1e3
    valu_ms = scores * VALU_CYCLES_PER_SCORE / (SIMDS * CLOCK_HZ) * 1e3
    bound = "valu" if valu_ms > mfma_ms else "mfma"
    return {"mfma_floor_ms": mfma_ms, "valu_floor_ms": valu_ms, "bound": bound,
            "bound_frac": max(mfma_ms, valu_ms) / kernel_ms}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_inputs(ts, B, Hq, Hkv, Sq, Sk, D, seed, sigma_q=1.0, copies=1):
    """Upload `copies` distinct input sets (copy 0 is the config's seeded data)."""
    bufs = []
    for c in range(copies):
        Q, K, V = ts.synth_normal_qkv(B * Hq, B * Hkv, Sq, Sk, D, seed + 0x10000 * c,
                                      sigma_q=sigma_q)
        bufs.append((ts.DeviceBuffer.from_array(Q), ts.DeviceBuffer.from_array(K),
                     ts.DeviceBuffer.from_array(V), ts.DeviceBuffer(B * Hq * Sq * D * 4),
                     (Q, K, V) if c == 0 else None))
    return bufs


def prepack(ts, bufs, B, Hkv, Sk, D):
    """Replace each copy's row-major V by V^T [Hkv][D][Sk] made on the device by pack_v_full
    (the operator the reference runs outside the timed attention, flash.c:1070-1089)."""
    out = []
    for q, k, v, o, host in bufs:
        vp = ts.DeviceBuffer(v.nbytes)
        ts.pack_v_full(v, vp, B * Hkv, Sk, D)
        ts.synchronize()
        v.free()
        out.append((q, k, vp, o, host))
    return out


def time_pack_v(ts, bufs, B, Hkv, Sk, D, steps=24):
    """Kernel ms of one pack_v_full over the workload's V (HIP events). The inputs rotate
    through copies of V's size totalling more than 2x the 256 MiB Infinity Cache, as the
    attention calls' inputs do, so every call reads V from HBM."""
    v = bufs[0][2]
    n = max(2, -(-2 * INFINITY_CACHE // v.nbytes) + 1)
    pool = [ts.DeviceBuffer(v.nbytes) for _ in range(n)]
    try:
        for p in pool:
            p.fill_bytes(0x3c)
        with ts.DeviceBuffer(v.nbytes) as vp:
            ts.pack_v_full(pool[0], vp, B * Hkv, Sk, D)
            ts.synchronize()
            e0, e1 = ts.Event(), ts.Event()
            e0.record()
            for i in range(steps):
                ts.pack_v_full(pool[(i + 1) % n], vp, B * Hkv, Sk, D)
            e1.record()
            ts.synchronize()
            return e0.elapsed_ms(e1) / steps
    finally:
        for p in pool:
            p.free()


# Untimed warmup runs at least `warmup` calls and at least this long: after the host-side work
# between legs (uploads, oracle checks) the GPU is idle, and its clock then takes about 40 ms
# of work to settle (measured from idle with `bench.py --ramp`: the first 10-call windows of
# c3 4k run 1.06, 0.90, 0.887 ms/call, then stay at 0.89). A few calls of warmup leave most of
# a short timed window inside that ramp.
WARMUP_MIN_S = 0.2


def time_calls(ts, bufs, B, Hq, Hkv, Sq, Sk, D, causal, bk, scratch, steps, warmup, vp=0):
    """Returns (wall ms per step, HIP-event kernel ms per step). vp=1: V buffers hold V^T."""
    n = len(bufs)
    i, t0 = 0, time.perf_counter()
    while i < warmup or time.perf_counter() - t0 < WARMUP_MIN_S:
        q, k, v, o, _ = bufs[i % n]
        ts.attn_flash(q, k, v, o, B * Hq, B * Hkv, Sq, Sk, D, causal, bk, scratch, vp)
        i += 1
        if i % 16 == 0:
            ts.synchronize()  # the host clock above then tracks the GPU's work
    ts.synchronize()
    e0, e1 = ts.Event(), ts.Event()
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        q, k, v, o, _ = bufs[i % n]
        ts.attn_flash(q, k, v, o, B * Hq, B * Hkv, Sq, Sk, D, causal, bk, scratch, vp)
    e1.record()
    ts.synchronize()
    t1 = time.perf_counter()
    return (t1 - t0) * 1e3 / steps, e0.elapsed_ms(e1) / steps


def parity(ts, o, bufs, B, Hq, Hkv, Sq, Sk, D, causal, ref_cap, nthreads):
    """err/scale of copy 0 against the oracle on spread rows (reference pass rule)."""
    Q, K, V = bufs[0][4]
    O = bufs[0][3].download(np.float32)
    rows = o.ref_rowset(Sq, ref_cap)
    R = o.attn_ref(Q, K, V, B * Hq, B * Hkv, Sq, Sk, D, causal, rows, nthreads=nthreads)
    ok, mad, maxref, nbad = o.cmp_rows(R, O, B * Hq, Sq, D, rows)
    return {"err_over_scale": float(mad / maxref) if maxref else 0.0, "nbad": int(nbad),
            "pass": bool(ok), "rows_checked_per_head": int(len(rows))}


def traffic_from_profiles(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE), scaled by
    the copy-kernel calibration; read from the committed summary, or None."""
    p = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(p):
        return None
    for line in open(p):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def measured_peaks():
    """Run the roofline microbenchmark (MFMA with constant and with random operands, HBM
    stream read); returns its JSON fields or {} if the tool is not built."""
    import subprocess
    from transfer_station_amd import build as b
    tool = b.tool_path("roofline_bench")
    out = {}
    for mode in ("mfma", "read"):
        try:
            r = subprocess.run([tool, mode, "2048"] if mode == "read" else [tool, mode],
                               capture_output=True, text=True, timeout=120)
            if r.returncode == 0:
                out.update(json.loads(r.stdout.strip().splitlines()[-1]))
        except (OSError, subprocess.SubprocessError, ValueError):
            pass
    return out


# A GPU box grants one GPU's job a share of 16 host cores, whatever os.cpu_count() reports
# there; the all-cores leg uses every core this process may run on, up to that share.
BOX_CPU_SHARE = 16


def host_threads():
    """(threads to use, cores this process may run on, cores the host reports)."""
    allowed = len(os.sched_getaffinity(0))
    return min(BOX_CPU_SHARE, allowed), allowed, os.cpu_count() or allowed


def cpu_baseline(o, ts, budget_s=16.0):
    """The oracle on the headline workload's rows, 1 thread and all allowed threads."""
    B, Hq, Hkv, S, D = 4, 32, 8, 4096, 128
    Q, K, V = ts.synth_normal_qkv(B * Hq, B * Hkv, S, S, D, SEED0 + 3)
    flop_per_row = 4.0 * S * D
    out = {}
    nthreads, allowed, host = host_threads()
    for label, nt in (("1", 1), ("all", nthreads)):
        # grow the row sample (up to 64 rows of each of the B*Hq heads) until the run takes a
        # meaningful time, within the budget
        ref_cap, heads, dt = 2, 1, 0.0
        while True:
            rows = o.ref_rowset(S, ref_cap)
            t0 = time.perf_counter()
            o.attn_ref(Q[: heads * S * D], K[: max(1, heads // 4) * S * D],
                       V[: max(1, heads // 4) * S * D], heads, max(1, heads // 4), S, S, D, 0,
                       rows, nthreads=nt)
            dt = time.perf_counter() - t0
            if dt > budget_s / 4 or (ref_cap >= 64 and heads >= B * Hq):
                break
            if ref_cap < 64:
                ref_cap *= 2
            else:
                heads = min(2 * heads, B * Hq)
        nrows = len(rows) * heads
        out[label] = {"rows": nrows, "seconds": dt, "tflops": nrows * flop_per_row / dt / 1e12,
                      "threads": nt}
    allc = out["all"]
    full_flop = 4.0 * B * Hq * S * S * D
    # config 2 (decode) is small enough to run whole on the CPU: every row, all threads
    Bd, Hqd, Hkvd, Skd, Dd = 64, 32, 8, 4096, 128
    Qd, Kd, Vd = ts.synth_normal_qkv(Bd * Hqd, Bd * Hkvd, 1, Skd, Dd, SEED0 + 2)
    t0 = time.perf_counter()
    o.attn_ref(Qd, Kd, Vd, Bd * Hqd, Bd * Hkvd, 1, Skd, Dd, 0, nthreads=nthreads)
    c2_s = time.perf_counter() - t0
    return {"value": allc["tflops"], "unit": "TFLOP/s", "cores": allc["threads"],
            "cores_allowed": allowed, "host_cpu_count": host,
            "cores_note": "all-cores leg = min(%d, cores in this process's affinity mask); "
                          "%d is the host-core share a one-GPU job gets on the GPU box"
                          % (BOX_CPU_SHARE, BOX_CPU_SHARE),
            "kind": "port",
            "sample": "oracle attn_ref (flash.c:262-314 restated in C, gcc -O2, OpenMP over "
                      "(head,row)) on %d spread query rows of config 3 @4k (Sk=4096, D=128), "
                      "%.2f s; single-thread: %.4f TFLOP/s on %d rows" %
                      (allc["rows"], allc["seconds"], out["1"]["tflops"], out["1"]["rows"]),
            "value_1core": out["1"]["tflops"],
            "c3_4k_full_problem_seconds_extrapolated": {
                "all_threads": full_flop / (allc["tflops"] * 1e12),
                "single_thread": full_flop / (out["1"]["tflops"] * 1e12)},
            "c2_decode_full_problem_seconds_measured": {"all_threads": c2_s,
                                                        "threads": nthreads}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--bk", type=int, default=128)
    ap.add_argument("--no-extra", action="store_true", help="headline only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-peaks", action="store_true",
                    help="skip the roofline microbenchmark (e.g. under a profiler)")
    ap.add_argument("--ramp", action="store_true",
                    help="instead of the benchmark: ms per call of the headline workload in "
                         "10-call windows from an idle GPU (the clock ramp the warmup covers)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        sys.exit("bench.py: this build measures ONE GPU only (the path shards over (batch, "
                 "kv-head) units with no communication; multi-GPU runs are not part of it)")

    import transfer_station_amd as ts
    from oracle import oracle as o

    info = ts.device_info()
    log("device:", info)
    nthreads = host_threads()[0]

    # ---- headline: config 3 @ 4k --------------------------------------------------------------
    B, Hq, Hkv, S, D = 4, 32, 8, 4096, 128
    flops = 4.0 * B * Hq * S * S * D
    in_bytes = (B * Hq * S * D + 2 * B * Hkv * S * D) * 2
    copies = max(1, -(-2 * INFINITY_CACHE // in_bytes) + 0)
    log("headline: c3 GQA prefill 4k, %d input copies (%.0f MiB each)" %
        (copies, in_bytes / 2 ** 20))
    bufs = make_inputs(ts, B, Hq, Hkv, S, S, D, SEED0 + 3, copies=copies)
    scratch = ts.DeviceBuffer(ts.attn_flash_scratch_bytes(D, args.bk))
    if args.ramp:
        for causal in (0, 1):
            time.sleep(3.0)  # idle, as between the legs
            wins, i, t0 = [], 0, time.perf_counter()
            while time.perf_counter() - t0 < 0.4:
                e0, e1 = ts.Event(), ts.Event()
                e0.record()
                for _ in range(10):
                    q, k, v, o_, _ = bufs[i % len(bufs)]
                    ts.attn_flash(q, k, v, o_, B * Hq, B * Hkv, S, S, D, causal, args.bk, scratch)
                    i += 1
                e1.record()
                ts.synchronize()
                wins.append([round((time.perf_counter() - t0) * 1e3, 1),
                             round(e0.elapsed_ms(e1) / 10, 4)])
            print(json.dumps({"ramp": "c3 4k" + (" causal" if causal else ""),
                              "windows_ms_since_idle_and_ms_per_call": wins}), flush=True)
        return
    wall_ms, kern_ms = time_calls(ts, bufs, B, Hq, Hkv, S, S, D, 0, args.bk, scratch, args.steps,
                                  args.warmup)
    value = flops / (wall_ms * 1e-3) / 1e12
    achieved = flops / (kern_ms * 1e-3) / 1e12
    head_parity = parity(ts, o, bufs, B, Hq, Hkv, S, S, D, 0, 8, nthreads)
    log("headline: %.3f ms/step wall, %.3f ms kernel -> %.1f TFLOP/s (%.1f%% of peak); %s" %
        (wall_ms, kern_ms, achieved, 100 * achieved / MFMA_BF16_PEAK_TFLOPS, head_parity))
    traffic = traffic_from_profiles("attn_prefill_c3_4k_traffic.txt")

    extra = {}
    if not args.no_extra:
        # ---- the same workload, causal (useful work = unmasked pairs only) ---------------------
        cflops = 4.0 * B * Hq * D * (S * (S + 1) // 2)
        w, k = time_calls(ts, bufs, B, Hq, Hkv, S, S, D, 1, args.bk, scratch, 20, 3)
        pc = parity(ts, o, bufs, B, Hq, Hkv, S, S, D, 1, 8, nthreads)
        extra["c3_gqa_prefill_4k_causal"] = {
            "kernel_ms": k, "TFLOP_s": cflops / (k * 1e-3) / 1e12,
            "mfma_frac": cflops / (k * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "flop_note": "4*D per unmasked (q,k) pair", "parity": pc,
            **bounds(cflops, cflops / (4.0 * D), k)}
        log("c3 4k causal:", extra["c3_gqa_prefill_4k_causal"])
        # ---- the same workload with a pre-packed V^T (v_prepacked=1) ---------------------------
        pk_ms = time_pack_v(ts, bufs, B, Hkv, S, D)
        bufs = prepack(ts, bufs, B, Hkv, S, D)
        w, k = time_calls(ts, bufs, B, Hq, Hkv, S, S, D, 0, args.bk, scratch, 20, 3, vp=1)
        pv = parity(ts, o, bufs, B, Hq, Hkv, S, S, D, 0, 8, nthreads)
        extra["c3_gqa_prefill_4k_v_prepacked"] = {
            "kernel_ms": k, "TFLOP_s": flops / (k * 1e-3) / 1e12,
            "mfma_frac": flops / (k * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "pack_v_full_ms": pk_ms,
            "pack_v_full_GB_s": 2 * B * Hkv * S * D * 2 / (pk_ms * 1e-3) / 1e9, "parity": pv}
        log("c3 4k v_prepacked:", extra["c3_gqa_prefill_4k_v_prepacked"])
    for b in bufs:
        for x in b[:4]:
            x.free()

    if not args.no_extra:
        # ---- config 2: GQA decode (HBM-bound) ------------------------------------------------
        Bd, Hqd, Hkvd, Skd, Dd = 64, 32, 8, 4096, 128
        dbytes = (Bd * Hqd * Dd + 2 * Bd * Hkvd * Skd * Dd) * 2 + Bd * Hqd * Dd * 4
        db = make_inputs(ts, Bd, Hqd, Hkvd, 1, Skd, Dd, SEED0 + 2, copies=1)
        w, k = time_calls(ts, db, Bd, Hqd, Hkvd, 1, Skd, Dd, 0, args.bk, scratch, 50, 5)
        p2 = parity(ts, o, db, Bd, Hqd, Hkvd, 1, Skd, Dd, 0, 0, nthreads)
        extra["c2_gqa_decode"] = {"kernel_us": k * 1e3, "wall_us": w * 1e3,
                                  "GB_s": dbytes / (k * 1e-3) / 1e9,
                                  "hbm_frac": dbytes / (k * 1e-3) / 1e9 / HBM_PEAK_GBPS,
                                  "bytes_per_call": dbytes, "parity": p2,
                                  "traffic": traffic_from_profiles(
                                      "attn_decode_c2_traffic.txt")}
        log("c2 decode:", extra["c2_gqa_decode"])
        db = prepack(ts, db, Bd, Hkvd, Skd, Dd)
        w, k = time_calls(ts, db, Bd, Hqd, Hkvd, 1, Skd, Dd, 0, args.bk, scratch, 50, 5, vp=1)
        extra["c2_gqa_decode_v_prepacked"] = {
            "kernel_us": k * 1e3, "GB_s": dbytes / (k * 1e-3) / 1e9,
            "hbm_frac": dbytes / (k * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "parity": parity(ts, o, db, Bd, Hqd, Hkvd, 1, Skd, Dd, 0, 0, nthreads)}
        log("c2 decode v_prepacked:", extra["c2_gqa_decode_v_prepacked"])
        for b in db:
            for x in b[:4]:
                x.free()
        # ---- config 3 at 1k/2k, config 4, config 5, config 1 --------------------------------
        # (name, B, Hq, Hkv, Sq, Sk, D, sigma_q, seed index, bks, causal); qwen3_4k_causal is the
        # reference's own --long case (flash.c:1312-1314), causal, useful flops only; the last
        # one is a serving shape outside the benchmark configurations (a 512-query chunk over
        # 8192 keys, batch 1: few query tiles, so the key range is split over workgroups and merged).
        # bk does not select the GPU's key tile (it is fixed by D), so every bk runs one kernel:
        # a case with several bk values is timed once, at the first, and the outputs at the
        # other bk values are checked to be bit-identical to it.
        cases = [("c3_gqa_prefill_1k", 4, 32, 8, 1024, 1024, 128, 1.0, 3, [args.bk], 0),
                 ("c3_gqa_prefill_2k", 4, 32, 8, 2048, 2048, 128, 1.0, 3, [args.bk], 0),
                 ("c4_mqa_prefill_2k", 8, 16, 1, 2048, 2048, 128, 1.0, 4, [args.bk], 0),
                 ("c5_ragged_gqa", 2, 24, 6, 1000, 4000, 64, 4.0, 5, [128, 32, 64, 256, 512], 0),
                 ("c1_mha_256", 1, 4, 4, 256, 256, 64, 1.0, 1, [128], 0),
                 ("qwen3_4k_causal", 1, 16, 8, 4096, 4096, 128, 1.0, 6, [args.bk], 1),
                 ("chunked_prefill_512x8192_causal", 1, 32, 8, 512, 8192, 128, 1.0, 7, [args.bk],
                  1)]
        for name, Bc, Hqc, Hkvc, Sq, Sk, Dc, sq, ci, bks, cz in cases:
            pairs = Sq * Sk if not cz else sum(min(Sk, max(0, Sk - Sq + i + 1)) for i in range(Sq))
            fl = 4.0 * Bc * Hqc * pairs * Dc
            cb = make_inputs(ts, Bc, Hqc, Hkvc, Sq, Sk, Dc, SEED0 + ci, sigma_q=sq, copies=1)
            sc = ts.DeviceBuffer(ts.attn_flash_scratch_bytes(Dc, max(bks)))
            w, k = time_calls(ts, cb, Bc, Hqc, Hkvc, Sq, Sk, Dc, cz, bks[0], sc, 20, 3)
            res = {"bk": bks[0], "kernel_ms": k, "TFLOP_s": fl / (k * 1e-3) / 1e12,
                   "mfma_frac": fl / (k * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS}
            res.update(bounds(fl, Bc * Hqc * pairs, k))
            res["parity"] = parity(ts, o, cb, Bc, Hqc, Hkvc, Sq, Sk, Dc, cz, 8, nthreads)
            if len(bks) > 1:
                q, kk, v, out, _ = cb[0]
                first = out.download(np.float32)
                same = []
                for bk in bks[1:]:
                    ts.attn_flash(q, kk, v, out, Bc * Hqc, Bc * Hkvc, Sq, Sk, Dc, cz, bk, sc, 0)
                    ts.synchronize()
                    same.append(bool(np.array_equal(out.download(np.float32), first)))
                res["bk_note"] = ("bk does not select the key tile: one kernel for every bk, "
                                  "timed once; O at bk %s bit-identical to bk %d: %s"
                                  % (bks[1:], bks[0], same))
                res["bk_outputs_identical"] = all(same)
            extra[name] = res
            log(name, res)
            for b in cb:
                for x in b[:4]:
                    x.free()
            sc.free()

    peaks = {} if args.no_peaks else measured_peaks()
    log("measured peaks:", peaks)
    cpu = None if args.no_cpu else cpu_baseline(o, ts)
    if cpu:
        log("cpu baseline:", cpu)
    line = {
        "metric": "TFLOP/s & % bf16 MFMA peak, GQA 4k prefill; decode HBM GB/s",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V, fp32 O)",
        "config": {"workload": "c3 GQA prefill B4 Hq32 Hkv8 D128 Sq=Sk=4096 non-causal",
                   "global_batch": B, "seq_len": S, "parallelism": "single GPU",
                   "bk": args.bk, "input_copies": copies},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3),
                     "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic,
                     "kernel_ms": round(kern_ms, 4), "flop_per_launch": flops,
                     "valu_issue_floor_ms": round(bounds(flops, flops / (4.0 * D),
                                                         kern_ms)["valu_floor_ms"], 4),
                     "measured_peaks": peaks,
                     "frac_of_measured_random_operand_peak":
                         (round(achieved / peaks["mfma32x32x16_bf16_random_operands_tflops"], 4)
                          if peaks.get("mfma32x32x16_bf16_random_operands_tflops") else None)},
        "cpu_baseline": cpu,
        "parity": head_parity,
        "device": info,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
