"""Phase timeline of the persistent prefill (attn_prefill_persist_kernel), from stamps written
inside the kernel.

    python -m transfer_station_amd.phases [--shape Hq,Hkv,Sq,Sk,D[,causal]] [--json] [--items]

The stamps exist only in libattn_flash_stamps.so, the library built a second time with
ATTN_PHASE_STAMPS=1 (transfer_station_amd/build.py); the product library has none of that code.
Wave 0 of every workgroup records the GPU's 100 MHz real-time counter at kernel entry, when the
first item's Q and key tile have arrived, at four points of every item (its start, the end of
its first key tile, the start and the end of its last key tile) and once its final O stores have
completed. The summary splits the kernel's time into the reference's kind of phases for this
kernel: the prologue (Q and the first tile, one HBM burst from every CU), the steady key loop
(per 128-key tile), the extra time of an item's first and last tiles (the previous item's O
stores and the next item's Q and first tile overlap them), and the tail (the final O stores).
The per-phase timers of the reference (flash.c:695-706, 822-849) have no counterpart in one
fused launch; this is the attribution that replaces them.
"""
import argparse
import ctypes
import json
import time

import numpy as np

from . import attn as ts
from . import build as _build

TICK_US = 0.01  # s_memrealtime runs at 100 MHz
KT, BQ = 128, 256  # the persistent kernel's key tile and item rows (128 with key halves)


def items_of(b, nwg, nunits, g, nqt, causal, swap=None):
    """(query tile) of each item of workgroup b, in order: the kernel's item mapping
    (attn_prefill_persist_kernel's `item`), restated. swap(qt) (key halves): whether a pair
    whose heavy tile is qt runs its light tile first."""
    x, xi, R = b & 7, b >> 3, nwg >> 3
    per, rem = nunits >> 3, nunits & 7
    xb = x * (per + 1) if x < rem else rem * (per + 1) + (x - rem) * per
    nx = per + (1 if x < rem else 0)
    nu = (nx - xi + R - 1) // R if xi < nx else 0
    out = []
    for k in range(2 * nu if causal else nu):
        if causal:
            npair = nqt >> 1
            P = xb + xi + (k >> 1) * R
            rr = P - (P // (g * npair)) * (g * npair)
            pp = rr // g
            first, second = nqt - 1 - pp, pp
            if swap is not None and swap(first):
                first, second = second, first
            out.append(second if k & 1 else first)
        else:
            L = xb + xi + k * R
            rr = L - (L // (g * nqt)) * (g * nqt)
            out.append(rr // g)
    return out


def key_tiles(qt, Sq, Sk, causal, bq=BQ):
    if causal:
        return (Sk - Sq + min(Sq - 1, qt * bq + bq - 1)) // KT + 1
    return (Sk + KT - 1) // KT


def summarize(stamps, slots, Hq, Hkv, Sq, Sk, causal, kh=False):
    """Phase times in microseconds from the (workgroups, slots) stamp array. kh: the key-halves
    variant (128-row items, each pair's item of even key-tile count first)."""
    nwg = stamps.shape[0]
    bq = 128 if kh else BQ
    g, nqt = Hq // Hkv, (Sq + bq - 1) // bq
    nunits = Hq * nqt // (2 if causal else 1)
    swap = (lambda qt: key_tiles(qt, Sq, Sk, causal, bq) % 2 == 1) if kh else None
    busy = [b for b in range(nwg) if items_of(b, nwg, nunits, g, nqt, causal, swap)]
    # workgroups without items return before their first stamp
    t = (stamps.astype(np.int64) - int(stamps[busy, 0].min())) * TICK_US
    prologue, first_x, last_x, tile, tail, gaps, ends = [], [], [], [], [], [], []
    by_k = {}  # item index -> (key tiles, first-tile extra, last-tile extra) per workgroup
    for b in busy:
        qts = items_of(b, nwg, nunits, g, nqt, causal, swap)
        per_tile = []
        for k, qt in enumerate(qts):
            s = t[b, 2 + 4 * k: 6 + 4 * k]
            n = key_tiles(qt, Sq, Sk, causal, bq)
            if n > 2:
                per_tile.append((s[2] - s[1]) / (n - 2))
            if k + 1 < len(qts):
                gaps.append(t[b, 2 + 4 * (k + 1)] - s[3])
        mid = float(np.median(per_tile)) if per_tile else float("nan")
        tile.extend(per_tile)
        prologue.append(t[b, 1] - t[b, 0])
        for k, qt in enumerate(qts):
            s = t[b, 2 + 4 * k: 6 + 4 * k]
            n = key_tiles(qt, Sq, Sk, causal, bq)
            first_x.append(s[1] - s[0] - mid)
            d = by_k.setdefault(k, ([], [], []))
            d[0].append(n)
            d[1].append(s[1] - s[0] - mid)
            if n > 1:  # (an item of one tile: first only)
                last_x.append(s[3] - s[2] - mid)
                d[2].append(s[3] - s[2] - mid)
        tail.append(t[b, slots - 1] - t[b, 2 + 4 * (len(qts) - 1) + 3])
        ends.append(t[b, slots - 1])

    def stat(v):
        v = np.asarray(v, dtype=np.float64)
        v = v[np.isfinite(v)]
        if v.size == 0:
            return None
        return {"median": round(float(np.median(v)), 3), "min": round(float(v.min()), 3),
                "max": round(float(v.max()), 3)}

    return {
        "workgroups": len(busy),
        "entry_spread_us": round(float(t[busy, 0].max()), 3),
        "prologue_us": stat(prologue),
        "key_tile_us": stat(tile),
        "first_tile_extra_us": stat(first_x),
        "last_tile_extra_us": stat(last_x),
        "between_items_us": stat(gaps),
        "tail_us": stat(tail),
        "span_us": round(float(max(ends)), 3),
        # per item index of a workgroup: the median key-tile count and first / last tile extras
        "items": [{"item": k, "key_tiles": float(np.median(d[0])),
                   "first_tile_extra_us": stat(d[1]), "last_tile_extra_us": stat(d[2])}
                  for k, d in sorted(by_k.items())],
    }


def summarize_tiles(stamps, slots):
    """Phase times in microseconds of the per-tile prefill kernel (attn_prefill_fast_kernel: one
    item per workgroup) from its stamps: slot 0 entry, 1 Q and first tile in, 2 after the first
    tile, 3 after the last, 4 after the key halves' hand-over, slots - 1 stores complete; slot 6
    the CU, slot 7 the key tiles."""
    busy = np.nonzero(stamps[:, 0])[0]
    base = int(stamps[busy, 0].min())
    t = (stamps[busy].astype(np.int64) - base) * TICK_US
    ntile = stamps[busy, 7].astype(np.int64)
    cu = stamps[busy, 6].astype(np.int64)
    end = t[:, slots - 1]
    many = ntile > 1
    per_tile = (t[many, 3] - t[many, 2]) / (ntile[many] - 1)

    def stat(v):
        v = np.asarray(v, dtype=np.float64)
        if v.size == 0:
            return None
        return {"median": round(float(np.median(v)), 3), "min": round(float(v.min()), 3),
                "max": round(float(v.max()), 3)}

    # per CU: its workgroups in entry order; a CU idles from its last workgroup's end to the
    # kernel's end, and between a workgroup's end and the next one's entry when it runs one at a
    # time
    span = float(end.max())
    idle_end, wg_per_cu, gaps = [], [], []
    for c in np.unique(cu):
        m = cu == c
        e0, e1 = t[m, 0], end[m]
        order = np.argsort(e0)
        wg_per_cu.append(int(m.sum()))
        idle_end.append(span - float(e1.max()))
        for a, b in zip(order[:-1], order[1:]):
            if e0[b] >= e1[a]:
                gaps.append(e0[b] - e1[a])
    return {
        "workgroups": int(busy.size), "cus": int(np.unique(cu).size),
        "workgroups_per_cu": stat(wg_per_cu),
        "entry_spread_us": round(float(t[:, 0].max()), 3),
        "prologue_us": stat(t[:, 1] - t[:, 0]),
        "first_tile_us": stat(t[:, 2] - t[:, 1]),
        "key_tile_us": stat(per_tile),
        "key_halves_handover_us": stat(t[:, 4] - t[:, 3]),
        "epilogue_us": stat(end - t[:, 4]),
        "gap_between_workgroups_us": stat(gaps),
        "cu_idle_at_end_us": stat(idle_end),
        "span_us": round(span, 3),
    }


def _stamps_lib():
    path = _build.stamps_lib_path()
    L = ctypes.CDLL(path)
    c = ctypes
    L.attn_flash.restype = None
    L.attn_flash.argtypes = [c.c_void_p] * 4 + [c.c_int] * 7 + [c.c_void_p, c.c_int, c.c_void_p]
    L.attn_flash_scratch_bytes.restype = c.c_size_t
    L.attn_flash_scratch_bytes.argtypes = [c.c_int, c.c_int]
    L.attn_flash_plan.restype = c.c_int
    L.attn_flash_plan.argtypes = [c.c_int] * 8 + [c.c_char_p, c.c_size_t]
    L.attn_hip_phase_stamps.restype = c.c_int
    L.attn_hip_phase_stamps.argtypes = [c.c_void_p]
    return L


def timeline(Hq, Hkv, Sq, Sk, D, causal=0, seed=0x12345678, warm_s=0.3):
    """Runs the shape on the stamps library (after warm_s seconds of warmup, the clock ramp) and
    returns (summary, stamps); the summary also holds the kernel time of both libraries."""
    L = _stamps_lib()
    buf = ctypes.create_string_buffer(4096)
    if L.attn_flash_plan(Hq, Hkv, Sq, Sk, D, causal, 128, 0, buf, len(buf)) < 0:
        raise RuntimeError("attn_flash_plan failed")
    plan = ts.parse_plan(buf.value.decode())
    kernel = plan[0][0]
    if not kernel.startswith(("attn_prefill_persist_kernel", "attn_prefill_fast_kernel")):
        raise ValueError("this shape runs no stamped prefill kernel: %s" % (plan,))
    nwg = int(plan[0][2])
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, seed)
    bq, bk, bv = (ts.DeviceBuffer.from_array(a) for a in (Q, K, V))
    bo = ts.DeviceBuffer(Hq * Sq * D * 4)
    scr = ts.DeviceBuffer(ts.attn_flash_scratch_bytes(D, 128))
    st = ts.DeviceBuffer(nwg * 64 * 8)
    try:
        slots = L.attn_hip_phase_stamps(ctypes.c_void_p(st.ptr))
        if slots <= 0 or nwg * slots * 8 > st.nbytes:
            raise RuntimeError("libattn_flash_stamps.so has no phase stamps")

        def run(fn, n):
            e0, e1 = ts.Event(), ts.Event()
            e0.record()
            for _ in range(n):
                fn(bq.ptr, bk.ptr, bv.ptr, bo.ptr, Hq, Hkv, Sq, Sk, D, causal, 128, scr.ptr, 0,
                   None)
            e1.record()
            ts.synchronize()
            return e0.elapsed_ms(e1) / n

        lib = ts.lib()
        st.fill_bytes(0)  # workgroups without items keep zeros
        run(lib.attn_flash, 3)  # the product library's first launches load its code
        t0 = time.time()
        while time.time() - t0 < warm_s:
            run(L.attn_flash, 10)
        ms_stamps = run(L.attn_flash, 20)
        ms_product = run(lib.attn_flash, 20)
        run(L.attn_flash, 10)  # back to back: the stamps hold the last call's, warm
        stamps = st.download(np.uint64, nwg * slots).reshape(nwg, slots)
        if kernel.startswith("attn_prefill_persist_kernel"):
            kh = kernel.replace(" ", "").endswith(",true>")  # <DP, CAUSAL, KH>
            summary = summarize(stamps, slots, Hq, Hkv, Sq, Sk, causal, kh)
        else:
            summary = summarize_tiles(stamps, slots)
        summary.update({"shape": [Hq, Hkv, Sq, Sk, D, causal], "kernel": kernel,
                        "plan": [" ".join((k, n)).strip() for k, n, _, _ in plan],
                        "kernel_ms_stamps_build": round(ms_stamps, 4),
                        "kernel_ms_product": round(ms_product, 4)})
        return summary, stamps
    finally:
        for x in (bq, bk, bv, bo, scr, st):
            x.free()


LABELS = (("cus", "CUs"), ("workgroups_per_cu", "workgroups per CU"),
          ("entry_spread_us", "entry spread"),
          ("prologue_us", "prologue (Q + first tile)"),
          ("first_tile_us", "first key tile"),
          ("key_tile_us", "key tile, steady"),
          ("first_tile_extra_us", "first tile of an item, extra"),
          ("last_tile_extra_us", "last tile of an item, extra"),
          ("between_items_us", "between items"),
          ("key_halves_handover_us", "key halves' hand-over"),
          ("epilogue_us", "epilogue (O or partial stores)"),
          ("tail_us", "tail (final O stores)"),
          ("gap_between_workgroups_us", "gap between workgroups"),
          ("cu_idle_at_end_us", "CU idle before the end"),
          ("span_us", "span of the stamps"))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--shape", action="append",
                    help="Hq,Hkv,Sq,Sk,D[,causal] (repeatable; default: config 3 at 1k, 4k and "
                         "4k causal, the Qwen3 4k causal case and config 5)")
    ap.add_argument("--json", action="store_true", help="one JSON line per shape")
    ap.add_argument("--items", action="store_true",
                    help="persistent kernel: also the first / last tile extras by item index")
    args = ap.parse_args()
    shapes = [tuple(int(v) for v in s.split(",")) for s in args.shape] if args.shape else [
        (128, 32, 1024, 1024, 128, 0), (128, 32, 4096, 4096, 128, 0),
        (128, 32, 4096, 4096, 128, 1), (16, 8, 4096, 4096, 128, 1), (48, 12, 1000, 4000, 64, 0)]
    for s in shapes:
        s = s + (0,) * (6 - len(s))
        summary, _ = timeline(*s)
        if args.json:
            print(json.dumps(summary), flush=True)
            continue
        print("shape Hq=%d Hkv=%d Sq=%d Sk=%d D=%d causal=%d: kernel %.4f ms (product library "
              "%.4f ms), %d workgroups" % (s + (summary["kernel_ms_stamps_build"],
                                                summary["kernel_ms_product"],
                                                summary["workgroups"])))
        print("  plan: %s" % "; ".join(summary["plan"]))
        for key, label in LABELS:
            v = summary.get(key)
            if v is None:
                continue
            if isinstance(v, dict):
                print("  %-31s %9.2f  (min %.2f, max %.2f)" % (label, v["median"], v["min"],
                                                              v["max"]))
            else:
                print("  %-31s %9.2f" % (label, v))
        for it in (summary.get("items") or []) if args.items else []:
            f, l = it["first_tile_extra_us"], it["last_tile_extra_us"]
            print("  item %d (%3.0f key tiles): first tile extra %5.2f, last tile extra %s" % (
                it["item"], it["key_tiles"], f["median"] if f else float("nan"),
                "%5.2f" % l["median"] if l else "  -"))
        print(flush=True)


if __name__ == "__main__":
    main()
