"""Python host mirror of the reference's attention interface, over the C ABI.

Same names, argument meaning and error behaviour as the reference's C entry points
(flash.c:679 attn_flash_scratch_bytes, flash.c:715 pack_v_full, flash.c:727-729
attn_flash; attn_flash_pick_bk per README.md:138-140,359-436): an invalid bk aborts the
process, exactly as in the reference. Tensors are device buffers (DeviceBuffer or raw
device addresses as int); bf16 is carried as uint16 bit patterns, O as float32.
"""
import ctypes

import numpy as np

from ._lib import check, lib

ATTN_BK_MIN = 16
ATTN_BK_MAX = 4096
ATTN_BK_DEFAULT = 128
ATTN_SCRATCH_ALIGN = 64
ATTN_D_MAX = 256
ATTN_NOALLOC_D_MAX = 128
ATTN_NOALLOC_SCRATCH_BYTES = 34078720


class AttnTimes(ctypes.Structure):
    """struct attn_times (flash.c:704-706)."""
    _fields_ = [("packv", ctypes.c_double), ("qxk", ctypes.c_double),
                ("softmax", ctypes.c_double), ("sxv", ctypes.c_double)]


class DeviceBuffer:
    """A device allocation owned by Python (hipMalloc through the library)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().attn_dev_malloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ValueError("upload larger than the buffer")
        check(lib().attn_dev_memcpy_htod(self.ptr, arr.ctypes.data, arr.nbytes), "hipMemcpy H2D")

    def download(self, dtype, count=None):
        dtype = np.dtype(dtype)
        if count is None:
            count = self.nbytes // dtype.itemsize
        out = np.empty(count, dtype)
        check(lib().attn_dev_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes), "hipMemcpy D2H")
        return out

    def fill_bytes(self, value):
        check(lib().attn_dev_memset(self.ptr, int(value), self.nbytes), "hipMemset")

    def free(self):
        if self.ptr:
            check(lib().attn_dev_free(self.ptr), "hipFree")
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _addr(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


# ---- the reference's entry points -----------------------------------------------------------
def attn_flash_scratch_bytes(D, bk):
    return int(lib().attn_flash_scratch_bytes(int(D), int(bk)))


def attn_flash_pick_bk(D, l2_bytes):
    return int(lib().attn_flash_pick_bk(int(D), int(l2_bytes)))


def attn_flash(Q, K, V, O, Hq, Hkv, Sq, Sk, D, causal, bk, scratch, v_prepacked=0, tm=None):
    """Stream-ordered launch; O is valid after synchronize() (or on return when tm is set)."""
    lib().attn_flash(_addr(Q), _addr(K), _addr(V), _addr(O), int(Hq), int(Hkv), int(Sq),
                     int(Sk), int(D), int(bool(causal)), int(bk), _addr(scratch),
                     int(v_prepacked), ctypes.byref(tm) if tm is not None else None)


def attn_flash_noalloc(Q, K, V, O, Hq, Hkv, Sq, Sk, D, causal, bk, v_prepacked=0):
    """attn_flash without a scratch argument: the split-K partials go to the library's static
    device array (no allocation). D above ATTN_NOALLOC_D_MAX aborts. Calls that overlap on one
    GPU race on that array."""
    lib().attn_flash_noalloc(_addr(Q), _addr(K), _addr(V), _addr(O), int(Hq), int(Hkv), int(Sq),
                             int(Sk), int(D), int(bool(causal)), int(bk), int(v_prepacked))


def attn_flash_plan(Hq, Hkv, Sq, Sk, D, causal, bk=ATTN_BK_DEFAULT, v_prepacked=0):
    """The kernels an attn_flash call with these arguments launches on the current device, as
    a list of (kernel, notes, grid, block) from the library's host-side choice; nothing is
    launched."""
    buf = ctypes.create_string_buffer(4096)
    n = lib().attn_flash_plan(int(Hq), int(Hkv), int(Sq), int(Sk), int(D), int(bool(causal)),
                              int(bk), int(v_prepacked), buf, len(buf))
    if n < 0:
        raise RuntimeError("attn_flash_plan: the plan does not fit the buffer")
    return parse_plan(buf.value.decode())


def parse_plan(text):
    """Lines "name[<template arguments>] [notes] grid=x[,y,z] block=n" -> a list of
    (name, notes, grid, block)."""
    out = []
    for line in text.splitlines():
        head, _, tail = line.partition(" grid=")
        grid, _, block = tail.partition(" block=")
        # the kernel name runs to its closing '>' when it has template arguments, else to the
        # first space; the notes follow it
        first = head.split(" ", 1)[0]
        cut = head.index(">") + 1 if "<" in first else len(first)
        out.append((head[:cut], head[cut:].strip(), grid, int(block)))
    return out


def pack_v_full(V, Vp, Hkv, Sk, D):
    lib().pack_v_full(_addr(V), _addr(Vp), int(Hkv), int(Sk), int(D))


def set_stream(stream):
    lib().attn_flash_set_stream(stream)


def get_stream():
    return lib().attn_flash_get_stream()


# ---- device plumbing ------------------------------------------------------------------------
def synchronize():
    check(lib().attn_dev_synchronize(), "hipDeviceSynchronize")


def device_count():
    n = ctypes.c_int(0)
    err = lib().attn_dev_count(ctypes.byref(n))
    return n.value if err == 0 else 0


def device_info():
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(256)
    cus, clk, l2 = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(lib().attn_dev_info(name, 256, arch, 256, ctypes.byref(cus), ctypes.byref(clk),
                              ctypes.byref(l2)), "hipGetDeviceProperties")
    return {"name": name.value.decode(), "arch": arch.value.decode(), "cus": cus.value,
            "clock_khz": clk.value, "l2_bytes": l2.value}


class Event:
    """A HIP event recorded on the calling thread's attn_flash stream."""

    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().attn_dev_event_create(ctypes.byref(p)), "hipEventCreate")
        self.ev = p.value

    def record(self):
        check(lib().attn_dev_event_record(self.ev), "hipEventRecord")

    def elapsed_ms(self, stop):
        ms = ctypes.c_float()
        check(lib().attn_dev_event_elapsed_ms(self.ev, stop.ev, ctypes.byref(ms)),
              "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            lib().attn_dev_event_destroy(self.ev)
        except Exception:
            pass


# ---- synthetic inputs -----------------------------------------------------------------------
def synth_normal_bf16(n, seed, counter0=0, sigma=1.0):
    out = np.empty(int(n), np.uint16)
    lib().attn_synth_normal_bf16(out.ctypes.data, out.size, int(seed), int(counter0),
                                 float(sigma))
    return out


def synth_normal_qkv(Hq, Hkv, Sq, Sk, D, seed, sigma_q=1.0, sigma_kv=1.0):
    """Q, K, V drawn from one counter stream in that order (Q, then K, then V)."""
    nq, nk = Hq * Sq * D, Hkv * Sk * D
    return (synth_normal_bf16(nq, seed, 0, sigma_q), synth_normal_bf16(nk, seed, nq, sigma_kv),
            synth_normal_bf16(nk, seed, nq + nk, sigma_kv))


def synth_lcg_qkv(Hq, Hkv, Sq, Sk, D, seed=0x12345678):
    """The reference's per-case data (flash.c:1030,1050-1061)."""
    st = ctypes.c_uint32(seed)
    arrs = []
    for n in (Hq * Sq * D, Hkv * Sk * D, Hkv * Sk * D):
        a = np.empty(n, np.uint16)
        lib().attn_synth_lcg_bf16(ctypes.byref(st), a.ctypes.data, n)
        arrs.append(a)
    return tuple(arrs)


def run_attention(Qh, Kh, Vh, Hq, Hkv, Sq, Sk, D, causal, bk=ATTN_BK_DEFAULT, v_prepacked=0,
                  prepack_v=False):
    """Host arrays in, host O out: uploads, runs attn_flash once, downloads.

    v_prepacked=1: Vh is already V^T [Hkv][D][Sk]. prepack_v=True: Vh is row-major V; it is
    transposed on the device by pack_v_full into a second buffer and attn_flash runs with
    v_prepacked=1 (the reference's --prepack-v flow, flash.c:1074-1082)."""
    if prepack_v and v_prepacked:
        raise ValueError("prepack_v packs a row-major V; do not combine it with v_prepacked=1")
    with DeviceBuffer.from_array(Qh) as dq, DeviceBuffer.from_array(Kh) as dk, \
            DeviceBuffer.from_array(Vh) as dv, DeviceBuffer(Hq * Sq * D * 4) as do, \
            DeviceBuffer(attn_flash_scratch_bytes(D, bk)) as ds, \
            DeviceBuffer(dv.nbytes if prepack_v else 1) as dvp:
        do.fill_bytes(0xFF)  # NaN poison: every row must be written
        if prepack_v:
            dvp.fill_bytes(0xFF)
            pack_v_full(dv, dvp, Hkv, Sk, D)
            attn_flash(dq, dk, dvp, do, Hq, Hkv, Sq, Sk, D, causal, bk, ds, 1)
        else:
            attn_flash(dq, dk, dv, do, Hq, Hkv, Sq, Sk, D, causal, bk, ds, v_prepacked)
        synchronize()
        return do.download(np.float32, Hq * Sq * D)
