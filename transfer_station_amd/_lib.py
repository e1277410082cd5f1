"""ctypes binding of libattn_flash.so (the C ABI declared in include/attn_flash.h and
include/attn_devutil.h). Loading fails loudly when the library has not been built: there
is no CPU or Python fallback for any entry point."""
import ctypes
import os

from . import build as _build

_lib = None

# Every symbol the headers declare, with (restype, argtypes).
_c = ctypes
_SIGNATURES = {
    # include/attn_flash.h
    "attn_flash_scratch_bytes": (_c.c_size_t, [_c.c_int, _c.c_int]),
    "attn_flash_pick_bk": (_c.c_int, [_c.c_int, _c.c_size_t]),
    "attn_flash": (None, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_void_p] + [_c.c_int] * 7 +
                   [_c.c_void_p, _c.c_int, _c.c_void_p]),
    "pack_v_full": (None, [_c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_int]),
    "attn_flash_noalloc": (None, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_void_p] +
                           [_c.c_int] * 8),
    "attn_flash_plan": (_c.c_int, [_c.c_int] * 8 + [_c.c_char_p, _c.c_size_t]),
    "attn_flash_set_stream": (None, [_c.c_void_p]),
    "attn_flash_get_stream": (_c.c_void_p, []),
    # include/attn_devutil.h
    "attn_dev_count": (_c.c_int, [_c.POINTER(_c.c_int)]),
    "attn_dev_malloc": (_c.c_int, [_c.POINTER(_c.c_void_p), _c.c_size_t]),
    "attn_dev_free": (_c.c_int, [_c.c_void_p]),
    "attn_dev_memcpy_htod": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_size_t]),
    "attn_dev_memcpy_dtoh": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_size_t]),
    "attn_dev_memcpy_dtod": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_size_t]),
    "attn_dev_memset": (_c.c_int, [_c.c_void_p, _c.c_int, _c.c_size_t]),
    "attn_dev_synchronize": (_c.c_int, []),
    "attn_dev_info": (_c.c_int, [_c.c_char_p, _c.c_size_t, _c.c_char_p, _c.c_size_t,
                                 _c.POINTER(_c.c_int), _c.POINTER(_c.c_int),
                                 _c.POINTER(_c.c_int)]),
    "attn_dev_event_create": (_c.c_int, [_c.POINTER(_c.c_void_p)]),
    "attn_dev_event_destroy": (_c.c_int, [_c.c_void_p]),
    "attn_dev_event_record": (_c.c_int, [_c.c_void_p]),
    "attn_dev_event_elapsed_ms": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.POINTER(_c.c_float)]),
    "attn_synth_normal_bf16": (None, [_c.c_void_p, _c.c_size_t, _c.c_uint64, _c.c_uint64,
                                      _c.c_double]),
    "attn_synth_lcg_bf16": (None, [_c.POINTER(_c.c_uint32), _c.c_void_p, _c.c_size_t]),
    "attn_synth_f32_to_bf16": (_c.c_uint16, [_c.c_float]),
}


def exported_symbols():
    return sorted(_SIGNATURES)


def lib():
    """The loaded library. Raises if it is missing (build it with __graft_entry__.build())."""
    global _lib
    if _lib is None:
        path = _build.lib_path()
        if not os.path.exists(path):
            raise RuntimeError("libattn_flash.so is not built (%s); run __graft_entry__.build() "
                               "-- there is no fallback path" % path)
        L = ctypes.CDLL(path)
        for name, (res, args) in _SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


class HipError(RuntimeError):
    pass


def check(err, what):
    if err != 0:
        raise HipError("%s failed with hipError_t %d" % (what, err))
