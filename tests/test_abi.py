"""CPU tests of the C ABI: the library loads and exports every declared symbol, the host
functions that need no GPU reproduce the reference's documented answers, and invalid
arguments abort exactly where the reference aborts (flash.c:641-647,680,764)."""
import os
import re
import signal
import subprocess
import sys

import pytest

import transfer_station_amd as ts
from transfer_station_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for hdr in ("attn_flash.h", "attn_devutil.h"):
        text = open(os.path.join(ROOT, "include", hdr)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", text):
            name = m.group(1)
            if name not in ("if", "sizeof", "defined"):
                names.add(name)
    return names


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    declared = _declared_functions()
    assert "attn_flash" in declared and "attn_flash_pick_bk" in declared
    for name in declared:
        assert hasattr(L, name), name
    assert declared == set(_lib.exported_symbols())


def test_header_constants_match_reference():
    text = open(os.path.join(ROOT, "include", "attn_flash.h")).read()
    for k, v in (("ATTN_BK_MIN", 16), ("ATTN_BK_MAX", 4096), ("ATTN_BK_DEFAULT", 128),
                 ("ATTN_SCRATCH_ALIGN", 64)):
        assert re.search(r"#define %s %d\b" % (k, v), text), k
    assert (ts.ATTN_BK_MIN, ts.ATTN_BK_MAX, ts.ATTN_BK_DEFAULT) == (16, 4096, 128)


# ---- attn_flash_pick_bk (README.md:359-436; EXEC_LOG:854-875, 989-1011) ----------------------
INT_MAX = 2 ** 31 - 1
SIZE_MAX = 2 ** 64 - 1


def test_pick_bk_documented_answers():
    assert [ts.attn_flash_pick_bk(128, m << 20) for m in (1, 2, 4, 8)] == [256, 512, 1024, 2048]
    assert [ts.attn_flash_pick_bk(d, 1 << 20) for d in (64, 128, 256, 512)] == [512, 256, 128, 64]
    assert ts.attn_flash_pick_bk(128, 0) == 16
    assert ts.attn_flash_pick_bk(128, SIZE_MAX) == 4096
    assert ts.attn_flash_pick_bk(INT_MAX, 2 * 10 ** 12) == 16
    assert ts.attn_flash_pick_bk(INT_MAX, 2 ** 50) == 4096
    assert ts.attn_flash_pick_bk(0, 1 << 20) == ts.attn_flash_pick_bk(1, 1 << 20)
    assert ts.attn_flash_pick_bk(-5, 1 << 20) == ts.attn_flash_pick_bk(1, 1 << 20)


def test_pick_bk_against_exact_integer_model():
    """The bound holds at the pick and fails at the next power of two (exact big integers)."""
    def ws(D, bk):
        return 6 * bk * (D + 64) + 6 * 64 * D + 4 * D + 12 * 64
    Ds = [1, 2, 3, 7, 40, 64, 100, 128, 256, 512, 1000, 10 ** 5, INT_MAX - 65, INT_MAX - 64,
          INT_MAX - 63, INT_MAX - 1, INT_MAX]
    L2s = [0, 4096, 65536, 1 << 20, 3 << 20, 16 << 20, 64 << 20, 2 * 10 ** 12, 2 ** 50, SIZE_MAX]
    for D in Ds:
        prev = None
        for l2 in L2s:
            got = ts.attn_flash_pick_bk(D, l2)
            assert got & (got - 1) == 0 and 16 <= got <= 4096
            want = 16
            bk = 16
            while bk <= 4096 and 2 * ws(D, bk) <= l2:
                want = bk
                bk *= 2
            assert got == want, (D, l2)
            if prev is not None:
                assert got >= prev  # non-decreasing in l2
            prev = got


# ---- scratch contract ----------------------------------------------------------------------------
def test_scratch_bytes_contract():
    for D in (1, 40, 64, 127, 128):
        sizes = [ts.attn_flash_scratch_bytes(D, 1 << e) for e in range(4, 13)]
        assert all(s % ts.ATTN_SCRATCH_ALIGN == 0 for s in sizes)
        assert sizes == sorted(sizes)  # monotone non-decreasing in bk
    assert ts.attn_flash_scratch_bytes(128, 128) >= ts.attn_flash_scratch_bytes(64, 128)
    # capacity: 65536 split slots of (m, l, acc[D]) fp32
    assert ts.attn_flash_scratch_bytes(128, 128) >= 65536 * (128 + 2) * 4


# ---- aborts (each in its own process, like the reference's subprocess-per-case checks) -------
def _run_py(code):
    return subprocess.run([sys.executable, "-c", "import sys; sys.path.insert(0, %r)\n" % ROOT +
                           code], capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize("bk", [0, -8, 3, 8, 100, 4095, 8192])
def test_bad_bk_aborts_at_both_doors(bk):
    r = _run_py("import transfer_station_amd as ts; ts.attn_flash_scratch_bytes(128, %d)" % bk)
    assert r.returncode == -signal.SIGABRT
    assert "bk=%d is invalid" % bk in r.stderr
    r = _run_py("import transfer_station_amd as ts\n"
                "ts.attn_flash(0, 0, 0, 0, 4, 4, 8, 8, 64, 0, %d, 0)" % bk)
    assert r.returncode == -signal.SIGABRT
    assert "attn_flash: bk=%d is invalid" % bk in r.stderr


@pytest.mark.parametrize("args,msg", [
    ("1, 2, 3, 4, 6, 4, 8, 8, 64, 0, 128, 64", "Hq % Hkv"),
    ("1, 2, 3, 4, 4, 0, 8, 8, 64, 0, 128, 64", "Hkv >= 1"),
    ("1, 2, 3, 4, 4, 4, 0, 8, 64, 0, 128, 64", "Sq >= 1"),
    ("1, 2, 3, 4, 4, 4, 8, 0, 64, 0, 128, 64", "Sk >= 1"),
    ("1, 2, 3, 4, 4, 4, 8, 8, 0, 0, 128, 64", "D=0 is invalid"),
    ("1, 2, 3, 4, 4, 4, 8, 8, 257, 0, 128, 64", "D=257 is invalid"),
    ("1, 2, 3, 4, 4, 4, 8, 8, 64, 0, 128, 0", "scratch must be"),
    ("1, 2, 3, 4, 4, 4, 8, 8, 64, 0, 128, 65", "scratch must be"),
    ("0, 2, 3, 4, 4, 4, 8, 8, 64, 0, 128, 64", "device pointers"),
])
def test_bad_shapes_abort(args, msg):
    r = _run_py("import transfer_station_amd as ts; ts.attn_flash(%s)" % args)
    assert r.returncode == -signal.SIGABRT
    assert msg in r.stderr


def test_noalloc_static_scratch_size():
    """The static array of attn_flash_noalloc is the layout of attn_flash's scratch at its largest
    D, so every D it accepts carves the same slots as a caller's scratch would."""
    text = open(os.path.join(ROOT, "include", "attn_flash.h")).read()
    m = re.search(r"#define ATTN_NOALLOC_SCRATCH_BYTES (\d+)u", text)
    assert m and int(m.group(1)) == ts.ATTN_NOALLOC_SCRATCH_BYTES
    assert re.search(r"#define ATTN_NOALLOC_D_MAX %d\b" % ts.ATTN_NOALLOC_D_MAX, text)
    for bk in (16, 128, 4096):
        assert ts.attn_flash_scratch_bytes(ts.ATTN_NOALLOC_D_MAX, bk) == \
            ts.ATTN_NOALLOC_SCRATCH_BYTES
    assert all(ts.attn_flash_scratch_bytes(d, 128) <= ts.ATTN_NOALLOC_SCRATCH_BYTES
               for d in range(1, ts.ATTN_NOALLOC_D_MAX + 1))


@pytest.mark.parametrize("args,msg", [
    ("1, 2, 3, 4, 4, 4, 8, 8, 129, 0, 128", "D=129 is invalid -- the static scratch holds"),
    ("1, 2, 3, 4, 4, 4, 8, 8, 256, 0, 128", "D=256 is invalid -- the static scratch holds"),
    ("1, 2, 3, 4, 4, 4, 8, 8, 64, 0, 100", "attn_flash_noalloc: bk=100 is invalid"),
    ("1, 2, 3, 4, 6, 4, 8, 8, 64, 0, 128", "Hq % Hkv"),
    ("0, 2, 3, 4, 4, 4, 8, 8, 64, 0, 128", "device pointers"),
])
def test_noalloc_rejects_before_any_device_call(args, msg):
    r = _run_py("import transfer_station_amd as ts; ts.attn_flash_noalloc(%s)" % args)
    assert r.returncode == -signal.SIGABRT
    assert msg in r.stderr


def test_bad_d_aborts_in_size_query():
    r = _run_py("import transfer_station_amd as ts; ts.attn_flash_scratch_bytes(0, 128)")
    assert r.returncode == -signal.SIGABRT and "D=0 is invalid" in r.stderr


def test_library_missing_fails_loudly(tmp_path, monkeypatch):
    from transfer_station_amd import build
    monkeypatch.setattr(build, "lib_path", lambda: str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.lib()


def test_parse_plan_lines():
    text = ("attn_decode_kernel<128, false, true, false, false> nsplit=64 nrb=1 grid=512 block=256\n"
            "attn_mergew_kernel nsplit=64 grid=8 block=256\n"
            "attn_merge2_kernel grid=8,2,1 block=256\n")
    assert ts.parse_plan(text) == [
        ("attn_decode_kernel<128, false, true, false, false>", "nsplit=64 nrb=1", "512", 256),
        ("attn_mergew_kernel", "nsplit=64", "8", 256),
        ("attn_merge2_kernel", "", "8,2,1", 256)]


def test_plan_checks_arguments_before_any_device_call():
    r = _run_py("import transfer_station_amd as ts; ts.attn_flash_plan(4, 4, 8, 8, 64, 0, 100)")
    assert r.returncode == -signal.SIGABRT and "bk" in r.stderr
