"""CPU checks of the generated gfx950 code of this repository's own build (no GPU needed).

The LDS-DMA kernels (the fast prefill and the V^T decode) order their DMA and their LDS reads
themselves: each wave waits for its own DMA (vmcnt(0)) right before the barrier that ends a tile.
The compiler can also add vmcnt waits on the DMA in flight before LDS reads inside the key loop
(it does so for a kernel that makes no out-of-line call, since it cannot tell the two tile
buffers apart), which serialises each tile with the next tile's load: 3-15% slower on the
prefill shapes. This test reads the disassembly of the built library and fails if any such
wait appears after a kernel's first MFMA.
"""
import os
import re
import shutil
import subprocess

import pytest

from transfer_station_amd import build as _build

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
OBJDUMP = os.path.join(ROCM, "llvm", "bin", "llvm-objdump")


@pytest.fixture(scope="module")
def funcs(tmp_path_factory):
    """Instruction lists by function name of the built library's gfx950 code object."""
    tmp_path = tmp_path_factory.mktemp("codegen")
    lib = _build.lib_path()
    if not os.path.exists(lib):
        pytest.skip("library not built")
    if not os.access(OBJDUMP, os.X_OK):
        pytest.skip("llvm-objdump not found under %s" % ROCM)
    # --offloading writes the bundled code objects next to its input: work on a copy.
    copy = os.path.join(str(tmp_path), "lib.so")
    shutil.copy(lib, copy)
    subprocess.run([OBJDUMP, "--offloading", copy], cwd=str(tmp_path), check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    objs = [f for f in os.listdir(str(tmp_path)) if f.endswith("gfx950")]
    assert len(objs) == 1, os.listdir(str(tmp_path))
    out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", os.path.join(str(tmp_path), objs[0])],
                         check=True, stdout=subprocess.PIPE, universal_newlines=True).stdout
    funcs, cur = {}, None
    for line in out.split("\n"):
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if m:
            cur = funcs.setdefault(m.group(1), [])
            continue
        if cur is not None and line.startswith("\t"):
            ins = line.strip().split("//")[0].strip()
            if ins:
                cur.append(ins)
    return funcs


def test_lds_dma_kernels_have_no_compiler_dma_waits(funcs):
    kernels = {n: ins for n, ins in funcs.items()
               if "attn_prefill_fast_kernel" in n or "attn_decode_vt_kernel" in n}
    assert len(kernels) >= 40, sorted(funcs)[:5]
    bad = {}
    for name, ins in kernels.items():
        first = next((i for i, x in enumerate(ins) if x.startswith("v_mfma")), None)
        assert first is not None, name
        for i in range(first, len(ins)):
            if ins[i].startswith("s_waitcnt") and "vmcnt" in ins[i]:
                nxt = [y for y in ins[i + 1:i + 6] if not y.startswith(("s_waitcnt", "s_nop"))]
                if nxt and nxt[0].startswith("ds_read"):
                    bad.setdefault(name, []).append(i)
    assert not bad, "vmcnt waits before LDS reads in the key loop of %d kernels, e.g. %s" % (
        len(bad), sorted(bad)[0])


def test_kernels_make_only_the_deliberate_library_call(funcs):
    """HIP's id builtins are out-of-line calls in this build; the kernels read the ids directly,
    except one threadIdx.x in each LDS-DMA kernel (the call that keeps the loop above free of
    compiler DMA waits): the fast and persistent prefills and the V^T decode."""
    for name, ins in funcs.items():
        if not name.startswith("_Z") or "attn_" not in name:
            continue
        calls = sum(1 for x in ins if x.startswith("s_swappc"))
        want = 1 if any(k in name for k in ("attn_prefill_fast_kernel", "attn_prefill_persist_kernel",
                                            "attn_decode_vt_kernel")) else 0
        assert calls == want, (name, calls)
