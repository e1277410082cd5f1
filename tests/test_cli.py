"""The command-line harness (tests/harness/flash_cli): the option names, verdict lines and exit
codes of the reference's `flash` program (flash.c:1151-1156,1177-1321), run against
libattn_flash.so.

CPU tests cover everything that ends before the first device call: argument errors (exit 2),
the refused --no-softmax, and the attn_flash_pick_bk self-test. GPU tests run the default
suite, a custom shape, the Qwen3 --long sweep, --prepack-v and --sweep-bk, and read the
verdict of every case line."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "tests", "harness")
CLI = os.path.join(HARNESS, "flash_cli")
CASE_LINE = re.compile(r"^(?P<name>.{17}) H=\s*(?P<hq>\d+)/(?P<hkv>\d+)\s*\(g\d+\) Sq=(?P<sq>\d+)\s+"
                       r"Sk=(?P<sk>\d+)\s+D=\s*(?P<d>\d+) bk=(?P<bk>\d+)\s+(?P<mode>causal|full)\s+\| "
                       r"err/scale=(?P<err>\S+) \|.* -> (?P<verdict>.*)$")


@pytest.fixture(scope="module")
def cli():
    if not os.path.exists(CLI):
        r = subprocess.run(["make", "-s", "-C", HARNESS], capture_output=True, text=True)
        assert r.returncode == 0, r.stdout + r.stderr
    return CLI


def run(cli, *args, timeout=300):
    r = subprocess.run([cli] + list(args), capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-4000:], flush=True)
    return r


# ---- host-only paths -------------------------------------------------------------------------
@pytest.mark.parametrize("args,needle", [
    (["--bk", "48"], "--bk 48 rejected"),
    (["--bk", "8"], "--bk 8 rejected"),
    (["--bk", "8192"], "--bk 8192 rejected"),
    (["--bk", "x"], "wants an integer"),
    (["--bk"], "needs a value"),
    (["--shape", "3,2,8,8,64"], "Hq a multiple of Hkv"),
    (["--shape", "4,4,0,8,64"], "must be positive"),
    (["--shape", "4,4"], "wants 5 to 7 comma-separated integers"),
    (["--shape", "4,4,8,8,64,"], "wants 5 to 7 comma-separated integers"),
    (["--shape", "4,4,8,8,64,1,8,9"], "wants 5 to 7 comma-separated integers"),
    (["--shape", "4,4,8,8,257"], "above ATTN_D_MAX=256"),
    (["--shape", "4,4,8,8,64,1,-1"], "ref_cap must be >= 0"),
    (["--iters", "3.5"], "wants an integer"),
    (["--iters", "-5"], "must be >= 0"),
    (["--warmup", "-1"], "must be >= 0"),
    (["--llc-mb", "-16"], "must be >= 0"),
    (["--normal", "-1"], "wants a non-negative integer"),
    (["--bench-secs", "fast"], "wants a number"),
    (["--frobnicate"], "unrecognised option '--frobnicate'"),
    (["--no-softmax"], "--no-softmax is rejected"),
])
def test_bad_arguments_exit_2(cli, args, needle):
    r = run(cli, *args)
    assert r.returncode == 2
    assert needle in r.stdout


def test_check_pick_bk(cli):
    r = run(cli, "--check-pick-bk")
    assert r.returncode == 0
    assert "PICK_BK OK, 0 checks failed" in r.stdout


def test_help_lists_every_reference_flag(cli):
    r = run(cli, "--help")
    assert r.returncode == 0
    for flag in ("--long", "--shape", "--bk", "--prepack-v", "--iters", "--warmup",
                 "--bench-secs", "--llc-mb", "--no-softmax", "--sweep-bk", "--check-pick-bk"):
        assert flag in r.stdout, flag


# ---- on the GPU ------------------------------------------------------------------------------
def case_lines(out):
    return [m for m in (CASE_LINE.match(l) for l in out.splitlines()) if m]


@pytest.mark.gpu
@pytest.mark.parametrize("extra", [[], ["--prepack-v"], ["--bk", "16"], ["--bk", "4096"],
                                   ["--normal", "7"]],
                         ids=["default", "prepack-v", "bk16", "bk4096", "normal-data"])
def test_default_suite(cli, extra):
    r = run(cli, "--bench-secs", "0.05", "--llc-mb", "16", *extra)
    assert r.returncode == 0, r.stdout
    lines = case_lines(r.stdout)
    assert len(lines) == 9
    assert all(m.group("verdict") == "PASS" for m in lines)
    assert "=== ALL PASS ===" in r.stdout
    if "--prepack-v" in extra:
        assert all("sep-packv=" in m.group(0) for m in lines)


@pytest.mark.gpu
def test_long_qwen3_sweep(cli):
    r = run(cli, "--long", "--iters", "5", "--warmup", "1", "--llc-mb", "64")
    assert r.returncode == 0, r.stdout
    lines = case_lines(r.stdout)
    assert [m.group("name").strip() for m in lines[-3:]] == ["qwen3 1k", "qwen3 2k", "qwen3 4k"]
    assert all("[ref:8 rows spread" in m.group(0) for m in lines[-3:])


@pytest.mark.gpu
def test_custom_shape_decode_and_iters(cli):
    r = run(cli, "--shape", "32,8,1,4096,128,0,0", "--iters", "7", "--llc-mb", "64")
    assert r.returncode == 0, r.stdout
    (m,) = case_lines(r.stdout)
    assert m.group("mode") == "full" and m.group("sq") == "1" and " x7 " in m.group(0)


@pytest.mark.gpu
def test_sweep_bk(cli):
    r = run(cli, "--sweep-bk", "--bench-secs", "0.05", "--llc-mb", "16")
    assert r.returncode == 0, r.stdout
    rows = [l.split() for l in r.stdout.splitlines() if re.match(r"^\s+\d+\s+\d+\s", l)]
    assert [int(x[0]) for x in rows] == [16 << i for i in range(9)]
    assert all(x[-1] == "PASS" for x in rows)
    assert "every bk runs the same kernel" in r.stdout
    assert "spread over bk:" in r.stdout and "attn_flash_pick_bk(D=128" in r.stdout
