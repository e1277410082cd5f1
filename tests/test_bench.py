"""CPU checks of bench.py's host logic (no GPU): the roofline floors it reports and its refusal
of more than one GPU."""
import importlib.util
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_floors_pick_the_binding_roofline():
    b = _bench()
    # config 5 (D = 64): half the MFMA work per score of D = 128, the same softmax per score
    scores = 48 * 1000 * 4000
    r = b.bounds(4.0 * 64 * scores, scores, 0.0648)
    assert r["bound"] == "valu"
    assert abs(r["mfma_floor_ms"] - 4.0 * 64 * scores / 2.5e15 * 1e3) < 1e-12
    assert abs(r["valu_floor_ms"] - scores * 18 / 64 / (1024 * 2.4e9) * 1e3) < 1e-12
    assert abs(r["bound_frac"] - r["valu_floor_ms"] / 0.0648) < 1e-12
    # the headline (D = 128): the MFMA floor binds, 0.44 ms at 2.5 PFLOP/s
    scores = 128 * 4096 * 4096
    r = b.bounds(4.0 * 128 * scores, scores, 0.88)
    assert r["bound"] == "mfma" and abs(r["mfma_floor_ms"] - 0.43980465) < 1e-6
    assert r["valu_floor_ms"] < r["mfma_floor_ms"]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "ONE GPU only" in (r.stdout + r.stderr)
