"""attn_flash_noalloc, the allocation-free variant of attn_flash: its split-K partials live in the
library's static device array instead of a caller's scratch. Each case runs two calls in a row
through the C ABI, the second with a smaller input (so stale partials of the first call would
show), and each output must equal attn_flash's with a caller-owned scratch bit for bit (same
kernels, same splits, same slot layout), and pass the oracle on spread rows. Every case takes a
path that writes partials: attn_flash's scratch, poisoned before its call, must have changed."""
import sys

import numpy as np
import pytest

import transfer_station_amd as ts

pytestmark = pytest.mark.gpu

SEED0 = 0x12345678


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu_present():
    assert ts.device_count() >= 1, "no HIP device visible: GPU tests must run on the MI355X box"


def run_both(Hq, Hkv, Sq, Sk, D, causal, seed, v_prepacked=0):
    """(O from attn_flash with its own scratch, O from attn_flash_noalloc, host inputs, bytes of
    attn_flash's scratch that its call changed)."""
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, seed)
    Vin = V.reshape(Hkv, Sk, D).transpose(0, 2, 1).copy().ravel() if v_prepacked else V
    outs = []
    with ts.DeviceBuffer.from_array(Q) as dq, ts.DeviceBuffer.from_array(K) as dk, \
            ts.DeviceBuffer.from_array(Vin) as dv, ts.DeviceBuffer(Hq * Sq * D * 4) as do, \
            ts.DeviceBuffer(ts.attn_flash_scratch_bytes(D, 128)) as ds:
        do.fill_bytes(0xFF)
        ds.fill_bytes(0xFF)
        ts.attn_flash(dq, dk, dv, do, Hq, Hkv, Sq, Sk, D, causal, 128, ds, v_prepacked)
        ts.synchronize()
        outs.append(do.download(np.float32))
        changed = int(np.count_nonzero(ds.download(np.uint8) != 0xFF))
        do.fill_bytes(0xFF)
        ts.attn_flash_noalloc(dq, dk, dv, do, Hq, Hkv, Sq, Sk, D, causal, 128, v_prepacked)
        ts.synchronize()
        outs.append(do.download(np.float32))
    return outs[0], outs[1], (Q, K, V), changed


# (label, Hq, Hkv, Sq, Sk, D, causal, v_prepacked): pairs of a larger then a smaller call, each
# on a path that writes partial slots and merges them: split-K decode (row-major V and V^T),
# the causal prefill's split of its upper query tiles, the prefill key split of small grids, and
# the slot-balanced head split (D <= 64; MHA grids whose 192-row workgroups would not fit one
# per CU).
PAIRS = [
    (("decode split 32k", 32, 8, 1, 32768, 128, 0, 0),
     ("decode split 4k", 32, 8, 1, 4096, 128, 0, 0)),
    (("prefill causal split 2k", 8, 2, 2048, 2048, 128, 1, 0),
     ("prefill causal split 2k MQA", 4, 1, 2048, 2048, 128, 1, 0)),
    (("prefill key split 8k causal", 32, 8, 512, 8192, 128, 1, 0),
     ("prefill key split 4k", 16, 4, 512, 4096, 128, 0, 0)),
    (("prefill head split D64", 48, 48, 1000, 4000, 64, 0, 0),
     ("prefill head split D40", 46, 46, 1000, 2056, 40, 0, 0)),
    (("decode split 8k D64 V^T", 16, 4, 4, 8192, 64, 1, 1),
     ("decode split 1k D40", 8, 2, 2, 1000, 40, 0, 0)),
]


@pytest.mark.parametrize("pair", PAIRS, ids=[p[0][0] for p in PAIRS])
def test_noalloc_matches_attn_flash_twice(oracle, pair):
    for i, (label, Hq, Hkv, Sq, Sk, D, causal, vt) in enumerate(pair):
        say("noalloc case %s (call %d): Hq=%d Hkv=%d Sq=%d Sk=%d D=%d causal=%d vt=%d" %
            (label, i + 1, Hq, Hkv, Sq, Sk, D, causal, vt))
        ref, got, (Q, K, V), changed = run_both(Hq, Hkv, Sq, Sk, D, causal, SEED0 + 17 * i, vt)
        say("   %d scratch bytes written by attn_flash" % changed)
        assert changed > 0, label  # the case must exercise the partial slots
        assert np.all(np.isfinite(got)), label
        assert np.array_equal(ref, got), label
        rows = oracle.ref_rowset(Sq, 8)
        R = oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, rows, nthreads=8)
        ok, mad, maxref, nbad = oracle.cmp_rows(R, got, Hq, Sq, D, rows)
        say("   bit-identical to attn_flash; err/scale=%.2e nbad=%d -> %s" %
            (mad / maxref if maxref else 0.0, nbad, "PASS" if ok else "FAIL"))
        assert ok, (label, mad, maxref, nbad)
