"""GPU parity: the HIP kernels, called through the C ABI (libattn_flash.so), against the CPU
oracle on identical bf16 bit patterns, with the reference's pass rule
nbad == 0 and max|O - O_ref| <= 8e-3 * max|O_ref| over the checked rows (flash.c:935-980).

Outputs are poisoned with NaN before each call, so an unwritten row is a failure. Large
configurations check the reference's spread rows (flash.c:900-913), which always include
row Sq-1 (every key block and every rescale)."""
import os
import sys

import numpy as np
import pytest

import transfer_station_amd as ts

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NT = min(16, os.cpu_count() or 1)
SEED0 = 0x12345678


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu_present():
    n = ts.device_count()
    assert n >= 1, "no HIP device visible: GPU tests must run on the MI355X box"


def check(oracle, name, Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk=128, ref_cap=0, O=None):
    say("case %s: Hq=%d Hkv=%d Sq=%d Sk=%d D=%d causal=%d bk=%d" % (name, Hq, Hkv, Sq, Sk, D,
                                                                     causal, bk))
    if O is None:
        O = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk)
    rows = oracle.ref_rowset(Sq, ref_cap)
    R = oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, rows, nthreads=NT)
    ok, mad, maxref, nbad = oracle.cmp_rows(R, O, Hq, Sq, D, rows)
    say("   err/scale=%.2e nbad=%d -> %s" % (mad / maxref if maxref else 0.0, nbad,
                                            "PASS" if ok else "FAIL"))
    assert ok, (name, mad, maxref, nbad)
    return O


# ---- the reference's short suite (LCG data, every row) ---------------------------------------
SUITE = [
    ("MHA prefill", 4, 4, 8, 8, 64, 0),
    ("MHA prefil.causal", 4, 4, 8, 8, 64, 1),
    ("GQA prefill", 8, 2, 8, 8, 64, 0),
    ("GQA prefil.causal", 8, 2, 8, 8, 64, 1),
    ("MHA decode(Sq=1)", 4, 4, 1, 16, 64, 0),
    ("GQA decode(Sq=1)", 8, 2, 1, 16, 64, 0),
    ("MQA prefill", 8, 1, 8, 8, 64, 0),
    ("odd + multiblock", 6, 3, 130, 70, 40, 1),
    ("GQA big head_dim", 8, 2, 4, 12, 128, 0),
]


@pytest.mark.parametrize("bk", [16, 32, 64, 128, 256, 4096])
@pytest.mark.parametrize("case", SUITE, ids=[c[0] for c in SUITE])
def test_reference_suite(oracle, case, bk):
    name, Hq, Hkv, Sq, Sk, D, causal = case
    Q, K, V = ts.synth_lcg_qkv(Hq, Hkv, Sq, Sk, D)
    check(oracle, name, Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk)


def test_golden_fixtures_direct():
    import json
    from oracle import oracle as o
    man = json.load(open(os.path.join(GOLD, "manifest.json")))
    for m in man:
        z = np.load(os.path.join(GOLD, m["file"]))
        if m["data"] == "lcg":
            Q, K, V = o.lcg_qkv(m["Hq"], m["Hkv"], m["Sq"], m["Sk"], m["D"], m["seed"])
        else:
            Q, K, V = z["Q"], z["K"], z["V"]
        say("fixture %s" % m["name"])
        O = ts.run_attention(Q, K, V, m["Hq"], m["Hkv"], m["Sq"], m["Sk"], m["D"], m["causal"])
        G = z["O"]
        assert np.isfinite(O).all()
        err = np.abs(O - G).max() / np.abs(G).max()
        say("   err/scale vs float64 = %.2e" % err)
        assert err <= 8e-3, m["name"]


# ---- the benchmark configurations c1-c5 --------------------------------------------------------
def test_c1_mha_256(oracle):
    Q, K, V = ts.synth_normal_qkv(4, 4, 256, 256, 64, SEED0 + 1)
    check(oracle, "c1 MHA", Q, K, V, 4, 4, 256, 256, 64, 0, 128)


def test_c2_gqa_decode(oracle):
    B, Hq, Hkv, Sk, D = 64, 32, 8, 4096, 128
    Q, K, V = ts.synth_normal_qkv(B * Hq, B * Hkv, 1, Sk, D, SEED0 + 2)
    check(oracle, "c2 GQA decode", Q, K, V, B * Hq, B * Hkv, 1, Sk, D, 0, 128)


@pytest.mark.parametrize("Hkv,Sk", [(8, 4096), (8, 1000), (2, 777), (1, 64)])
def test_decode_split_paths(oracle, Hkv, Sk):
    """Few kv heads -> the key range is split over workgroups and merged (attn_merge_kernel)."""
    Hq, D = Hkv * 4, 128
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, 1, Sk, D, SEED0 + 20 + Sk)
    check(oracle, "decode split", Q, K, V, Hq, Hkv, 1, Sk, D, 0, 128)
    # g*Sq = 16 rows: the largest query block the decode tile holds, causal
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, 4, Sk, D, SEED0 + 21 + Sk)
    check(oracle, "decode split causal Sq=4", Q, K, V, Hq, Hkv, 4, Sk, D, 1, 128)


@pytest.mark.parametrize("Hq,Hkv,Sq,Sk,D,causal", [
    (32, 4, 8, 1000, 128, 1),   # g*Sq = 64: four 16-row blocks (speculative decoding, GQA 8)
    (64, 1, 1, 3000, 128, 0),   # MQA decode with 64 query heads
    (8, 2, 5, 300, 64, 1),      # 20 rows: a partial second block
    (6, 3, 17, 200, 40, 1),     # 34 rows, D = 40
    (16, 2, 3, 4096, 128, 0),   # 24 rows, split over the key range
    (4, 4, 17, 64, 64, 0),      # g = 1, Sq = 17
])
def test_decode_row_blocks(oracle, Hq, Hkv, Sq, Sk, D, causal):
    """Up to 64 query rows per kv head (g*Sq) take the split-K decode kernel in 16-row blocks
    while there are fewer kv heads than CUs."""
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 60 + Sq)
    check(oracle, "decode row blocks", Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128)


@pytest.mark.parametrize("Hq,Hkv,Sq,Sk,D,causal", [
    (2048, 512, 1, 4104, 128, 0),  # 33 steps: a one-step last group, met mid-walk by most WGs
    (8, 2, 1, 1000, 128, 0),       # 8 splits of one step each
    (64, 16, 1, 6000, 128, 0),     # 24 splits of 2 steps, the last split one partial step
    (512, 128, 1, 2600, 64, 1),    # D = 64: 2 tiles rows of 16; splits of 6 steps (4 + 2)
    (256, 64, 4, 3000, 128, 1),    # 16 rows, causal mask in the last steps, 3-step splits
    (96, 8, 4, 5000, 96, 1),       # D = 96 on 128-wide tiles, 3 row blocks
    (40, 8, 2, 1000, 40, 0),       # D = 40 on 64-wide tiles
])
def test_decode_vt_groups(oracle, Hq, Hkv, Sq, Sk, D, causal):
    """The V^T decode kernel walks the keys in groups of four 128-key steps, starting at a
    different group per workgroup, and multiplies each group's V^T tiles one interval after
    scoring it. Step counts that leave a partial last group (met in the middle of the walk by
    most workgroups), splits of one to six steps, head dims that leave zero tile rows and
    several row blocks must all give the row-major kernel's bits and the oracle's answer."""
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 110 + Sk)
    O = check(oracle, "decode V^T groups", Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128)
    Ot = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, prepack_v=True)
    assert np.array_equal(O.view(np.uint32), Ot.view(np.uint32))


@pytest.mark.parametrize("Hq,Hkv,Sq,Sk,D,causal", [
    (1024, 256, 8, 300, 64, 1),   # 32 rows per kv head, 256 kv heads: packed prefill
    (2048, 512, 16, 520, 128, 0), # 64 rows, 512 kv heads
    (1024, 256, 4, 777, 128, 1),  # 16 rows: decode at any kv-head count
])
def test_short_queries_many_kv_heads(oracle, Hq, Hkv, Sq, Sk, D, causal):
    """Decode-sized query blocks (g*Sq <= 64) over at least as many kv heads as CUs go to the
    packed prefill tiles (up to 16 rows, to decode); the answer is the same either way."""
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 90 + Sq)
    check(oracle, "short queries, many kv heads", Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128,
          ref_cap=4)


@pytest.mark.parametrize("S", [1024, 2048, 4096])
def test_c3_gqa_prefill(oracle, S):
    B, Hq, Hkv, D = 4, 32, 8, 128
    Q, K, V = ts.synth_normal_qkv(B * Hq, B * Hkv, S, S, D, SEED0 + 3)
    check(oracle, "c3 GQA prefill %d" % S, Q, K, V, B * Hq, B * Hkv, S, S, D, 0, 128, ref_cap=8)


def test_c4_mqa_prefill(oracle):
    B, Hq, Hkv, S, D = 8, 16, 1, 2048, 128
    Q, K, V = ts.synth_normal_qkv(B * Hq, B * Hkv, S, S, D, SEED0 + 4)
    check(oracle, "c4 MQA prefill", Q, K, V, B * Hq, B * Hkv, S, S, D, 0, 128, ref_cap=8)


@pytest.mark.parametrize("bk", [32, 64, 128, 256, 512])
def test_c5_ragged_softmax_stress(oracle, bk):
    B, Hq, Hkv, Sq, Sk, D = 2, 24, 6, 1000, 4000, 64
    Q, K, V = ts.synth_normal_qkv(B * Hq, B * Hkv, Sq, Sk, D, SEED0 + 5, sigma_q=4.0)
    check(oracle, "c5 ragged", Q, K, V, B * Hq, B * Hkv, Sq, Sk, D, 0, bk, ref_cap=16)


def test_qwen3_causal_long(oracle):
    """The reference's --long case shape (flash.c:1312-1314) at 1k, causal, spread rows."""
    Q, K, V = ts.synth_lcg_qkv(16, 8, 1024, 1024, 128)
    check(oracle, "qwen3 1k causal", Q, K, V, 16, 8, 1024, 1024, 128, 1, 128, ref_cap=8)


# ---- causal grids of one or two 128-row tiles per CU (the reference's Qwen3 shapes): the causal
# key split (the heavier tiles' key ranges in two workgroups, merged through the scratch), key
# halves, and their persistent variant (Qwen3 4k) ------------------------------------------------
@pytest.mark.parametrize("shape", [
    (16, 8, 4096, 4096, 128, 8),   # the reference's --long qwen3 4k
    (16, 8, 2048, 2048, 128, 8),
    (8, 2, 1000, 3000, 128, 0),    # Sk > Sq, every row
    (4, 4, 700, 300, 64, 0),       # Sq > Sk: rows below Sq - Sk attend nothing
    (6, 3, 600, 600, 40, 0),       # D = 40 on the 64-wide tiles (zero columns 40..63)
    (8, 4, 1500, 1500, 96, 8),     # D = 96 on the 96-wide tiles
    (8, 2, 900, 1100, 80, 8),      # D = 80 on the 96-wide tiles
], ids=["qwen3-4k", "qwen3-2k", "sk>sq", "sq>sk", "d40", "d96", "d80"])
def test_causal_split_small_grid(oracle, shape):
    Hq, Hkv, Sq, Sk, D, cap = shape
    Q, K, V = ts.synth_lcg_qkv(Hq, Hkv, Sq, Sk, D)
    O = check(oracle, "causal small grid", Q, K, V, Hq, Hkv, Sq, Sk, D, 1, 128, ref_cap=cap)
    if Sq > Sk:
        assert np.all(O.reshape(Hq, Sq, D)[:, :Sq - Sk] == 0.0)
    again = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, 1, 128)
    assert np.array_equal(O.view(np.uint32), again.view(np.uint32))


# ---- tails, head_dim, masks -----------------------------------------------------------------------
@pytest.mark.parametrize("D", [64, 96, 128])
@pytest.mark.parametrize("causal", [0, 1])
@pytest.mark.parametrize("bk", [32, 64, 128])
def test_tail_probe(oracle, bk, causal, D):
    """The reference's tail probe (README:550-554): Sk around multiples of bk, at each tile
    width the fast kernel is built for."""
    for Sk in (1, bk - 1, bk, bk + 1, 2 * bk, 2 * bk + 1, 70):
        for Sq in (40, 1):
            Q, K, V = ts.synth_lcg_qkv(4, 2, Sq, Sk, D)
            check(oracle, "tail", Q, K, V, 4, 2, Sq, Sk, D, causal, bk)


@pytest.mark.parametrize("D", [1, 2, 3, 7, 8, 16, 24, 33, 40, 63, 64, 65, 72, 100, 127, 128, 129,
                               160, 200, 255, 256])
def test_head_dim_sweep(oracle, D):
    for Sq, Hq, Hkv in ((37, 4, 2), (1, 8, 2)):
        Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, 150, D, 1000 + D)
        check(oracle, "D sweep", Q, K, V, Hq, Hkv, Sq, 150, D, 1, 64)


# ---- head dims past 128 (up to ATTN_D_MAX = 256): the general prefill kernel on 32-key tiles
# and the 256-wide decode kernel ----------------------------------------------------------------
@pytest.mark.parametrize("shape", [
    (8, 2, 300, 700, 256, 1, 64, 0),     # GQA prefill, causal, bk 64
    (16, 4, 200, 333, 256, 0, 4096, 0),  # prefill, Sk % 8 != 0, one scratch for the largest bk
    (32, 8, 1, 4096, 256, 0, 128, 0),    # split-K decode
    (8, 1, 5, 1001, 192, 1, 128, 0),     # decode row blocks, D = 192
    (8, 2, 300, 640, 256, 1, 128, 1),    # prefill from V^T
    (8, 2, 1, 2048, 256, 0, 128, 1),     # decode from V^T
    (8, 2, 200, 500, 224, 1, 16, 0),     # causal key split, D = 224, bk 16
    (6, 3, 130, 70, 200, 1, 128, 0),     # general kernel (D % 8 != 0)
], ids=["prefill-causal", "prefill-ragged", "decode", "decode-d192", "prefill-vt", "decode-vt",
        "bk16-split-d224", "general-d200"])
def test_head_dim_256(oracle, shape):
    Hq, Hkv, Sq, Sk, D, causal, bk, vt = shape
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 256 + Sk)
    if vt:
        vt_host = np.ascontiguousarray(V.reshape(Hkv, Sk, D).transpose(0, 2, 1)).ravel()
        O = ts.run_attention(Q, K, vt_host, Hq, Hkv, Sq, Sk, D, causal, bk, v_prepacked=1)
    else:
        O = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk)
    check(oracle, "D=%d" % D, Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk, ref_cap=8, O=O)


# ---- short query blocks under GQA (Sq below a workgroup's rows, g*Sq > 64): the g heads' rows
# of a kv head are packed into shared query tiles --------------------------------------------------
@pytest.mark.parametrize("shape", [
    (32, 8, 17, 1000, 128, 1, 0),   # 68 rows per kv head, causal
    (32, 8, 40, 333, 128, 0, 0),    # 160 rows, Sk % 8 != 0
    (64, 4, 5, 700, 64, 1, 0),      # g = 16, 80 rows
    (16, 2, 100, 100, 96, 1, 0),    # Sq == Sk causal, D = 96
    (8, 1, 200, 4096, 128, 1, 0),   # MQA, 1600 rows in 8-wave tiles
    (32, 8, 33, 640, 128, 1, 1),    # V^T input
    (24, 6, 50, 500, 256, 1, 0),    # D = 256
    (32, 8, 40, 20, 128, 1, 0),     # Sq > Sk: each head's first 20 rows attend nothing
    (16, 1, 60, 7, 64, 1, 0),       # MQA, Sk below one key tile
], ids=["g4-sq17", "g4-sq40", "g16-sq5", "g8-sq100-d96", "mqa-sq200", "vt", "d256", "sq>sk",
        "mqa-sk7"])
def test_gqa_packed_short_queries(oracle, shape):
    Hq, Hkv, Sq, Sk, D, causal, vt = shape
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 700 + Sq)
    if vt:
        vt_host = np.ascontiguousarray(V.reshape(Hkv, Sk, D).transpose(0, 2, 1)).ravel()
        O = ts.run_attention(Q, K, vt_host, Hq, Hkv, Sq, Sk, D, causal, 128, v_prepacked=1)
    else:
        O = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128)
    check(oracle, "packed", Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128, O=O)
    if causal and Sq > Sk:
        assert np.all(O.reshape(Hq, Sq, D)[:, :Sq - Sk] == 0.0)


def test_sk_one_copies_v(oracle):
    """Sk = 1: a one-element softmax. The kernels evaluate p = 2^(s*c - m*c) with one fma, so
    p at the row max is 1 within 2^-23 (not exactly 1, unlike the reference's exp(s - m)):
    O equals V[0] to within a few ulp (and bf16(p) == 1 exactly)."""
    for Sq in (1, 50):
        Q, K, V = ts.synth_normal_qkv(8, 2, Sq, 1, 128, 7)
        O = ts.run_attention(Q, K, V, 8, 2, Sq, 1, 128, 0).reshape(8, Sq, 128)
        Vf = oracle.bf16_to_f32(V).reshape(2, 128)
        for h in range(8):
            want = np.broadcast_to(Vf[h // 4], (Sq, 128))
            assert np.all(np.abs(O[h] - want) <= 2.0 ** -21 * np.abs(want))


def test_fully_masked_causal_rows_are_zero():
    Q, K, V = ts.synth_lcg_qkv(6, 3, 130, 70, 40)
    O = ts.run_attention(Q, K, V, 6, 3, 130, 70, 40, 1).reshape(6, 130, 40)
    assert np.all(O[:, :60] == 0.0) and np.isfinite(O).all()
    Q, K, V = ts.synth_normal_qkv(8, 2, 300, 20, 128, 8)
    O = ts.run_attention(Q, K, V, 8, 2, 300, 20, 128, 1).reshape(8, 300, 128)
    assert np.all(O[:, :280] == 0.0) and np.all(np.abs(O[:, 280:]).max(axis=2) > 0)


# ---- invariants (GPU against GPU) ------------------------------------------------------------------
def test_gqa_equals_mha_with_repeated_kv_bitwise():
    Hq, Hkv, Sq, Sk, D = 16, 4, 200, 333, 128
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, 11)
    g = Hq // Hkv
    Kr = np.repeat(K.reshape(Hkv, 1, -1), g, axis=1).reshape(-1)
    Vr = np.repeat(V.reshape(Hkv, 1, -1), g, axis=1).reshape(-1)
    for causal in (0, 1):
        a = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal)
        b = ts.run_attention(Q, Kr, Vr, Hq, Hq, Sq, Sk, D, causal)
        assert np.array_equal(a, b)


def test_batch_fold_bitwise_and_determinism():
    B, Hq, Hkv, Sq, Sk, D = 3, 8, 2, 150, 260, 64
    Q, K, V = ts.synth_normal_qkv(B * Hq, B * Hkv, Sq, Sk, D, 12)
    folded = ts.run_attention(Q, K, V, B * Hq, B * Hkv, Sq, Sk, D, 1)
    again = ts.run_attention(Q, K, V, B * Hq, B * Hkv, Sq, Sk, D, 1)
    assert np.array_equal(folded, again)  # run-to-run bitwise (no LDS races)
    nq, nk = Hq * Sq * D, Hkv * Sk * D
    for b in range(B):
        one = ts.run_attention(Q[b * nq:(b + 1) * nq], K[b * nk:(b + 1) * nk],
                               V[b * nk:(b + 1) * nk], Hq, Hkv, Sq, Sk, D, 1)
        assert np.array_equal(folded[b * nq:(b + 1) * nq], one)


@pytest.mark.parametrize("Hq,Hkv,Sq,Sk,D,causal,ref_cap", [
    (32, 8, 512, 8192, 128, 0, 8),   # chunked prefill: 128 query tiles, key range in 4 parts
    (32, 8, 512, 8192, 128, 1, 8),   # the same, causal (the keys before the block dominate)
    (64, 8, 128, 8192, 128, 1, 8),   # 8 parts
    (8, 1, 1024, 8192, 128, 0, 8),   # MQA
    (16, 4, 256, 4096, 64, 0, 0),    # D = 64 (software-pipelined tiles inside each part)
    (8, 2, 512, 1024, 128, 1, 0),    # causal, Sk - Sq == Sq: the shortest tiles get empty parts
    (6, 3, 200, 777, 36, 0, 0),      # general kernel (D % 8 != 0): no split, the same answer
])
def test_prefill_key_split(oracle, Hq, Hkv, Sq, Sk, D, causal, ref_cap):
    """Grids that fill at most half of one round of resident workgroups split each query tile's
    key tiles into parts whose partials (m, l, acc) attn_mergew_kernel combines. Every row that
    the reference's row set picks is checked, with the V^T input giving the same bits where
    both inputs take the fast kernel (D % 8 == 0 and Sk % 8 == 0)."""
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 70 + Sq)
    O = check(oracle, "prefill key split", Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128,
              ref_cap=ref_cap)
    if D % 8 == 0 and Sk % 8 == 0:
        Ot = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, prepack_v=True)
        assert np.array_equal(O, Ot)


@pytest.mark.parametrize("Hq,Hkv,Sq,Sk,D,causal,ref_cap", [
    (16, 8, 4096, 4096, 128, 1, 8),   # Qwen3 4k causal: 512 tiles of 128 rows, two rounds
    (16, 8, 4096, 4200, 128, 1, 8),   # the same with keys before the query block
    (16, 8, 2048, 2048, 128, 0, 8),   # 256 tiles, one per CU
    (24, 8, 1000, 1000, 128, 0, 0),   # a ragged query tail, every row
    (16, 4, 2048, 2056, 96, 0, 8),    # the 96-wide tiles, a key tail in the second half
    (8, 1, 1024, 8192, 128, 0, 8),    # MQA, with the key split on top (4 parts)
    (16, 8, 1024, 4096, 128, 1, 8),   # causal with 3072 keys before the block: key split too
    (8, 2, 2048, 2048, 128, 1, 8),    # triangular causal, 128 tiles: the causal key split too
    (16, 8, 2048, 2048, 128, 1, 8),   # triangular causal, 256 tiles: no split (one round)
    (32, 8, 1024, 1000, 64, 0, 8),    # D = 64 (64-key halves of 128-key tiles), a key tail
    (16, 8, 2048, 2048, 64, 1, 8),    # D = 64, triangular causal
])
def test_prefill_key_halves(oracle, Hq, Hkv, Sq, Sk, D, causal, ref_cap):
    """Grids that would run 4-wave workgroups at D > 64 with at most one 128-row tile per CU,
    or exactly two (causal), run 8 waves per 128 rows instead: waves w and w + 4
    take the two 64-key halves of every 128-key tile and combine (m, l, o) through LDS. The rows
    the reference's row set picks are checked against the oracle; the V^T input gives the same
    bits (within the tolerance where row-major V takes the persistent variant and V^T the
    per-tile kernel: Qwen3 4k), and a second call repeats them."""
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 110 + Sq + Sk)
    O = check(oracle, "prefill key halves", Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128,
              ref_cap=ref_cap)
    Ot = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, prepack_v=True)
    if ts.attn_flash_plan(Hq, Hkv, Sq, Sk, D, causal)[0][0].startswith("attn_prefill_persist"):
        assert np.abs(O - Ot).max() <= 8e-3 * np.abs(O).max()
    else:
        assert np.array_equal(O.view(np.uint32), Ot.view(np.uint32))
    again = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128)
    assert np.array_equal(O.view(np.uint32), again.view(np.uint32))


HEAD_SPLIT_CASES = [
    (48, 12, 1000, 4000, 64, 4.0, 8),  # config 5: 384 tiles (the last 16 heads halved); 252 x 192
    (40, 10, 1000, 4000, 64, 1.0, 8),  # 320 tiles (24 heads halved); 210 x 192 rows
    (20, 5, 1800, 2056, 40, 1.0, 0),   # D = 40 on the 64-wide tiles, a key tail, every row
    (40, 40, 1000, 4000, 64, 1.0, 8),  # MHA: 6 workgroups per head, the last of 40 rows
]


@pytest.mark.parametrize("Hq,Hkv,Sq,Sk,D,sigma_q,ref_cap", HEAD_SPLIT_CASES)
def test_prefill_head_split(oracle, Hq, Hkv, Sq, Sk, D, sigma_q, ref_cap):
    """Non-causal D <= 64 grids of one to two 128-row tiles per CU (where the 4-wave grid would
    run the last heads' tiles as key halves merged through the scratch) run as 12-wave key-halves
    workgroups of 192 rows of a kv head's packed row space (32-row blocks straddle query heads;
    each kv head's last workgroup is part empty), one per CU. The rows the reference's row set
    picks are checked against the oracle; the V^T input takes the same kernel and gives the same
    bits, and a second call repeats them."""
    if ts.device_info()["cus"] == 256:
        plan = ts.attn_flash_plan(Hq, Hkv, Sq, Sk, D, 0)
        assert [p[0] for p in plan] == ["attn_prefill_fast_kernel<64, 128, 12, false, false, true>"]
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 90 + Hq, sigma_q=sigma_q)
    O = check(oracle, "prefill 12 waves", Q, K, V, Hq, Hkv, Sq, Sk, D, 0, 128, ref_cap=ref_cap)
    Ot = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, 0, prepack_v=True)
    assert np.array_equal(O.view(np.uint32), Ot.view(np.uint32))
    again = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, 0, 128)
    assert np.array_equal(O.view(np.uint32), again.view(np.uint32))


_HSPLIT_SCRIPT = r"""
import sys, numpy as np
sys.path.insert(0, %r)
import transfer_station_amd as ts
from oracle import oracle as o
for (Hq, Hkv, Sq, Sk, D, sigma_q, cap) in %r:
    plan = ts.attn_flash_plan(Hq, Hkv, Sq, Sk, D, 0)
    print("head split case", Hq, Hkv, Sq, Sk, D, plan, flush=True)
    if ts.device_info()["cus"] == 256:
        assert [p[0] for p in plan] == ["attn_prefill_fast_kernel<64, 128, 4, false, false, false>",
                                        "attn_merge2_kernel"], plan
        assert "hsplit=0" not in plan[0][1].split(), plan
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, 90 + Hq, sigma_q=sigma_q)
    O = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, 0, 128)
    rows = o.ref_rowset(Sq, cap)
    R = o.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, 0, rows, nthreads=8)
    ok, mad, maxref, nbad = o.cmp_rows(R, O, Hq, Sq, D, rows)
    print("   err/scale", mad / maxref, nbad, flush=True)
    assert ok
    Ot = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, 0, prepack_v=True)
    assert np.array_equal(O.view(np.uint32), Ot.view(np.uint32))
print("OK")
"""


def test_prefill_head_split_4_waves():
    """The same grids with the 12-wave workgroups turned off (ATTN_PREFILL_W12=0, in a child
    process) take 4-wave workgroups with the slot-balanced head split: whole tiles in the CUs'
    first slots, the last heads' tiles as two key halves merged through the scratch
    (attn_merge2_kernel)."""
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, ATTN_PREFILL_W12="0")
    r = subprocess.run([sys.executable, "-c", _HSPLIT_SCRIPT % (root, HEAD_SPLIT_CASES[:3])],
                       env=env, capture_output=True, text=True, timeout=240)
    say(r.stdout[-2000:] + r.stderr[-2000:])
    assert r.returncode == 0 and r.stdout.strip().endswith("OK")


@pytest.mark.parametrize("Hq,Hkv,Sq,Sk,D,causal", [
    (8, 2, 300, 1504, 128, 0),    # 8-wave workgroups, 128-key tiles
    (8, 2, 500, 1504, 128, 1),    # 4-wave workgroups, 64-key tiles, causal
    (8, 2, 600, 2104, 64, 0),
    (4, 1, 1024, 1024, 128, 1),   # causal small grid: upper query tiles split over two items
    (128, 32, 1024, 1504, 128, 0),  # the persistent prefill (12 key tiles per item)
    (128, 32, 1024, 1024, 128, 1),  # the causal persistent prefill (pairs of 2 + 8, 4 + 6 tiles)
    (64, 16, 1024, 1024, 128, 1),  # the persistent prefill with key halves (pairs of 8 + 1 ...)
    (24, 6, 1500, 2104, 64, 0),    # 12 waves on key halves, 192 packed rows, pipelined halves
])
def test_score_jumps_between_key_tiles(oracle, Hq, Hkv, Sq, Sk, D, causal):
    """Each query row gets a first coordinate of +4 or -4 and each key a first coordinate that
    steps with its 64-key block, by amounts from under the rescale margin to far past it: up
    to 2^600 against a max from an earlier block, beyond fp32's range. Rows of either sign see
    their maximum rise in later key tiles by every size of jump, and fall. That is the path on
    which the running max, its rescale and the tile-sum test must all hold. Every row is
    checked (the spread rows on the persistent grid); the V^T input must give the same bits,
    or, where row-major V takes the persistent prefill and V^T the per-tile kernel, agree
    within the tolerance."""
    rng = np.random.default_rng(21)
    steps = np.array([0, 1, -3, 6, 60, 2, -40, 300, 301, 5, -300, 700, 0, 1200, 20, 1300, 8],
                     dtype=np.float32)
    q = oracle.bf16_to_f32(ts.synth_normal_bf16(Hq * Sq * D, 31, 0)).reshape(Hq * Sq, D)
    q[:, 0] = np.where(rng.random(Hq * Sq) < 0.5, -4.0, 4.0)
    k = oracle.bf16_to_f32(ts.synth_normal_bf16(Hkv * Sk * D, 31, Hq * Sq * D)).reshape(Hkv, Sk, D)
    k[:, :, 0] = steps[(np.arange(Sk) // 64) % len(steps)]
    Q = oracle.f32_to_bf16(q).reshape(-1)
    K = oracle.f32_to_bf16(k).reshape(-1)
    V = ts.synth_normal_bf16(Hkv * Sk * D, 32, 0)
    persist = ts.attn_flash_plan(Hq, Hkv, Sq, Sk, D, causal)[0][0].startswith("attn_prefill_persist")
    O = check(oracle, "score jumps", Q, K, V, Hq, Hkv, Sq, Sk, D, causal,
              ref_cap=8 if persist else 0)
    Ot = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, prepack_v=True)
    if persist:
        assert np.abs(O - Ot).max() <= 8e-3 * np.abs(O).max()
    else:
        assert np.array_equal(O, Ot)


def test_key_permutation_invariance(oracle):
    Hq, Hkv, Sq, Sk, D = 4, 2, 64, 500, 64
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, 13)
    perm = np.random.default_rng(0).permutation(Sk)
    Kp = K.reshape(Hkv, Sk, D)[:, perm].reshape(-1).copy()
    Vp = V.reshape(Hkv, Sk, D)[:, perm].reshape(-1).copy()
    a = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, 0)
    b = ts.run_attention(Q, Kp, Vp, Hq, Hkv, Sq, Sk, D, 0)
    rows = np.arange(Sq, dtype=np.int32)
    assert oracle.cmp_rows(a, b, Hq, Sq, D, rows)[0]


@pytest.mark.parametrize("D,Sk", [(128, 1000), (64, 4000), (256, 333), (200, 150)])
def test_bk_invariance(oracle, D, Sk):
    """The reference's result is bk-invariant within the tolerance (README:354-357). Here bk is
    validated and sizes the scratch but never picks the key tile, so O is bit-identical at
    every bk, on the fast, the D > 128 and the general (D % 8 != 0) kernels alike."""
    Hq, Hkv, Sq = 8, 2, 300
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, 14)
    base = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, 1, 128)
    check(oracle, "bk invariance D=%d" % D, Q, K, V, Hq, Hkv, Sq, Sk, D, 1, 128, ref_cap=8, O=base)
    for bk in (16, 32, 64, 256, 1024, 4096):
        other = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, 1, bk)
        assert np.array_equal(base, other), bk


# ---- the other entry points ------------------------------------------------------------------------
@pytest.mark.parametrize("Hkv,Sk,D,offset", [
    (3, 77, 40, 0),     # element-wise path (Sk % 8 != 0)
    (3, 80, 40, 0),     # 16-byte path, partial 64-column tile
    (1, 200, 64, 0),    # 16-byte path, partial key tile (72 of 128 keys)
    (2, 136, 96, 0),    # 16-byte path, one 8-key chunk in the last key tile, 32 of 64 columns
    (2, 4096, 128, 0),  # 16-byte path, full tiles
    (2, 8, 8, 0),       # 16-byte path, one chunk per row
    (2, 64, 64, 2),     # misaligned by one element: element-wise path
    (65535 + 7, 8, 8, 0),  # more kv heads than one launch's z range: two launches
    (65535 + 2, 9, 7, 0),  # the same on the element-wise path
])
def test_pack_v_full_transposes_exactly(Hkv, Sk, D, offset):
    rng = np.random.default_rng(Sk * 1000 + D)
    V = rng.integers(0, 1 << 16, size=Hkv * Sk * D, dtype=np.uint16)
    guard = 256
    with ts.DeviceBuffer(V.nbytes + offset) as dv, ts.DeviceBuffer(V.nbytes + offset + guard) as dp:
        dv.upload(np.concatenate([np.zeros(offset // 2, np.uint16), V]))
        dp.fill_bytes(0x5A)
        ts.pack_v_full(dv.ptr + offset, dp.ptr + offset, Hkv, Sk, D)
        ts.synchronize()
        raw = dp.download(np.uint8)
        got = raw[offset:offset + V.nbytes].view(np.uint16).reshape(Hkv, D, Sk)
    assert np.array_equal(got, V.reshape(Hkv, Sk, D).transpose(0, 2, 1))
    assert np.all(raw[:offset] == 0x5A) and np.all(raw[offset + V.nbytes:] == 0x5A)


# ---- v_prepacked = 1: V^T [Hkv][D][Sk] input (flash.c:751-753,770,812-833) -----------------------
# The reference changes only V's stride when V is pre-packed, so the math is identical. Here the
# V^T operand of the P.V MFMA holds the same values in the same positions either way, so O is
# bit-identical whenever both layouts run the same kernel. They do not when D % 8 == 0 and
# Sk % 8 != 0 (a V^T row is then not 16-byte aligned and the prefill takes the general kernel
# while row-major V takes the fast one): those cases are held to the oracle tolerance only.
VT_CASES = [
    # name, Hq, Hkv, Sq, Sk, D, causal, bk
    ("fast D128 partial tile", 8, 2, 300, 1000, 128, 0, 128),
    ("fast D128 causal", 8, 2, 513, 1024, 128, 1, 64),
    ("fast D128 kt128 causal", 8, 2, 700, 1000, 128, 1, 128),
    ("fast D64 kt128 causal", 4, 4, 257, 520, 64, 1, 256),
    ("fast D64 bk16 Sk<KT", 4, 2, 100, 24, 64, 0, 16),
    ("D40 causal Sk%8!=0", 6, 3, 130, 70, 40, 1, 128),
    ("fast D96 causal", 8, 2, 300, 640, 96, 1, 128),
    ("fast D80 bk64", 8, 4, 200, 512, 80, 0, 64),
    ("fast D40 bk32", 6, 3, 130, 72, 40, 1, 32),
    ("general D128 Sk%8!=0", 8, 2, 200, 333, 128, 0, 128),
    ("general D64 Sk%8!=0 causal", 4, 1, 64, 77, 64, 1, 32),
    ("general D7", 4, 2, 40, 50, 7, 0, 64),
    ("decode Sq=1 split", 8, 2, 1, 2048, 128, 0, 128),
    ("decode Sq=2 causal", 4, 1, 2, 1000, 64, 1, 128),
    ("decode Sk%8!=0", 8, 1, 2, 4099, 128, 1, 128),
    ("decode D40", 4, 2, 1, 300, 40, 0, 128),
    ("decode 40 rows", 8, 1, 5, 999, 128, 1, 128),
    ("decode 64 rows Sk%8!=0", 32, 4, 8, 1001, 128, 0, 128),
]


@pytest.mark.parametrize("case", VT_CASES, ids=[c[0] for c in VT_CASES])
def test_v_prepacked(oracle, case):
    name, Hq, Hkv, Sq, Sk, D, causal, bk = case
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 40 + Sk)
    base = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk)
    packed = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk, prepack_v=True)
    vt_host = np.ascontiguousarray(V.reshape(Hkv, Sk, D).transpose(0, 2, 1)).ravel()
    direct = ts.run_attention(Q, K, vt_host, Hq, Hkv, Sq, Sk, D, causal, bk, v_prepacked=1)
    assert np.array_equal(packed.view(np.uint32), direct.view(np.uint32))
    rows = (Hq // Hkv) * Sq
    decode = rows <= 16 or (rows <= 64 and Hkv < 256)  # the host's choice on 256 CUs
    same_kernel = decode or D % 8 != 0 or Sk % 8 == 0
    if same_kernel:
        nd = int(np.count_nonzero(packed.view(np.uint32) != base.view(np.uint32)))
        say("   v_prepacked vs row-major: %d differing outputs" % nd)
        assert nd == 0
    check(oracle, "v_prepacked " + name, Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk, O=packed)


def test_v_prepacked_c3_4k(oracle):
    """The headline shape with a pre-packed V. Row-major V runs the persistent prefill there and
    V^T the per-tile kernel, whose last key tile of a row block keeps the lazy row max: the two
    agree on every row to the oracle tolerance, not bit for bit."""
    B, Hq, Hkv, S, D = 4, 32, 8, 4096, 128
    Q, K, V = ts.synth_normal_qkv(B * Hq, B * Hkv, S, S, D, SEED0 + 3)
    base = ts.run_attention(Q, K, V, B * Hq, B * Hkv, S, S, D, 0, 128)
    packed = ts.run_attention(Q, K, V, B * Hq, B * Hkv, S, S, D, 0, 128, prepack_v=True)
    assert np.isfinite(packed).all() and np.isfinite(base).all()
    assert np.abs(packed - base).max() <= 8e-3 * np.abs(base).max()
    check(oracle, "v_prepacked c3 4k", Q, K, V, B * Hq, B * Hkv, S, S, D, 0, 128, ref_cap=8,
          O=packed)


def test_scratch_canary():
    """Nothing is written past attn_flash_scratch_bytes (the reference's canary guard,
    EXEC_LOG:517-569): 64 KiB of 0x5A after the block must survive split decode, merge and
    prefill calls at every bk."""
    D = 128
    sbytes = ts.attn_flash_scratch_bytes(D, 4096)
    guard = 64 << 10
    cases = [(32, 1, 1, 4096, 0), (8, 2, 4, 3000, 1), (8, 2, 300, 1000, 1)]
    with ts.DeviceBuffer(sbytes + guard) as ds:
        ds.fill_bytes(0x5A)
        for bk in (16, 128, 4096):
            for Hq, Hkv, Sq, Sk, causal in cases:
                Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, 31)
                with ts.DeviceBuffer.from_array(Q) as dq, ts.DeviceBuffer.from_array(K) as dk, \
                        ts.DeviceBuffer.from_array(V) as dv, ts.DeviceBuffer(Hq * Sq * D * 4) as do:
                    ts.attn_flash(dq, dk, dv, do, Hq, Hkv, Sq, Sk, D, causal, bk, ds)
                    ts.synchronize()
        tail = ds.download(np.uint8)[sbytes:]
    assert tail.size == guard and np.all(tail == 0x5A)


def test_timing_struct_and_scratch_reuse(oracle):
    Hq, Hkv, Sq, Sk, D = 8, 2, 1, 2048, 128
    bk_max = 4096
    sbytes = ts.attn_flash_scratch_bytes(D, bk_max)
    tm = ts.AttnTimes()
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, 15)
    rows = np.arange(Sq, dtype=np.int32)
    R = oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, 0, rows)
    with ts.DeviceBuffer(sbytes) as ds, ts.DeviceBuffer.from_array(Q) as dq, \
            ts.DeviceBuffer.from_array(K) as dk, ts.DeviceBuffer.from_array(V) as dv, \
            ts.DeviceBuffer(Hq * Sq * D * 4) as do:
        ds.fill_bytes(0xFF)  # poisoned scratch: the kernels must initialise what they read
        for bk in (64, 512, 4096, 16):  # one scratch sized for the largest bk serves all
            do.fill_bytes(0xFF)
            ts.attn_flash(dq, dk, dv, do, Hq, Hkv, Sq, Sk, D, 0, bk, ds, 0, tm)
            O = do.download(np.float32)
            assert oracle.cmp_rows(R, O, Hq, Sq, D, rows)[0], bk
    assert tm.qxk > 0 and tm.packv == 0 and tm.softmax == 0 and tm.sxv == 0


# ---- tiling variants (the GPU analogue of the reference's VL sweep, README:502-508) ----------------
_WAVES_SCRIPT = r"""
import sys, numpy as np
sys.path.insert(0, %r)
import transfer_station_amd as ts
from oracle import oracle as o
for (Hq, Hkv, Sq, Sk, D, causal, bk) in [(32, 8, 1024, 1024, 128, 0, 128), (16, 8, 2048, 2048, 128, 1, 128),
                                         (24, 6, 1000, 4000, 64, 0, 128), (8, 2, 700, 900, 128, 1, 64)]:
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, 77)
    O = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk)
    rows = o.ref_rowset(Sq, 8)
    R = o.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, rows, nthreads=8)
    ok, mad, maxref, nbad = o.cmp_rows(R, O, Hq, Sq, D, rows)
    print("waves case", Hq, Hkv, Sq, Sk, D, causal, bk, mad / maxref, nbad, flush=True)
    assert ok
print("OK")
"""


@pytest.mark.parametrize("waves,kh", [("4", "1"), ("4", "0"), ("4", "2"), ("8", "1")])
def test_forced_wave_counts(waves, kh):
    """Every workgroup shape of the fast kernel (4 waves x 32 rows, 8 waves x 32 rows, 8 waves
    on key halves of 128 rows), forced through ATTN_PREFILL_WAVES and ATTN_PREFILL_KH in a child
    process, on shapes that normally take another; KH=2 puts key halves under the causal key
    split as well."""
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, ATTN_PREFILL_WAVES=waves, ATTN_PREFILL_KH=kh)
    r = subprocess.run([sys.executable, "-c", _WAVES_SCRIPT % root], env=env, capture_output=True,
                       text=True, timeout=240)
    say(r.stdout[-2000:] + r.stderr[-2000:])
    assert r.returncode == 0 and r.stdout.strip().endswith("OK")


# ---- which kernels each configuration takes (attn_flash_plan) --------------------------------------
# (label, Hq, Hkv, Sq, Sk, D, causal, v_prepacked, [(kernel, required note), ...] in launch order):
# the benchmark configurations c1-c5, the reference's Qwen3 --long case, a chunked-prefill
# serving shape and a long-context split decode, as the host-side choice takes them on a
# 256-CU MI355X.
PLANS = [
    ("c1 MHA 256", 4, 4, 256, 256, 64, 0, 0,
     [("attn_prefill_fast_kernel<64, 128, 4, false, false, false>", "nsplit=1")]),
    ("c2 GQA decode", 2048, 512, 1, 4096, 128, 0, 0,
     [("attn_decode_kernel<128, false, true, false, true>", "nsplit=1")]),
    ("c2 GQA decode, V^T", 2048, 512, 1, 4096, 128, 0, 1,
     [("attn_decode_vt_kernel<128, false, true>", "nsplit=1")]),
    ("c3 1k", 128, 32, 1024, 1024, 128, 0, 0, [("attn_prefill_persist_kernel<128, false, false>", "units=512")]),
    ("c3 2k", 128, 32, 2048, 2048, 128, 0, 0, [("attn_prefill_persist_kernel<128, false, false>", "units=1024")]),
    ("c3 4k", 128, 32, 4096, 4096, 128, 0, 0, [("attn_prefill_persist_kernel<128, false, false>", "units=2048")]),
    ("c3 4k causal", 128, 32, 4096, 4096, 128, 1, 0,
     [("attn_prefill_persist_kernel<128, true, false>", "units=1024")]),
    ("c3 1k causal", 128, 32, 1024, 1024, 128, 1, 0,
     [("attn_prefill_persist_kernel<128, true, false>", "units=256")]),
    ("96 heads at 1536 causal (288 pairs: uneven)", 96, 24, 1536, 1536, 128, 1, 0,
     [("attn_prefill_fast_kernel<128, 64, 4, true, false, false>", "nsplit=1")]),
    ("c3 4k, V^T", 128, 32, 4096, 4096, 128, 0, 1,
     [("attn_prefill_fast_kernel<128, 128, 8, false, true, false>", "nsplit=1")]),
    ("c4 MQA 2k", 128, 8, 2048, 2048, 128, 0, 0, [("attn_prefill_persist_kernel<128, false, false>", "units=1024")]),
    ("c5 ragged D 64", 48, 12, 1000, 4000, 64, 0, 0,
     [("attn_prefill_fast_kernel<64, 128, 12, false, false, true>", "pack=1")]),
    ("c5 ragged D 64, V^T", 48, 12, 1000, 4000, 64, 0, 1,
     [("attn_prefill_fast_kernel<64, 128, 12, false, true, true>", "pack=1")]),
    ("48 MHA heads of 1000 rows at D 64 (288 workgroups of 192 rows: head split)",
     48, 48, 1000, 4000, 64, 0, 0,
     [("attn_prefill_fast_kernel<64, 128, 4, false, false, false>", "hsplit=16"),
      ("attn_merge2_kernel", "")]),
    ("Qwen3 4k causal", 16, 8, 4096, 4096, 128, 1, 0,
     [("attn_prefill_persist_kernel<128, true, true>", "units=256")]),
    ("Qwen3 4k causal, V^T", 16, 8, 4096, 4096, 128, 1, 1,
     [("attn_prefill_fast_kernel<128, 128, 8, true, true, true>", "nsplit=1")]),
    ("chunked 512 over 8192, causal", 32, 8, 512, 8192, 128, 1, 0,
     [("attn_prefill_fast_kernel<128, 128, 8, true, false, true>", "nsplit=2"),
      ("attn_merge2_kernel", "")]),
    ("batch-1 decode 32k", 32, 8, 1, 32768, 128, 0, 0,
     [("attn_decode_kernel<128, false, true, false, false>", "nsplit=64"),
      ("attn_mergew_kernel", "nsplit=64")]),
]


@pytest.mark.parametrize("case", PLANS, ids=[c[0] for c in PLANS])
def test_kernel_plan(case):
    """attn_flash_plan records, without launching, the kernels a call takes; a change in the
    host-side choice shows here as a failure rather than only as a slower bench line. The
    persistent prefill takes one workgroup per CU."""
    if ts.device_info()["cus"] != 256:
        pytest.skip("the kernel choice is pinned for a 256-CU MI355X")
    label, Hq, Hkv, Sq, Sk, D, causal, vt, want = case
    plan = ts.attn_flash_plan(Hq, Hkv, Sq, Sk, D, causal, 128, vt)
    say("plan %s: %s" % (label, plan))
    assert [k for k, _, _, _ in plan] == [k for k, _ in want], label
    for (k, notes, grid, block), (_, need) in zip(plan, want):
        assert need in notes.split() or need == "", (label, k, notes)
        if k.startswith("attn_prefill_persist_kernel"):
            assert grid == "256" and block == 512, (label, grid, block)


_PERSIST_SCRIPT = r"""
import sys, numpy as np
sys.path.insert(0, %r)
import transfer_station_amd as ts
from oracle import oracle as o
out = []
for i, (Hq, Hkv, Sq, Sk, D, sigma, causal) in enumerate(%r):
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, 313 + i, sigma_q=sigma)
    O = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128)
    rows = o.ref_rowset(Sq, 8)
    R = o.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, rows, nthreads=8)
    ok, mad, maxref, nbad = o.cmp_rows(R, O, Hq, Sq, D, rows)
    print("persist case", Hq, Hkv, Sq, Sk, D, sigma, causal, mad / maxref, nbad, flush=True)
    assert ok
    out.append(O)
np.savez(%r, *out)
print("OK")
"""

# Shapes that take the persistent prefill on a 256-CU part (97 <= D <= 128, at least two 256-row
# items per CU, an even number of 128-key tiles per item; causal: Sk >= Sq and an even number of
# query tiles), as (Hq, Hkv, Sq, Sk, D, sigma_q, causal). Non-causal: uneven items per
# workgroup, a ragged last query tile, two key tiles (the first tile followed by the last),
# D = 104, peaked scores (sigma_q = 4: the lazy-sum recompute), MHA with an item count that no
# XCD divides, MQA-like sharing (one kv head for 64 query heads). Causal (pairs of query tiles):
# a ragged last query tile and key tail, keys before the query block with peaked scores,
# D = 104, and GQA 4 at 2k. Key halves (causal, exactly two 128-row tiles per CU, one pair per
# workgroup): Qwen3 4k, GQA 4 at 2k with D = 104, keys before the query block (a whole tile, with
# peaked scores, and 76 keys: pairs of odd and even counts either way round), MQA-like sharing
# (one kv head for 128 query heads). V^T (prepacked) keeps the per-tile kernel.
PERSIST_CASES = [
    (128, 32, 1000, 1000, 128, 1.0, 0),
    (256, 16, 512, 256, 128, 1.0, 0),
    (256, 64, 520, 250, 104, 1.0, 0),
    (192, 48, 700, 900, 128, 4.0, 0),
    (131, 131, 1024, 512, 128, 1.0, 0),
    (128, 2, 1024, 1024, 128, 1.0, 0),
    (128, 32, 1000, 1000, 128, 1.0, 1),
    (128, 32, 1024, 2048, 128, 4.0, 1),
    (128, 32, 1024, 1024, 104, 1.0, 1),
    (64, 16, 2048, 2048, 128, 1.0, 1),
    (16, 8, 4096, 4096, 128, 1.0, 1),
    (32, 8, 2048, 2048, 104, 1.0, 1),
    (64, 16, 1024, 1152, 128, 4.0, 1),
    (64, 8, 1024, 1100, 128, 1.0, 1),
    (128, 1, 512, 512, 128, 1.0, 1),
]


def test_persistent_prefill(tmp_path):
    """The persistent prefill against the oracle on the spread rows, and on every row against
    the per-tile 8-wave kernel that ATTN_PREFILL_PERSIST=0 selects instead (child processes),
    to the same tolerance. They are not bit-identical: the persistent kernel's last key tile
    of an item always takes a fresh row max (its Q registers are reloaded for the next item
    mid-tile, so it cannot recompute), where the per-tile kernel keeps the running max unless
    the row sum would pass its cap."""
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = {}
    for p in ("1", "0"):
        path = str(tmp_path / ("persist%s.npz" % p))
        env = dict(os.environ, ATTN_PREFILL_PERSIST=p)
        r = subprocess.run([sys.executable, "-c", _PERSIST_SCRIPT % (root, PERSIST_CASES, path)],
                           env=env, capture_output=True, text=True, timeout=300)
        say(r.stdout[-2000:] + r.stderr[-2000:])
        assert r.returncode == 0 and r.stdout.strip().endswith("OK")
        with np.load(path) as z:
            res[p] = [z[k] for k in sorted(z.files, key=lambda f: int(f.split("_")[1]))]
    for case, a, b in zip(PERSIST_CASES, res["1"], res["0"]):
        assert np.isfinite(a).all() and np.isfinite(b).all(), case  # NaN poison: all written
        dev, scale = float(np.abs(a - b).max()), float(np.abs(b).max())
        say("   persistent vs per-tile %s: max|diff|/scale = %.2e" % (case, dev / scale))
        assert dev <= 8e-3 * scale, case


_DECODE_NT_SCRIPT = r"""
import sys, numpy as np
sys.path.insert(0, %r)
import transfer_station_amd as ts
out = []
for i, (Hq, Hkv, Sq, Sk, D, causal, vt) in enumerate([(256, 64, 1, 4096, 128, 0, 0),
                                                      (256, 32, 8, 1024, 128, 1, 0),
                                                      (64, 8, 2, 6000, 64, 1, 0),
                                                      (256, 64, 1, 4096, 128, 0, 1),
                                                      (96, 8, 4, 5000, 96, 1, 1)]):
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, 91 + i)
    if vt:
        V = np.ascontiguousarray(V.reshape(Hkv, Sk, D).transpose(0, 2, 1)).ravel()
    out.append(ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, 128, v_prepacked=vt))
np.savez(%r, *out)
print("OK")
"""


def test_decode_nt_policy_is_bit_identical(tmp_path):
    """The decode kernels' load policy (non-temporal or ordinary K/V, forced through
    ATTN_DECODE_NT in child processes) changes caching only: O is bit-identical either way, on
    row-block and single-block grids, row-major V and V^T."""
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = {}
    for nt in ("0", "1"):
        path = str(tmp_path / ("nt%s.npz" % nt))
        env = dict(os.environ, ATTN_DECODE_NT=nt)
        r = subprocess.run([sys.executable, "-c", _DECODE_NT_SCRIPT % (root, path)], env=env,
                           capture_output=True, text=True, timeout=240)
        say(r.stdout[-2000:] + r.stderr[-2000:])
        assert r.returncode == 0 and r.stdout.strip().endswith("OK")
        with np.load(path) as z:
            res[nt] = [z[k] for k in sorted(z.files, key=lambda f: int(f.split("_")[1]))]
    for a, b in zip(res["0"], res["1"]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- seeded random shapes over every kernel and staging path ---------------------------------
def _random_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice([64, 128, 64, 128, 32, 80, 96]))
        Hkv = int(rng.integers(1, 4))
        g = int(rng.choice([1, 2, 4, 8, 16]))
        Sq = int(rng.choice([1, 2, 3, 7])) if rng.random() < 0.35 else int(rng.integers(8, 700))
        Sk = int(rng.integers(1, 1500))
        if rng.random() < 0.5:
            Sk = max(8, Sk - Sk % 8)  # V^T inputs take the fast kernel only when Sk % 8 == 0
        causal = int(rng.random() < 0.5)
        bk = int(rng.choice([16, 32, 64, 128, 256, 512]))
        vt = int(rng.random() < 0.3)
        cases.append((i, g * Hkv, Hkv, Sq, Sk, D, causal, bk, vt))
    return cases


RANDOM_CASES = _random_cases(40, 0x5EED)


@pytest.mark.parametrize("case", RANDOM_CASES, ids=["r%02d" % c[0] for c in RANDOM_CASES])
def test_random_shapes(oracle, case):
    """Seeded random shapes (GQA group 1-16, Sq 1-700, Sk 1-1500 with and without Sk % 8,
    D in {32, 64, 80, 96, 128}, causal or not, bk 16-512, row-major V or V^T) against the
    oracle: decode, prefill fast and general kernels, tails and the causal key split."""
    i, Hq, Hkv, Sq, Sk, D, causal, bk, vt = case
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 1000 + i)
    if vt:
        vt_host = np.ascontiguousarray(V.reshape(Hkv, Sk, D).transpose(0, 2, 1)).ravel()
        O = ts.run_attention(Q, K, vt_host, Hq, Hkv, Sq, Sk, D, causal, bk, v_prepacked=1)
    else:
        O = ts.run_attention(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk)
    check(oracle, "random %d%s" % (i, " V^T" if vt else ""), Q, K, V, Hq, Hkv, Sq, Sk, D, causal,
          bk, ref_cap=8, O=O)


# ---- a kv head past 2 GiB: K and V exceed a buffer's 31-bit range, so the prefill takes the
# general kernel (64-bit element offsets), and decode and the V^T path read past 2 GiB as well --
def _spread_bf16(n, seed):
    """n finite bf16 values: random sign and mantissa, magnitude in [2^-7, 2), so that an offset
    that wrapped at 2^31 bytes would read different values."""
    x = np.random.default_rng(seed).integers(0, 1 << 16, size=n, dtype=np.uint16)
    e = (np.uint16(120) + ((x >> np.uint16(7)) & np.uint16(7))) << np.uint16(7)
    return (x & np.uint16(0x807F)) | e


@pytest.fixture(scope="module")
def kv_over_2gib():
    """One kv head (D = 128) whose K is 2^31 + 18 KiB bytes, made once for the cases below."""
    D = 128
    Sk = (1 << 31) // (2 * D) + 72
    say("generating K and V of %d keys x %d (2 x %.2f GB)" % (Sk, D, Sk * D * 2 / 1e9))
    return Sk, D, _spread_bf16(Sk * D, 11), _spread_bf16(Sk * D, 12)


@pytest.mark.parametrize("Hq,Sq,causal,prepack", [
    (2, 40, 1, False),   # prefill, general kernel, causal
    (2, 1, 0, False),    # split-K decode
    (2, 40, 0, True),    # prefill from V^T packed on the device
], ids=["prefill-causal", "decode", "prefill-vt"])
def test_kv_head_over_2gib(oracle, kv_over_2gib, Hq, Sq, causal, prepack):
    Sk, D, K, V = kv_over_2gib
    Q = _spread_bf16(Hq * Sq * D, 13)
    say("running Hq=%d Sq=%d causal=%d prepack_v=%d" % (Hq, Sq, causal, prepack))
    O = ts.run_attention(Q, K, V, Hq, 1, Sq, Sk, D, causal, 128, prepack_v=prepack)
    check(oracle, "kv head over 2 GiB", Q, K, V, Hq, 1, Sq, Sk, D, causal, 128, ref_cap=2, O=O)


def _random_cases_wide(n, seed):
    """Head dims past 128 (odd ones on the general kernel), short query blocks that pack the
    GQA heads' rows, and many kv heads (the decode / packed-prefill choice)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice([136, 160, 192, 200, 224, 256, 130, 250, 64, 128]))
        if rng.random() < 0.3:
            Hkv, g = int(rng.integers(256, 300)), int(rng.choice([2, 4, 8]))
            Sq = int(rng.integers(1, 17))
            Sk = int(rng.integers(1, 200))
        else:
            Hkv, g = int(rng.integers(1, 4)), int(rng.choice([1, 2, 4, 8, 16]))
            Sq = int(rng.integers(1, 65)) if rng.random() < 0.6 else int(rng.integers(65, 300))
            Sk = int(rng.integers(1, 900))
        causal = int(rng.random() < 0.5)
        bk = int(rng.choice([16, 32, 64, 128, 256]))
        cases.append((i, g * Hkv, Hkv, Sq, Sk, D, causal, bk))
    return cases


WIDE_CASES = _random_cases_wide(24, 0xD256)


@pytest.mark.parametrize("case", WIDE_CASES, ids=["w%02d" % c[0] for c in WIDE_CASES])
def test_random_shapes_wide(oracle, case):
    """Seeded random shapes over head dims 130-256, packed short query blocks and many kv
    heads, against the oracle."""
    i, Hq, Hkv, Sq, Sk, D, causal, bk = case
    Q, K, V = ts.synth_normal_qkv(Hq, Hkv, Sq, Sk, D, SEED0 + 2000 + i)
    check(oracle, "wide random %d" % i, Q, K, V, Hq, Hkv, Sq, Sk, D, causal, bk, ref_cap=4)


@pytest.mark.parametrize("shape", [(128, 32, 1024, 1024, 128, 0), (16, 8, 4096, 4096, 128, 1)],
                         ids=["c3 1k", "Qwen3 4k causal, key halves"])
def test_persistent_phase_stamps(shape):
    """The stamps build of the persistent prefill (transfer_station_amd/phases.py) records, per
    workgroup, times that never run backwards, whose span is the kernel's duration, at the
    product library's speed within 15%."""
    from transfer_station_amd import phases
    s, st = phases.timeline(*shape)
    say("phases %s: %s" % (shape, s))
    assert s["kernel"].startswith("attn_prefill_persist_kernel")
    busy = st[:, 0] > 0
    assert busy.sum() == s["workgroups"] > 0
    used = [0, 1] + [2 + i for i in range(8)] + [st.shape[1] - 1]  # two items per workgroup here
    seq = st[busy][:, used].astype(np.int64)
    assert (np.diff(seq, axis=1) >= 0).all()
    ms = s["kernel_ms_product"]
    assert 0.5 * ms <= s["span_us"] * 1e-3 <= 1.5 * ms
    assert abs(s["kernel_ms_stamps_build"] / ms - 1) <= 0.15
