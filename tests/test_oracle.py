"""CPU tests that pin the oracle (oracle/attn_oracle.c) before anything is checked against it.

Each check is chosen so that a plausible mistake in the oracle -- a dropped term, a wrong
sign, index or mask offset, a transposed operand -- fails it: float64 fixtures built by a
different implementation, the reference's own published numbers, and closed forms."""
import json
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _manifest():
    with open(os.path.join(GOLD, "manifest.json")) as f:
        return json.load(f)


# ---- bf16 rounding (flash.c:78-92) -----------------------------------------------------------
def test_bf16_rne_exhaustive(oracle):
    """All 2^32 fp32 patterns against an independent nearest-even definition (in C, threaded)."""
    chunks = [(i << 28, ((i + 1) << 28) - 1) for i in range(16)]
    with ThreadPoolExecutor(8) as ex:
        bad = sum(ex.map(lambda c: oracle.bf16_selfcheck(*c), chunks))
    assert bad == 0


def test_bf16_specials(oracle):
    f = oracle.lib().orc_f32_to_bf16
    assert f(1.0) == 0x3F80 and f(-2.0) == 0xC000 and f(0.0) == 0
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> even (1.0)
    assert f(np.float32(1.0 + 2.0 ** -8)) == 0x3F80
    assert f(np.float32(1.0 + 3 * 2.0 ** -8)) == 0x3F82
    # Inf stays Inf, NaN is truncated (stays NaN), max finite rounds up to Inf
    assert f(float("inf")) == 0x7F80
    nan = oracle.lib().orc_f32_to_bf16(float("nan"))
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0
    assert f(np.float32(3.4028235e38)) == 0x7F80


# ---- generators --------------------------------------------------------------------------------
def test_lcg_matches_fixture_hashes(oracle):
    import hashlib
    for m in _manifest():
        if m["data"] != "lcg":
            continue
        Q, K, V = oracle.lcg_qkv(m["Hq"], m["Hkv"], m["Sq"], m["Sk"], m["D"], m["seed"])
        sha = hashlib.sha256(Q.tobytes() + K.tobytes() + V.tobytes()).hexdigest()
        assert sha == m["sha256_qkv"], m["name"]


def test_normal_generator_moments(oracle):
    x = oracle.bf16_to_f32(oracle.normal_bf16(1 << 20, 0x12345679, 0, 1.0)).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1.0) < 5e-3
    assert abs((x ** 3).mean()) < 2e-2 and abs((x ** 4).mean() - 3.0) < 3e-2
    y = oracle.bf16_to_f32(oracle.normal_bf16(1 << 18, 7, 0, 4.0)).astype(np.float64)
    assert abs(y.std() - 4.0) < 4e-2
    # disjoint counters give disjoint (independent) draws; equal counters repeat exactly
    a = oracle.normal_bf16(1000, 7, 0, 1.0)
    b = oracle.normal_bf16(1000, 7, 500, 1.0)
    assert np.array_equal(a[500:], b[:500]) and not np.array_equal(a[:500], b[:500])


def test_product_generators_match_oracle(oracle):
    import transfer_station_amd as ts
    for seed, c0, sig in ((0x12345679, 0, 1.0), (0x1234567D, 123457, 4.0)):
        assert np.array_equal(ts.synth_normal_bf16(50000, seed, c0, sig),
                              oracle.normal_bf16(50000, seed, c0, sig))
    for got, want in zip(ts.synth_lcg_qkv(6, 3, 130, 70, 40), oracle.lcg_qkv(6, 3, 130, 70, 40)):
        assert np.array_equal(got, want)


# ---- the attention oracle ------------------------------------------------------------------------
@pytest.mark.parametrize("m", _manifest(), ids=lambda m: m["name"])
def test_oracle_vs_float64_fixture(oracle, m):
    z = np.load(os.path.join(GOLD, m["file"]))
    if m["data"] == "lcg":
        Q, K, V = oracle.lcg_qkv(m["Hq"], m["Hkv"], m["Sq"], m["Sk"], m["D"], m["seed"])
    else:
        Q, K, V = z["Q"], z["K"], z["V"]
    O = oracle.attn_ref(Q, K, V, m["Hq"], m["Hkv"], m["Sq"], m["Sk"], m["D"], m["causal"])
    G = z["O"].astype(np.float32)
    scale = np.abs(G).max()
    assert np.isfinite(O).all()
    assert np.abs(O - G).max() <= 5e-6 * scale, m["name"]


def test_reference_known_answer_odd_multiblock(oracle):
    """EXEC_LOG_2026-07-16.md:378-389: maxref 9.882812e-01 and 360 exactly-zero rows."""
    Q, K, V = oracle.lcg_qkv(6, 3, 130, 70, 40)
    O = oracle.attn_ref(Q, K, V, 6, 3, 130, 70, 40, 1).reshape(6, 130, 40)
    assert float(np.abs(O).max()) == 0.98828125
    assert np.all(O[:, :60, :] == 0.0)  # rows with Sk-Sq+i < 0 attend nothing
    assert np.all(np.abs(O[:, 60:, :]).max(axis=2) > 0)


def test_reference_known_answer_gflop(oracle):
    """flash_long.log:32-34: useful GFLOP 4.30 / 17.19 / 68.74 for qwen3 causal Hq=16 D=128."""
    got = [4 * 16 * 128 * oracle.attn_pairs(s, s, 1) / 1e9 for s in (1024, 2048, 4096)]
    assert [round(g, 2) for g in got] == [4.30, 17.19, 68.74]
    for Sq, Sk in ((1, 1), (5, 3), (3, 5), (130, 70), (7, 7)):
        brute = sum(1 for i in range(Sq) for j in range(Sk) if j <= Sk - Sq + i)
        assert oracle.attn_pairs(Sq, Sk, 1) == brute
        assert oracle.attn_pairs(Sq, Sk, 0) == Sq * Sk


def test_ref_rowset(oracle):
    assert list(oracle.ref_rowset(10, 0)) == list(range(10))
    assert list(oracle.ref_rowset(10, 10)) == list(range(10))
    assert list(oracle.ref_rowset(10, 1)) == [9]
    r = oracle.ref_rowset(4096, 8)
    assert r[0] == 0 and r[-1] == 4095 and len(r) == 8 and np.all(np.diff(r) > 0)
    assert list(oracle.ref_rowset(1000, 3)) == [0, 499, 999]


def test_closed_forms(oracle):
    rng = np.random.default_rng(3)
    bf = lambda a: oracle.f32_to_bf16(a.astype(np.float32))
    # Sk = 1: every row copies V[0] exactly (p = 1, inv = 1)
    Hq, Hkv, Sq, D = 4, 2, 5, 24
    Q = bf(rng.standard_normal(Hq * Sq * D))
    K = bf(rng.standard_normal(Hkv * D))
    V = bf(rng.standard_normal(Hkv * D))
    O = oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, 1, D, 0).reshape(Hq, Sq, D)
    Vf = oracle.bf16_to_f32(V).reshape(Hkv, D)
    for h in range(Hq):
        assert np.array_equal(O[h], np.broadcast_to(Vf[h // 2], (Sq, D)))
    # causal with Sq == Sk: row 0 copies V[0]
    Sk = Sq
    K = bf(rng.standard_normal(Hkv * Sk * D))
    V = bf(rng.standard_normal(Hkv * Sk * D))
    O = oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, 1).reshape(Hq, Sq, D)
    Vf = oracle.bf16_to_f32(V).reshape(Hkv, Sk, D)
    for h in range(Hq):
        assert np.array_equal(O[h, 0], Vf[h // 2, 0])
    # constant V: O == V up to the fp32 rounding of sum(p)*inv
    V = bf(np.full(Hkv * Sk * D, 0.75))
    O = oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, 0)
    assert np.abs(O - 0.75).max() < 1e-6


def test_gqa_equals_mha_with_repeated_kv(oracle):
    rng = np.random.default_rng(5)
    Hq, Hkv, Sq, Sk, D = 8, 2, 9, 21, 32
    bf = lambda n: oracle.f32_to_bf16(rng.standard_normal(n).astype(np.float32))
    Q, K, V = bf(Hq * Sq * D), bf(Hkv * Sk * D), bf(Hkv * Sk * D)
    Kr = np.repeat(K.reshape(Hkv, 1, Sk * D), Hq // Hkv, axis=1).reshape(-1)
    Vr = np.repeat(V.reshape(Hkv, 1, Sk * D), Hq // Hkv, axis=1).reshape(-1)
    for causal in (0, 1):
        a = oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, causal)
        b = oracle.attn_ref(Q, Kr, Vr, Hq, Hq, Sq, Sk, D, causal)
        assert np.array_equal(a, b)


def test_batch_folds_into_heads(oracle):
    rng = np.random.default_rng(6)
    B, Hq, Hkv, Sq, Sk, D = 3, 4, 2, 6, 11, 16
    bf = lambda n: oracle.f32_to_bf16(rng.standard_normal(n).astype(np.float32))
    Q, K, V = bf(B * Hq * Sq * D), bf(B * Hkv * Sk * D), bf(B * Hkv * Sk * D)
    folded = oracle.attn_ref(Q, K, V, B * Hq, B * Hkv, Sq, Sk, D, 1)
    nq, nk = Hq * Sq * D, Hkv * Sk * D
    for b in range(B):
        one = oracle.attn_ref(Q[b * nq:(b + 1) * nq], K[b * nk:(b + 1) * nk],
                              V[b * nk:(b + 1) * nk], Hq, Hkv, Sq, Sk, D, 1)
        assert np.array_equal(folded[b * nq:(b + 1) * nq], one)


def test_multithreaded_oracle_is_bit_identical(oracle):
    Q, K, V = oracle.lcg_qkv(6, 3, 130, 70, 40)
    rows = oracle.ref_rowset(130, 0)
    a = oracle.attn_ref(Q, K, V, 6, 3, 130, 70, 40, 1, rows, nthreads=1)
    b = oracle.attn_ref(Q, K, V, 6, 3, 130, 70, 40, 1, rows, nthreads=4)
    assert np.array_equal(a, b)


# ---- tolerance teeth (flash.c:935-980; README:584-585, 601-621; EXEC_LOG:394-407) ------------
def test_cmp_rows_teeth(oracle):
    Q, K, V = oracle.lcg_qkv(8, 2, 64, 512, 64)
    rows = oracle.ref_rowset(64, 8)
    O = oracle.attn_ref(Q, K, V, 8, 2, 64, 512, 64, 0, rows)
    ok, mad, maxref, nbad = oracle.cmp_rows(O, O, 8, 64, 64, rows)
    assert ok and mad == 0 and nbad == 0
    assert not oracle.cmp_rows(O, O * np.float32(1.01), 8, 64, 64, rows)[0]
    assert oracle.cmp_rows(O, O * np.float32(1.007), 8, 64, 64, rows)[0]
    bad = O.copy()
    bad[rows[0] * 64] = np.nan
    ok, _, _, nbad = oracle.cmp_rows(O, bad, 8, 64, 64, rows)
    assert not ok and nbad == 1
    # a dropped last key block (128 keys) is caught on the spread rows
    Kd = K.reshape(2, 512, 64)[:, :384].reshape(-1).copy()
    Vd = V.reshape(2, 512, 64)[:, :384].reshape(-1).copy()
    Od = oracle.attn_ref(Q, Kd, Vd, 8, 2, 64, 384, 64, 0, rows)
    assert not oracle.cmp_rows(O, Od, 8, 64, 64, rows)[0]


def test_oracle_rejects_bad_shapes(oracle):
    Q = np.zeros(64, np.uint16)
    with pytest.raises(ValueError):
        oracle.attn_ref(Q, Q, Q, 3, 2, 1, 1, 8, 0)


# ---- a second, independent library restatement: torch SDPA in float64 on the CPU -------------
TORCH_CASES = [
    # Hq, Hkv, Sq, Sk, D, causal
    (4, 4, 8, 8, 64, 0),
    (8, 2, 37, 53, 40, 1),   # Sk > Sq: bottom-right causal keeps Sk-Sq extra keys per row
    (6, 3, 130, 70, 40, 1),  # Sk < Sq: the first 60 rows attend nothing
    (8, 1, 5, 200, 128, 0),  # MQA
    (4, 2, 1, 300, 128, 1),  # decode row
]


@pytest.mark.parametrize("case", TORCH_CASES, ids=[str(c) for c in TORCH_CASES])
def test_oracle_vs_torch_sdpa_float64(oracle, case):
    """The oracle against torch.nn.functional.scaled_dot_product_attention (float64, GQA by
    explicit head repetition, bottom-right causal mask built explicitly, fully masked rows
    set to 0 as flash.c:851-860 writes them). Independent of the numpy fixtures."""
    torch = pytest.importorskip("torch")
    Hq, Hkv, Sq, Sk, D, causal = case
    Q, K, V = oracle.normal_qkv(Hq, Hkv, Sq, Sk, D, seed=4242 + Sq)
    R = oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, causal).reshape(Hq, Sq, D).astype(np.float64)
    f = lambda x, H, S: torch.from_numpy(oracle.bf16_to_f32(x).astype(np.float64).reshape(H, S, D))
    q, k, v = f(Q, Hq, Sq), f(K, Hkv, Sk), f(V, Hkv, Sk)
    g = Hq // Hkv
    k = k.repeat_interleave(g, dim=0)
    v = v.repeat_interleave(g, dim=0)
    i = torch.arange(Sq).unsqueeze(1)
    j = torch.arange(Sk).unsqueeze(0)
    allowed = (j <= Sk - Sq + i) if causal else torch.ones(Sq, Sk, dtype=torch.bool)
    bias = torch.zeros(Sq, Sk, dtype=torch.float64).masked_fill(~allowed, float("-inf"))
    s = (q @ k.transpose(1, 2)) * (1.0 / np.sqrt(np.float32(D)).astype(np.float64)) + bias
    empty = ~allowed.any(dim=1)
    s[:, empty, :] = 0.0  # keep softmax finite on rows that attend nothing; zeroed below
    T = torch.softmax(s, dim=-1) @ v
    T[:, empty, :] = 0.0
    T = T.numpy()
    scale = np.abs(T).max()
    err = np.abs(R - T).max() / scale
    assert np.isfinite(R).all() and err < 1e-5, err
    # The same comparison through SDPA itself where no row is empty.
    if not bool(empty.any()):
        sd = torch.nn.functional.scaled_dot_product_attention(
            q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0), attn_mask=allowed,
            scale=float(1.0 / np.sqrt(np.float32(D)))).squeeze(0).numpy()
        assert np.abs(R - sd).max() / np.abs(sd).max() < 1e-5


def test_attn_ref_rejects_short_arrays(oracle):
    """The C oracle indexes raw pointers, so its wrapper refuses arrays smaller than the shape
    they are passed with, and rows outside [0, Sq)."""
    Hq, Hkv, Sq, Sk, D = 4, 2, 5, 7, 8
    Q = np.zeros(Hq * Sq * D, np.uint16)
    K = np.zeros(Hkv * Sk * D, np.uint16)
    V = np.zeros(Hkv * Sk * D, np.uint16)
    oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, 0)
    for args in ((Q[:-1], K, V), (Q, K[:-1], V), (Q, K, V[:-1])):
        with pytest.raises(ValueError):
            oracle.attn_ref(*args, Hq, Hkv, Sq, Sk, D, 0)
    with pytest.raises(ValueError):
        oracle.attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, 0, rows=np.array([0, Sq], np.int32))
