"""Generate the golden fixtures in this directory (run from the repo root):

    python tests/golden/make_golden.py

Each fixture holds an attention output computed in float64 with numpy -- matrix
products, a masked max, exp and a normalised sum -- an implementation independent of
the C oracle's scalar loops, following the reference's semantics (flash.c:262-314):
kv = h // (Hq//Hkv), scale = float32(1/sqrtf(D)), bottom-right causal mask j <= Sk-Sq+i,
a row with no admissible key is a zero row. The inputs are the reference's LCG data
(flash.c:867-871, 1030, 1050-1061; regenerated here with exact integer arithmetic, so the
fixture also pins the generator through a SHA-256 of the bytes) or, for the N(0,1)
cases, bf16 arrays stored in the fixture itself.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def lcg_bf16(state, n):
    """Reference LCG, vectorised per step is not possible (it is sequential): plain loop."""
    out = np.empty(n, np.uint16)
    s = state
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        v = np.float32(((s >> 8) & 0xFFFF)) / np.float32(32768.0) - np.float32(1.0)
        u = int(np.array(v, np.float32).view(np.uint32))
        if (u & 0x7F800000) == 0x7F800000:
            out[i] = u >> 16
        else:
            out[i] = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF) >> 16
    return out, s


def lcg_qkv(Hq, Hkv, Sq, Sk, D, seed=0x12345678):
    Q, s = lcg_bf16(seed, Hq * Sq * D)
    K, s = lcg_bf16(s, Hkv * Sk * D)
    V, s = lcg_bf16(s, Hkv * Sk * D)
    return Q, K, V


def bf16_to_f64(h):
    return (h.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def attn_f64(Q, K, V, Hq, Hkv, Sq, Sk, D, causal):
    q = bf16_to_f64(Q).reshape(Hq, Sq, D)
    k = bf16_to_f64(K).reshape(Hkv, Sk, D)
    v = bf16_to_f64(V).reshape(Hkv, Sk, D)
    g = Hq // Hkv
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    i = np.arange(Sq)[:, None]
    j = np.arange(Sk)[None, :]
    allowed = (j <= (Sk - Sq + i)) if causal else np.ones((Sq, Sk), bool)
    O = np.zeros((Hq, Sq, D))
    for h in range(Hq):
        kv = h // g
        s = (q[h] @ k[kv].T) * scale
        s = np.where(allowed, s, -np.inf)
        mx = s.max(axis=1, keepdims=True)
        mx = np.where(np.isfinite(mx), mx, 0.0)
        p = np.where(allowed, np.exp(s - mx), 0.0)
        tot = p.sum(axis=1, keepdims=True)
        w = np.divide(p, tot, out=np.zeros_like(p), where=tot > 0)
        O[h] = w @ v[kv]
    return O.reshape(-1)


# The reference's short suite, the union of the shipped and documented versions
# (flash.c:1287-1299; README:524-532): name, Hq, Hkv, Sq, Sk, D, causal.
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

# Small N(0,1)/ragged/causal cases whose inputs are stored with the fixture.
# name, Hq, Hkv, Sq, Sk, D, causal, sigma_q
STORED = [
    ("c1 MHA 256", 4, 4, 256, 256, 64, 0, 1.0),
    ("ragged causal Sk<Sq", 4, 2, 77, 45, 64, 1, 1.0),
    ("ragged full peaked", 6, 2, 45, 300, 64, 0, 4.0),
    ("decode gqa causal Sq=2", 8, 2, 2, 333, 128, 1, 1.0),
]


def normal_bf16(rng, n, sigma):
    x = (rng.standard_normal(n) * sigma).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def main():
    manifest = []
    for name, Hq, Hkv, Sq, Sk, D, causal in SUITE:
        Q, K, V = lcg_qkv(Hq, Hkv, Sq, Sk, D)
        sha = hashlib.sha256(Q.tobytes() + K.tobytes() + V.tobytes()).hexdigest()
        O = attn_f64(Q, K, V, Hq, Hkv, Sq, Sk, D, causal)
        fn = "suite_%s.npz" % "".join(ch if ch.isalnum() else "_" for ch in name)
        np.savez_compressed(os.path.join(HERE, fn), O=O.astype(np.float32))
        manifest.append(dict(file=fn, name=name, data="lcg", seed=0x12345678, Hq=Hq, Hkv=Hkv,
                             Sq=Sq, Sk=Sk, D=D, causal=causal, sha256_qkv=sha))
    rng = np.random.default_rng(20260716)
    for name, Hq, Hkv, Sq, Sk, D, causal, sq in STORED:
        Q = normal_bf16(rng, Hq * Sq * D, sq)
        K = normal_bf16(rng, Hkv * Sk * D, 1.0)
        V = normal_bf16(rng, Hkv * Sk * D, 1.0)
        O = attn_f64(Q, K, V, Hq, Hkv, Sq, Sk, D, causal)
        fn = "stored_%s.npz" % "".join(ch if ch.isalnum() else "_" for ch in name)
        np.savez_compressed(os.path.join(HERE, fn), Q=Q, K=K, V=V, O=O.astype(np.float32))
        manifest.append(dict(file=fn, name=name, data="stored", Hq=Hq, Hkv=Hkv, Sq=Sq, Sk=Sk,
                             D=D, causal=causal))
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print("wrote %d fixtures" % len(manifest), file=sys.stderr)


if __name__ == "__main__":
    main()
