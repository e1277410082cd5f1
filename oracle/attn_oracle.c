/* attn_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement, in plain C99, of the reference's scalar verification path for the
 * bf16 flash-attention forward (liujiang833/transfer_station, flash.c). It is the
 * checker for the HIP kernels and the "reference CPU path" timed beside them. Only the
 * tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product library never links or calls it.
 *
 * Pinning (what proves each function right, independently of this file):
 *   orc_f32_to_bf16 / orc_bf16_to_f32  exhaustive 2^32 check against an independent
 *                                      nearest-even rounding written with double
 *                                      arithmetic (tests/test_oracle.py, oracle_selftest)
 *   orc_lcg_bf16                       the reference's published maxref 0.98828125 of the
 *                                      "odd + multiblock" case (EXEC_LOG_2026-07-16.md:378-389)
 *   orc_attn_ref / orc_attn_ref_mt     numpy float64 golden fixtures (tests/golden/), plus
 *                                      closed forms: Sk=1 -> O=V[0] exactly, constant V ->
 *                                      O=V, zero rows for fully-masked causal rows, GQA ==
 *                                      MHA with K/V repeated
 *   orc_attn_pairs                     the reference's published useful GFLOP 4.30 / 17.19 /
 *                                      68.74 (flash_long.log:32-34) and a brute-force count
 *   orc_ref_rowset                     spread-row properties (first 0, last Sq-1, sorted)
 *   orc_cmp_rows                       tolerance teeth: x1.01 scaling fails, x1.007 passes,
 *                                      one NaN fails (README:584-585, EXEC_LOG:394-407)
 *   orc_normal_bf16                    moments of the sample, and the product generator
 *                                      must agree with it bit for bit
 * Nothing here is "parity unpinned".
 *
 * Build: oracle/Makefile (gcc -O2, no -ffast-math: the summation order is the point).
 */
#include "attn_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- bf16 <-> fp32 on bits (flash.c:78-92) ----------------------------------------
 * Round to nearest, ties to even, by adding 0x7fff plus the kept lsb. An all-ones
 * exponent (Inf/NaN) is truncated, not rounded, so a NaN payload never carries into
 * the exponent. Widening is a 16-bit left shift. */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7f800000u) == 0x7f800000u)
        return (uint16_t)(u >> 16);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* Vector forms for the Python side. */
void orc_f32_to_bf16_n(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++)
        out[i] = orc_f32_to_bf16(in[i]);
}

/* Self-check of the rounding helper over every fp32 bit pattern, against a second,
 * independent definition: the nearest of the two bf16 neighbours (truncation t and
 * its successor), measured exactly in double, ties broken toward the even mantissa.
 * Returns the number of mismatches (Inf/NaN inputs excluded: they truncate by
 * definition and are checked separately by the tests). */
long orc_bf16_selfcheck(uint32_t lo, uint32_t hi) {
    long bad = 0;
    for (uint64_t v = lo; v <= hi; v++) {
        uint32_t u = (uint32_t)v;
        if ((u & 0x7f800000u) == 0x7f800000u)
            continue;
        float f;
        memcpy(&f, &u, sizeof f);
        uint16_t t = (uint16_t)(u >> 16); /* truncation toward zero in magnitude */
        uint16_t t1 = (uint16_t)(t + 1);  /* next magnitude up (may become Inf: fine) */
        double x = fabs((double)f);
        double a = fabs((double)orc_bf16_to_f32(t)), b = fabs((double)orc_bf16_to_f32(t1));
        if ((t1 & 0x7f80u) == 0x7f80u) /* successor is Inf: it stands for 2^128 here */
            b = ldexp(1.0, 128);
        uint16_t want;
        if (x - a < b - x)
            want = t;
        else if (x - a > b - x)
            want = t1;
        else
            want = (t & 1u) ? t1 : t;
        if (orc_f32_to_bf16(f) != want)
            bad++;
    }
    return bad;
}

/* ---- the reference's LCG data mode (flash.c:867-871, 1030, 1050-1061) ---------------
 * state <- state*1664525 + 1013904223 (mod 2^32); value = ((state>>8)&0xffff)/32768 - 1,
 * a uniform on [-1,1) with 16 bits; each value is rounded to bf16. One case seeds the
 * state with 0x12345678 and draws Q, then K, then V, straight through. */
void orc_lcg_bf16(uint32_t *state, uint16_t *out, size_t n) {
    uint32_t s = *state;
    for (size_t i = 0; i < n; i++) {
        s = s * 1664525u + 1013904223u;
        float v = (float)((s >> 8) & 0xffffu) / 32768.0f - 1.0f;
        out[i] = orc_f32_to_bf16(v);
    }
    *state = s;
}

/* ---- seeded N(0, sigma^2) data mode (the data of the benchmark configurations) ------
 * Element c of a stream (Q at counters [0,nq), K at [nq,nq+nk), V after) takes two
 * counter-based splitmix64 outputs x_j = mix(seed + (2c+j+1)*0x9E3779B97F4A7C15),
 * j = 0,1; U1 = ((x_0>>11)+0.5)*2^-53 in (0,1), U2 = (x_1>>11)*2^-53 in [0,1);
 * n = sqrt(-2 ln U1) * cos(2 pi U2) (Box-Muller, cosine branch), all in double;
 * value = (float)(sigma*n), then bf16 RNE. */
static uint64_t orc_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void orc_normal_bf16(uint16_t *out, size_t n, uint64_t seed, uint64_t counter0, double sigma) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i++) {
        uint64_t c = counter0 + i;
        uint64_t x0 = orc_mix64(seed + (2 * c + 1) * 0x9E3779B97F4A7C15ull);
        uint64_t x1 = orc_mix64(seed + (2 * c + 2) * 0x9E3779B97F4A7C15ull);
        double u1 = ((double)(x0 >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        double u2 = (double)(x1 >> 11) * (1.0 / 9007199254740992.0);
        double v = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = orc_f32_to_bf16((float)(sigma * v));
    }
}

/* ---- fp32 attention oracle (flash.c:262-314) -----------------------------------------
 * Layouts: Q,O [Hq][Sq][D], K,V [Hkv][Sk][D], bf16 as uint16 bits, O fp32. Only the
 * listed rows are computed and written. For each query head h the kv head is
 * h / (Hq/Hkv). Row i attends keys j <= Sk-Sq+i when causal (bottom-right aligned),
 * all keys otherwise. Scores: fp32 dot over d in order, then times 1/sqrtf(D); softmax
 * with expf(s - rowmax), denominator summed in key order; a row with no admissible key
 * yields a zero row (sum==0 -> inv 0). Output: fp32 sum over keys in order of
 * (p*inv) * V. */
static void orc_one_row(const uint16_t *Qh, const uint16_t *Kh, const uint16_t *Vh, float *Orow,
                        int Sq, int Sk, int D, int causal, int i, float scale, float *s) {
    int lim = causal ? (Sk - Sq + i) : (Sk - 1);
    float mx = -INFINITY;
    for (int j = 0; j < Sk; j++) {
        if (j > lim) {
            s[j] = -INFINITY;
            continue;
        }
        float a = 0.0f;
        const uint16_t *q = Qh + (size_t)i * D, *k = Kh + (size_t)j * D;
        for (int d = 0; d < D; d++)
            a += orc_bf16_to_f32(q[d]) * orc_bf16_to_f32(k[d]);
        a *= scale;
        s[j] = a;
        if (a > mx)
            mx = a;
    }
    float sum = 0.0f;
    for (int j = 0; j < Sk; j++) {
        if (s[j] == -INFINITY) {
            s[j] = 0.0f;
        } else {
            s[j] = expf(s[j] - mx);
            sum += s[j];
        }
    }
    float inv = (sum > 0.0f) ? 1.0f / sum : 0.0f;
    for (int j = 0; j < Sk; j++)
        s[j] *= inv;
    for (int d = 0; d < D; d++) {
        float a = 0.0f;
        for (int j = 0; j < Sk; j++)
            a += s[j] * orc_bf16_to_f32(Vh[(size_t)j * D + d]);
        Orow[d] = a;
    }
}

/* Returns 0 on success, -1 on a bad shape or allocation failure. */
int orc_attn_ref(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O, int Hq,
                 int Hkv, int Sq, int Sk, int D, int causal, const int *rows, int nrows) {
    if (Hq < 1 || Hkv < 1 || Hq % Hkv || Sq < 1 || Sk < 1 || D < 1)
        return -1;
    int group = Hq / Hkv;
    float scale = 1.0f / sqrtf((float)D);
    float *s = (float *)malloc(sizeof(float) * (size_t)Sk);
    if (!s)
        return -1;
    for (int h = 0; h < Hq; h++) {
        int kv = h / group;
        const uint16_t *Qh = Q + (size_t)h * Sq * D;
        const uint16_t *Kh = K + (size_t)kv * Sk * D, *Vh = V + (size_t)kv * Sk * D;
        for (int t = 0; t < nrows; t++) {
            int i = rows[t];
            orc_one_row(Qh, Kh, Vh, O + ((size_t)h * Sq + i) * D, Sq, Sk, D, causal, i, scale, s);
        }
    }
    free(s);
    return 0;
}

/* Same arithmetic per row, with the (head, row) pairs spread over nthreads OpenMP
 * threads: identical bits to orc_attn_ref, used for the all-cores CPU baseline. */
int orc_attn_ref_mt(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O, int Hq,
                    int Hkv, int Sq, int Sk, int D, int causal, const int *rows, int nrows,
                    int nthreads) {
    if (Hq < 1 || Hkv < 1 || Hq % Hkv || Sq < 1 || Sk < 1 || D < 1)
        return -1;
    int group = Hq / Hkv;
    float scale = 1.0f / sqrtf((float)D);
    long total = (long)Hq * nrows;
    int failed = 0;
#ifdef _OPENMP
    if (nthreads < 1)
        nthreads = omp_get_max_threads();
#pragma omp parallel num_threads(nthreads) reduction(| : failed)
#endif
    {
        float *s = (float *)malloc(sizeof(float) * (size_t)Sk);
        if (!s) {
            failed = 1;
        } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
            for (long p = 0; p < total; p++) {
                int h = (int)(p / nrows), t = (int)(p % nrows);
                int kv = h / group, i = rows[t];
                orc_one_row(Q + (size_t)h * Sq * D, K + (size_t)kv * Sk * D,
                            V + (size_t)kv * Sk * D, O + ((size_t)h * Sq + i) * D, Sq, Sk, D,
                            causal, i, scale, s);
            }
            free(s);
        }
    }
    (void)nthreads;
    return failed ? -1 : 0;
}

/* ---- useful score pairs (flash.c:874-887); FLOPs = 4*Hq*D*pairs (flash.c:1149) ------- */
double orc_attn_pairs(int Sq, int Sk, int causal) {
    if (!causal)
        return (double)Sq * (double)Sk;
    double n = 0.0;
    for (int i = 0; i < Sq; i++) {
        long cnt = (long)Sk - Sq + i + 1;
        if (cnt > Sk)
            cnt = Sk;
        if (cnt < 0)
            cnt = 0;
        n += (double)cnt;
    }
    return n;
}

/* ---- spread row sample (flash.c:900-913) ---------------------------------------------
 * ref_cap <= 0 or >= Sq: every row. ref_cap == 1: only row Sq-1. Otherwise ref_cap rows
 * t*(Sq-1)/(ref_cap-1) (64-bit product, truncating division), first 0, last Sq-1. */
int orc_ref_rowset(int Sq, int ref_cap, int *rows) {
    if (ref_cap <= 0 || ref_cap >= Sq) {
        for (int i = 0; i < Sq; i++)
            rows[i] = i;
        return Sq;
    }
    if (ref_cap == 1) {
        rows[0] = Sq - 1;
        return 1;
    }
    for (int t = 0; t < ref_cap; t++)
        rows[t] = (int)(((int64_t)t * (Sq - 1)) / (ref_cap - 1));
    return ref_cap;
}

/* ---- tolerance compare (flash.c:935-980) ----------------------------------------------
 * Over the listed rows of every head: non-finite elements (in either array) are counted
 * in nbad and skipped; mad = max |k - r| and maxref = max |r| over the finite rest.
 * Pass iff nbad == 0 and mad <= tol * maxref (the reference's tol is 8e-3). */
#define ORC_TOL 8e-3f
float orc_tol(void) { return ORC_TOL; }

int orc_cmp_rows_tol(const float *Oref, const float *Odut, int Hq, int Sq, int D, const int *rows,
                     int nrows, float tol, float *mad_o, float *maxref_o, long *nbad_o) {
    float mad = 0.0f, maxref = 0.0f;
    long nbad = 0;
    for (int h = 0; h < Hq; h++)
        for (int t = 0; t < nrows; t++)
            for (int d = 0; d < D; d++) {
                size_t idx = ((size_t)h * Sq + rows[t]) * D + d;
                float r = Oref[idx], k = Odut[idx];
                if (!isfinite(k) || !isfinite(r)) {
                    nbad++;
                    continue;
                }
                float ad = fabsf(k - r);
                if (ad > mad)
                    mad = ad;
                if (fabsf(r) > maxref)
                    maxref = fabsf(r);
            }
    *mad_o = mad;
    *maxref_o = maxref;
    *nbad_o = nbad;
    return (nbad == 0) && (mad <= tol * maxref);
}

int orc_cmp_rows(const float *Oref, const float *Odut, int Hq, int Sq, int D, const int *rows,
                 int nrows, float *mad_o, float *maxref_o, long *nbad_o) {
    return orc_cmp_rows_tol(Oref, Odut, Hq, Sq, D, rows, nrows, ORC_TOL, mad_o, maxref_o, nbad_o);
}
