/* flash_cli.c -- TEST HARNESS: the reference's command-line benchmark on one MI355X.
 *
 * Mirrors the reference's `flash` program (liujiang833/transfer_station flash.c:1177-1321,
 * per-case driver run_case flash.c:1030-1175): same flags, same default suite, same
 * verdict line, same exit codes (0 all pass, 1 a case failed, 2 bad arguments). It drives
 * libattn_flash.so through its C ABI exactly as a C caller of the reference would, and checks
 * every case against the CPU oracle (oracle/attn_oracle.c, the reference's fp32 attn_ref
 * restated), which is why it lives under tests/ and is never part of the library.
 *
 * Differences from the reference harness, each deliberate:
 *   - Buffers are device memory. The cold-input pool holds ncopies copies at distinct
 *     addresses, sized so their total input is >= 2x the cache to overflow (flash.c:982-991);
 *     copy 0 holds the case's LCG data, the others are device-side duplicates of it (what
 *     makes a call cold is the address, not the values), so building the pool costs no host
 *     generation. The pool label reads "hbm" instead of "ddr".
 *   - --llc-mb 0 autodetects the GPU's last-level caches: the L2 the runtime reports plus the
 *     MI355X's 256 MiB Infinity Cache (not reported by the runtime).
 *   - Timing: calls are launched back to back in batches bracketed by HIP events; s/it is
 *     the mean device time per call. The GPU kernel is one fused launch, so the per-phase
 *     split is reported the way attn_times documents it: all of it in qk.
 *   - O is poisoned with NaN before the checked call, so an unwritten row fails.
 *   - --no-softmax is refused (exit 2): a kernel variant that skips work exists only for
 *     profiling experiments, never in the library.
 *   - The default suite is the union of the shipped and the documented suites: the 7
 *     prefill shapes plus the two Sq=1 decode shapes (README.md:524-532).
 *   - Added: --sweep-bk (one shape over every legal bk with one scratch sized for the largest,
 *     README.md:193-216,445-478) and --check-pick-bk (attn_flash_pick_bk's documented
 *     answers and an exact model check, README.md:359-436).
 */
#define _POSIX_C_SOURCE 200809L
#include "attn_devutil.h"
#include "attn_flash.h"
#include "attn_oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static int g_warmup = 3;
static int g_iters = 0;
static double g_bench_secs = 0.5;
static size_t g_llc_bytes = (size_t)512 * 1024 * 1024;
#define BENCH_MIN_REPS 3
#define BENCH_DDR_MULT 2u
#define BENCH_MAX_COPIES 8192
#define POOL_ALIGN 256u
#define INFINITY_CACHE_BYTES ((size_t)256 * 1024 * 1024)

static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

static void hip_or_die(int err, const char *what) {
    if (err != 0) {
        printf("HIP error %d in %s\n", err, what);
        exit(1);
    }
}

static size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

static size_t detect_llc_bytes(void) {
    int l2 = 0;
    if (attn_dev_info(NULL, 0, NULL, 0, NULL, NULL, &l2) != 0 || l2 < 0)
        l2 = 0;
    return (size_t)l2 + INFINITY_CACHE_BYTES;
}

/* Device pool of ncopies input sets: Q, K, V (and V^T when pre-packing) and O per copy. */
struct pool {
    int ncopies;
    size_t q_b, kv_b, o_b, stride;
    char *base;
};

static char *pool_at(const struct pool *p, int c, int which) {
    /* which: 0 Q, 1 K, 2 V, 3 Vp, 4 O */
    size_t off = (size_t)c * p->stride;
    size_t q = round_up(p->q_b, POOL_ALIGN), kv = round_up(p->kv_b, POOL_ALIGN);
    switch (which) {
    case 0: return p->base + off;
    case 1: return p->base + off + q;
    case 2: return p->base + off + q + kv;
    case 3: return p->base + off + q + 2 * kv;
    default: return p->base + off + q + 3 * kv;
    }
}

/* Times `fn(arg, i)` on the device: warmup untimed calls, then batches bracketed by HIP events
 * until --iters calls, or >= BENCH_MIN_REPS calls and >= --bench-secs of wall clock. Returns
 * the mean device seconds per call; *reps_o receives the call count. */
typedef void (*call_fn)(void *arg, int i);

static double time_device(call_fn fn, void *arg, int *reps_o) {
    void *e0 = NULL, *e1 = NULL;
    hip_or_die(attn_dev_event_create(&e0), "event create");
    hip_or_die(attn_dev_event_create(&e1), "event create");
    for (int w = 0; w < g_warmup; w++)
        fn(arg, w);
    hip_or_die(attn_dev_synchronize(), "synchronize");
    int reps = 0, batch = 1;
    double dev_s = 0.0, t0 = now_s();
    for (;;) {
        int n = batch;
        if (g_iters > 0 && reps + n > g_iters)
            n = g_iters - reps;
        hip_or_die(attn_dev_event_record(e0), "event record");
        for (int i = 0; i < n; i++)
            fn(arg, reps + i);
        hip_or_die(attn_dev_event_record(e1), "event record");
        float ms = 0.f;
        hip_or_die(attn_dev_event_elapsed_ms(e0, e1, &ms), "event elapsed");
        dev_s += 1e-3 * (double)ms;
        reps += n;
        if (g_iters > 0 ? (reps >= g_iters)
                        : (reps >= BENCH_MIN_REPS && now_s() - t0 >= g_bench_secs))
            break;
        if (batch < 256)
            batch *= 2;
    }
    attn_dev_event_destroy(e0);
    attn_dev_event_destroy(e1);
    *reps_o = reps;
    return dev_s / reps;
}

struct case_ctx {
    const struct pool *p;
    int Hq, Hkv, Sq, Sk, D, causal, bk, prepack_v;
    void *scratch;
};

static void call_attn(void *arg, int i) {
    const struct case_ctx *c = (const struct case_ctx *)arg;
    int k = i % c->p->ncopies;
    attn_flash((const uint16_t *)pool_at(c->p, k, 0), (const uint16_t *)pool_at(c->p, k, 1),
               (const uint16_t *)pool_at(c->p, k, c->prepack_v ? 3 : 2),
               (float *)pool_at(c->p, k, 4), c->Hq, c->Hkv, c->Sq, c->Sk, c->D, c->causal,
               c->bk, c->scratch, c->prepack_v, NULL);
}

static void call_pack(void *arg, int i) {
    const struct case_ctx *c = (const struct case_ctx *)arg;
    int k = i % c->p->ncopies;
    pack_v_full((const uint16_t *)pool_at(c->p, k, 2), (uint16_t *)pool_at(c->p, k, 3), c->Hkv,
                c->Sk, c->D);
}

/* Builds the case's data and device pool. Returns 0, or -1 on allocation failure. */
static int make_case(struct pool *p, uint16_t **Qh, uint16_t **Kh, uint16_t **Vh, int Hq, int Hkv,
                     int Sq, int Sk, int D) {
    size_t nq = (size_t)Hq * Sq * D, nk = (size_t)Hkv * Sk * D;
    *Qh = malloc(nq * 2);
    *Kh = malloc(nk * 2);
    *Vh = malloc(nk * 2);
    if (!*Qh || !*Kh || !*Vh)
        return -1;
    uint32_t rng = 0x12345678u; /* flash.c:1032: every case restarts the generator */
    attn_synth_lcg_bf16(&rng, *Qh, nq);
    attn_synth_lcg_bf16(&rng, *Kh, nk);
    attn_synth_lcg_bf16(&rng, *Vh, nk);

    size_t in_bytes = (nq + 2 * nk) * 2;
    size_t target = (size_t)BENCH_DDR_MULT * g_llc_bytes;
    long nc = (long)((target + in_bytes - 1) / in_bytes);
    if (nc < 1)
        nc = 1;
    if (nc > BENCH_MAX_COPIES)
        nc = BENCH_MAX_COPIES;
    p->ncopies = (int)nc;
    p->q_b = nq * 2;
    p->kv_b = nk * 2;
    p->o_b = nq * 4;
    p->stride = round_up(p->q_b, POOL_ALIGN) + 3 * round_up(p->kv_b, POOL_ALIGN) +
                round_up(p->o_b, POOL_ALIGN);
    void *base = NULL;
    if (attn_dev_malloc(&base, p->stride * (size_t)p->ncopies) != 0)
        return -1;
    p->base = (char *)base;
    hip_or_die(attn_dev_memcpy_htod(pool_at(p, 0, 0), *Qh, p->q_b), "upload Q");
    hip_or_die(attn_dev_memcpy_htod(pool_at(p, 0, 1), *Kh, p->kv_b), "upload K");
    hip_or_die(attn_dev_memcpy_htod(pool_at(p, 0, 2), *Vh, p->kv_b), "upload V");
    for (int c = 1; c < p->ncopies; c++) {
        hip_or_die(attn_dev_memcpy_dtod(pool_at(p, c, 0), pool_at(p, 0, 0), p->q_b), "pool Q");
        hip_or_die(attn_dev_memcpy_dtod(pool_at(p, c, 1), pool_at(p, 0, 1), p->kv_b), "pool K");
        hip_or_die(attn_dev_memcpy_dtod(pool_at(p, c, 2), pool_at(p, 0, 2), p->kv_b), "pool V");
    }
    return 0;
}

static void free_case(struct pool *p, uint16_t *Qh, uint16_t *Kh, uint16_t *Vh) {
    if (p->base)
        attn_dev_free(p->base);
    p->base = NULL;
    free(Qh);
    free(Kh);
    free(Vh);
}

/* Correctness of one attn_flash call on copy 0 against the oracle over the spread rows.
 * Returns the pass flag; fills err/scale and the non-finite count. */
static int check_case(const struct case_ctx *c, const uint16_t *Qh, const uint16_t *Kh,
                      const uint16_t *Vh, int ref_cap, float *err_o, long *nbad_o, int *nrows_o) {
    size_t no = (size_t)c->Hq * c->Sq * c->D;
    float *Oref = calloc(no, 4), *O = malloc(no * 4);
    int *rows = malloc(sizeof(int) * (size_t)c->Sq);
    if (!Oref || !O || !rows) {
        printf("host allocation failed\n");
        exit(1);
    }
    int nrows = orc_ref_rowset(c->Sq, ref_cap, rows);
    orc_attn_ref_mt(Qh, Kh, Vh, Oref, c->Hq, c->Hkv, c->Sq, c->Sk, c->D, c->causal, rows, nrows,
                    0);
    hip_or_die(attn_dev_memset(pool_at(c->p, 0, 4), 0xFF, c->p->o_b), "poison O");
    call_attn((void *)c, 0);
    hip_or_die(attn_dev_synchronize(), "synchronize");
    hip_or_die(attn_dev_memcpy_dtoh(O, pool_at(c->p, 0, 4), no * 4), "download O");
    float mad = 0.f, maxref = 0.f;
    long nbad = 0;
    int ok = orc_cmp_rows(Oref, O, c->Hq, c->Sq, c->D, rows, nrows, &mad, &maxref, &nbad);
    *err_o = maxref > 0 ? mad / maxref : 0.f;
    *nbad_o = nbad;
    *nrows_o = nrows;
    free(Oref);
    free(O);
    free(rows);
    return ok;
}

static int run_case(const char *name, int Hq, int Hkv, int Sq, int Sk, int D, int causal,
                    int ref_cap, int bk, int prepack_v) {
    struct pool p = {0};
    uint16_t *Qh = NULL, *Kh = NULL, *Vh = NULL;
    if (make_case(&p, &Qh, &Kh, &Vh, Hq, Hkv, Sq, Sk, D) != 0) {
        printf("%-17s allocation failed\n", name);
        free_case(&p, Qh, Kh, Vh);
        return 0;
    }
    void *scratch = NULL;
    hip_or_die(attn_dev_malloc(&scratch, attn_flash_scratch_bytes(D, bk)), "scratch");
    struct case_ctx c = {&p, Hq, Hkv, Sq, Sk, D, causal, bk, prepack_v, scratch};

    double tpack = 0.0;
    if (prepack_v) {
        for (int k = 0; k < p.ncopies; k++)
            call_pack(&c, k);
        int preps = 0;
        tpack = time_device(call_pack, &c, &preps);
    }
    float err = 0.f;
    long nbad = 0;
    int nrows = 0;
    int ok = check_case(&c, Qh, Kh, Vh, ref_cap, &err, &nbad, &nrows);

    int reps = 0;
    double tdot = time_device(call_attn, &c, &reps);

    char reflbl[48] = "";
    if (nrows < Sq)
        snprintf(reflbl, sizeof reflbl, " [ref:%d rows spread 0..%d]", nrows, Sq - 1);
    char verdict[40];
    if (nbad)
        snprintf(verdict, sizeof verdict, "*** FAIL (%ld non-finite) ***", nbad);
    else
        snprintf(verdict, sizeof verdict, "%s", ok ? "PASS" : "*** FAIL ***");
    char packlbl[40] = "";
    if (prepack_v)
        snprintf(packlbl, sizeof packlbl, " sep-packv=%.6fs", tpack);
    double gflop = 4.0 * (double)Hq * D * orc_attn_pairs(Sq, Sk, causal) / 1e9;
    double pool_mib = (double)p.ncopies * (double)(p.q_b + 2 * p.kv_b) / (1024.0 * 1024.0);
    printf("%-17s H=%2d/%-2d(g%d) Sq=%-4d Sk=%-4d D=%3d bk=%-4d %s | err/scale=%.1e | %7.2f GFLOP "
           "%11.6fs/it x%-5d %9.2f GFLOP/s | pv/qk/sm/sv=%.6f/%.6f/%.6f/%.6f | hbm %dx=%.0fMiB%s%s "
           "-> %s\n",
           name, Hq, Hkv, Hq / Hkv, Sq, Sk, D, bk, causal ? "causal" : "full  ", err, gflop, tdot,
           reps, gflop / tdot, 0.0, tdot, 0.0, 0.0, p.ncopies, pool_mib, packlbl, reflbl,
           verdict);
    fflush(stdout);
    attn_dev_free(scratch);
    free_case(&p, Qh, Kh, Vh);
    return ok;
}

/* One shape over every legal bk, with ONE scratch sized for the largest bk and poisoned
 * first (README.md:193-216): each bk checked against the oracle and timed. Prints the
 * fastest bk next to attn_flash_pick_bk's analytic answer for the device's L2. */
static int sweep_bk(int Hq, int Hkv, int Sq, int Sk, int D, int causal, int ref_cap,
                    int prepack_v) {
    struct pool p = {0};
    uint16_t *Qh = NULL, *Kh = NULL, *Vh = NULL;
    if (make_case(&p, &Qh, &Kh, &Vh, Hq, Hkv, Sq, Sk, D) != 0) {
        printf("sweep: allocation failed\n");
        free_case(&p, Qh, Kh, Vh);
        return 0;
    }
    const size_t sbytes = attn_flash_scratch_bytes(D, ATTN_BK_MAX);
    void *scratch = NULL;
    hip_or_die(attn_dev_malloc(&scratch, sbytes), "scratch");
    hip_or_die(attn_dev_memset(scratch, 0xFF, sbytes), "poison scratch");
    double gflop = 4.0 * (double)Hq * D * orc_attn_pairs(Sq, Sk, causal) / 1e9;
    printf("--- bk sweep: Hq=%d Hkv=%d Sq=%d Sk=%d D=%d %s, one scratch of %zu B (sized for "
           "bk=%d) ---\n",
           Hq, Hkv, Sq, Sk, D, causal ? "causal" : "full", sbytes, ATTN_BK_MAX);
    printf("%6s %10s %12s %12s %10s  %s\n", "bk", "scratch B", "err/scale", "s/it", "GFLOP/s",
           "verdict");
    int all = 1, best_bk = 0;
    double best_t = 0.0;
    struct case_ctx c = {&p, Hq, Hkv, Sq, Sk, D, causal, 0, prepack_v, scratch};
    if (prepack_v)
        for (int k = 0; k < p.ncopies; k++)
            call_pack(&c, k);
    for (int bk = ATTN_BK_MIN; bk <= ATTN_BK_MAX; bk *= 2) {
        c.bk = bk;
        float err = 0.f;
        long nbad = 0;
        int nrows = 0;
        int ok = check_case(&c, Qh, Kh, Vh, ref_cap, &err, &nbad, &nrows);
        int reps = 0;
        double t = time_device(call_attn, &c, &reps);
        printf("%6d %10zu %12.1e %12.6f %10.1f  %s\n", bk, attn_flash_scratch_bytes(D, bk), err, t,
               gflop / t, ok ? "PASS" : "*** FAIL ***");
        fflush(stdout);
        all &= ok;
        if (best_bk == 0 || t < best_t) {
            best_bk = bk;
            best_t = t;
        }
    }
    int l2 = 0;
    attn_dev_info(NULL, 0, NULL, 0, NULL, NULL, &l2);
    printf("fastest bk=%d (%.6f s/it); attn_flash_pick_bk(D=%d, L2=%d B) = %d (analytic model)\n",
           best_bk, best_t, D, l2, attn_flash_pick_bk(D, (size_t)(l2 > 0 ? l2 : 0)));
    attn_dev_free(scratch);
    free_case(&p, Qh, Kh, Vh);
    return all;
}

/* attn_flash_pick_bk self-test (README.md:359-436): the documented answers, the worked
 * example's bound, the edge cases, and an exact 128-bit restatement of the model over a grid
 * of (D, l2). Host only. */
static int pick_model_exact(long long D, unsigned long long l2) {
    const unsigned __int128 BQm = 64;
    unsigned __int128 d = D < 1 ? 1 : (unsigned __int128)D;
    unsigned __int128 per_bk = 6 * (d + BQm), fixed = 6 * BQm * d + 4 * d + 12 * BQm;
    int best = ATTN_BK_MIN;
    for (int bk = ATTN_BK_MIN; bk <= ATTN_BK_MAX; bk *= 2) {
        if (2 * (per_bk * (unsigned __int128)bk + fixed) > (unsigned __int128)l2)
            break;
        best = bk;
    }
    return best;
}

static int check_pick_bk(void) {
    int fails = 0;
#define EXPECT(cond, ...)                                                                          \
    do {                                                                                           \
        if (!(cond)) {                                                                             \
            fails++;                                                                               \
            printf("  FAIL: " __VA_ARGS__);                                                        \
            printf("\n");                                                                          \
        }                                                                                          \
    } while (0)
    const int want_l2[4] = {256, 512, 1024, 2048};
    for (int i = 0; i < 4; i++) {
        int got = attn_flash_pick_bk(128, ((size_t)1 << 20) << i);
        EXPECT(got == want_l2[i], "pick_bk(128, %d MiB) = %d, documented %d", 1 << i, got,
               want_l2[i]);
    }
    const int dd[4] = {64, 128, 256, 512}, want_d[4] = {512, 256, 128, 64};
    for (int i = 0; i < 4; i++) {
        int got = attn_flash_pick_bk(dd[i], (size_t)1 << 20);
        EXPECT(got == want_d[i], "pick_bk(%d, 1 MiB) = %d, documented %d", dd[i], got, want_d[i]);
    }
    /* worked example: 2*(1152*bk + 50432) <= 2^20 holds at 256 and fails at 512 */
    EXPECT(2.0 * (1152.0 * 256 + 50432.0) <= 1048576.0, "bound at bk=256");
    EXPECT(2.0 * (1152.0 * 512 + 50432.0) > 1048576.0, "bound at bk=512");
    EXPECT(attn_flash_pick_bk(128, 0) == ATTN_BK_MIN, "l2=0 must give the floor");
    EXPECT(attn_flash_pick_bk(128, SIZE_MAX) == ATTN_BK_MAX, "l2=SIZE_MAX must give the cap");
    EXPECT(attn_flash_pick_bk(0, 1 << 20) == attn_flash_pick_bk(1, 1 << 20), "D<1 clamps to 1");
    EXPECT(attn_flash_pick_bk(-5, 1 << 20) == attn_flash_pick_bk(1, 1 << 20), "D<1 clamps to 1");
    const long long Ds[] = {1, 2, 40, 64, 100, 128, 256, 1024, 65536, 1LL << 24, 2147483647LL};
    const unsigned long long L2s[] = {0ull, 1ull, 4096ull, 1ull << 20, 3ull << 20, 1ull << 22,
                                      256ull << 20, 1ull << 40, 2000000000000ull,
                                      18446744073709551615ull};
    int checked = 0;
    for (size_t i = 0; i < sizeof Ds / sizeof Ds[0]; i++)
        for (size_t j = 0; j < sizeof L2s / sizeof L2s[0]; j++) {
            int got = attn_flash_pick_bk((int)Ds[i], (size_t)L2s[j]);
            int want = pick_model_exact(Ds[i], L2s[j]);
            EXPECT(got == want, "pick_bk(%lld, %llu) = %d, exact model %d", Ds[i], L2s[j], got,
                   want);
            EXPECT(got >= ATTN_BK_MIN && got <= ATTN_BK_MAX && (got & (got - 1)) == 0,
                   "pick_bk(%lld, %llu) = %d is not a power of two in range", Ds[i], L2s[j], got);
            checked++;
        }
#undef EXPECT
    printf("PICK_BK %s, %d checks failed (%d exact-model combinations)\n", fails ? "FAILED" : "OK",
           fails, checked);
    return fails == 0;
}

static void usage(const char *argv0) {
    printf("usage: %s [--long] [--shape Hq,Hkv,Sq,Sk,D[,causal[,ref_cap]]] [--bk N]\n", argv0);
    printf("       %*s [--prepack-v] [--iters N] [--warmup N] [--bench-secs S] [--llc-mb N]\n",
           (int)strlen(argv0), "");
    printf("       %*s [--sweep-bk] [--check-pick-bk]\n", (int)strlen(argv0), "");
    printf("  (no args)       run the default suite (7 prefill + 2 decode shapes)\n");
    printf("  --shape ...     run ONE case of the given shape instead of the suite, then exit;\n");
    printf("                  causal defaults to 1, ref_cap to 8. Qwen3 1k prefill, on its own:\n");
    printf("                  --shape 16,8,1024,1024,128,1\n");
    printf("  --bk N          key-block size N (power of two in [%d,%d]); default %d. RUNTIME.\n",
           ATTN_BK_MIN, ATTN_BK_MAX, ATTN_BK_DEFAULT);
    printf("  --long          also run the Qwen3 1k/2k/4k prefill sweep\n");
    printf("  --prepack-v     transpose V with the SEPARATE pack_v_full operator before attention\n");
    printf("                  (attn_flash runs v_prepacked=1)\n");
    printf("  --iters N       time exactly N runs per case (default: adaptive to --bench-secs)\n");
    printf("  --warmup N      untimed warmup runs before timing (default 3)\n");
    printf("  --bench-secs S  adaptive: keep timing a case until S seconds elapse (default 0.5)\n");
    printf("  --llc-mb N      cache (MiB) the input pool must overflow so calls stream from HBM\n");
    printf("                  (default 512; 0 = the device's L2 + 256 MiB Infinity Cache)\n");
    printf("  --sweep-bk      one shape (--shape, default 4,2,128,1024,128,0) over every legal\n");
    printf("                  bk with one scratch sized for bk=%d; prints the fastest bk\n",
           ATTN_BK_MAX);
    printf("  --check-pick-bk self-test attn_flash_pick_bk's cache model (host only)\n");
    printf("  --no-softmax    not available in this build (exits 2)\n");
}

int main(int argc, char **argv) {
    int longrun = 0, prepack_v = 0, bk = ATTN_BK_DEFAULT, sweep = 0, pickcheck = 0;
    int shq = 0, shkv = 0, ssq = 0, ssk = 0, sd = 0, scausal = 1, srefcap = 8, have_shape = 0;
    setvbuf(stdout, NULL, _IOLBF, 0);
    for (int i = 1; i < argc; i++) {
        if (!strcmp(argv[i], "--long"))
            longrun = 1;
        else if (!strcmp(argv[i], "--prepack-v"))
            prepack_v = 1;
        else if (!strcmp(argv[i], "--sweep-bk"))
            sweep = 1;
        else if (!strcmp(argv[i], "--check-pick-bk"))
            pickcheck = 1;
        else if (!strcmp(argv[i], "--no-softmax")) {
            printf("--no-softmax: not available. This build keeps no work-skipping kernel "
                   "variant; per-phase attribution comes from rocprofv3 counters instead.\n");
            return 2;
        } else if (!strcmp(argv[i], "--bk") && i + 1 < argc)
            bk = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--shape") && i + 1 < argc) {
            scausal = 1;
            srefcap = 8;
            int n = sscanf(argv[++i], "%d,%d,%d,%d,%d,%d,%d", &shq, &shkv, &ssq, &ssk, &sd,
                           &scausal, &srefcap);
            if (n < 5) {
                printf("bad --shape: need Hq,Hkv,Sq,Sk,D[,causal[,ref_cap]]\n");
                return 2;
            }
            have_shape = 1;
        } else if (!strcmp(argv[i], "--iters") && i + 1 < argc)
            g_iters = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--warmup") && i + 1 < argc)
            g_warmup = atoi(argv[++i]);
        else if (!strcmp(argv[i], "--bench-secs") && i + 1 < argc)
            g_bench_secs = atof(argv[++i]);
        else if (!strcmp(argv[i], "--llc-mb") && i + 1 < argc) {
            size_t mb = strtoul(argv[++i], NULL, 10);
            g_llc_bytes = mb ? mb * 1024u * 1024u : 0; /* 0: autodetect once a device is up */
        } else if (!strcmp(argv[i], "--help") || !strcmp(argv[i], "-h")) {
            usage(argv[0]);
            return 0;
        } else {
            printf("unknown argument: %s\n", argv[i]);
            usage(argv[0]);
            return 2;
        }
    }
    if (bk < ATTN_BK_MIN || bk > ATTN_BK_MAX || (bk & (bk - 1)) != 0) {
        printf("bad --bk %d: must be a power of two in [%d, %d]\n", bk, ATTN_BK_MIN, ATTN_BK_MAX);
        return 2;
    }
    if (have_shape && (shq < 1 || shkv < 1 || shq % shkv != 0 || ssq < 1 || ssk < 1 || sd < 1)) {
        printf("bad --shape %d,%d,%d,%d,%d: need Hq>=1, Hkv>=1, Hq%%Hkv==0, Sq>=1, Sk>=1, D>=1\n",
               shq, shkv, ssq, ssk, sd);
        return 2;
    }
    if (have_shape && sd > ATTN_D_MAX) {
        printf("bad --shape: D=%d exceeds ATTN_D_MAX=%d of this build\n", sd, ATTN_D_MAX);
        return 2;
    }
    if (g_warmup < 0)
        g_warmup = 0;
    if (g_iters < 0)
        g_iters = 0;
    if (g_bench_secs <= 0)
        g_bench_secs = 0.5;
    if (pickcheck)
        return check_pick_bk() ? 0 : 1;

    int ndev = 0;
    if (attn_dev_count(&ndev) != 0 || ndev < 1) {
        printf("no HIP device visible: this harness runs on an MI355X\n");
        return 1;
    }
    if (g_llc_bytes == 0)
        g_llc_bytes = detect_llc_bytes();
    char name[128] = "", arch[64] = "";
    int cus = 0, clk = 0, l2 = 0;
    attn_dev_info(name, sizeof name, arch, sizeof arch, &cus, &clk, &l2);
    printf("=== FLASH bf16 attention (online softmax, gfx950 MFMA vs fp32 ref) ===\n");
    printf("device: %s (%s), %d CUs, %d MHz, L2 %d KiB\n", name, arch, cus, clk / 1000, l2 / 1024);
    printf("bk=%d (RUNTIME, --bk N to change; scratch %zu B at D=128); V-pack: %s\n", bk,
           attn_flash_scratch_bytes(128, bk),
           prepack_v ? "SEPARATE operator (v_prepacked=1)" : "inside kernel (LDS transposed reads)");
    printf("per-phase times pv/qk/sm/sv = packv / qxk / softmax / sxv, seconds (one fused kernel: "
           "all of it in qk)\n");
    {
        char tdesc[64];
        if (g_iters > 0)
            snprintf(tdesc, sizeof tdesc, "%d timed runs/case", g_iters);
        else
            snprintf(tdesc, sizeof tdesc, "adaptive >=%.2gs/case (min %d)", g_bench_secs,
                     BENCH_MIN_REPS);
        printf("timing: %d warmup + %s, mean device time per call (HIP events); HBM-cold input "
               "pool >= %ux LLC=%.1f MiB (per line: /it = mean seconds, xN = runs, hbm Cx=MiB = "
               "pool)\n",
               g_warmup, tdesc, BENCH_DDR_MULT, (double)g_llc_bytes / (1024.0 * 1024.0));
    }
    if (sweep) {
        int ok = have_shape ? sweep_bk(shq, shkv, ssq, ssk, sd, scausal, srefcap, prepack_v)
                            : sweep_bk(4, 2, 128, 1024, 128, 0, 0, prepack_v);
        printf("=== %s ===\n", ok ? "ALL PASS" : "SOME FAILED");
        return ok ? 0 : 1;
    }
    if (have_shape) {
        int ok = run_case("custom shape", shq, shkv, ssq, ssk, sd, scausal, srefcap, bk, prepack_v);
        printf("=== %s ===\n", ok ? "ALL PASS" : "SOME FAILED");
        return ok ? 0 : 1;
    }
    int all = 1;
    all &= run_case("MHA prefill", 4, 4, 8, 8, 64, 0, 0, bk, prepack_v);
    all &= run_case("MHA prefil.causal", 4, 4, 8, 8, 64, 1, 0, bk, prepack_v);
    all &= run_case("GQA prefill", 8, 2, 8, 8, 64, 0, 0, bk, prepack_v);
    all &= run_case("GQA prefil.causal", 8, 2, 8, 8, 64, 1, 0, bk, prepack_v);
    all &= run_case("MHA decode(Sq=1)", 4, 4, 1, 16, 64, 0, 0, bk, prepack_v);
    all &= run_case("GQA decode(Sq=1)", 8, 2, 1, 16, 64, 0, 0, bk, prepack_v);
    all &= run_case("MQA prefill", 8, 1, 8, 8, 64, 0, 0, bk, prepack_v);
    all &= run_case("odd + multiblock", 6, 3, 130, 70, 40, 1, 0, bk, prepack_v);
    all &= run_case("GQA big head_dim", 8, 2, 4, 12, 128, 0, 0, bk, prepack_v);
    if (longrun) {
        printf("--- Qwen3 prefill sweep: Hq=16 Hkv=8 (GQA group=2) D=128 causal ---\n");
        printf("  GFLOP = causal-correct USEFUL flops = 4*Hq*D*#{(i,j): j<=i}\n");
        printf("  [ref:N rows spread 0..Sq-1]: the fp32 ref checks N rows spread over the whole\n");
        printf("  sequence, including row Sq-1, which attends every key block.\n");
        all &= run_case("qwen3 1k", 16, 8, 1024, 1024, 128, 1, 8, bk, prepack_v);
        all &= run_case("qwen3 2k", 16, 8, 2048, 2048, 128, 1, 8, bk, prepack_v);
        all &= run_case("qwen3 4k", 16, 8, 4096, 4096, 128, 1, 8, bk, prepack_v);
    } else
        printf("(default = 9 short shapes; --shape Hq,Hkv,Sq,Sk,D[,causal]: one custom case,\n"
               " e.g. --shape 16,8,1024,1024,128,1 for qwen3 1k; --long: Qwen3 1k/2k/4k sweep;\n"
               " --bk/--prepack-v/--iters/--warmup/--bench-secs/--llc-mb: tune the benchmark)\n");
    printf("=== %s ===\n", all ? "ALL PASS" : "SOME FAILED");
    return all ? 0 : 1;
}
