/* flash_cli.c -- TEST HARNESS: command-line benchmark and self-check of libattn_flash.so.
 *
 * Interface kept from the reference's `flash` program (liujiang833/transfer_station,
 * flash.c:1177-1321 as a specification only): the option names, the default suite's shapes,
 * the per-case verdict line (flash.c:1151-1156) and the exit status (0 every case passed,
 * 1 a case failed, 2 the command line was rejected). Scripts that drive the reference's
 * `flash` therefore drive this program unchanged. The program itself is organised around
 * three tables: the option table (parser and --help are generated from it), the suite table,
 * and one `bench` record per case (pool, scratch, check, timing).
 *
 * Every case is checked against the CPU oracle (oracle/attn_oracle.c), which is why this
 * program lives under tests/ and is never part of the library.
 *
 * How this harness differs from the reference's, on purpose:
 *   - Inputs live in device memory. A pool of copies at distinct addresses, together at
 *     least twice the last-level cache, makes every timed call read cold inputs
 *     (flash.c:982-991). Copy 0 holds the LCG data (with --normal, seeded N(0,1) data); the
 *     rest are device-side duplicates, since what makes a call cold is its addresses, not its
 *     values. The pool is labelled "hbm".
 *   - --llc-mb 0 sizes the pool from the device: its L2 plus the MI355X's 256 MiB Infinity
 *     Cache (which the runtime does not report).
 *   - Times are device times from HIP events around batches of back-to-back calls. One fused
 *     kernel has no per-phase split, so the line reports all of it as qk (attn_times's rule).
 *   - O is filled with NaN before the checked call, so a row the kernel never writes fails.
 *   - --no-softmax is rejected (exit 2). A kernel variant that skips work on purpose is kept
 *     out of committed code; per-phase cost comes from rocprofv3 counters instead.
 *   - The default suite adds the two Sq = 1 decode shapes documented in README.md:524-532 to
 *     the seven shipped prefill shapes.
 *   - Extra modes: --sweep-bk (one shape at every legal bk, one scratch sized for the largest,
 *     README.md:193-216,445-478) and --check-pick-bk (attn_flash_pick_bk's documented answers
 *     plus an exact wide-integer model, README.md:359-436).
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

#define EXIT_ALL_PASS 0
#define EXIT_CASE_FAILED 1
#define EXIT_BAD_USAGE 2

#define MIN_TIMED_CALLS 3
#define POOL_CACHE_MULTIPLE 2u /* pool input bytes >= this many times the cache */
#define POOL_MAX_COPIES 8192
#define POOL_ALIGN 256u
#define MI355X_INFINITY_CACHE ((size_t)256 << 20)
#define MAX_BATCH 256

/* ---- configuration, filled by the option table ---------------------------------------------- */
struct config {
    int suite_long, prepack_v, sweep, pick_selftest, help, no_softmax;
    int bk, iters, warmup, llc_mib;
    long normal_seed; /* -1: the reference's LCG data */
    double min_secs;
    const char *shape_text;
};

static struct config cfg = {
    .bk = ATTN_BK_DEFAULT, .iters = 0, .warmup = 3, .llc_mib = 512, .normal_seed = -1,
    .min_secs = 0.5,
};

enum opt_kind { OPT_SWITCH, OPT_INT, OPT_LONG, OPT_REAL, OPT_TEXT };

struct opt {
    const char *name;
    enum opt_kind kind;
    void *target;
    const char *metavar; /* shown in --help after the name; NULL for switches */
    const char *help;    /* lines separated by '\n' */
};

static const struct opt options[] = {
    {"--shape", OPT_TEXT, &cfg.shape_text, "Hq,Hkv,Sq,Sk,D[,causal[,ref_cap]]",
     "one case of this shape instead of the suite (causal 1 and ref_cap 8 when left out;\n"
     "ref_cap 0 checks every row). Qwen3 1k: --shape 16,8,1024,1024,128,1"},
    {"--bk", OPT_INT, &cfg.bk, "N",
     "key-block size passed to attn_flash: a power of two, 16 to 4096 (default 128).\n"
     "It sizes the scratch; the GPU's key tile does not depend on it, so O is the same"},
    {"--long", OPT_SWITCH, &cfg.suite_long, NULL,
     "after the suite, the causal Qwen3 prefill at 1k, 2k and 4k tokens"},
    {"--prepack-v", OPT_SWITCH, &cfg.prepack_v, NULL,
     "make V^T once per pool copy with pack_v_full (timed on its own) and call attn_flash\n"
     "with v_prepacked = 1"},
    {"--iters", OPT_INT, &cfg.iters, "N", "time exactly N calls per case (0: run by --bench-secs)"},
    {"--warmup", OPT_INT, &cfg.warmup, "N", "untimed calls before the timed ones (default 3)"},
    {"--bench-secs", OPT_REAL, &cfg.min_secs, "S",
     "without --iters: keep timing until S seconds and at least 3 calls (default 0.5)"},
    {"--normal", OPT_LONG, &cfg.normal_seed, "SEED",
     "instead of the reference's LCG data, seeded N(0,1) bf16 Q, K, V drawn from one counter\n"
     "stream in that order (the benchmark's generator; bench.py's config 3 data: SEED 305419899)"},
    {"--llc-mb", OPT_INT, &cfg.llc_mib, "N",
     "cache size in MiB that the input pool must exceed twice over (default 512;\n"
     "0: the device's L2 plus its 256 MiB Infinity Cache)"},
    {"--sweep-bk", OPT_SWITCH, &cfg.sweep, NULL,
     "time and check one shape (--shape, else 4,2,128,1024,128,0) at every legal bk with a\n"
     "single scratch sized for bk = 4096"},
    {"--check-pick-bk", OPT_SWITCH, &cfg.pick_selftest, NULL,
     "host-only self-test of attn_flash_pick_bk against its documented answers"},
    {"--no-softmax", OPT_SWITCH, &cfg.no_softmax, NULL,
     "rejected here (exit 2): no work-skipping kernel variant is built"},
    {"--help", OPT_SWITCH, &cfg.help, NULL, "print this text"},
};
#define NOPTIONS ((int)(sizeof options / sizeof options[0]))

static void print_help(const char *prog) {
    printf("%s: bf16 flash-attention forward on the GPU, checked against the fp32 CPU oracle\n",
           prog);
    printf("Without options it runs the 9-shape suite and prints one verdict line per case.\n\n");
    for (int i = 0; i < NOPTIONS; i++) {
        const struct opt *o = &options[i];
        char head[64];
        snprintf(head, sizeof head, "%s%s%s", o->name, o->metavar ? " " : "",
                 o->metavar ? o->metavar : "");
        const char *line = o->help;
        int first = 1;
        while (*line) {
            const char *nl = strchr(line, '\n');
            int len = nl ? (int)(nl - line) : (int)strlen(line);
            if (first && strlen(head) <= 20)
                printf("  %-20s %.*s\n", head, len, line);
            else {
                if (first)
                    printf("  %s\n", head);
                printf("  %-20s %.*s\n", "", len, line);
            }
            first = 0;
            line += len + (nl ? 1 : 0);
        }
    }
    printf("\nExit status: 0 all cases passed, 1 a case failed, 2 bad command line.\n");
}

static const struct opt *find_option(const char *name) {
    for (int i = 0; i < NOPTIONS; i++)
        if (strcmp(options[i].name, name) == 0)
            return &options[i];
    if (strcmp(name, "-h") == 0)
        return find_option("--help");
    return NULL;
}

/* Parses a whole decimal number (no trailing text). */
static int whole_int(const char *s, long *out) {
    char *end = NULL;
    long v = strtol(s, &end, 10);
    if (end == s || *end != '\0')
        return 0;
    *out = v;
    return 1;
}

/* Returns 1 when argv was understood, else prints why and returns 0. */
static int parse_args(int argc, char **argv) {
    for (int i = 1; i < argc; i++) {
        const struct opt *o = find_option(argv[i]);
        if (!o) {
            printf("flash_cli: unrecognised option '%s' (--help lists them)\n", argv[i]);
            return 0;
        }
        if (o->kind == OPT_SWITCH) {
            *(int *)o->target = 1;
            continue;
        }
        if (i + 1 >= argc) {
            printf("flash_cli: option %s needs a value (%s)\n", o->name, o->metavar);
            return 0;
        }
        const char *val = argv[++i];
        if (o->kind == OPT_TEXT) {
            *(const char **)o->target = val;
        } else if (o->kind == OPT_INT) {
            long v;
            if (!whole_int(val, &v) || v < -2147483647L || v > 2147483647L) {
                printf("flash_cli: option %s wants an integer, got '%s'\n", o->name, val);
                return 0;
            }
            *(int *)o->target = (int)v;
        } else if (o->kind == OPT_LONG) {
            long v;
            if (!whole_int(val, &v) || v < 0) {
                printf("flash_cli: option %s wants a non-negative integer, got '%s'\n", o->name, val);
                return 0;
            }
            *(long *)o->target = v;
        } else {
            char *end = NULL;
            double v = strtod(val, &end);
            if (end == val || *end != '\0') {
                printf("flash_cli: option %s wants a number, got '%s'\n", o->name, val);
                return 0;
            }
            *(double *)o->target = v;
        }
    }
    return 1;
}

/* ---- shapes ------------------------------------------------------------------------------- */
struct shape {
    const char *label;
    int Hq, Hkv, Sq, Sk, D, causal, ref_cap;
};

/* The reference's seven prefill shapes, its two documented decode shapes, and the causal
 * Qwen3 sweep (16 query heads over 8 kv heads, head dim 128). */
static const struct shape suite[] = {
    {"MHA prefill", 4, 4, 8, 8, 64, 0, 0},
    {"MHA prefil.causal", 4, 4, 8, 8, 64, 1, 0},
    {"GQA prefill", 8, 2, 8, 8, 64, 0, 0},
    {"GQA prefil.causal", 8, 2, 8, 8, 64, 1, 0},
    {"MHA decode(Sq=1)", 4, 4, 1, 16, 64, 0, 0},
    {"GQA decode(Sq=1)", 8, 2, 1, 16, 64, 0, 0},
    {"MQA prefill", 8, 1, 8, 8, 64, 0, 0},
    {"odd + multiblock", 6, 3, 130, 70, 40, 1, 0},
    {"GQA big head_dim", 8, 2, 4, 12, 128, 0, 0},
};
static const struct shape qwen3_sweep[] = {
    {"qwen3 1k", 16, 8, 1024, 1024, 128, 1, 8},
    {"qwen3 2k", 16, 8, 2048, 2048, 128, 1, 8},
    {"qwen3 4k", 16, 8, 4096, 4096, 128, 1, 8},
};
#define COUNT(a) ((int)(sizeof(a) / sizeof((a)[0])))

/* --shape text -> shape; 1 on success, else prints the reason and returns 0. */
static int parse_shape(const char *text, struct shape *s) {
    long f[7] = {0, 0, 0, 0, 0, 1, 8};
    int n = 0, dangling = 0;
    const char *p = text;
    while (n < 7) {
        char *end = NULL;
        f[n] = strtol(p, &end, 10);
        if (end == p)
            break;
        n++;
        dangling = 0;
        p = end;
        if (*p != ',')
            break;
        p++;
        dangling = 1;
    }
    if (n < 5 || dangling || *p != '\0') {
        printf("flash_cli: --shape wants 5 to 7 comma-separated integers "
               "Hq,Hkv,Sq,Sk,D[,causal[,ref_cap]], got '%s'\n", text);
        return 0;
    }
    for (int i = 0; i < 7; i++)
        if (f[i] < -2147483647L || f[i] > 2147483647L) {
            printf("flash_cli: --shape '%s': a field is out of range\n", text);
            return 0;
        }
    s->label = "custom shape";
    s->Hq = (int)f[0];
    s->Hkv = (int)f[1];
    s->Sq = (int)f[2];
    s->Sk = (int)f[3];
    s->D = (int)f[4];
    s->causal = (int)f[5];
    s->ref_cap = (int)f[6];
    if (s->Hq < 1 || s->Hkv < 1 || s->Sq < 1 || s->Sk < 1 || s->D < 1 || s->Hq % s->Hkv != 0) {
        printf("flash_cli: --shape '%s' rejected: heads, lengths and D must be positive and "
               "Hq a multiple of Hkv\n", text);
        return 0;
    }
    if (s->D > ATTN_D_MAX) {
        printf("flash_cli: --shape '%s' rejected: D=%d is above ATTN_D_MAX=%d\n", text, s->D,
               ATTN_D_MAX);
        return 0;
    }
    if (s->ref_cap < 0) {
        printf("flash_cli: --shape '%s' rejected: ref_cap must be >= 0\n", text);
        return 0;
    }
    return 1;
}

static int bk_is_legal(int bk) {
    return bk >= ATTN_BK_MIN && bk <= ATTN_BK_MAX && (bk & (bk - 1)) == 0;
}

/* ---- device helpers ----------------------------------------------------------------------- */
static void must(int err, const char *what) {
    if (err != 0) {
        printf("flash_cli: HIP error %d during %s\n", err, what);
        exit(EXIT_CASE_FAILED);
    }
}

static double wall_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

static size_t pad(size_t n) { return (n + POOL_ALIGN - 1) / POOL_ALIGN * POOL_ALIGN; }

/* ---- one case: host data, device pool, scratch -------------------------------------------- */
enum slot { SLOT_Q, SLOT_K, SLOT_V, SLOT_VT, SLOT_O, NSLOTS };

struct bench {
    struct shape s;
    int bk;
    uint16_t *hq, *hk, *hv; /* host copies of copy 0 (LCG data) for the oracle */
    size_t nq, nkv;         /* elements */
    size_t bytes[NSLOTS];
    size_t offset[NSLOTS];
    size_t copy_stride;
    int copies;
    char *pool;
    void *scratch;
};

static char *slot_ptr(const struct bench *b, int copy, enum slot s) {
    return b->pool + (size_t)copy * b->copy_stride + b->offset[s];
}

/* Allocates and fills everything a case needs; 0 on success. */
static int bench_open(struct bench *b, const struct shape *s, int bk, size_t cache_bytes,
                      size_t scratch_bytes) {
    memset(b, 0, sizeof *b);
    b->s = *s;
    b->bk = bk;
    b->nq = (size_t)s->Hq * s->Sq * s->D;
    b->nkv = (size_t)s->Hkv * s->Sk * s->D;
    b->hq = malloc(b->nq * 2);
    b->hk = malloc(b->nkv * 2);
    b->hv = malloc(b->nkv * 2);
    if (!b->hq || !b->hk || !b->hv)
        return -1;
    if (cfg.normal_seed >= 0) {
        /* N(0,1) bf16, one counter stream: Q, then K, then V */
        const uint64_t seed = (uint64_t)cfg.normal_seed;
        attn_synth_normal_bf16(b->hq, b->nq, seed, 0, 1.0);
        attn_synth_normal_bf16(b->hk, b->nkv, seed, b->nq, 1.0);
        attn_synth_normal_bf16(b->hv, b->nkv, seed, b->nq + b->nkv, 1.0);
    } else {
        /* The reference's data: its LCG restarted at 0x12345678 for every case (flash.c:1030),
         * drawn Q, then K, then V. */
        uint32_t state = 0x12345678u;
        attn_synth_lcg_bf16(&state, b->hq, b->nq);
        attn_synth_lcg_bf16(&state, b->hk, b->nkv);
        attn_synth_lcg_bf16(&state, b->hv, b->nkv);
    }

    b->bytes[SLOT_Q] = b->nq * 2;
    b->bytes[SLOT_K] = b->bytes[SLOT_V] = b->bytes[SLOT_VT] = b->nkv * 2;
    b->bytes[SLOT_O] = b->nq * 4;
    size_t off = 0;
    for (int i = 0; i < NSLOTS; i++) {
        b->offset[i] = off;
        off += pad(b->bytes[i]);
    }
    b->copy_stride = off;
    const size_t per_call = b->bytes[SLOT_Q] + 2 * b->bytes[SLOT_K];
    const size_t want = POOL_CACHE_MULTIPLE * cache_bytes;
    size_t copies = (want + per_call - 1) / per_call;
    b->copies = (int)(copies < 1 ? 1 : (copies > POOL_MAX_COPIES ? POOL_MAX_COPIES : copies));

    void *p = NULL;
    if (attn_dev_malloc(&p, b->copy_stride * (size_t)b->copies) != 0)
        return -1;
    b->pool = p;
    must(attn_dev_memcpy_htod(slot_ptr(b, 0, SLOT_Q), b->hq, b->bytes[SLOT_Q]), "upload Q");
    must(attn_dev_memcpy_htod(slot_ptr(b, 0, SLOT_K), b->hk, b->bytes[SLOT_K]), "upload K");
    must(attn_dev_memcpy_htod(slot_ptr(b, 0, SLOT_V), b->hv, b->bytes[SLOT_V]), "upload V");
    for (int c = 1; c < b->copies; c++)
        for (int sl = SLOT_Q; sl <= SLOT_V; sl++)
            must(attn_dev_memcpy_dtod(slot_ptr(b, c, sl), slot_ptr(b, 0, sl), b->bytes[sl]),
                 "pool copy");
    if (attn_dev_malloc(&b->scratch, scratch_bytes) != 0)
        return -1;
    return 0;
}

static void bench_close(struct bench *b) {
    if (b->scratch)
        attn_dev_free(b->scratch);
    if (b->pool)
        attn_dev_free(b->pool);
    free(b->hq);
    free(b->hk);
    free(b->hv);
    memset(b, 0, sizeof *b);
}

static void call_attention(const struct bench *b, int i) {
    const int c = i % b->copies;
    const struct shape *s = &b->s;
    attn_flash((const uint16_t *)slot_ptr(b, c, SLOT_Q), (const uint16_t *)slot_ptr(b, c, SLOT_K),
               (const uint16_t *)slot_ptr(b, c, cfg.prepack_v ? SLOT_VT : SLOT_V),
               (float *)slot_ptr(b, c, SLOT_O), s->Hq, s->Hkv, s->Sq, s->Sk, s->D, s->causal,
               b->bk, b->scratch, cfg.prepack_v, NULL);
}

static void call_pack(const struct bench *b, int i) {
    const int c = i % b->copies;
    pack_v_full((const uint16_t *)slot_ptr(b, c, SLOT_V), (uint16_t *)slot_ptr(b, c, SLOT_VT),
                b->s.Hkv, b->s.Sk, b->s.D);
}

/* Mean device seconds per call of `op`: warmup calls, then batches (doubling up to MAX_BATCH)
 * between two HIP events, until --iters calls or, without it, MIN_TIMED_CALLS calls and
 * --bench-secs of wall time. The warmup runs --warmup calls and, when --warmup is above 0, at
 * least WARMUP_MIN_S seconds: after the host-side setup the GPU is idle, and its clock takes
 * about 40 ms of work to settle (bench.py --ramp measures it), which a few calls do not cover. */
#define WARMUP_MIN_S 0.2
struct timing {
    double per_call;
    int calls;
};

static struct timing measure(const struct bench *b, void (*op)(const struct bench *, int)) {
    void *start = NULL, *stop = NULL;
    must(attn_dev_event_create(&start), "event");
    must(attn_dev_event_create(&stop), "event");
    const double w0 = wall_seconds();
    for (int i = 0; i < cfg.warmup || (cfg.warmup > 0 && wall_seconds() - w0 < WARMUP_MIN_S);
         i++) {
        op(b, i);
        if (i % 16 == 15)
            must(attn_dev_synchronize(), "warmup"); /* the wall clock then tracks the GPU */
    }
    must(attn_dev_synchronize(), "warmup");
    struct timing t = {0.0, 0};
    double device_s = 0.0;
    const double t0 = wall_seconds();
    for (int batch = 1;; batch = batch < MAX_BATCH ? 2 * batch : MAX_BATCH) {
        if (cfg.iters > 0 && t.calls + batch > cfg.iters)
            batch = cfg.iters - t.calls;
        must(attn_dev_event_record(start), "event record");
        for (int i = 0; i < batch; i++)
            op(b, t.calls + i);
        must(attn_dev_event_record(stop), "event record");
        float ms = 0.f;
        must(attn_dev_event_elapsed_ms(start, stop, &ms), "event time");
        device_s += (double)ms * 1e-3;
        t.calls += batch;
        const int done = cfg.iters > 0
                             ? t.calls >= cfg.iters
                             : (t.calls >= MIN_TIMED_CALLS && wall_seconds() - t0 >= cfg.min_secs);
        if (done)
            break;
    }
    attn_dev_event_destroy(start);
    attn_dev_event_destroy(stop);
    t.per_call = device_s / t.calls;
    return t;
}

/* Checked call on copy 0 against the oracle over the spread rows (ref_cap, flash.c:900-913). */
struct check {
    int pass, rows;
    long nonfinite;
    float err_scale;
};

static struct check verify(const struct bench *b) {
    const struct shape *s = &b->s;
    struct check r = {0, 0, 0, 0.f};
    float *want = calloc(b->nq, sizeof(float)), *got = malloc(b->nq * sizeof(float));
    int *rows = malloc(sizeof(int) * (size_t)s->Sq);
    if (!want || !got || !rows) {
        printf("flash_cli: host memory exhausted\n");
        exit(EXIT_CASE_FAILED);
    }
    r.rows = orc_ref_rowset(s->Sq, s->ref_cap, rows);
    orc_attn_ref_mt(b->hq, b->hk, b->hv, want, s->Hq, s->Hkv, s->Sq, s->Sk, s->D, s->causal,
                    rows, r.rows, 0);
    must(attn_dev_memset(slot_ptr(b, 0, SLOT_O), 0xFF, b->bytes[SLOT_O]), "poison O");
    call_attention(b, 0);
    must(attn_dev_synchronize(), "checked call");
    must(attn_dev_memcpy_dtoh(got, slot_ptr(b, 0, SLOT_O), b->bytes[SLOT_O]), "download O");
    float mad = 0.f, maxref = 0.f;
    r.pass = orc_cmp_rows(want, got, s->Hq, s->Sq, s->D, rows, r.rows, &mad, &maxref,
                          &r.nonfinite);
    r.err_scale = maxref > 0.f ? mad / maxref : 0.f;
    free(want);
    free(got);
    free(rows);
    return r;
}

static double useful_gflop(const struct shape *s) {
    return 4.0 * (double)s->Hq * (double)s->D * orc_attn_pairs(s->Sq, s->Sk, s->causal) * 1e-9;
}

/* The verdict line: field order and format are the reference's (flash.c:1151-1156), with the
 * pool labelled "hbm" and per-phase times as attn_times reports them (all in qk). */
static void report(const struct bench *b, const struct check *ck, const struct timing *t,
                   double pack_s) {
    const struct shape *s = &b->s;
    char rowsnote[48] = "", packnote[40] = "", verdict[40];
    if (ck->rows < s->Sq)
        snprintf(rowsnote, sizeof rowsnote, " [ref:%d rows spread 0..%d]", ck->rows, s->Sq - 1);
    if (cfg.prepack_v)
        snprintf(packnote, sizeof packnote, " sep-packv=%.6fs", pack_s);
    if (ck->nonfinite)
        snprintf(verdict, sizeof verdict, "*** FAIL (%ld non-finite) ***", ck->nonfinite);
    else
        snprintf(verdict, sizeof verdict, "%s", ck->pass ? "PASS" : "*** FAIL ***");
    const double gf = useful_gflop(s);
    const double pool_mib =
        (double)b->copies * (double)(b->bytes[SLOT_Q] + 2 * b->bytes[SLOT_K]) / 1048576.0;
    printf("%-17s H=%2d/%-2d(g%d) Sq=%-4d Sk=%-4d D=%3d bk=%-4d %s | err/scale=%.1e | %7.2f GFLOP "
           "%11.6fs/it x%-5d %9.2f GFLOP/s | pv/qk/sm/sv=%.6f/%.6f/%.6f/%.6f | hbm %dx=%.0fMiB%s%s "
           "-> %s\n",
           s->label, s->Hq, s->Hkv, s->Hq / s->Hkv, s->Sq, s->Sk, s->D, b->bk,
           s->causal ? "causal" : "full  ", ck->err_scale, gf, t->per_call, t->calls,
           gf / t->per_call, 0.0, t->per_call, 0.0, 0.0, b->copies, pool_mib, packnote, rowsnote,
           verdict);
    fflush(stdout);
}

static size_t g_cache_bytes;

/* Pack every copy's V^T (so each timed call reads its own), then time the pack itself. */
static double prepare_vt(const struct bench *b) {
    if (!cfg.prepack_v)
        return 0.0;
    for (int c = 0; c < b->copies; c++)
        call_pack(b, c);
    return measure(b, call_pack).per_call;
}

static int run_one(const struct shape *s) {
    struct bench b;
    if (bench_open(&b, s, cfg.bk, g_cache_bytes, attn_flash_scratch_bytes(s->D, cfg.bk)) != 0) {
        printf("%-17s could not allocate its buffers\n", s->label);
        bench_close(&b);
        return 0;
    }
    const double pack_s = prepare_vt(&b);
    const struct check ck = verify(&b);
    const struct timing t = measure(&b, call_attention);
    report(&b, &ck, &t, pack_s);
    bench_close(&b);
    return ck.pass;
}

/* ---- --sweep-bk ----------------------------------------------------------------------------- */
/* One scratch sized for the largest bk and poisoned first serves every bk (the size is
 * non-decreasing in bk, README.md:193-216). bk does not select the GPU's key tile, so every
 * row runs the same kernel: the sweep shows that the result and the time do not depend on bk. */
static int sweep_bk(const struct shape *s) {
    struct bench b;
    const size_t big = attn_flash_scratch_bytes(s->D, ATTN_BK_MAX);
    if (bench_open(&b, s, ATTN_BK_MAX, g_cache_bytes, big) != 0) {
        printf("sweep: could not allocate its buffers\n");
        bench_close(&b);
        return 0;
    }
    must(attn_dev_memset(b.scratch, 0xFF, big), "poison scratch");
    printf("--- bk sweep: Hq=%d Hkv=%d Sq=%d Sk=%d D=%d %s; one %zu-byte scratch (bk=%d size) "
           "serves every bk ---\n",
           s->Hq, s->Hkv, s->Sq, s->Sk, s->D, s->causal ? "causal" : "full", big, ATTN_BK_MAX);
    printf("note: the key tile is fixed by D, so every bk runs the same kernel\n");
    printf("%6s %10s %12s %12s %10s  %s\n", "bk", "scratch B", "err/scale", "s/it", "GFLOP/s",
           "verdict");
    prepare_vt(&b);
    const double gf = useful_gflop(s);
    int all = 1;
    double tmin = 0.0, tmax = 0.0;
    for (int bk = ATTN_BK_MIN; bk <= ATTN_BK_MAX; bk <<= 1) {
        b.bk = bk;
        const struct check ck = verify(&b);
        const struct timing t = measure(&b, call_attention);
        printf("%6d %10zu %12.1e %12.6f %10.1f  %s\n", bk, attn_flash_scratch_bytes(s->D, bk),
               ck.err_scale, t.per_call, gf / t.per_call, ck.pass ? "PASS" : "*** FAIL ***");
        fflush(stdout);
        all = all && ck.pass;
        tmin = (bk == ATTN_BK_MIN || t.per_call < tmin) ? t.per_call : tmin;
        tmax = (bk == ATTN_BK_MIN || t.per_call > tmax) ? t.per_call : tmax;
    }
    int l2 = 0;
    attn_dev_info(NULL, 0, NULL, 0, NULL, NULL, &l2);
    printf("spread over bk: %.1f%% (one kernel; run-to-run noise). attn_flash_pick_bk(D=%d, "
           "L2=%d B) = %d from the reference's cache model\n",
           tmin > 0 ? 100.0 * (tmax - tmin) / tmin : 0.0, s->D, l2,
           attn_flash_pick_bk(s->D, (size_t)(l2 > 0 ? l2 : 0)));
    bench_close(&b);
    return all;
}

/* ---- --check-pick-bk (host only) ------------------------------------------------------------ */
/* The cache model restated in 128-bit arithmetic, where nothing can overflow. */
static int pick_exact(long long D, unsigned long long l2) {
    typedef unsigned __int128 u128;
    const u128 rows = 64, d = D < 1 ? 1 : (u128)D;
    int best = ATTN_BK_MIN;
    for (int bk = ATTN_BK_MIN; bk <= ATTN_BK_MAX; bk <<= 1) {
        const u128 ws = 6 * (u128)bk * (d + rows) + 6 * rows * d + 4 * d + 12 * rows;
        if (2 * ws > (u128)l2)
            break;
        best = bk;
    }
    return best;
}

static int pick_failures;
static void expect(int ok, const char *what) {
    if (!ok) {
        pick_failures++;
        printf("  FAIL: %s\n", what);
    }
}

static int pick_selftest(void) {
    char msg[160];
    /* Documented answers: D = 128 over 1/2/4/8 MiB, and four D at 1 MiB. */
    static const struct { int D; size_t l2; int want; } known[] = {
        {128, 1u << 20, 256}, {128, 2u << 20, 512}, {128, 4u << 20, 1024}, {128, 8u << 20, 2048},
        {64, 1u << 20, 512},  {256, 1u << 20, 128}, {512, 1u << 20, 64},
    };
    for (int i = 0; i < COUNT(known); i++) {
        const int got = attn_flash_pick_bk(known[i].D, known[i].l2);
        snprintf(msg, sizeof msg, "pick_bk(%d, %zu) = %d, documented %d", known[i].D, known[i].l2,
                 got, known[i].want);
        expect(got == known[i].want, msg);
    }
    /* The worked example's bound for D = 128 at 1 MiB: 2*(1152*bk + 50432) fits at 256 only. */
    expect(2 * (1152L * 256 + 50432) <= (1L << 20), "worked example holds at bk = 256");
    expect(2 * (1152L * 512 + 50432) > (1L << 20), "worked example fails at bk = 512");
    expect(attn_flash_pick_bk(128, 0) == ATTN_BK_MIN, "an empty cache gives the floor");
    expect(attn_flash_pick_bk(128, SIZE_MAX) == ATTN_BK_MAX, "SIZE_MAX gives the cap");
    expect(attn_flash_pick_bk(0, 1u << 20) == attn_flash_pick_bk(1, 1u << 20), "D = 0 acts as 1");
    expect(attn_flash_pick_bk(-5, 1u << 20) == attn_flash_pick_bk(1, 1u << 20), "D < 0 acts as 1");
    static const long long dims[] = {1, 2, 40, 64, 100, 128, 256, 1024, 65536, 1LL << 24,
                                     2147483647LL};
    static const unsigned long long caches[] = {
        0ull, 1ull, 4096ull, 1ull << 20, 3ull << 20, 1ull << 22, 256ull << 20, 1ull << 40,
        2000000000000ull, 18446744073709551615ull};
    int combos = 0;
    for (int i = 0; i < COUNT(dims); i++)
        for (int j = 0; j < COUNT(caches); j++, combos++) {
            const int got = attn_flash_pick_bk((int)dims[i], (size_t)caches[j]);
            const int want = pick_exact(dims[i], caches[j]);
            snprintf(msg, sizeof msg, "pick_bk(%lld, %llu) = %d, exact model %d", dims[i],
                     caches[j], got, want);
            expect(got == want && bk_is_legal(got), msg);
        }
    printf("PICK_BK %s, %d checks failed (%d exact-model combinations)\n",
           pick_failures ? "FAILED" : "OK", pick_failures, combos);
    return pick_failures == 0;
}

/* ---- main ----------------------------------------------------------------------------------- */
static void print_banner(void) {
    char name[128] = "", arch[64] = "";
    int cus = 0, khz = 0, l2 = 0;
    attn_dev_info(name, sizeof name, arch, sizeof arch, &cus, &khz, &l2);
    printf("=== FLASH bf16 attention (online softmax, gfx950 MFMA vs fp32 ref) ===\n");
    printf("device %s [%s]: %d CUs, %d MHz, L2 %d KiB\n", name, arch, cus, khz / 1000, l2 / 1024);
    printf("bk=%d (a runtime argument; scratch %zu B at D=128). V enters as %s\n", cfg.bk,
           attn_flash_scratch_bytes(128, cfg.bk),
           cfg.prepack_v ? "V^T from pack_v_full (v_prepacked=1)"
                         : "row-major V (transposed on LDS reads)");
    if (cfg.iters > 0)
        printf("timing: %d warmup calls, then %d timed calls per case", cfg.warmup, cfg.iters);
    else
        printf("timing: %d warmup calls, then at least %d calls and %.2g s per case", cfg.warmup,
               MIN_TIMED_CALLS, cfg.min_secs);
    printf("; s/it is mean device time (HIP events). Inputs rotate over a pool >= %ux %.1f MiB, "
           "shown as 'hbm copies x MiB'. pv/qk/sm/sv: one fused kernel, so all time is in qk\n",
           POOL_CACHE_MULTIPLE, (double)g_cache_bytes / 1048576.0);
}

int main(int argc, char **argv) {
    setvbuf(stdout, NULL, _IOLBF, 0);
    if (!parse_args(argc, argv))
        return EXIT_BAD_USAGE;
    if (cfg.help) {
        print_help(argv[0]);
        return EXIT_ALL_PASS;
    }
    if (cfg.no_softmax) {
        printf("flash_cli: --no-softmax is rejected: this build ships no kernel variant that "
               "skips work; measure phases with rocprofv3 counters instead\n");
        return EXIT_BAD_USAGE;
    }
    if (!bk_is_legal(cfg.bk)) {
        printf("flash_cli: --bk %d rejected: bk must be a power of two from %d to %d\n", cfg.bk,
               ATTN_BK_MIN, ATTN_BK_MAX);
        return EXIT_BAD_USAGE;
    }
    struct shape custom;
    if (cfg.shape_text && !parse_shape(cfg.shape_text, &custom))
        return EXIT_BAD_USAGE;
    if (cfg.iters < 0 || cfg.warmup < 0 || cfg.llc_mib < 0) {
        printf("flash_cli: --iters, --warmup and --llc-mb must be >= 0 (got %d, %d, %d)\n",
               cfg.iters, cfg.warmup, cfg.llc_mib);
        return EXIT_BAD_USAGE;
    }
    if (!(cfg.min_secs > 0.0))
        cfg.min_secs = 0.5;
    if (cfg.pick_selftest)
        return pick_selftest() ? EXIT_ALL_PASS : EXIT_CASE_FAILED;

    int ndev = 0;
    if (attn_dev_count(&ndev) != 0 || ndev < 1) {
        printf("flash_cli: no HIP device is visible; run this on the GPU\n");
        return EXIT_CASE_FAILED;
    }
    if (cfg.llc_mib > 0) {
        g_cache_bytes = (size_t)cfg.llc_mib << 20;
    } else {
        int l2 = 0;
        if (attn_dev_info(NULL, 0, NULL, 0, NULL, NULL, &l2) != 0 || l2 < 0)
            l2 = 0;
        g_cache_bytes = (size_t)l2 + MI355X_INFINITY_CACHE;
    }
    print_banner();

    int all = 1;
    if (cfg.sweep) {
        static const struct shape sweep_default = {"sweep", 4, 2, 128, 1024, 128, 0, 0};
        all = sweep_bk(cfg.shape_text ? &custom : &sweep_default);
    } else if (cfg.shape_text) {
        all = run_one(&custom);
    } else {
        for (int i = 0; i < COUNT(suite); i++)
            all = run_one(&suite[i]) && all;
        if (cfg.suite_long) {
            printf("--- causal Qwen3 prefill: 16 query heads on 8 kv heads (g2), D=128; GFLOP "
                   "counts useful (unmasked) pairs only; each case checks 8 rows spread over "
                   "0..Sq-1, the last of which sees every key ---\n");
            for (int i = 0; i < COUNT(qwen3_sweep); i++)
                all = run_one(&qwen3_sweep[i]) && all;
        } else {
            printf("(--long adds the causal Qwen3 1k/2k/4k prefill; --shape runs one case of "
                   "your own; --help lists every option)\n");
        }
    }
    printf("=== %s ===\n", all ? "ALL PASS" : "SOME FAILED");
    return all ? EXIT_ALL_PASS : EXIT_CASE_FAILED;
}
