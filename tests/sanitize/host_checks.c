/* host_checks.c -- CPU-only sanitizer driver for the host C code (built by the Makefile
 * here with -fsanitize=address,undefined; run by tests/test_sanitize.py).
 *
 * It links the real host layer (attn_flash.c, attn_synth.c) and the real oracle
 * (attn_oracle.c). The HIP launchers and the few HIP runtime calls the host layer makes are
 * replaced by stand-ins defined below. A stand-in launcher never touches Q/K/V/O (fake
 * addresses); instead it writes every scratch slot the real kernel could write, given the
 * split count and layout the host layer chose, into the caller's scratch, which this driver
 * allocates on the host at exactly attn_flash_scratch_bytes(D, bk). A wrong carve, a split
 * count past the slot capacity or a size that disagrees with the layout is then a heap
 * overflow that AddressSanitizer reports; integer overflow or a bad shift in the size and
 * split arithmetic is reported by UBSan. The oracle is exercised on small shapes, including
 * the edge cases its tests pin (Sk = 1, fully masked causal rows, odd D).
 *
 * Prints "HOST_CHECKS OK" and exits 0 when every check passes.
 */
#define _POSIX_C_SOURCE 200809L
#include "attn_devutil.h"
#include "attn_flash.h"
#include "attn_oracle.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int failures;
#define CHECK(cond, ...)                                                                           \
    do {                                                                                           \
        if (!(cond)) {                                                                             \
            failures++;                                                                            \
            printf("FAIL %s:%d: ", __FILE__, __LINE__);                                            \
            printf(__VA_ARGS__);                                                                   \
            printf("\n");                                                                          \
        }                                                                                          \
    } while (0)

/* ---- stand-ins for the HIP runtime calls attn_flash.c makes ----------------------------- */
static int fake_event_storage[2];
const char *hipGetErrorString(hipError_t e) {
    (void)e;
    return "stand-in";
}
hipError_t hipEventCreate(hipEvent_t *ev) {
    static int n;
    *ev = (hipEvent_t)(void *)&fake_event_storage[n++ & 1];
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t ev, hipStream_t st) {
    (void)ev;
    (void)st;
    return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t ev) {
    (void)ev;
    return hipSuccess;
}
hipError_t hipEventElapsedTime(float *ms, hipEvent_t a, hipEvent_t b) {
    (void)a;
    (void)b;
    *ms = 2.0f;
    return hipSuccess;
}

/* ---- stand-ins for the HIP launchers (attn_kernels.hip) --------------------------------- */
#define SLOTS 65536 /* the partial-slot capacity the scratch layout promises */

struct last_call {
    int decode_calls, merge_calls, prefill_calls, pack_calls;
    int nsplit, kps, nrb;
    long merge_rows;
};
static struct last_call lc;

/* attn_flash_plan: while a plan is recorded the real launchers write kernel lines instead of
 * launching; these stand-ins then touch no partials (the scratch is a stand-in address). */
static char *g_plan;
static size_t g_plan_len, g_plan_pos;
void attn_hip_plan_begin(char *buf, size_t len) {
    g_plan = buf;
    g_plan_len = len;
    g_plan_pos = 0;
    buf[0] = '\0';
}
long attn_hip_plan_end(void) {
    g_plan = NULL;
    return (long)g_plan_pos;
}
static void plan_line(const char *what) {
    const size_t n = strlen(what);
    if (g_plan_pos + n + 2 <= g_plan_len) {
        memcpy(g_plan + g_plan_pos, what, n);
        g_plan_pos += n;
        g_plan[g_plan_pos++] = '\n';
        g_plan[g_plan_pos] = '\0';
    }
}

/* Writes slots [0, n) of the (m, l, acc[D]) partial arrays, as a kernel storing n partials. */
static void touch_partials(float *pm, float *pl, float *pacc, long n, int D) {
    if (g_plan)
        return;
    for (long s = 0; s < n; s++) {
        pm[s] = -1.0f;
        pl[s] = 1.0f;
    }
    memset(pacc, 0x3f, sizeof(float) * (size_t)n * (size_t)D);
}

int attn_hip_launch_prefill(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O,
                            int Hq, int Hkv, int Sq, int Sk, int D, int causal, int vec, int vt,
                            int dp, float c, float *pm, float *pl, float *pacc, long slots,
                            void *stream) {
    (void)Q, (void)K, (void)V, (void)O, (void)Sq, (void)Sk, (void)causal, (void)vec, (void)vt,
        (void)c, (void)stream;
    lc.prefill_calls++;
    if (g_plan)
        plan_line("prefill");
    CHECK(Hq % Hkv == 0 && D <= dp && (dp == 64 || dp == 128 || dp == 256), "prefill args");
    CHECK(slots == SLOTS, "prefill slot capacity %ld", slots);
    /* A causal split may use any of the slots: write all of them. */
    touch_partials(pm, pl, pacc, slots, D);
    return 0;
}

int attn_hip_launch_decode(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O,
                           float *pm, float *pl, float *pacc, int Hq, int Hkv, int Sq, int Sk,
                           int D, int causal, int vec, int vt, int dp, float c, int nsplit,
                           int kps, int nrb, void *stream) {
    (void)Q, (void)K, (void)V, (void)O, (void)causal, (void)vec, (void)vt, (void)c, (void)stream;
    lc.decode_calls++;
    if (g_plan)
        plan_line("decode");
    lc.nsplit = nsplit;
    lc.kps = kps;
    lc.nrb = nrb;
    const long g = Hq / Hkv;
    CHECK(D <= dp, "decode dp");
    CHECK(nsplit >= 1 && kps >= 1, "decode split %d x %d", nsplit, kps);
    CHECK(kps % 128 == 0, "keys per split %d not a multiple of 128", kps);
    CHECK((long)nsplit * kps >= Sk && (long)(nsplit - 1) * kps < Sk,
          "splits %d x %d do not tile Sk = %d exactly", nsplit, kps, Sk);
    CHECK((long)nrb * 16 >= g * Sq && (long)(nrb - 1) * 16 < g * Sq, "row blocks %d for %ld rows",
          nrb, g * Sq);
    if (nsplit > 1) {
        const long partials = (long)Hq * Sq * nsplit;
        CHECK(partials <= SLOTS, "%ld partials exceed %d slots", partials, SLOTS);
        touch_partials(pm, pl, pacc, partials, D);
    }
    return 0;
}

int attn_hip_launch_merge(const float *pm, const float *pl, const float *pacc, float *O, int rows,
                          int D, int nsplit, float c, int Sq, void *stream) {
    (void)O, (void)c, (void)Sq, (void)stream;
    lc.merge_calls++;
    lc.merge_rows = rows;
    CHECK(nsplit == lc.nsplit, "merge nsplit %d, decode nsplit %d", nsplit, lc.nsplit);
    if (g_plan) {
        plan_line("merge");
        return 0;
    }
    /* Read every partial the merge reads. */
    double acc = 0.0;
    const long n = (long)rows * nsplit;
    for (long s = 0; s < n; s++)
        acc += pm[s] + pl[s];
    for (long i = 0; i < n * D; i++)
        acc += pacc[i];
    CHECK(isfinite(acc), "merge read");
    return 0;
}

int attn_hip_launch_pack_v(const uint16_t *V, uint16_t *Vp, int Hkv, int Sk, int D,
                           void *stream) {
    (void)V, (void)Vp, (void)stream;
    lc.pack_calls++;
    CHECK(Hkv >= 1 && Sk >= 1 && D >= 1, "pack args");
    return 0;
}

int attn_hip_device_cus(void) { return 256; }

static void *g_static;
int attn_hip_static_scratch(void **ptr, size_t *bytes) {
    if (!g_static)
        g_static = aligned_alloc(256, ATTN_NOALLOC_SCRATCH_BYTES);
    *ptr = g_static;
    *bytes = ATTN_NOALLOC_SCRATCH_BYTES;
    return 0;
}

/* ---- checks of the host layer ----------------------------------------------------------- */
#define FAKE(p) ((const uint16_t *)(uintptr_t)(p))

static void check_scratch_sizes(void) {
    for (int D = 1; D <= ATTN_D_MAX; D++) {
        size_t prev = 0;
        for (int bk = ATTN_BK_MIN; bk <= ATTN_BK_MAX; bk <<= 1) {
            const size_t n = attn_flash_scratch_bytes(D, bk);
            CHECK(n % ATTN_SCRATCH_ALIGN == 0, "size %zu not aligned", n);
            CHECK(n >= prev, "size not monotone in bk");
            CHECK(n >= (size_t)SLOTS * (size_t)(D + 2) * 4, "size below the slot capacity");
            prev = n;
        }
    }
    CHECK(attn_flash_scratch_bytes(ATTN_NOALLOC_D_MAX, 128) == ATTN_NOALLOC_SCRATCH_BYTES,
          "static scratch constant");
}

static void check_pick_bk(void) {
    static const int dims[] = {-2147483647 - 1, -5, 0, 1, 40, 128, 4096, 1 << 20, 2147483647};
    static const size_t caches[] = {0, 1, 4096, 1u << 20, (size_t)1 << 40, SIZE_MAX};
    for (size_t i = 0; i < sizeof dims / sizeof dims[0]; i++)
        for (size_t j = 0; j < sizeof caches / sizeof caches[0]; j++) {
            const int bk = attn_flash_pick_bk(dims[i], caches[j]);
            CHECK(bk >= ATTN_BK_MIN && bk <= ATTN_BK_MAX && (bk & (bk - 1)) == 0,
                  "pick_bk(%d, %zu) = %d", dims[i], caches[j], bk);
        }
}

/* Every decode-routed shape: the split arithmetic, the partial slots it writes into a scratch
 * of exactly the advertised size, and the merge that reads them back. */
static void check_attention_calls(void) {
    static const int shapes[][6] = {
        /* Hq, Hkv, Sq, Sk, D, causal */
        {32, 8, 1, 4096, 128, 0},      {2048, 512, 1, 4096, 128, 0}, {32, 8, 1, 65536, 128, 1},
        {8, 8, 1, 1, 1, 0},            {64, 8, 2, 65536, 128, 1},    {16, 4, 4, 8192, 64, 1},
        {8, 2, 2, 1000, 40, 0},        {1, 1, 16, 5, 256, 1},        {4096, 64, 1, 300000, 256, 0},
        {64, 1, 1, 2147483, 16, 0},    {3, 3, 1, 129, 7, 0},         {256, 256, 64, 4096, 128, 1},
        {128, 32, 4096, 4096, 128, 0}, {16, 8, 2048, 2048, 128, 1},  {48, 12, 1000, 4000, 64, 0},
    };
    const int nshapes = (int)(sizeof shapes / sizeof shapes[0]);
    for (int i = 0; i < nshapes; i++) {
        const int Hq = shapes[i][0], Hkv = shapes[i][1], Sq = shapes[i][2], Sk = shapes[i][3];
        const int D = shapes[i][4], causal = shapes[i][5];
        for (int bk = ATTN_BK_MIN; bk <= ATTN_BK_MAX; bk <<= 4) {
            const size_t bytes = attn_flash_scratch_bytes(D, bk);
            void *scratch = aligned_alloc(ATTN_SCRATCH_ALIGN, bytes);
            CHECK(scratch != NULL, "host scratch");
            memset(&lc, 0, sizeof lc);
            struct attn_times tm = {0, 0, 0, 0};
            attn_flash(FAKE(0x1000), FAKE(0x2000), FAKE(0x3000), (float *)(uintptr_t)0x4000, Hq,
                       Hkv, Sq, Sk, D, causal, bk, scratch, i & 1, (i % 3 == 0) ? &tm : NULL);
            CHECK(lc.decode_calls + lc.prefill_calls == 1, "one attention launch per call");
            if (lc.decode_calls)
                CHECK(lc.merge_calls == (lc.nsplit > 1), "merge iff split");
            if (lc.merge_calls)
                CHECK(lc.merge_rows == (long)Hq * Sq, "merge rows");
            if (i % 3 == 0)
                CHECK(tm.qxk == 2e-3 && tm.packv == 0.0 && tm.softmax == 0.0 && tm.sxv == 0.0,
                      "tm accumulates the event time into qxk only");
            free(scratch);
        }
        if (D <= ATTN_NOALLOC_D_MAX) {
            memset(&lc, 0, sizeof lc);
            attn_flash_noalloc(FAKE(0x1000), FAKE(0x2000), FAKE(0x3000),
                               (float *)(uintptr_t)0x4000, Hq, Hkv, Sq, Sk, D, causal, 128, 0);
            CHECK(lc.decode_calls + lc.prefill_calls == 1, "noalloc: one launch");
        }
    }
    memset(&lc, 0, sizeof lc);
    pack_v_full(FAKE(0x1000), (uint16_t *)(uintptr_t)0x2000, 7, 1000, 40);
    CHECK(lc.pack_calls == 1, "pack_v_full launches once");
}

/* ---- checks of the oracle --------------------------------------------------------------- */
static void check_oracle(void) {
    /* spread rows stay in range, start at 0 and end at Sq-1 */
    for (int Sq = 1; Sq <= 300; Sq += 7)
        for (int cap = -1; cap <= Sq + 2; cap++) {
            int *rows = malloc(sizeof(int) * (size_t)Sq);
            const int n = orc_ref_rowset(Sq, cap, rows);
            CHECK(n >= 1 && n <= Sq, "rowset count");
            for (int t = 0; t < n; t++)
                CHECK(rows[t] >= 0 && rows[t] < Sq && (t == 0 || rows[t] > rows[t - 1]),
                      "rowset(%d,%d) row %d", Sq, cap, rows[t]);
            CHECK(rows[n - 1] == Sq - 1, "rowset ends at Sq-1");
            free(rows);
        }
    /* attention on small shapes, every row; Sk = 1 copies V[0]; masked rows are zero */
    static const int shapes[][6] = {{1, 1, 1, 1, 1, 0},   {4, 2, 7, 1, 3, 1}, {6, 3, 13, 5, 40, 1},
                                    {2, 1, 5, 9, 17, 0},  {8, 8, 3, 64, 64, 1}};
    for (size_t i = 0; i < sizeof shapes / sizeof shapes[0]; i++) {
        const int Hq = shapes[i][0], Hkv = shapes[i][1], Sq = shapes[i][2], Sk = shapes[i][3];
        const int D = shapes[i][4], causal = shapes[i][5];
        const size_t nq = (size_t)Hq * Sq * D, nk = (size_t)Hkv * Sk * D;
        uint16_t *Q = malloc(nq * 2), *K = malloc(nk * 2), *V = malloc(nk * 2);
        float *O = malloc(nq * 4), *O2 = malloc(nq * 4);
        int *rows = malloc(sizeof(int) * (size_t)Sq);
        uint32_t st = 0x12345678u;
        orc_lcg_bf16(&st, Q, nq);
        orc_lcg_bf16(&st, K, nk);
        orc_lcg_bf16(&st, V, nk);
        const int n = orc_ref_rowset(Sq, 0, rows);
        CHECK(orc_attn_ref(Q, K, V, O, Hq, Hkv, Sq, Sk, D, causal, rows, n) == 0, "attn_ref");
        CHECK(orc_attn_ref_mt(Q, K, V, O2, Hq, Hkv, Sq, Sk, D, causal, rows, n, 3) == 0,
              "attn_ref_mt");
        CHECK(memcmp(O, O2, nq * 4) == 0, "single- and multi-threaded oracle agree bitwise");
        for (int h = 0; h < Hq; h++)
            for (int r = 0; r < Sq; r++) {
                const float *o = O + ((size_t)h * Sq + r) * D;
                const int kv = h / (Hq / Hkv);
                if (causal && Sk - Sq + r < 0) {
                    for (int d = 0; d < D; d++)
                        CHECK(o[d] == 0.0f, "masked row is zero");
                } else if (Sk == 1) {
                    for (int d = 0; d < D; d++)
                        CHECK(o[d] == orc_bf16_to_f32(V[(size_t)kv * D + d]), "Sk=1 copies V[0]");
                }
            }
        float mad, maxref;
        long nbad;
        CHECK(orc_cmp_rows(O, O2, Hq, Sq, D, rows, n, &mad, &maxref, &nbad) && mad == 0.0f,
              "cmp_rows of equal arrays");
        free(Q), free(K), free(V), free(O), free(O2), free(rows);
    }
    for (int Sq = 1; Sq < 40; Sq += 3)
        for (int Sk = 1; Sk < 40; Sk += 5) {
            double brute = 0;
            for (int i = 0; i < Sq; i++)
                for (int j = 0; j < Sk; j++)
                    brute += (j <= Sk - Sq + i);
            CHECK(orc_attn_pairs(Sq, Sk, 1) == brute && orc_attn_pairs(Sq, Sk, 0) == (double)Sq * Sk,
                  "pairs(%d,%d)", Sq, Sk);
        }
    uint16_t buf[4096], buf2[4096];
    orc_normal_bf16(buf, 4096, 7, 123, 2.0);
    attn_synth_normal_bf16(buf2, 4096, 7, 123, 2.0);
    CHECK(memcmp(buf, buf2, sizeof buf) == 0, "product and oracle normal generators agree");
    uint32_t s1 = 99, s2 = 99;
    orc_lcg_bf16(&s1, buf, 4096);
    attn_synth_lcg_bf16(&s2, buf2, 4096);
    CHECK(s1 == s2 && memcmp(buf, buf2, sizeof buf) == 0, "LCG generators agree");
}

/* attn_flash_plan runs the host-side choice with stand-in pointers and touches no memory: a
 * prefill, a split decode (with its merge) and a short buffer. */
static void check_plan(void) {
    char buf[256];
    int n = attn_flash_plan(128, 32, 4096, 4096, 128, 0, 128, 0, buf, sizeof buf);
    CHECK(n > 0 && strcmp(buf, "prefill\n") == 0, "plan of a prefill: %d '%s'", n, buf);
    n = attn_flash_plan(32, 8, 1, 32768, 128, 0, 128, 0, buf, sizeof buf);
    CHECK(n > 0 && strcmp(buf, "decode\nmerge\n") == 0, "plan of a split decode: %d '%s'", n,
          buf);
}

int main(void) {
    check_scratch_sizes();
    check_plan();
    check_pick_bk();
    check_attention_calls();
    check_oracle();
    free(g_static);
    if (failures) {
        printf("HOST_CHECKS FAILED: %d\n", failures);
        return 1;
    }
    printf("HOST_CHECKS OK\n");
    return 0;
}
