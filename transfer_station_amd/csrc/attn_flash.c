/* attn_flash.c -- C host layer of the MI355X bf16 flash-attention forward.
 *
 * Validates exactly as the reference does (bk aborts at both doors, flash.c:641-647,680,764),
 * plus the tightenings listed in include/attn_flash.h, chooses the kernel (MFMA prefill, or
 * split-K decode + merge when a kv head has at most 64 query rows g*Sq, in 16-row blocks),
 * and launches it on the calling thread's stream. It allocates nothing per call: the decode
 * partials live in the caller's scratch, exactly as the reference's tiles do.
 */
#define __HIP_PLATFORM_AMD__ 1
#include "attn_flash.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* HIP launchers (attn_kernels.hip). Each returns a hipError_t. */
int attn_hip_launch_prefill(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O,
                            int Hq, int Hkv, int Sq, int Sk, int D, int causal, int vec, int vt,
                            int dp, float c, float *pm, float *pl, float *pacc, long slots,
                            void *stream);
int attn_hip_launch_decode(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O,
                           float *pm, float *pl, float *pacc, int Hq, int Hkv, int Sq, int Sk,
                           int D, int causal, int vec, int vt, int dp, float c, int nsplit,
                           int kps, int nrb, void *stream);
int attn_hip_launch_merge(const float *pm, const float *pl, const float *pacc, float *O, int rows,
                          int D, int nsplit, float c, int Sq, void *stream);
int attn_hip_launch_pack_v(const uint16_t *V, uint16_t *Vp, int Hkv, int Sk, int D, void *stream);
int attn_hip_device_cus(void);
void attn_hip_plan_begin(char *buf, size_t len);
long attn_hip_plan_end(void);
int attn_hip_static_scratch(void **ptr, size_t *bytes);

/* ---- device scratch layout ---------------------------------------------------------------
 * Split-K partial slots, one per (query row, split): m[ATTN_SLOTS], l[ATTN_SLOTS] and
 * acc[ATTN_SLOTS][D], each sub-buffer starting on a 256-byte boundary. The slot count is a
 * fixed capacity, so the size depends only on D (and trivially on bk), never on Sq/Sk; the
 * decode path caps its split count at ATTN_SLOTS / (Hq*Sq) and runs unsplit below 2, as does
 * the key split of an under-filled prefill grid, and the causal prefill splits the key range of
 * its heavier query tiles only when their rows fit. */
#define ATTN_SLOTS 65536
#define ATTN_SUB_ALIGN 256

static size_t align_up(size_t x, size_t a) { return (x + a - 1) & ~(a - 1); }

struct attn_carve {
    float *m, *l, *acc;
};

/* Measures when base == NULL, else also carves. One function, so the reported size and the
 * carve the kernels use cannot disagree (the reference's single-source-of-truth rule,
 * flash.c:658-672). */
static size_t attn_layout(void *base, int D, struct attn_carve *cv) {
    size_t off = 0;
    size_t om = off;
    off = align_up(off + sizeof(float) * ATTN_SLOTS, ATTN_SUB_ALIGN);
    size_t ol = off;
    off = align_up(off + sizeof(float) * ATTN_SLOTS, ATTN_SUB_ALIGN);
    size_t oa = off;
    off = align_up(off + sizeof(float) * (size_t)ATTN_SLOTS * (size_t)D, ATTN_SUB_ALIGN);
    if (base && cv) {
        cv->m = (float *)((char *)base + om);
        cv->l = (float *)((char *)base + ol);
        cv->acc = (float *)((char *)base + oa);
    }
    return off;
}

/* bk contract (flash.c:641-647): a power of two in [ATTN_BK_MIN, ATTN_BK_MAX]. The range
 * test runs first, so bk-1 is never evaluated for bk <= 0. */
static void attn_bk_check(int bk, const char *who) {
    if (bk < ATTN_BK_MIN || bk > ATTN_BK_MAX || (bk & (bk - 1)) != 0) {
        fprintf(stderr, "%s: bk=%d is invalid -- bk must be a POWER OF TWO in [%d, %d]\n", who, bk,
                ATTN_BK_MIN, ATTN_BK_MAX);
        abort();
    }
}

static void attn_d_check(int D, const char *who) {
    if (D < 1 || D > ATTN_D_MAX) {
        fprintf(stderr, "%s: D=%d is invalid -- head_dim must be in [1, %d]\n", who, D,
                ATTN_D_MAX);
        abort();
    }
}

static void attn_fail(const char *who, const char *what) {
    fprintf(stderr, "%s: %s\n", who, what);
    abort();
}

static void attn_hip_check(int err, const char *who) {
    if (err != 0) {
        fprintf(stderr, "%s: HIP error %d (%s)\n", who, err, hipGetErrorString((hipError_t)err));
        abort();
    }
}

size_t attn_flash_scratch_bytes(int D, int bk) {
    attn_bk_check(bk, "attn_flash_scratch_bytes");
    attn_d_check(D, "attn_flash_scratch_bytes");
    return attn_layout(NULL, D, NULL);
}

/* Documented cache model (README.md:359-436 of the reference): working set of one key block
 *   ws(D, bk) = 6*bk*(D + BQm) + 6*BQm*D + 4*D + 12*BQm,  BQm = 64,
 * computed in size_t with D widened before any arithmetic; the answer is the largest power
 * of two bk in [16, 4096] with 2*ws <= l2_bytes, scanning upward and stopping at the first
 * failure, and never less than 16. D < 1 is treated as 1. */
int attn_flash_pick_bk(int D, size_t l2_bytes) {
    const size_t BQm = 64;
    size_t d = (D < 1) ? (size_t)1 : (size_t)D;
    size_t per_bk = 6u * (d + BQm);
    size_t fixed = 6u * BQm * d + 4u * d + 12u * BQm;
    int best = ATTN_BK_MIN;
    for (int bk = ATTN_BK_MIN; bk <= ATTN_BK_MAX; bk *= 2) {
        size_t ws = per_bk * (size_t)bk + fixed;
        if (ws > SIZE_MAX / 2 || 2u * ws > l2_bytes)
            break;
        best = bk;
    }
    return best;
}

/* ---- streams ---------------------------------------------------------------------------- */
static _Thread_local void *t_stream = NULL;
void attn_flash_set_stream(void *stream) { t_stream = stream; }
void *attn_flash_get_stream(void) { return t_stream; }

/* ---- tile and split selection ------------------------------------------------------------ */
#define ATTN_DECODE_ROWS 16     /* query rows the decode MFMA tile holds (one row block) */
#define ATTN_DECODE_MAX_ROWS 64 /* g*Sq rows per kv head up to which decode can beat prefill */

/* Decode (split-K over the key range, 16-row blocks) or prefill for g*Sq rows per kv head.
 * Up to one row block decode streams K/V at the HBM rate. Up to 64 rows it wins while the
 * prefill grid (one packed query tile per kv head) would be smaller than the GPU, since
 * split-K spreads few kv heads over many workgroups; with at least as many kv heads as CUs
 * the prefill's MFMA tiles win. Measured, Sk = 4096, 32-64 rows per kv head: 512 kv heads
 * prefill 1.4-2.1x faster; 32-64 kv heads decode 1.7-2x faster. */
static int attn_use_decode(int Hkv, int group, int Sq) {
    /* ATTN_PATH=decode or =prefill (read once) forces the kernel for tuning sweeps, decode only
     * where its row blocks apply (g*Sq <= 64). */
    static int forced = -1;
    if (forced < 0) {
        const char *e = getenv("ATTN_PATH");
        forced = (e && !strcmp(e, "decode")) ? 1 : ((e && !strcmp(e, "prefill")) ? 2 : 0);
    }
    const long rows = (long)group * Sq;
    if (forced == 2 || (forced == 1 && rows <= ATTN_DECODE_MAX_ROWS))
        return forced == 1;
    if (rows <= ATTN_DECODE_ROWS)
        return 1;
    return rows <= ATTN_DECODE_MAX_ROWS && Hkv < attn_hip_device_cus();
}
#define ATTN_DECODE_TARGET_WG 512
#define ATTN_DECODE_MIN_KEYS 128 /* keys per split: one 32-key tile per wave, 4 waves */

static void attn_decode_split(int Hq, int Hkv, int Sq, int Sk, int nrb, int *nsplit_o,
                              int *kps_o) {
    long rows = (long)Hq * Sq;
    long cap = ATTN_SLOTS / (rows > 0 ? rows : 1);
    long want = (ATTN_DECODE_TARGET_WG + (long)Hkv * nrb - 1) / ((long)Hkv * nrb);
    long by_len = (Sk + ATTN_DECODE_MIN_KEYS - 1) / ATTN_DECODE_MIN_KEYS;
    long ns = want;
    if (ns > by_len)
        ns = by_len;
    if (ns > cap)
        ns = cap;
    if (ns < 2)
        ns = 1;
    /* keys per split: a multiple of 128 covering Sk in ns pieces */
    long kps = (Sk + ns - 1) / ns;
    kps = (kps + ATTN_DECODE_MIN_KEYS - 1) / ATTN_DECODE_MIN_KEYS * ATTN_DECODE_MIN_KEYS;
    ns = (Sk + kps - 1) / kps;
    *nsplit_o = (int)ns;
    *kps_o = (int)kps;
}

static int attn_dp_for_d(int D) { return (D <= 64) ? 64 : (D <= 128 ? 128 : 256); }

/* ---- timing events (only when the caller asks for tm) ------------------------------------- */
static _Thread_local hipEvent_t t_ev0 = NULL, t_ev1 = NULL;

static void attn_events(void) {
    if (!t_ev0)
        attn_hip_check(hipEventCreate(&t_ev0), "attn_flash(tm)");
    if (!t_ev1)
        attn_hip_check(hipEventCreate(&t_ev1), "attn_flash(tm)");
}

/* Argument checks shared by both attention entry points. bk keeps the reference's contract
 * (validated here, scratch sized with it), but the key tile is the hardware's: 128 keys up to
 * D = 128, 64 beyond, whatever bk says. In the reference bk is a cache-blocking knob whose
 * result is bk-invariant within the tolerance (README.md:354-357); on the GPU a smaller tile is
 * only slower. */
static void attn_check_args(const char *who, const uint16_t *Q, const uint16_t *K,
                            const uint16_t *V, const float *O, int Hq, int Hkv, int Sq, int Sk,
                            int D, int bk) {
    attn_bk_check(bk, who);
    attn_d_check(D, who);
    if (Hkv < 1 || Hq < 1 || Hq % Hkv != 0)
        attn_fail(who, "need Hq >= 1, Hkv >= 1 and Hq % Hkv == 0");
    if (Sq < 1 || Sk < 1)
        attn_fail(who, "need Sq >= 1 and Sk >= 1");
    if (!Q || !K || !V || !O)
        attn_fail(who, "Q, K, V and O must be device pointers");
}

/* Kernel choice and launches on the calling thread's stream; `scratch` holds the split-K
 * partial slots (attn_layout at this D). */
static void attn_run(const char *who, const uint16_t *Q, const uint16_t *K, const uint16_t *V,
                     float *O, int Hq, int Hkv, int Sq, int Sk, int D, int causal, void *scratch,
                     int v_prepacked, struct attn_times *tm) {
    void *st = t_stream;
    const int group = Hq / Hkv;
    const float scale = 1.0f / sqrtf((float)D);
    const float c = scale * 1.44269504088896341f;
    const int dp = attn_dp_for_d(D);
    /* v_prepacked (flash.c:751-753,770): V is V^T [Hkv][D][Sk], rows of stride Sk. 16-byte
     * vector loads then also need Sk % 8 == 0 (each d row starting 16-byte aligned). */
    const int vt = v_prepacked ? 1 : 0;
    const int vec = (D % 8 == 0) && (!vt || Sk % 8 == 0) &&
                    ((((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V | (uintptr_t)O) & 15u) == 0);

    if (tm) {
        attn_events();
        attn_hip_check(hipEventRecord(t_ev0, (hipStream_t)st), who);
    }
    if (attn_use_decode(Hkv, group, Sq)) {
        const int nrb = (group * Sq + ATTN_DECODE_ROWS - 1) / ATTN_DECODE_ROWS;
        int nsplit, kps;
        attn_decode_split(Hq, Hkv, Sq, Sk, nrb, &nsplit, &kps);
        struct attn_carve cv = {NULL, NULL, NULL};
        attn_layout(scratch, D, &cv);
        attn_hip_check(attn_hip_launch_decode(Q, K, V, O, cv.m, cv.l, cv.acc, Hq, Hkv, Sq, Sk, D,
                                              causal ? 1 : 0, vec, vt, dp, c, nsplit, kps, nrb,
                                              st),
                       who);
        if (nsplit > 1)
            attn_hip_check(
                attn_hip_launch_merge(cv.m, cv.l, cv.acc, O, Hq * Sq, D, nsplit, c, Sq, st), who);
    } else {
        struct attn_carve cv = {NULL, NULL, NULL};
        attn_layout(scratch, D, &cv);
        attn_hip_check(attn_hip_launch_prefill(Q, K, V, O, Hq, Hkv, Sq, Sk, D, causal ? 1 : 0,
                                               vec, vt, dp, c, cv.m, cv.l, cv.acc, ATTN_SLOTS,
                                               st),
                       who);
    }
    if (tm) {
        float ms = 0.f;
        attn_hip_check(hipEventRecord(t_ev1, (hipStream_t)st), who);
        attn_hip_check(hipEventSynchronize(t_ev1), who);
        attn_hip_check(hipEventElapsedTime(&ms, t_ev0, t_ev1), who);
        tm->qxk += (double)ms * 1e-3;
    }
}

void attn_flash(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O, int Hq,
                int Hkv, int Sq, int Sk, int D, int causal, int bk, void *scratch,
                int v_prepacked, struct attn_times *tm) {
    static const char *who = "attn_flash";
    attn_check_args(who, Q, K, V, O, Hq, Hkv, Sq, Sk, D, bk);
    if (!scratch || ((uintptr_t)scratch % ATTN_SCRATCH_ALIGN) != 0)
        attn_fail(who, "scratch must be non-NULL and ATTN_SCRATCH_ALIGN-aligned");
    attn_run(who, Q, K, V, O, Hq, Hkv, Sq, Sk, D, causal, scratch, v_prepacked, tm);
}

/* No hipMalloc and no events: the partial slots are the library's static device array, whose
 * address is resolved once per device (attn_hip_static_scratch). */
void attn_flash_noalloc(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O,
                        int Hq, int Hkv, int Sq, int Sk, int D, int causal, int bk,
                        int v_prepacked) {
    static const char *who = "attn_flash_noalloc";
    attn_check_args(who, Q, K, V, O, Hq, Hkv, Sq, Sk, D, bk);
    if (D > ATTN_NOALLOC_D_MAX) {
        fprintf(stderr,
                "%s: D=%d is invalid -- the static scratch holds partials for D <= %d "
                "(use attn_flash with a caller-owned scratch)\n",
                who, D, ATTN_NOALLOC_D_MAX);
        abort();
    }
    void *scratch = NULL;
    size_t bytes = 0;
    attn_hip_check(attn_hip_static_scratch(&scratch, &bytes), who);
    if (bytes < attn_layout(NULL, D, NULL) || ((uintptr_t)scratch % ATTN_SCRATCH_ALIGN) != 0)
        attn_fail(who, "static scratch is smaller than its layout or misaligned");
    attn_run(who, Q, K, V, O, Hq, Hkv, Sq, Sk, D, causal, scratch, v_prepacked, NULL);
}

/* The host-side kernel choice of attn_flash for these arguments, recorded instead of launched:
 * no device memory is read or written. Stand-in pointers are 256-aligned and non-NULL, as a
 * caller's tensors and scratch are, so every alignment- and scratch-dependent choice is the one
 * attn_flash makes. */
int attn_flash_plan(int Hq, int Hkv, int Sq, int Sk, int D, int causal, int bk, int v_prepacked,
                    char *buf, size_t len) {
    static const char *who = "attn_flash_plan";
    const uint16_t *p = (const uint16_t *)(uintptr_t)ATTN_SCRATCH_ALIGN;
    attn_check_args(who, p, p, p, (const float *)p, Hq, Hkv, Sq, Sk, D, bk);
    if (!buf || len == 0)
        attn_fail(who, "buf must be non-NULL and len above 0");
    attn_hip_plan_begin(buf, len);
    attn_run(who, p, p, p, (float *)p, Hq, Hkv, Sq, Sk, D, causal, (void *)p, v_prepacked, NULL);
    const long n = attn_hip_plan_end();
    return n < 0 || n > 0x7fffffffL ? -1 : (int)n;
}

void pack_v_full(const uint16_t *V, uint16_t *Vp, int Hkv, int Sk, int D) {
    static const char *who = "pack_v_full";
    if (Hkv < 1 || Sk < 1 || D < 1)
        attn_fail(who, "need Hkv >= 1, Sk >= 1 and D >= 1");
    if (!V || !Vp)
        attn_fail(who, "V and Vp must be device pointers");
    attn_hip_check(attn_hip_launch_pack_v(V, Vp, Hkv, Sk, D, t_stream), who);
}
