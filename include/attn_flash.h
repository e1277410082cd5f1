/* attn_flash.h -- C ABI of the MI355X (gfx950) bf16 flash-attention forward.
 *
 * Drop-in for the C entry points of the reference's AArch64 kernel
 * (liujiang833/transfer_station, flash.c). Same names and parameter lists; the
 * differences are deliberate and listed here:
 *   - Q, K, V, O and scratch are DEVICE pointers (hipMalloc'd or equivalent).
 *   - Work is stream-ordered on the calling thread's stream (attn_flash_set_stream,
 *     default: the null stream). O is valid once that stream has synchronised. When
 *     `tm` is non-NULL the call synchronises itself and O is valid on return, as in
 *     the reference.
 *   - Validation aborts (stderr message, then abort()) on an invalid bk exactly like
 *     the reference, and additionally on Hq%Hkv != 0, Hkv < 1, Sq < 1, Sk < 1,
 *     D outside [1, ATTN_D_MAX], a NULL or misaligned scratch, and HIP errors.
 *   - The scratch keeps the reference's contract (caller-owned, size depends only on
 *     (D, bk), monotone in bk, the kernel allocates nothing and keeps no state) but its
 *     content is the GPU's: split-K partials (m, l, acc[D]), 65536 slots, for the decode
 *     path and for prefills too small to fill the GPU, whose key ranges are split (34 MB at
 *     D = 128).
 *   - bk is validated and sizes the scratch but does not pick the key tile: the GPU's
 *     tile is fixed by D (128 keys up to D = 128, 64 beyond), so O is bit-identical at
 *     every bk. The reference's result is bk-invariant within its tolerance.
 *
 * Layouts (row-major, bf16 stored as uint16_t bits, O fp32):
 *   Q, O [Hq][Sq][D];  K, V [Hkv][Sk][D];  V^T when v_prepacked=1: [Hkv][D][Sk].
 *   A batch folds into the head axes: call with Hq' = B*Hq and Hkv' = B*Hkv.
 */
#ifndef ATTN_FLASH_H
#define ATTN_FLASH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Key-block bounds and default (flash.c:132-134). bk must be a power of two in
 * [ATTN_BK_MIN, ATTN_BK_MAX]; anything else aborts. */
#define ATTN_BK_MIN 16
#define ATTN_BK_MAX 4096
#define ATTN_BK_DEFAULT 128

/* Required scratch alignment in bytes (flash.c:607). hipMalloc already returns
 * 256-byte aligned memory. */
#define ATTN_SCRATCH_ALIGN 64

/* Largest head dimension the compiled kernels accept (the reference has no bound). */
#define ATTN_D_MAX 256

/* Optional per-call timing (flash.c:704-706). The GPU kernel is one fused launch, so the
 * whole kernel time (HIP events, seconds) is ADDED to qxk; packv, softmax and sxv are
 * left unchanged (no per-phase split is fabricated). */
struct attn_times {
    double packv, qxk, softmax, sxv;
};

/* Bytes of device scratch attn_flash() needs for this head_dim and key-block size
 * (replaces flash.c:679 attn_flash_scratch_bytes). Depends only on (D, bk), never on
 * Sq/Sk; non-decreasing in bk. Aborts on an invalid bk (flash.c:641-647) or D. */
size_t attn_flash_scratch_bytes(int D, int bk);

/* Largest power-of-two bk in [16, 4096] whose modelled per-key-block working set,
 * double-buffered, fits l2_bytes (spec: README.md:138-140,359-436 of the reference;
 * the function is absent from the shipped flash.c). Pure host function. */
int attn_flash_pick_bk(int D, size_t l2_bytes);

/* The attention forward (replaces flash.c:727-729 attn_flash).
 *   O[h][i][:] = softmax_j(scale * Q[h][i]·K[kv][j]) · V[kv][j][:], kv = h / (Hq/Hkv),
 *   scale = 1/sqrtf(D); causal masks keys j > Sk-Sq+i (bottom-right aligned); a row with
 *   no admissible key is written as zeros. P is rounded to bf16 (RNE) before P·V; the
 *   softmax denominator sums the unrounded fp32 p. */
void attn_flash(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O, int Hq,
                int Hkv, int Sq, int Sk, int D, int causal, int bk, void *scratch,
                int v_prepacked, struct attn_times *tm);

/* Separate V -> V^T operator: Vp[kv][d][k] = V[kv][k][d] (replaces flash.c:715-718
 * pack_v_full). Device pointers, stream-ordered like attn_flash. */
void pack_v_full(const uint16_t *V, uint16_t *Vp, int Hkv, int Sk, int D);

/* Allocation-free variant of attn_flash. No counterpart in the reference: it is for callers
 * that cannot allocate device memory or own a scratch (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same arguments and semantics as attn_flash,
 * without scratch and tm; the split-K partials go to a static device array of
 * ATTN_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs on until the process
 * ends (the layout of attn_flash's scratch at D = ATTN_NOALLOC_D_MAX, so the kernels, the splits
 * and the output are those of attn_flash). It calls no hipMalloc, hipFree or other allocating
 * routine. D above ATTN_NOALLOC_D_MAX is rejected (stderr message, then abort), as is everything
 * attn_flash rejects. Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams, other threads) race and must be serialised by the caller. */
#define ATTN_NOALLOC_D_MAX 128
#define ATTN_NOALLOC_SCRATCH_BYTES 34078720u /* = attn_flash_scratch_bytes(128, any bk) */
void attn_flash_noalloc(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O, int Hq,
                        int Hkv, int Sq, int Sk, int D, int causal, int bk, int v_prepacked);

/* Kernel plan of an attn_flash call (no counterpart in the reference: introspection for tests
 * and integrators, who can see which kernels a shape takes on the current device). Runs
 * attn_flash's host-side choice for these arguments and, instead of launching, writes one line
 * per kernel the call would launch -- "name<template arguments> [notes] grid=x block=n" -- into
 * buf, NUL-terminated. Returns the length written, or -1 when buf is too small. Reads and writes
 * no device memory; the argument checks are attn_flash's (tensors and scratch aside). */
int attn_flash_plan(int Hq, int Hkv, int Sq, int Sk, int D, int causal, int bk, int v_prepacked,
                    char *buf, size_t len);

/* Stream selection for the calling thread (no counterpart in the reference, which has
 * no device). `stream` is a hipStream_t; NULL selects the null stream. */
void attn_flash_set_stream(void *stream);
void *attn_flash_get_stream(void);

#ifdef __cplusplus
}
#endif

#endif /* ATTN_FLASH_H */
