/* attn_devutil.h -- device plumbing and synthetic-data helpers exported by the same library.
 *
 * No counterpart in the reference (it has no device and allocates with aligned_alloc in its
 * harness, flash.c:1047-1066). These exist so tests, the benchmark and a C or Python driver
 * can own device buffers and time launches without a second runtime. They are NOT on the
 * attention hot path and attn_flash never calls them.
 */
#ifndef ATTN_DEVUTIL_H
#define ATTN_DEVUTIL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Device memory. Every function returns 0 on success or the hipError_t code. */
int attn_dev_count(int *n);
int attn_dev_malloc(void **p, size_t bytes);
int attn_dev_free(void *p);
int attn_dev_memcpy_htod(void *dst, const void *src, size_t bytes);
int attn_dev_memcpy_dtoh(void *dst, const void *src, size_t bytes);
int attn_dev_memcpy_dtod(void *dst, const void *src, size_t bytes);
int attn_dev_memset(void *dst, int value, size_t bytes);
int attn_dev_synchronize(void);
/* Device name, gfx arch, CU count, max engine clock (kHz), L2 bytes. */
int attn_dev_info(char *name, size_t name_len, char *arch, size_t arch_len, int *cus,
                  int *clock_khz, int *l2_bytes);

/* Events recorded on the calling thread's attn_flash stream (attn_flash_set_stream). */
int attn_dev_event_create(void **ev);
int attn_dev_event_destroy(void *ev);
int attn_dev_event_record(void *ev);
int attn_dev_event_elapsed_ms(void *start, void *stop, float *ms); /* waits for stop */

/* Synthetic bf16 data (host memory), the benchmark's input generators:
 *  normal: element c uses counter-based splitmix64 (seed, 2c+1), (seed, 2c+2) -> two
 *          53-bit uniforms -> Box-Muller cosine branch in double -> sigma*n -> float -> bf16
 *          RNE. Counters let Q, K, V occupy disjoint ranges of one stream.
 *  lcg:    the reference's generator (flash.c:867-871): state*1664525 + 1013904223,
 *          ((state>>8)&0xffff)/32768 - 1, then bf16 RNE; state is updated in place. */
void attn_synth_normal_bf16(uint16_t *out, size_t n, uint64_t seed, uint64_t counter0,
                            double sigma);
void attn_synth_lcg_bf16(uint32_t *state, uint16_t *out, size_t n);
uint16_t attn_synth_f32_to_bf16(float f);

#ifdef __cplusplus
}
#endif

#endif /* ATTN_DEVUTIL_H */
