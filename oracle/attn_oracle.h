/* attn_oracle.h -- TEST INFRASTRUCTURE ONLY: prototypes of the CPU oracle (attn_oracle.c).
 * Only tests, __graft_entry__.smoke() and bench.py's CPU-baseline leg may use it. */
#ifndef ATTN_ORACLE_H
#define ATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_lcg_bf16(uint32_t *state, uint16_t *out, size_t n);
void orc_normal_bf16(uint16_t *out, size_t n, uint64_t seed, uint64_t counter0, double sigma);
int orc_attn_ref(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O, int Hq,
                 int Hkv, int Sq, int Sk, int D, int causal, const int *rows, int nrows);
int orc_attn_ref_mt(const uint16_t *Q, const uint16_t *K, const uint16_t *V, float *O, int Hq,
                    int Hkv, int Sq, int Sk, int D, int causal, const int *rows, int nrows,
                    int nthreads);
double orc_attn_pairs(int Sq, int Sk, int causal);
int orc_ref_rowset(int Sq, int ref_cap, int *rows);
float orc_tol(void);
int orc_cmp_rows(const float *Oref, const float *Odut, int Hq, int Sq, int D, const int *rows,
                 int nrows, float *mad_o, float *maxref_o, long *nbad_o);

#endif /* ATTN_ORACLE_H */
