// roofline_bench.hip -- measured roofline denominators for MI355X (gfx950), the counterpart of
// the reference's SVE BFDOT peak microbenchmark (bfdot_peak.cpp:1-132): independent chains of
// the compute primitive the kernel uses, timed long enough to be steady, reported as a rate.
//
//   roofline_bench                 all measurements, one JSON line
//   roofline_bench mfma            bf16 MFMA peak (v_mfma_f32_32x32x16_bf16, 16x16x32_bf16)
//   roofline_bench clock           MFMA-only rate and shader clock, constant vs random operands
//   roofline_bench copy <MiB>      one float4 copy of <MiB> MiB (PMC calibration: known bytes)
//   roofline_bench read <MiB>      streaming read of <MiB> MiB, ordinary and non-temporal loads
//   roofline_bench mix             the headline prefill kernel's per-tile instruction mix, with parts removed
//   roofline_bench ldsprobe        the split-K decode kernel's LDS access patterns, one kernel each
//                                  (run under rocprofv3 --pmc SQ_LDS_BANK_CONFLICT for conflicts)
//
// Grid shapes are fixed at launch and every index is bounded by the buffer sizes below.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;

#define CHECK(x)                                                                                   \
    do {                                                                                           \
        hipError_t e_ = (x);                                                                       \
        if (e_ != hipSuccess) {                                                                    \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_));     \
            exit(1);                                                                               \
        }                                                                                          \
    } while (0)

// Four independent accumulation chains per wave keep the matrix pipe issuing back to back.
__global__ __launch_bounds__(256) void mfma32_peak(float *out, int iters) {
    bf16x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = (__bf16)(float)((threadIdx.x + i) & 7);
        b[i] = (__bf16)(float)((threadIdx.x * 3 + i) & 7);
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
    }
    float s = 0.f;
    for (int i = 0; i < 16; ++i)
        s += c0[i] + c1[i] + c2[i] + c3[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Same chains as mfma32_peak but with random bf16 operands that change every step (operand
// bits toggle as in a real attention tile; constant operands draw less power and can clock
// higher). r holds 64 random u32 per lane-slot, read from registers after one load.
__global__ __launch_bounds__(256) void mfma32_peak_random(const unsigned *r, float *out, int iters) {
    typedef __attribute__((ext_vector_type(4))) unsigned u4;
    // eight random operand registers per lane, cycled so that consecutive MFMAs see different
    // bits (as a real attention tile does); no VALU work in the loop
    bf16x8 op[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        u4 v = *(const u4 *)(r + ((threadIdx.x & 63) * 8 + k) * 4);
        v = (v & 0x80FF80FFu) | 0x3E003E00u; // bounded exponents, random sign and mantissa
        op[k] = __builtin_bit_cast(bf16x8, v);
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[k], op[k + 1], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[k + 1], op[(k + 2) & 7], c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[(k + 3) & 7], op[k], c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[(k + 5) & 7], op[(k + 6) & 7], c3, 0, 0, 0);
        }
    }
    float s = 0.f;
    for (int i = 0; i < 16; ++i)
        s += c0[i] + c1[i] + c2[i] + c3[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// MFMA-only chains (as mfma32_peak / mfma32_peak_random) that also record, for wave 0 of each
// block, the shader-clock ticks (s_memtime) and the 100 MHz real-time ticks (s_memrealtime)
// across the loop: their ratio is the clock the chip ran at under that load.
template <bool RANDOM>
__global__ __launch_bounds__(256) void mfma32_clock(const unsigned *r, float *out,
                                                   unsigned long long *clk, int iters) {
    typedef __attribute__((ext_vector_type(4))) unsigned u4;
    bf16x8 op[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        u4 v;
        if (RANDOM) {
            v = *(const u4 *)(r + ((threadIdx.x & 63) * 8 + k) * 4);
            v = (v & 0x80FF80FFu) | 0x3E003E00u;
        } else {
            v = u4{0x3F803F80u, 0x40003F80u, 0x3F804000u, 0x3F803F80u};
        }
        op[k] = __builtin_bit_cast(bf16x8, v);
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[k], op[k + 1], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[k + 1], op[(k + 2) & 7], c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[(k + 3) & 7], op[k], c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(op[(k + 5) & 7], op[(k + 6) & 7], c3, 0, 0, 0);
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.f;
    for (int i = 0; i < 16; ++i)
        s += c0[i] + c1[i] + c2[i] + c3[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clk[2 * blockIdx.x] = t1 - t0;
        clk[2 * blockIdx.x + 1] = r1 - r0;
    }
}

// One or two dependent accumulation chains per wave (how a single S^T chain is served).
template <int CH>
__global__ __launch_bounds__(256) void mfma32_chain(float *out, int iters) {
    bf16x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = (__bf16)(float)((threadIdx.x + i) & 7);
        b[i] = (__bf16)(float)((threadIdx.x * 3 + i) & 7);
    }
    f32x16 c[CH] = {};
    for (int it = 0; it < iters; ++it)
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int ch = 0; ch < CH; ++ch)
                c[ch] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[ch], 0, 0, 0);
    float s = 0.f;
    for (int ch = 0; ch < CH; ++ch)
        for (int i = 0; i < 16; ++i)
            s += c[ch][i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// One wave per SIMD: 2 MFMA chains plus NV independent VALU fma per MFMA, in program order.
template <int NV>
__global__ __launch_bounds__(256) void mfma_valu_coissue(float *out, int iters) {
    bf16x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = (__bf16)(float)((threadIdx.x + i) & 7);
        b[i] = (__bf16)(float)((threadIdx.x * 3 + i) & 7);
    }
    f32x16 c0 = {}, c1 = {};
    float v[16];
    for (int i = 0; i < 16; ++i)
        v[i] = 1.0f + threadIdx.x * 1e-3f + i;
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
#pragma unroll
        for (int k = 0; k < NV; ++k)
            v[k] = fmaf(v[k], 0.999f, 0.5f);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
#pragma unroll
        for (int k = 0; k < NV; ++k)
            v[8 + k % 8] = fmaf(v[8 + k % 8], 0.999f, 0.25f);
        if constexpr (NV > 0) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);
        }
    }
    float s = 0.f;
    for (int i = 0; i < 16; ++i)
        s += c0[i] + c1[i] + v[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Two waves per SIMD: waves 0-3 issue only MFMA (2 chains), waves 4-7 only VALU fma
// (NV per MFMA-equivalent step); measures how far a VALU wave slows an MFMA wave.
template <int NV, bool AG>
__global__ __launch_bounds__(512) void mfma_valu_split(float *out, int iters) {
    const int w = threadIdx.x >> 6;
    float s = 0.f;
    if (w < 4) {
        bf16x8 a, b;
        for (int i = 0; i < 8; ++i) {
            a[i] = (__bf16)(float)((threadIdx.x + i) & 7);
            b[i] = (__bf16)(float)((threadIdx.x * 3 + i) & 7);
        }
        f32x16 c0 = {}, c1 = {};
        for (int it = 0; it < iters; ++it) {
            if (AG) { // accumulators pinned in AGPRs
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c0) : "v"(a), "v"(b));
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c1) : "v"(a), "v"(b));
            } else {
                c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
            }
        }
        for (int i = 0; i < 16; ++i)
            s += c0[i] + c1[i];
    } else {
        float v[8];
        for (int i = 0; i < 8; ++i)
            v[i] = 1.0f + threadIdx.x * 1e-3f + i;
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int k = 0; k < 2 * NV; ++k)
                v[k % 8] = fmaf(v[k % 8], 0.999f, 0.5f);
        for (int i = 0; i < 8; ++i)
            s += v[i];
    }
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void mfma16_peak(float *out, int iters) {
    bf16x8 a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = (__bf16)(float)((threadIdx.x + i) & 7);
        b[i] = (__bf16)(float)((threadIdx.x * 3 + i) & 7);
    }
    f32x4 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c3, 0, 0, 0);
    }
    float s = 0.f;
    for (int i = 0; i < 4; ++i)
        s += c0[i] + c1[i] + c2[i] + c3[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// VALU issue rate: 8 independent chains of v_exp_f32 (transcendental) or v_fma_f32 per lane.
template <bool EXP>
__global__ __launch_bounds__(256) void valu_rate(float *out, int iters) {
    float x[8];
    for (int i = 0; i < 8; ++i)
        x[i] = -1.0f - 1e-3f * (threadIdx.x + i);
    for (int it = 0; it < iters; ++it)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            x[i] = EXP ? __builtin_amdgcn_exp2f(x[i]) - 1.5f : fmaf(x[i], 0.999f, -0.5f);
    float s = 0.f;
    for (int i = 0; i < 8; ++i)
        s += x[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// LDS read throughput: every lane reads 16 bytes (ds_read_b128) or 8 bytes transposed
// (ds_read_b64_tr_b16) per step from a 64 KiB tile; addresses stay inside the tile.
typedef __attribute__((ext_vector_type(4))) unsigned u32x4_t;
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
template <bool TR>
__global__ __launch_bounds__(256) void lds_rate(unsigned *out, unsigned long long *clk, int iters) {
    __shared__ __attribute__((aligned(16))) unsigned short tile[32768];
    for (int i = threadIdx.x; i < 32768; i += 256)
        tile[i] = (unsigned short)i;
    __syncthreads();
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    unsigned acc = 0;
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            // 16 KiB window per wave, rows of 256 B plus a 16 B pad (bank-conflict free)
            const int base = ((w * 8 + k) & 31) * 512 + ((it & 7) * 64);
            if (TR) {
                const int off = base + (lane & 15) * 136 / 4 * 4 + (lane >> 4) * 4;
                s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4_t *)(tile + (off & 32767 & ~3)));
                acc ^= (unsigned)v[0] ^ ((unsigned)v[3] << 16);
            } else {
                const int off = base + (lane & 15) * 136 + (lane >> 4) * 8;
                u32x4_t v = *(const u32x4_t *)(tile + (off & 32767 & ~7));
                acc ^= v[0] ^ v[3];
            }
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    out[blockIdx.x * blockDim.x + threadIdx.x] = acc;
    if (threadIdx.x == 0) {
        clk[2 * blockIdx.x] = t1 - t0;
        clk[2 * blockIdx.x + 1] = r1 - r0;
    }
}

// The per-tile instruction mix of the headline prefill kernel (attn_prefill_fast_kernel at
// D = 128, 128-key tiles, 8 waves = two per SIMD, one workgroup per CU) without its data
// dependencies on real inputs: per wave and tile, 32 MFMA of S^T = K.Q^T whose A operands are
// 16-byte LDS reads of a K tile, the softmax VALU on those accumulators (p = 2^(s c - m c),
// bf16 conversion, pairwise sums), 32 MFMA of O^T += V^T.P^T whose A operands are pairs of
// transposed 8-byte LDS reads of a V tile, then (DMA) the next tile's 64 KB by LDS-DMA from an
// L2-resident buffer and one barrier. LDS and register operands hold random bf16 (bounded
// exponents), so the MFMA operand bits toggle as in the kernel. Switches take parts away:
// REUSE = 2 reads each K and V fragment once for two MFMAs (half the LDS fragment bytes, as
// with 64 rows per wave), VALU = false drops the softmax (P is then the S bits), DMA = false the
// tile loads. The rate with everything on is the ceiling of this mix; each switch measures the
// share of one resource. Every LDS address stays inside the two 64 KB tile buffers and every
// DMA source offset inside src (64 KB per buffer, blocks of 1 KB per wave).
typedef __attribute__((ext_vector_type(4))) unsigned u32x4_m;
typedef __attribute__((ext_vector_type(4))) short s16x4_m;
template <int REUSE, int VALU, bool DMA>
__global__ __launch_bounds__(512, 1) void mix_tile(const unsigned short *src, float *out,
                                                   unsigned long long *clk, int tiles) {
    __shared__ __attribute__((aligned(1024))) unsigned short T[2][2][128 * 128]; // [buf][K,V]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l32 = lane & 31, hi = lane >> 5, g16 = lane >> 4, i16 = lane & 15;
    for (int i = tid; i < 2 * 2 * 128 * 128 / 8; i += 512)
        reinterpret_cast<u32x4_m *>(&T[0][0][0])[i] =
            reinterpret_cast<const u32x4_m *>(src)[i & (2 * 128 * 128 / 8 - 1)];
    bf16x8 qb[8];
    for (int k = 0; k < 8; ++k)
        qb[k] = __builtin_bit_cast(bf16x8, reinterpret_cast<const u32x4_m *>(src)[lane * 8 + k]);
    // fragment offsets as in the kernel's swizzled tiles (conflict-free)
    const int kperm = (l32 & ~12) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
    const int kfo = (kperm >> 3) * 8 * 128 + (kperm & 7) * 16 + ((hi ^ ((kperm >> 3) & 1)) * 8);
    const int vfo = hi * 8 * 128 + (i16 >> 2) * 32 + (2 * (g16 & 1) + ((i16 & 3) >> 1)) * 8 +
                    (i16 & 1) * 4;
    const float c = 0.1275f;
    float mrun = 4.0f, l = 0.f;
    f32x16 o[4] = {}, negm;
    for (int i = 0; i < 16; ++i)
        negm[i] = -mrun * c;
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int t = 0; t < tiles; ++t) {
        const int buf = t & 1;
        if (DMA) {
            // 64 KB per CU: each wave 4 K and 4 V blocks of 1 KB into the other buffer
            const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<unsigned short *>(src), (short)0, 2 * 128 * 128 * 2, 0x00020000);
            for (int k = 0; k < 4; ++k) {
                const int blk = w * 4 + k; // 0..31
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    r, (__attribute__((address_space(3))) void *)&T[buf ^ 1][0][blk * 512], 16,
                    (unsigned)(blk * 1024 + lane * 16), 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    r, (__attribute__((address_space(3))) void *)&T[buf ^ 1][1][blk * 512], 16,
                    (unsigned)(32768 + blk * 1024 + lane * 16), 0, 0, 0);
            }
        }
        const unsigned short *kb = &T[buf][0][kfo];
        f32x16 s[4];
        for (int st = 0; st < 4; ++st) {
            for (int i = 0; i < 16; ++i)
                s[st][i] = (VALU == 2) ? negm[i] : 0.f;
            for (int kk = 0; kk < 8; kk += REUSE) {
                const bf16x8 a = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4_m *>(kb + st * 32 * 128 + kk * 128));
                for (int j = 0; j < REUSE; ++j)
                    s[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qb[(kk + j + st) & 7], s[st],
                                                                    0, 0, 0);
            }
        }
        bf16x8 pk[8];
        if (VALU) {
            const float mc = mrun * c;
            float ps = 0.f;
            for (int st = 0; st < 4; ++st)
                for (int hh = 0; hh < 2; ++hh) {
                    float p[8];
                    for (int j = 0; j < 8; ++j) {
                        p[j] = __builtin_amdgcn_exp2f(VALU == 2 ? s[st][8 * hh + j]
                                                                : fmaf(s[st][8 * hh + j], c, -mc));
                        pk[2 * st + hh][j] = (__bf16)p[j];
                    }
                    ps += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
                }
            l += ps;
        } else {
            for (int st = 0; st < 4; ++st)
                for (int hh = 0; hh < 2; ++hh) {
                    u32x4_m v;
                    for (int j = 0; j < 4; ++j)
                        v[j] = (__builtin_bit_cast(unsigned, s[st][8 * hh + 2 * j]) & 0x807F807Fu) |
                               0x3C003C00u;
                    pk[2 * st + hh] = __builtin_bit_cast(bf16x8, v);
                }
        }
        const unsigned short *vb = &T[buf][1][vfo];
        for (int cc = 0; cc < 8; ++cc)
            for (int db = 0; db < 4; db += REUSE) {
                const unsigned short *p = vb + cc * 16 * 128 + db * 128;
                const s16x4_m lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4_m *)p);
                const s16x4_m hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4_m *)(p + 4 * 128));
                typedef __attribute__((ext_vector_type(8))) short s16x8;
                const s16x8 a8 = {lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                const bf16x8 a = __builtin_bit_cast(bf16x8, a8);
                for (int j = 0; j < REUSE; ++j)
                    o[db + j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pk[cc], o[db + j], 0, 0, 0);
            }
        if (DMA)
            __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float acc = l;
    for (int d = 0; d < 4; ++d)
        for (int i = 0; i < 16; ++i)
            acc += o[d][i];
    out[blockIdx.x * 512 + tid] = acc;
    if (tid == 0) {
        clk[2 * blockIdx.x] = t1 - t0;
        clk[2 * blockIdx.x + 1] = r1 - r0;
    }
}

// The same per-tile mix for one wave per SIMD with 64 query rows (4 waves per CU, 512
// registers each): every K and V fragment read from LDS feeds two MFMAs (the two 32-row
// blocks), the softmax covers 128 scores per lane. Per CU and tile the MFMA work equals
// mix_tile's; the LDS fragment bytes are half.
template <bool VALU>
__global__ __launch_bounds__(256, 1) void mix_tile_w64(const unsigned short *src, float *out,
                                                       unsigned long long *clk, int tiles) {
    __shared__ __attribute__((aligned(1024))) unsigned short T[2][2][128 * 128]; // [buf][K,V]
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int l32 = lane & 31, hi = lane >> 5, g16 = lane >> 4, i16 = lane & 15;
    for (int i = tid; i < 2 * 2 * 128 * 128 / 8; i += 256)
        reinterpret_cast<u32x4_m *>(&T[0][0][0])[i] =
            reinterpret_cast<const u32x4_m *>(src)[i & (2 * 128 * 128 / 8 - 1)];
    bf16x8 qb[2][8];
    for (int rb = 0; rb < 2; ++rb)
        for (int k = 0; k < 8; ++k)
            qb[rb][k] = __builtin_bit_cast(
                bf16x8, reinterpret_cast<const u32x4_m *>(src)[(lane * 8 + k + rb * 1024) & 4095]);
    const int kperm = (l32 & ~12) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
    const int kfo = (kperm >> 3) * 8 * 128 + (kperm & 7) * 16 + ((hi ^ ((kperm >> 3) & 1)) * 8);
    const int vfo = hi * 8 * 128 + (i16 >> 2) * 32 + (2 * (g16 & 1) + ((i16 & 3) >> 1)) * 8 +
                    (i16 & 1) * 4;
    const float c = 0.1275f;
    float mrun = 4.0f, l = 0.f;
    f32x16 o[2][4] = {};
    __syncthreads();
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int t = 0; t < tiles; ++t) {
        const int buf = t & 1;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<unsigned short *>(src), (short)0, 2 * 128 * 128 * 2, 0x00020000);
        for (int k = 0; k < 8; ++k) { // 64 KB per CU: each of 4 waves 8 K and 8 V blocks
            const int blk = w * 8 + k;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                r, (__attribute__((address_space(3))) void *)&T[buf ^ 1][0][blk * 512], 16,
                (unsigned)(blk * 1024 + lane * 16), 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                r, (__attribute__((address_space(3))) void *)&T[buf ^ 1][1][blk * 512], 16,
                (unsigned)(32768 + blk * 1024 + lane * 16), 0, 0, 0);
        }
        const unsigned short *kb = &T[buf][0][kfo];
        const unsigned short *vb = &T[buf][1][vfo];
        // per 32-key sub-tile: S for both row blocks, softmax, P.V
        for (int st = 0; st < 4; ++st) {
            f32x16 s[2];
            for (int rb = 0; rb < 2; ++rb)
                for (int i = 0; i < 16; ++i)
                    s[rb][i] = 0.f;
            for (int kk = 0; kk < 8; ++kk) {
                const bf16x8 a = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const u32x4_m *>(kb + st * 32 * 128 + kk * 128));
                for (int rb = 0; rb < 2; ++rb)
                    s[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qb[rb][kk], s[rb], 0, 0, 0);
            }
            bf16x8 pk[2][2];
            if (VALU) {
                const float mc = mrun * c;
                float ps = 0.f;
                for (int rb = 0; rb < 2; ++rb)
                    for (int hh = 0; hh < 2; ++hh) {
                        float p[8];
                        for (int j = 0; j < 8; ++j) {
                            p[j] = __builtin_amdgcn_exp2f(fmaf(s[rb][8 * hh + j], c, -mc));
                            pk[rb][hh][j] = (__bf16)p[j];
                        }
                        ps += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
                    }
                l += ps;
            } else {
                for (int rb = 0; rb < 2; ++rb)
                    for (int hh = 0; hh < 2; ++hh) {
                        u32x4_m v;
                        for (int j = 0; j < 4; ++j)
                            v[j] = (__builtin_bit_cast(unsigned, s[rb][8 * hh + 2 * j]) & 0x807F807Fu) |
                                   0x3C003C00u;
                        pk[rb][hh] = __builtin_bit_cast(bf16x8, v);
                    }
            }
            for (int hh = 0; hh < 2; ++hh)
                for (int db = 0; db < 4; ++db) {
                    const unsigned short *p = vb + (st * 2 + hh) * 16 * 128 + db * 128;
                    const s16x4_m lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4_m *)p);
                    const s16x4_m hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) s16x4_m *)(p + 4 * 128));
                    typedef __attribute__((ext_vector_type(8))) short s16x8;
                    const s16x8 a8 = {lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                    const bf16x8 a = __builtin_bit_cast(bf16x8, a8);
                    for (int rb = 0; rb < 2; ++rb)
                        o[rb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pk[rb][hh], o[rb][db],
                                                                            0, 0, 0);
                }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float acc = l;
    for (int rb = 0; rb < 2; ++rb)
        for (int d = 0; d < 4; ++d)
            for (int i = 0; i < 16; ++i)
                acc += o[rb][d][i];
    out[blockIdx.x * 512 + tid] = acc;
    if (tid == 0) {
        clk[2 * blockIdx.x] = t1 - t0;
        clk[2 * blockIdx.x + 1] = r1 - r0;
    }
}

// dst[i] = src[i] for i < n4 (float4 elements), grid-stride.
__global__ __launch_bounds__(256) void hbm_copy(const f32x4 *__restrict__ src,
                                                f32x4 *__restrict__ dst, size_t n4) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4;
         i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// Per-thread sums of src[i] for i < n4; one float per thread written to out.
// Each workgroup reads its contiguous share (n4 / gridDim.x elements, a multiple of 256 * 8)
// with 8 16-byte loads in flight per thread. NT: non-temporal loads (the cache policy for data
// read once, as the decode kernels use), which HBM streams faster.
template <bool NT>
__global__ __launch_bounds__(256) void hbm_read(const f32x4 *__restrict__ src, float *out,
                                                size_t n4) {
    const size_t per = n4 / gridDim.x;
    const f32x4 *p = src + blockIdx.x * per + threadIdx.x;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (size_t off = 0; off < per; off += 256 * 8) {
        f32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = NT ? __builtin_nontemporal_load(p + off + 256 * i) : p[off + 256 * i];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            acc += v[i];
    }
    out[blockIdx.x * blockDim.x + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

static double time_ms(hipEvent_t a, hipEvent_t b) {
    float ms = 0.f;
    CHECK(hipEventSynchronize(b));
    CHECK(hipEventElapsedTime(&ms, a, b));
    return ms;
}

static double run_mfma_random() {
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int blocks = cus * 8, threads = 256, iters = 5000;
    float *out;
    unsigned *r;
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
    CHECK(hipMalloc(&r, 64 * 8 * 4 * sizeof(unsigned)));
    unsigned h[2048];
    unsigned x = 0x12345678u;
    for (int i = 0; i < 2048; ++i) {
        x ^= x << 13; x ^= x >> 17; x ^= x << 5;
        h[i] = x;
    }
    CHECK(hipMemcpy(r, h, sizeof h, hipMemcpyHostToDevice));
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    double best = 0;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(a, 0));
        hipLaunchKernelGGL(mfma32_peak_random, dim3(blocks), dim3(threads), 0, 0, r, out, iters);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        double ms = time_ms(a, b);
        double flops = (double)blocks * (threads / 64) * iters * 16 * 32768.0;
        double tf = flops / (ms * 1e-3) / 1e12;
        if (tf > best)
            best = tf;
    }
    CHECK(hipFree(out));
    CHECK(hipFree(r));
    return best;
}

// TFLOP/s and the shader clock (GHz, from s_memtime over the 100 MHz s_memrealtime) of the
// MFMA-only loop with constant or random operands.
template <bool RANDOM> static void run_clock(double *tflops, double *ghz) {
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int blocks = cus * 8, threads = 256, iters = 5000;
    float *out;
    unsigned *r;
    unsigned long long *clk;
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
    CHECK(hipMalloc(&r, 64 * 8 * 4 * sizeof(unsigned)));
    CHECK(hipMalloc(&clk, (size_t)blocks * 2 * sizeof(unsigned long long)));
    unsigned h[2048];
    unsigned x = 0x12345678u;
    for (int i = 0; i < 2048; ++i) {
        x ^= x << 13; x ^= x >> 17; x ^= x << 5;
        h[i] = x;
    }
    CHECK(hipMemcpy(r, h, sizeof h, hipMemcpyHostToDevice));
    std::vector<unsigned long long> hc((size_t)blocks * 2);
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    *tflops = 0;
    *ghz = 0;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(a, 0));
        hipLaunchKernelGGL(mfma32_clock<RANDOM>, dim3(blocks), dim3(threads), 0, 0, r, out, clk,
                           iters);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        const double ms = time_ms(a, b);
        const double tf = (double)blocks * (threads / 64) * iters * 16 * 32768.0 / (ms * 1e-3) / 1e12;
        if (tf > *tflops) {
            *tflops = tf;
            CHECK(hipMemcpy(hc.data(), clk, hc.size() * sizeof(unsigned long long),
                            hipMemcpyDeviceToHost));
            double sum = 0;
            for (int i = 0; i < blocks; ++i)
                sum += (double)hc[2 * i] / (double)hc[2 * i + 1];
            *ghz = sum / blocks * 0.1; // real-time counter: 100 MHz
        }
    }
    CHECK(hipFree(out));
    CHECK(hipFree(r));
    CHECK(hipFree(clk));
}

static double run_mfma(int which) {
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int blocks = cus * 8, threads = 256, iters = 20000;
    float *out;
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    double flop_per_inst = (which == 32) ? 32.0 * 32 * 16 * 2 : 16.0 * 16 * 32 * 2;
    double best = 0;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(a, 0));
        if (which == 32)
            hipLaunchKernelGGL(mfma32_peak, dim3(blocks), dim3(threads), 0, 0, out, iters);
        else
            hipLaunchKernelGGL(mfma16_peak, dim3(blocks), dim3(threads), 0, 0, out, iters);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        double ms = time_ms(a, b);
        double flops = (double)blocks * (threads / 64) * iters * 4 * flop_per_inst;
        double tf = flops / (ms * 1e-3) / 1e12;
        if (tf > best)
            best = tf;
    }
    CHECK(hipFree(out));
    return best;
}

// Wave-instructions per clock per SIMD for v_exp_f32 (EXP) or v_fma_f32.
// TFLOP/s with CH dependent chains per wave, `wpb` waves per SIMD (blocks of 256 threads).
static double run_chain(int ch, int waves_per_simd) {
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int blocks = cus * waves_per_simd, threads = 256, iters = 5000;
    float *out;
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    double best = 0;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(a, 0));
        if (ch == 1)
            hipLaunchKernelGGL(mfma32_chain<1>, dim3(blocks), dim3(threads), 0, 0, out, iters * 4);
        else if (ch == 2)
            hipLaunchKernelGGL(mfma32_chain<2>, dim3(blocks), dim3(threads), 0, 0, out, iters * 2);
        else
            hipLaunchKernelGGL(mfma32_chain<4>, dim3(blocks), dim3(threads), 0, 0, out, iters);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        double ms = time_ms(a, b);
        double flops = (double)blocks * 4 * iters * 16 * 32768.0;
        double tf = flops / (ms * 1e-3) / 1e12;
        if (tf > best)
            best = tf;
    }
    CHECK(hipFree(out));
    return best;
}

static double run_coissue(int nv) {
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int blocks = cus, threads = 256, iters = 20000; // one wave per SIMD
    float *out;
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    double best = 0;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(a, 0));
        switch (nv) {
        case 0: hipLaunchKernelGGL(mfma_valu_coissue<0>, dim3(blocks), dim3(threads), 0, 0, out, iters); break;
        case 2: hipLaunchKernelGGL(mfma_valu_coissue<2>, dim3(blocks), dim3(threads), 0, 0, out, iters); break;
        case 4: hipLaunchKernelGGL(mfma_valu_coissue<4>, dim3(blocks), dim3(threads), 0, 0, out, iters); break;
        case 6: hipLaunchKernelGGL(mfma_valu_coissue<6>, dim3(blocks), dim3(threads), 0, 0, out, iters); break;
        default: hipLaunchKernelGGL(mfma_valu_coissue<8>, dim3(blocks), dim3(threads), 0, 0, out, iters); break;
        }
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        double ms = time_ms(a, b);
        double flops = (double)blocks * 4 * iters * 2 * 32768.0;
        double tf = flops / (ms * 1e-3) / 1e12;
        if (tf > best)
            best = tf;
    }
    CHECK(hipFree(out));
    return best;
}

template <bool AG>
static double run_split(int nv) {
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int blocks = cus, threads = 512, iters = 20000;
    float *out;
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    double best = 0;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(a, 0));
        switch (nv) {
        case 0: hipLaunchKernelGGL((mfma_valu_split<0, AG>), dim3(blocks), dim3(threads), 0, 0, out, iters); break;
        case 4: hipLaunchKernelGGL((mfma_valu_split<4, AG>), dim3(blocks), dim3(threads), 0, 0, out, iters); break;
        case 6: hipLaunchKernelGGL((mfma_valu_split<6, AG>), dim3(blocks), dim3(threads), 0, 0, out, iters); break;
        default: hipLaunchKernelGGL((mfma_valu_split<8, AG>), dim3(blocks), dim3(threads), 0, 0, out, iters); break;
        }
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        double ms = time_ms(a, b);
        double flops = (double)blocks * 4 * iters * 2 * 32768.0;
        double tf = flops / (ms * 1e-3) / 1e12;
        if (tf > best)
            best = tf;
    }
    CHECK(hipFree(out));
    return best;
}

// LDS bank-conflict probes: the split-K decode kernel's per-wave LDS access patterns, one kernel
// per pattern, so that rocprofv3 --pmc SQ_LDS_BANK_CONFLICT attributes the counts to each:
//   P = 0: the V tile stores, 8 ds_write_b128 per wave writing 32 key rows of 256 bytes at a
//          row stride of RS bytes (lane + 64 r -> row / 16, 16-byte chunk % 16);
//   P = 1: the transposed V reads, 16 ds_read_b64_tr_b16 per wave, lane (g = lane / 16,
//          r = lane % 16) at row 8g + r / 4 (and 4 rows on), bytes 8 (r % 4) + 32 db;
//   P = 2: the row exchanges, __shfl_xor by 16 and by 32.
// Each wave owns 32 rows of RS bytes; every address stays inside them.
template <int P, int RS>
__global__ __launch_bounds__(256) void lds_probe(unsigned *out, int iters) {
    constexpr int RE = RS / 2; // row stride in elements
    __shared__ __attribute__((aligned(16))) unsigned short tile[4 * 32 * RE];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int i = threadIdx.x; i < 4 * 32 * RE; i += 256)
        tile[i] = (unsigned short)i;
    __syncthreads();
    unsigned short *vt = &tile[w * 32 * RE];
    unsigned acc = lane;
    for (int it = 0; it < iters; ++it) {
        if constexpr (P == 0) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int cidx = lane + 64 * r, row = cidx / 16, col = (cidx % 16) * 8;
                const u32x4_t v = {(unsigned)it, (unsigned)r, acc, 0u};
                *reinterpret_cast<u32x4_t *>(&vt[row * RE + col]) = v;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        } else if constexpr (P == 1) {
            const int g = lane >> 4, r = lane & 15;
            const unsigned short *vb = &vt[(8 * g + (r >> 2)) * RE + 4 * (r & 3)];
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4_t *)(vb + db * 16));
                const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4_t *)(vb + db * 16 + 4 * RE));
                acc += (unsigned)(lo[0] ^ hi[3]);
            }
        } else {
            float x = (float)acc;
            x += __shfl_xor(x, 16);
            x += __shfl_xor(x, 32);
            acc = (unsigned)x;
        }
    }
    out[blockIdx.x * 256 + threadIdx.x] = acc;
}

// Runs each LDS probe once over 4 workgroups per CU; returns the probes' ms (rocprofv3 reads
// the counters).
static void run_lds_probes(double *ms) {
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int blocks = cus * 4, iters = 2000;
    unsigned *out;
    CHECK(hipMalloc(&out, (size_t)blocks * 256 * sizeof(unsigned)));
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    for (int k = 0; k < 5; ++k) {
        CHECK(hipEventRecord(a, 0));
        switch (k) {
        case 0: hipLaunchKernelGGL((lds_probe<0, 288>), dim3(blocks), dim3(256), 0, 0, out, iters); break;
        case 1: hipLaunchKernelGGL((lds_probe<1, 288>), dim3(blocks), dim3(256), 0, 0, out, iters); break;
        case 2: hipLaunchKernelGGL((lds_probe<2, 288>), dim3(blocks), dim3(256), 0, 0, out, iters); break;
        case 3: hipLaunchKernelGGL((lds_probe<0, 256>), dim3(blocks), dim3(256), 0, 0, out, iters); break;
        default: hipLaunchKernelGGL((lds_probe<1, 256>), dim3(blocks), dim3(256), 0, 0, out, iters); break;
        }
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        ms[k] = time_ms(a, b);
    }
    CHECK(hipFree(out));
}

static double run_valu(bool exp) {
    int cus = 0, clk_khz = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    CHECK(hipDeviceGetAttribute(&clk_khz, hipDeviceAttributeClockRate, 0));
    const int blocks = cus * 8, threads = 256, iters = 20000;
    float *out;
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    double best = 0;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(a, 0));
        if (exp)
            hipLaunchKernelGGL(valu_rate<true>, dim3(blocks), dim3(threads), 0, 0, out, iters);
        else
            hipLaunchKernelGGL(valu_rate<false>, dim3(blocks), dim3(threads), 0, 0, out, iters);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        double ms = time_ms(a, b);
        // per chain step: one v_exp + one v_add (EXP) or one v_fma; count the op of interest
        double wave_insts = (double)blocks * (threads / 64) * iters * 8;
        double per_simd_clk = wave_insts / (cus * 4.0) / (ms * 1e-3 * clk_khz * 1e3);
        if (per_simd_clk > best)
            best = per_simd_clk;
    }
    CHECK(hipFree(out));
    return best;
}

// Bytes per shader clock per CU delivered by LDS reads (clock from s_memtime over the 100 MHz
// s_memrealtime inside the kernel), with wpc waves per CU.
static double run_lds(bool tr, int wpc) {
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int blocks = cus * wpc / 4, threads = 256, iters = 4000;
    unsigned *out;
    unsigned long long *clk;
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(unsigned)));
    CHECK(hipMalloc(&clk, (size_t)blocks * 2 * sizeof(unsigned long long)));
    std::vector<unsigned long long> hc((size_t)blocks * 2);
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    double best = 0;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(a, 0));
        if (tr)
            hipLaunchKernelGGL(lds_rate<true>, dim3(blocks), dim3(threads), 0, 0, out, clk, iters);
        else
            hipLaunchKernelGGL(lds_rate<false>, dim3(blocks), dim3(threads), 0, 0, out, clk, iters);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        const double ms = time_ms(a, b);
        CHECK(hipMemcpy(hc.data(), clk, hc.size() * sizeof(unsigned long long),
                        hipMemcpyDeviceToHost));
        double ghz = 0;
        for (int i = 0; i < blocks; ++i)
            ghz += (double)hc[2 * i] / (double)hc[2 * i + 1] * 0.1 / blocks;
        const double bytes = (double)blocks * threads * iters * 8 * (tr ? 8 : 16);
        const double bpc = bytes / cus / (ms * 1e-3 * ghz * 1e9);
        if (bpc > best)
            best = bpc;
    }
    CHECK(hipFree(out));
    CHECK(hipFree(clk));
    return best;
}

// mix_tile over one workgroup per CU: TFLOP/s of its MFMA work, the shader clock (s_memtime
// over the 100 MHz s_memrealtime) and shader clocks per tile, best of three runs.
template <int REUSE, int VALU, bool DMA, bool W64 = false>
static void run_mix(double *tflops, double *ghz, double *clk_per_tile) {
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int blocks = cus, tiles = 2000;
    std::vector<unsigned short> h(2 * 128 * 128);
    unsigned x = 0x2468ace1u;
    for (auto &e : h) {
        x ^= x << 13; x ^= x >> 17; x ^= x << 5;
        e = (unsigned short)((x & 0x807Fu) | 0x3F00u); // random sign and mantissa, |v| in [0.5, 1)
    }
    unsigned short *src;
    float *out;
    unsigned long long *clk;
    CHECK(hipMalloc(&src, h.size() * 2));
    CHECK(hipMalloc(&out, (size_t)blocks * 512 * sizeof(float)));
    CHECK(hipMalloc(&clk, (size_t)blocks * 2 * sizeof(unsigned long long)));
    CHECK(hipMemcpy(src, h.data(), h.size() * 2, hipMemcpyHostToDevice));
    std::vector<unsigned long long> hc((size_t)blocks * 2);
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    *tflops = 0;
    for (int rep = 0; rep < 3; ++rep) {
        CHECK(hipEventRecord(a, 0));
        if (W64)
            hipLaunchKernelGGL((mix_tile_w64<VALU != 0>), dim3(blocks), dim3(256), 0, 0, src, out, clk,
                               tiles);
        else
            hipLaunchKernelGGL((mix_tile<REUSE, VALU, DMA>), dim3(blocks), dim3(512), 0, 0, src,
                               out, clk, tiles);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        const double ms = time_ms(a, b);
        const double tf = (double)blocks * 8 * 64 * tiles * 32768.0 / (ms * 1e-3) / 1e12;
        if (tf > *tflops) {
            *tflops = tf;
            CHECK(hipMemcpy(hc.data(), clk, hc.size() * sizeof(unsigned long long),
                            hipMemcpyDeviceToHost));
            double g = 0, cpt = 0;
            for (int i = 0; i < blocks; ++i) {
                g += (double)hc[2 * i] / (double)hc[2 * i + 1] * 0.1 / blocks;
                cpt += (double)hc[2 * i] / tiles / blocks;
            }
            *ghz = g;
            *clk_per_tile = cpt;
        }
    }
    CHECK(hipFree(src));
    CHECK(hipFree(out));
    CHECK(hipFree(clk));
}

static double run_stream(int copy, size_t mib, int reps, bool nt = false) {
    size_t bytes = mib << 20, n4 = bytes / 16;
    f32x4 *src, *dst;
    float *out;
    const int blocks = 256 * 16, threads = 256;
    CHECK(hipMalloc(&src, bytes));
    CHECK(hipMalloc(&dst, bytes));
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
    CHECK(hipMemset(src, 0, bytes));
    // hbm_read takes whole passes of 256 threads x 8 loads per workgroup: the bytes it reads
    // are rounded down to a multiple of blocks * 2048 elements (all of them from 128 MiB up).
    const size_t pass = (size_t)blocks * 256 * 8;
    const size_t n4r = n4 / pass * pass;
    if (!copy && n4r == 0) {
        fprintf(stderr, "read size must be at least %zu MiB\n", pass * 16 >> 20);
        exit(2);
    }
    const double moved = copy ? 2.0 * bytes : 16.0 * n4r;
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    double best = 0;
    for (int rep = 0; rep < reps; ++rep) {
        CHECK(hipEventRecord(a, 0));
        if (copy)
            hipLaunchKernelGGL(hbm_copy, dim3(blocks), dim3(threads), 0, 0, src, dst, n4);
        else if (nt)
            hipLaunchKernelGGL(hbm_read<true>, dim3(blocks), dim3(threads), 0, 0, src, out, n4r);
        else
            hipLaunchKernelGGL(hbm_read<false>, dim3(blocks), dim3(threads), 0, 0, src, out, n4r);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        double ms = time_ms(a, b);
        double gbs = moved / (ms * 1e-3) / 1e9;
        if (gbs > best)
            best = gbs;
    }
    CHECK(hipFree(src));
    CHECK(hipFree(dst));
    CHECK(hipFree(out));
    return best;
}

int main(int argc, char **argv) {
    const char *mode = argc > 1 ? argv[1] : "all";
    size_t mib = argc > 2 ? (size_t)atol(argv[2]) : 2048;
    if (mib < 1 || mib > 65536) {
        fprintf(stderr, "size must be 1..65536 MiB\n");
        return 2;
    }
    if (!strcmp(mode, "mfma")) {
        printf("{\"mfma32x32x16_bf16_tflops\": %.1f, \"mfma16x16x32_bf16_tflops\": %.1f, "
               "\"mfma32x32x16_bf16_random_operands_tflops\": %.1f}\n",
               run_mfma(32), run_mfma(16), run_mfma_random());
    } else if (!strcmp(mode, "clock")) {
        double tc, gc, tr, gr;
        run_clock<false>(&tc, &gc);
        run_clock<true>(&tr, &gr);
        printf("{\"mfma_const_operands_tflops\": %.1f, \"mfma_const_operands_ghz\": %.3f, "
               "\"mfma_random_operands_tflops\": %.1f, \"mfma_random_operands_ghz\": %.3f}\n",
               tc, gc, tr, gr);
    } else if (!strcmp(mode, "split")) {
        for (int nv = 0; nv <= 8; nv += (nv == 0 ? 4 : 2))
            printf("{\"valu_per_mfma_other_wave\": %d, \"mfma_tflops_vgpr_acc\": %.1f, "
                   "\"mfma_tflops_agpr_acc\": %.1f}\n",
                   nv, run_split<false>(nv), run_split<true>(nv));
    } else if (!strcmp(mode, "coissue")) {
        for (int nv = 0; nv <= 8; nv += 2)
            printf("{\"valu_per_mfma\": %d, \"one_wave_per_simd_mfma_tflops\": %.1f}\n", nv,
                   run_coissue(nv));
    } else if (!strcmp(mode, "chain")) {
        for (int w = 1; w <= 2; ++w)
            printf("{\"waves_per_simd\": %d, \"chain1_tflops\": %.1f, \"chain2_tflops\": %.1f, "
                   "\"chain4_tflops\": %.1f}\n",
                   w, run_chain(1, w), run_chain(2, w), run_chain(4, w));
    } else if (!strcmp(mode, "lds")) {
        for (int wpc = 4; wpc <= 8; wpc += 4) // 64 KB of LDS per block: at most 2 per CU
            printf("{\"waves_per_cu\": %d, \"lds_read_b128_bytes_per_clk_cu\": %.1f, "
                   "\"lds_read_tr_b64_bytes_per_clk_cu\": %.1f}\n",
                   wpc, run_lds(false, wpc), run_lds(true, wpc));
    } else if (!strcmp(mode, "mix")) {
        struct {
            const char *name;
            void (*fn)(double *, double *, double *);
        } v[] = {{"kernel mix (1 KB LDS per MFMA, softmax VALU, DMA)", run_mix<1, true, true>},
                 {"softmax without the fma (scale in Q, max in the accumulators)", run_mix<1, 2, true>},
                 {"half the LDS fragment reads", run_mix<2, true, true>},
                 {"no softmax VALU", run_mix<1, false, true>},
                 {"no DMA", run_mix<1, true, false>},
                 {"half LDS reads, no softmax VALU", run_mix<2, false, true>},
                 {"MFMA and LDS reads only", run_mix<1, false, false>},
                 {"one wave per SIMD, 64 rows (half the LDS fragment reads)", run_mix<2, true, true, true>},
                 {"one wave per SIMD, 64 rows, no softmax VALU", run_mix<2, false, true, true>}};
        for (auto &e : v) {
            double tf, g, cpt;
            e.fn(&tf, &g, &cpt);
            printf("{\"mix\": \"%s\", \"tflops\": %.1f, \"ghz\": %.3f, "
                   "\"shader_clocks_per_tile\": %.0f, \"mfma_clocks_per_tile\": 4096}\n",
                   e.name, tf, g, cpt);
        }
    } else if (!strcmp(mode, "ldsprobe")) {
        double ms[5];
        run_lds_probes(ms);
        printf("{\"lds_probe_ms\": {\"v_store_b128_rs288\": %.3f, \"v_read_tr_rs288\": %.3f, "
               "\"shfl_xor_16_32\": %.3f, \"v_store_b128_rs256\": %.3f, \"v_read_tr_rs256\": %.3f}}\n",
               ms[0], ms[1], ms[2], ms[3], ms[4]);
    } else if (!strcmp(mode, "valu")) {
        printf("{\"exp_chain_steps_per_simd_clk\": %.4f, \"fma_per_simd_clk\": %.4f}\n",
               run_valu(true), run_valu(false));
    } else if (!strcmp(mode, "copy")) {
        printf("{\"copy_mib\": %zu, \"copy_gbps\": %.1f}\n", mib, run_stream(1, mib, 1));
    } else if (!strcmp(mode, "read")) {
        printf("{\"read_mib\": %zu, \"read_gbps\": %.1f, \"read_nt_gbps\": %.1f}\n", mib,
               run_stream(0, mib, 5), run_stream(0, mib, 5, true));
    } else if (!strcmp(mode, "all")) {
        double m32 = run_mfma(32), m16 = run_mfma(16), mr = run_mfma_random();
        double cp = run_stream(1, mib, 5), rd = run_stream(0, mib, 5);
        printf("{\"mfma32x32x16_bf16_tflops\": %.1f, \"mfma16x16x32_bf16_tflops\": %.1f, "
               "\"mfma32x32x16_bf16_random_operands_tflops\": %.1f, "
               "\"copy_gbps\": %.1f, \"read_gbps\": %.1f, \"stream_mib\": %zu}\n",
               m32, m16, mr, cp, rd, mib);
    } else {
        fprintf(stderr, "usage: %s [all|mfma|clock|split|coissue|chain|lds|mix|ldsprobe|valu|copy MiB|read MiB]\n", argv[0]);
        return 2;
    }
    return 0;
}
