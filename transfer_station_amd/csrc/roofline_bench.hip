// roofline_bench.hip -- measured roofline denominators for MI355X (gfx950), the counterpart of
// the reference's SVE BFDOT peak microbenchmark (bfdot_peak.cpp:1-132): independent chains of
// the compute primitive the kernel uses, timed long enough to be steady, reported as a rate.
//
//   roofline_bench                 all measurements, one JSON line
//   roofline_bench mfma            bf16 MFMA peak (v_mfma_f32_32x32x16_bf16, 16x16x32_bf16)
//   roofline_bench copy <MiB>      one float4 copy of <MiB> MiB (PMC calibration: known bytes)
//   roofline_bench read <MiB>      streaming read of <MiB> MiB
//
// Grid shapes are fixed at launch and every index is bounded by the buffer sizes below.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

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

// dst[i] = src[i] for i < n4 (float4 elements), grid-stride.
__global__ __launch_bounds__(256) void hbm_copy(const f32x4 *__restrict__ src,
                                                f32x4 *__restrict__ dst, size_t n4) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4;
         i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// Per-thread sums of src[i] for i < n4; one float per thread written to out.
__global__ __launch_bounds__(256) void hbm_read(const f32x4 *__restrict__ src, float *out,
                                                size_t n4) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4;
         i += (size_t)gridDim.x * blockDim.x)
        acc += src[i];
    out[blockIdx.x * blockDim.x + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

static double time_ms(hipEvent_t a, hipEvent_t b) {
    float ms = 0.f;
    CHECK(hipEventSynchronize(b));
    CHECK(hipEventElapsedTime(&ms, a, b));
    return ms;
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

static double run_stream(int copy, size_t mib, int reps) {
    size_t bytes = mib << 20, n4 = bytes / 16;
    f32x4 *src, *dst;
    float *out;
    const int blocks = 256 * 16, threads = 256;
    CHECK(hipMalloc(&src, bytes));
    CHECK(hipMalloc(&dst, bytes));
    CHECK(hipMalloc(&out, (size_t)blocks * threads * sizeof(float)));
    CHECK(hipMemset(src, 0, bytes));
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    double best = 0;
    for (int rep = 0; rep < reps; ++rep) {
        CHECK(hipEventRecord(a, 0));
        if (copy)
            hipLaunchKernelGGL(hbm_copy, dim3(blocks), dim3(threads), 0, 0, src, dst, n4);
        else
            hipLaunchKernelGGL(hbm_read, dim3(blocks), dim3(threads), 0, 0, src, out, n4);
        CHECK(hipGetLastError());
        CHECK(hipEventRecord(b, 0));
        double ms = time_ms(a, b);
        double gbs = (copy ? 2.0 : 1.0) * bytes / (ms * 1e-3) / 1e9;
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
        printf("{\"mfma32x32x16_bf16_tflops\": %.1f, \"mfma16x16x32_bf16_tflops\": %.1f}\n",
               run_mfma(32), run_mfma(16));
    } else if (!strcmp(mode, "valu")) {
        printf("{\"exp_chain_steps_per_simd_clk\": %.4f, \"fma_per_simd_clk\": %.4f}\n",
               run_valu(true), run_valu(false));
    } else if (!strcmp(mode, "copy")) {
        printf("{\"copy_mib\": %zu, \"copy_gbps\": %.1f}\n", mib, run_stream(1, mib, 1));
    } else if (!strcmp(mode, "read")) {
        printf("{\"read_mib\": %zu, \"read_gbps\": %.1f}\n", mib, run_stream(0, mib, 5));
    } else if (!strcmp(mode, "all")) {
        double m32 = run_mfma(32), m16 = run_mfma(16);
        double cp = run_stream(1, mib, 5), rd = run_stream(0, mib, 5);
        printf("{\"mfma32x32x16_bf16_tflops\": %.1f, \"mfma16x16x32_bf16_tflops\": %.1f, "
               "\"copy_gbps\": %.1f, \"read_gbps\": %.1f, \"stream_mib\": %zu}\n",
               m32, m16, cp, rd, mib);
    } else {
        fprintf(stderr, "usage: %s [all|mfma|copy MiB|read MiB]\n", argv[0]);
        return 2;
    }
    return 0;
}
