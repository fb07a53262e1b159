// Sustained matrix-core throughput probe for gfx950 (MI355X): how fast v_mfma runs when the chip is held
// busy long enough to reach its steady clock, alone and with the per-MFMA side work of the attention
// kernel's key loop. Prints one JSON object. Used by bench.py (--probe) to put the attention kernel's
// roofline fraction next to what the chip actually sustains, since the 2.5 PFLOP/s dense fp16 figure
// assumes 2.4 GHz and a matrix-core-only load.
//
// Each wave runs 4 independent accumulator chains of 8 MFMAs per iteration; 2 workgroups of 4 waves per CU
// (2 waves per SIMD, like the attention kernel). Variants:
//   mfma32      v_mfma_f32_32x32x16_f16 on random fp16 operands
//   mfma16      v_mfma_f32_16x16x32_f16, same flops
//   mix32       mfma32 + per MFMA: one 1 KB ds_read_b128 operand, one v_exp_f32, two fp32 FMAs
//               (the attention key loop does 1 operand read, 1 exp2 and ~2.4 other VALU per MFMA)
//   mfma32_zero mfma32 on all-zero operands (operand toggling is a large share of the power)
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) half8 lds_half8;

constexpr int NIT = 4096, BLOCKS = 512, THREADS = 256, NOPS = 4096;

#define CK(x)                                                                          \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

// SHAPE 32: 32x32x16; 16: two 16x16x32 per step (same flops). MIX: + LDS read, exp, 2 FMA per step.
template <int SHAPE, bool MIX>
__global__ __launch_bounds__(THREADS, 2) void k_probe(float* out, const half8* ops) {
    __shared__ half8 sm[NOPS];  // 64 KB of operands
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < NOPS; i += THREADS) sm[i] = ops[(i * 7 + blockIdx.x) % NOPS];
    __syncthreads();
    half8 a[8], b[2];
#pragma unroll
    for (int i = 0; i < 8; i++) a[i] = ops[(threadIdx.x + 64 * i + blockIdx.x * 3) % NOPS];
    b[0] = ops[(threadIdx.x * 5 + 1) % NOPS];
    b[1] = ops[(threadIdx.x * 3 + 77) % NOPS];
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] = -1.0f + 0.001f * (threadIdx.x + i);
    floatx16 c[4] = {};
    const uint32_t vb = (uint32_t)(size_t)(lds_half8*)sm + lane * 16 + (w & 3) * 8192;
    for (int it = 0; it < NIT; it++) {
        half8 l[8];
        if constexpr (MIX) {
            const uint32_t off = (uint32_t)__builtin_amdgcn_readfirstlane((it & 3) * 2048);
#pragma unroll
            for (int k = 0; k < 8; k++) l[k] = *reinterpret_cast<const lds_half8*>((size_t)(vb + off + k * 1024));
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const half8 av = MIX ? l[k] : a[k];
            floatx16& acc = c[k & 3];
            if constexpr (SHAPE == 32) {
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b[k & 1], acc, 0, 0, 0);
            } else {
                floatx4 t0 = {acc[0], acc[1], acc[2], acc[3]}, t1 = {acc[4], acc[5], acc[6], acc[7]};
                t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b[k & 1], t0, 0, 0, 0);
                t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b[(k + 1) & 1], t1, 0, 0, 0);
                for (int i = 0; i < 4; i++) {
                    acc[i] = t0[i];
                    acc[i + 4] = t1[i];
                }
            }
            if constexpr (MIX) {
                x[k] = __builtin_amdgcn_exp2f(x[k]) - 1.0f;
                x[(k + 4) & 7] = x[(k + 4) & 7] * 0.999f + 0.001f;
                x[(k + 1) & 7] = x[(k + 1) & 7] * 0.998f + 0.002f;
            }
        }
        if ((it & 255) == 255)
            for (int q = 0; q < 4; q++) c[q] *= 0.5f;  // keep the accumulators bounded
    }
    float s = 0;
    for (int i = 0; i < 8; i++) s += x[i];
    for (int q = 0; q < 4; q++)
        for (int i = 0; i < 16; i++) s += c[q][i];
    out[blockIdx.x * THREADS + threadIdx.x] = s;
}

template <int SHAPE, bool MIX>
static double run(float* out, const half8* ops, double sustain_s) {
    auto k = k_probe<SHAPE, MIX>;
    hipLaunchKernelGGL(k, dim3(BLOCKS), dim3(THREADS), 0, 0, out, ops);
    CK(hipDeviceSynchronize());
    const auto t0 = std::chrono::steady_clock::now();
    while (std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() < sustain_s) {
        for (int r = 0; r < 10; r++) hipLaunchKernelGGL(k, dim3(BLOCKS), dim3(THREADS), 0, 0, out, ops);
        CK(hipDeviceSynchronize());
    }
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    const int reps = 20;
    CK(hipEventRecord(e0));
    for (int r = 0; r < reps; r++) hipLaunchKernelGGL(k, dim3(BLOCKS), dim3(THREADS), 0, 0, out, ops);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    CK(hipGetLastError());
    const double flops = (double)BLOCKS * (THREADS / 64) * NIT * 8 * 32768.0 * reps;
    return flops / (ms * 1e-3) / 1e12;
}

int main(int argc, char** argv) {
    const double sustain = argc > 1 ? atof(argv[1]) : 0.3;
    half8* ops;
    float* out;
    CK(hipMalloc(&ops, NOPS * sizeof(half8)));
    CK(hipMalloc(&out, BLOCKS * THREADS * sizeof(float)));
    static half8 h[NOPS];
    srand(1);
    for (int i = 0; i < NOPS; i++)
        for (int e = 0; e < 8; e++) h[i][e] = (_Float16)((rand() / (float)RAND_MAX) * 2 - 1);
    CK(hipMemcpy(ops, h, sizeof(h), hipMemcpyHostToDevice));
    const double m32 = run<32, false>(out, ops, sustain);
    const double m16 = run<16, false>(out, ops, sustain);
    const double x32 = run<32, true>(out, ops, sustain);
    CK(hipMemset(ops, 0, NOPS * sizeof(half8)));
    const double z32 = run<32, false>(out, ops, sustain);
    printf("{\"mfma32_tflops\": %.1f, \"mfma16_tflops\": %.1f, \"mix32_tflops\": %.1f, \"mfma32_zero_tflops\": %.1f}\n",
           m32, m16, x32, z32);
    return 0;
}
