// C++ harness in the shape of the reference's bench/tfa_test.cu: host Q,K ~ N(0,1.5), V ~ N(0,1) from
// std::mt19937(3), an fp32 reference computed here on the host (two passes per (query, head), as
// bench/tfa_test.cu:11-33 does on the GPU), kiln::attention / kiln::attention16 through the C ABI, and
// rel_l2 / max-abs / ms / TF per shape. Exit status 1 if any shape leaves the bars below; the error-path
// checks (throwing drop-in) run first.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "../../kiln_amd/host/kiln_gpu.hpp"

#define CK(x)                                                                              \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            std::exit(2);                                                                  \
        }                                                                                  \
    } while (0)

static void ref_attn(std::vector<float>& out, const std::vector<float>& q, const std::vector<float>& k,
                     const std::vector<float>& v, int T, int Tk, int H, int ld, int npad, int rows) {
    for (int t = 0; t < rows; t++)
        for (int h = 0; h < H; h++) {
            const float* qr = &q[(size_t)t * ld + h * 128];
            double m = npad ? 0.0 : -INFINITY;
            std::vector<double> s(Tk);
            for (int j = 0; j < Tk; j++) {
                double a = 0;
                for (int d = 0; d < 128; d++) a += (double)qr[d] * k[(size_t)j * ld + h * 128 + d];
                s[j] = a / std::sqrt(128.0);
                m = std::max(m, s[j]);
            }
            double l = npad * std::exp(-m), acc[128] = {0};
            for (int j = 0; j < Tk; j++) {
                double p = std::exp(s[j] - m);
                l += p;
                for (int d = 0; d < 128; d++) acc[d] += p * v[(size_t)j * ld + h * 128 + d];
            }
            for (int d = 0; d < 128; d++) out[(size_t)t * ld + h * 128 + d] = (float)(acc[d] / l);
        }
}

static float h2f(uint16_t h) {
    _Float16 x;
    std::memcpy(&x, &h, 2);
    return (float)x;
}

static bool run(int T, int Tk, int npad, const char* name, bool f16) {
    const int H = 16, ld = H * 128, rows = std::min(T, 256);
    std::mt19937 rng(3);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<float> Q((size_t)T * ld), K((size_t)Tk * ld), V((size_t)Tk * ld);
    for (auto& x : Q) x = nd(rng) * 1.5f;
    for (auto& x : K) x = nd(rng) * 1.5f;
    for (auto& x : V) x = nd(rng);
    float *dq, *dk, *dv, *o;
    CK(hipMalloc(&dq, Q.size() * 4));
    CK(hipMalloc(&dk, K.size() * 4));
    CK(hipMalloc(&dv, V.size() * 4));
    CK(hipMalloc(&o, Q.size() * 4));
    CK(hipMemcpy(dq, Q.data(), Q.size() * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(dk, K.data(), K.size() * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(dv, V.data(), V.size() * 4, hipMemcpyHostToDevice));
    auto go = [&] {
        if (f16) kiln::attention16((uint16_t*)o, ld, dq, ld, dk, ld, dv, ld, T, Tk, H, 128, npad);
        else kiln::attention(o, ld, dq, ld, dk, ld, dv, ld, T, Tk, H, 128, false, npad);
    };
    for (int i = 0; i < 3; i++) go();
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    CK(hipEventRecord(e0));
    const int reps = 10;
    for (int i = 0; i < reps; i++) go();
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    ms /= reps;
    std::vector<float> A((size_t)T * ld), B((size_t)T * ld);
    if (f16) {
        std::vector<uint16_t> Bh((size_t)T * ld);
        CK(hipMemcpy(Bh.data(), o, Bh.size() * 2, hipMemcpyDeviceToHost));
        for (size_t i = 0; i < Bh.size(); i++) B[i] = h2f(Bh[i]);
    } else {
        CK(hipMemcpy(B.data(), o, B.size() * 4, hipMemcpyDeviceToHost));
    }
    ref_attn(A, Q, K, V, T, Tk, H, ld, npad, rows);
    double num = 0, den = 0, mx = 0;
    for (size_t i = 0; i < (size_t)rows * ld; i++) {
        double d = B[i] - A[i];
        num += d * d;
        den += (double)A[i] * A[i];
        mx = std::max(mx, std::fabs(d));
    }
    double flop = 4.0 * T * Tk * 128 * H, rel = std::sqrt(num / den);
    // the reference publishes rel_l2 6.9e-4 for its tensor-core kernel (README.md:570) on these inputs
    bool ok = rel < 1.0e-3 && mx < 8e-3;
    printf("%s %-28s %7.3f ms  %6.1f TF  rel_l2 %.2e  max-abs %.2e  %s\n", f16 ? "attention16" : "attention  ", name, ms,
           flop / ms / 1e9, rel, mx, ok ? "ok" : "FAIL");
    CK(hipFree(dq));
    CK(hipFree(dk));
    CK(hipFree(dv));
    CK(hipFree(o));
    return ok;
}

int main() {
    // error behaviour of the drop-in: an unsupported head size throws like the reference's attention16
    bool threw = false;
    try {
        kiln::attention16(nullptr, 1024, nullptr, 1024, nullptr, 1024, nullptr, 1024, 8, 8, 16, 64);
    } catch (const std::runtime_error& e) {
        threw = true;
        printf("attention16(Dh=64) throws: %s\n", e.what());
    }
    if (!threw) return 1;
    bool ok = true;
    for (int f16 = 0; f16 < 2; f16++) {
        ok &= run(1536, 1536, 0, "self  512x768 (1536 tok)", f16);
        ok &= run(3952, 3952, 0, "self  832x1216 (3952 tok)", f16);
        ok &= run(1536, 26, 486, "cross 26 real + 486 pad", f16);
        ok &= run(1000, 1000, 0, "self  ragged 1000 tok", f16);
        ok &= run(1000, 77, 0, "cross ragged 77 keys", f16);
    }
    return ok ? 0 : 1;
}
