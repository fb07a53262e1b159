// Bandwidth-bound kernels around the attention call: per-head RMSNorm, rotate-half RoPE, NAG combine,
// and the exact fp32 attention used when the fp16 path does not apply (causal, Dh != 128, fp32 mode).
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "internal.hpp"

namespace kiln {

// Full-wave reductions on the VALU, the result in every lane: DPP within rows of 16 lanes (quad swaps, half-row
// and row mirrors), then v_permlane16_swap and v_permlane32_swap across rows (no LDS round trips).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float swap16(float v, bool mx) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return mx ? fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])) : __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap32(float v, bool mx) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return mx ? fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])) : __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    return swap32(swap16(v, false), false);
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return swap32(swap16(v, true), true);
}
// block of 256 threads (4 waves); red must hold 4 floats
__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}
__device__ __forceinline__ float block_max256(float v, float* red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// ---- RMSNorm over rows of `dim` (engine/src/kernels.cu:656-666): one wave per row ----
__global__ __launch_bounds__(256) void k_rmsnorm_rows(float* y, const float* x, const uint16_t* w, int rows, int dim,
                                                      float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * dim;
    float* yr = y + (size_t)row * dim;
    float s = 0.f;
    for (int i = lane; i < dim; i += 64) s += xr[i] * xr[i];
    const float r = rsqrtf(wave_sum(s) / (float)dim + eps);
    for (int i = lane; i < dim; i += 64) yr[i] = xr[i] * r * (w ? bf16_to_f32(w[i]) : 1.f);
}

hipError_t launch_rmsnorm_rows(float* y, const float* x, const uint16_t* w, int rows, int dim, float eps, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3((rows + 3) / 4), dim3(256), 0, s, y, x, w, rows, dim, eps);
    return hipGetLastError();
}

__device__ __forceinline__ float ldv(const float* p) { return *p; }
__device__ __forceinline__ float ldv(const _Float16* p) { return (float)*p; }
__device__ __forceinline__ void stv(float* p, float v) { *p = v; }
__device__ __forceinline__ void stv(_Float16* p, float v) { *p = (_Float16)v; }

// ---- modulated LayerNorm of the DiT block (engine/src/kernels.cu:678-697): one wave per row ----
// y = (x - mean) * rsqrt(var + eps) * (1 + scale) + shift, mean and var over the row (two passes, as the
// reference). Rows of up to 64 lanes x NC float4 chunks stay in registers: one HBM read, one write.
__device__ __forceinline__ void st4(float* p, floatx4 v) { *reinterpret_cast<floatx4*>(p) = v; }
__device__ __forceinline__ void st4(_Float16* p, floatx4 v) {
    half4 h = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    *reinterpret_cast<half4*>(p) = h;
}

// A wave normalizes LN_RPW consecutive rows with the modulation vectors loaded once (per row they would be twice
// the row's own bytes in L2 reads; 6912 x 2048 fp16 out: 15.4 -> 14.4 us against one row per wave).
constexpr int LN_RPW = 4;
template <typename OutT, int NC>
__global__ __launch_bounds__(256) void k_layernorm_mod_rows(OutT* y, const float* x, const float* scale,
                                                            const float* shift, int rows, int dim, float eps) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * LN_RPW;
    if (row0 >= rows) return;
    const int nc = dim / 4;
    floatx4 v[NC], sc[NC], sh[NC];  // a row and the modulation; the row's loads issued before its reductions
#pragma unroll
    for (int k = 0; k < NC; k++) {
        const int c = min(lane + 64 * k, nc - 1);
        sc[k] = *reinterpret_cast<const floatx4*>(scale + 4 * c);
        sh[k] = *reinterpret_cast<const floatx4*>(shift + 4 * c);
    }
    for (int row = row0; row < min(row0 + LN_RPW, rows); row++) {
    const float* xr = x + (size_t)row * dim;
    OutT* yr = y + (size_t)row * dim;
#pragma unroll
    for (int k = 0; k < NC; k++) {
        const int c = min(lane + 64 * k, nc - 1);
        v[k] = *reinterpret_cast<const floatx4*>(xr + 4 * c);
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NC; k++)
        if (lane + 64 * k < nc) s += (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]);
    const float mean = wave_sum(s) / (float)dim;
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < NC; k++)
        if (lane + 64 * k < nc)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float d = v[k][e] - mean;
                q += d * d;
            }
    const float r = rsqrtf(wave_sum(q) / (float)dim + eps);
#pragma unroll
    for (int k = 0; k < NC; k++) {
        const int c = lane + 64 * k;
        if (c < nc) {
            floatx4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = (v[k][e] - mean) * r * (1.f + sc[k][e]) + sh[k][e];
            st4(yr + 4 * c, o);
        }
    }
    }
}

// any dim / alignment: three passes over the row (the second and third hit the cache)
template <typename OutT>
__global__ __launch_bounds__(256) void k_layernorm_mod_any(OutT* y, const float* x, const float* scale,
                                                           const float* shift, int rows, int dim, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + (size_t)row * dim;
    OutT* yr = y + (size_t)row * dim;
    float s = 0.f;
    for (int i = lane; i < dim; i += 64) s += xr[i];
    const float mean = wave_sum(s) / (float)dim;
    float q = 0.f;
    for (int i = lane; i < dim; i += 64) {
        const float d = xr[i] - mean;
        q += d * d;
    }
    const float r = rsqrtf(wave_sum(q) / (float)dim + eps);
    for (int i = lane; i < dim; i += 64) stv(yr + i, (xr[i] - mean) * r * (1.f + scale[i]) + shift[i]);
}

template <typename OutT>
static hipError_t layernorm_mod_sel(OutT* y, const float* x, const float* scale, const float* shift, int rows, int dim,
                                    float eps, bool vec, hipStream_t s) {
    const dim3 grid((rows + 3) / 4), block(256), grid_rows((rows + 4 * LN_RPW - 1) / (4 * LN_RPW));
    const int nc = dim / 4;
    if (vec && nc <= 64 * 2) hipLaunchKernelGGL((k_layernorm_mod_rows<OutT, 2>), grid_rows, block, 0, s, y, x, scale, shift, rows, dim, eps);
    else if (vec && nc <= 64 * 4) hipLaunchKernelGGL((k_layernorm_mod_rows<OutT, 4>), grid_rows, block, 0, s, y, x, scale, shift, rows, dim, eps);
    else if (vec && nc <= 64 * 8) hipLaunchKernelGGL((k_layernorm_mod_rows<OutT, 8>), grid_rows, block, 0, s, y, x, scale, shift, rows, dim, eps);
    else if (vec && nc <= 64 * 16) hipLaunchKernelGGL((k_layernorm_mod_rows<OutT, 16>), grid_rows, block, 0, s, y, x, scale, shift, rows, dim, eps);
    else hipLaunchKernelGGL((k_layernorm_mod_any<OutT>), grid, block, 0, s, y, x, scale, shift, rows, dim, eps);
    return hipGetLastError();
}

hipError_t launch_layernorm_mod(void* y, DT out, const float* x, const float* scale, const float* shift, int rows,
                                int dim, float eps, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    const size_t osz = out == DT::F16 ? 2 : 4;
    auto al = [](const void* p, size_t a) { return ((uintptr_t)p % a) == 0; };
    const bool vec = dim % 4 == 0 && al(x, 16) && al(scale, 16) && al(shift, 16) && al(y, 4 * osz);
    if (out == DT::F16) return layernorm_mod_sel((_Float16*)y, x, scale, shift, rows, dim, eps, vec, s);
    return layernorm_mod_sel((float*)y, x, scale, shift, rows, dim, eps, vec, s);
}

// ---- gated residual (engine/src/kernels.cu:700-708): x += (gate ? gate[col] : 1) * y ----
__global__ __launch_bounds__(256) void k_add_gated4(float* x, const float* y, const float* gate, size_t n4, int dim4) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    floatx4 a = reinterpret_cast<floatx4*>(x)[i];
    const floatx4 b = reinterpret_cast<const floatx4*>(y)[i];
    const floatx4 g = gate ? reinterpret_cast<const floatx4*>(gate)[i % dim4] : floatx4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int e = 0; e < 4; e++) a[e] += g[e] * b[e];
    reinterpret_cast<floatx4*>(x)[i] = a;
}
__global__ __launch_bounds__(256) void k_add_gated1(float* x, const float* y, const float* gate, size_t n, int dim) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] += (gate ? gate[i % dim] : 1.f) * y[i];
}

hipError_t launch_add_gated(float* x, const float* y, const float* gate, int rows, int dim, hipStream_t s) {
    const size_t n = (size_t)rows * dim;
    if (n == 0) return hipSuccess;
    auto al = [](const void* p) { return ((uintptr_t)p % 16) == 0; };
    if (dim % 4 == 0 && al(x) && al(y) && (!gate || al(gate))) {
        const size_t n4 = n / 4;
        hipLaunchKernelGGL(k_add_gated4, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, x, y, gate, n4, dim / 4);
    } else {
        hipLaunchKernelGGL(k_add_gated1, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, y, gate, n, dim);
    }
    return hipGetLastError();
}

// ---- rotate-half RoPE (engine/src/kernels.cu:759-772): one thread per rotated pair ----
__global__ __launch_bounds__(256) void k_rope_half(float* x, int T, int H, int Dh, const float* ct, const float* st) {
    const int half = Dh / 2;
    const size_t n = (size_t)T * H * half;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const int i = (int)(idx % half);
    const size_t th = idx / half;
    const int t = (int)(th / H);
    float* p = x + th * Dh;
    const float c = ct[(size_t)t * half + i], sn = st[(size_t)t * half + i];
    const float a = p[i], b = p[i + half];
    p[i] = a * c - b * sn;
    p[i + half] = b * c + a * sn;
}

hipError_t launch_rope_half(float* x, int T, int H, int Dh, const float* c, const float* sn, hipStream_t s) {
    const size_t n = (size_t)T * H * (Dh / 2);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_rope_half, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, T, H, Dh, c, sn);
    return hipGetLastError();
}

// ---- NAG combine (engine/src/dit.cu:295-324): one block per token row, fp32 arithmetic ----

template <typename T>
__global__ __launch_bounds__(256) void k_nag(T* a, int lda, const T* an, int ldn, int dim, float s, float tau,
                                             float alpha) {
    __shared__ float red[4];
    T* p = a + (size_t)blockIdx.x * lda;
    const T* n = an + (size_t)blockIdx.x * ldn;
    float lp = 0.f, lg = 0.f;
    for (int i = threadIdx.x; i < dim; i += 256) {
        const float pi = ldv(p + i);
        const float g = pi * s - ldv(n + i) * (s - 1.f);
        lp += fabsf(pi);
        lg += fabsf(g);
    }
    const float tp = block_sum256(lp, red);
    const float tg = block_sum256(lg, red);
    const float ratio = tg / fmaxf(tp, 1e-12f);
    const float k = ratio > tau ? tau / ratio : 1.f;
    for (int i = threadIdx.x; i < dim; i += 256) {
        const float pi = ldv(p + i);
        const float g = pi * s - ldv(n + i) * (s - 1.f);
        stv(p + i, alpha * g * k + (1.f - alpha) * pi);
    }
}

// Row-per-wave NAG for rows of up to 64 x 8 x NAG_CH elements in 16-byte-aligned chunks of 8: every lane
// loads its chunks once (vector loads), the two L1 sums are wave reductions, and the blend is computed from
// the registers (one read pass instead of two).
constexpr int NAG_CH = 4;
template <typename T>
__global__ __launch_bounds__(256) void k_nag_rows(T* a, int lda, const T* an, int ldn, int T_, int dim, float s,
                                                  float tau, float alpha) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T_) return;
    T* p = a + (size_t)row * lda;
    const T* n = an + (size_t)row * ldn;
    float pv[NAG_CH][8], nv[NAG_CH][8], g[NAG_CH][8];
    // all loads issued before any use (chunks past the row re-read its first chunk and are masked)
#pragma unroll
    for (int c = 0; c < NAG_CH; c++) {
        const int i = (c * 64 + lane) * 8 < dim ? (c * 64 + lane) * 8 : 0;
        load8(p + i, pv[c]);
        load8(n + i, nv[c]);
    }
    float lp = 0.f, lg = 0.f;
#pragma unroll
    for (int c = 0; c < NAG_CH; c++) {
        const bool in = (c * 64 + lane) * 8 < dim;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            g[c][e] = pv[c][e] * s - nv[c][e] * (s - 1.f);
            lp += in ? fabsf(pv[c][e]) : 0.f;
            lg += in ? fabsf(g[c][e]) : 0.f;
        }
    }
    lp = wave_sum(lp);
    lg = wave_sum(lg);
    const float ratio = lg / fmaxf(lp, 1e-12f);
    const float k = ratio > tau ? tau / ratio : 1.f;
#pragma unroll
    for (int c = 0; c < NAG_CH; c++) {
        const int i = (c * 64 + lane) * 8;
        if (i < dim) {
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = alpha * g[c][e] * k + (1.f - alpha) * pv[c][e];
            if constexpr (std::is_same<T, float>::value) {
                *reinterpret_cast<floatx4*>(p + i) = floatx4{o[0], o[1], o[2], o[3]};
                *reinterpret_cast<floatx4*>(p + i + 4) = floatx4{o[4], o[5], o[6], o[7]};
            } else {
                *reinterpret_cast<half8*>(p + i) = to_half8(o);
            }
        }
    }
}

hipError_t launch_nag(void* a, int lda, const void* an, int ldn, DT dt, int T, int dim, float sc, float tau,
                      float alpha, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    const size_t esz = dt == DT::F16 ? 2 : 4;
    const bool vec = dim % 8 == 0 && dim <= 64 * 8 * NAG_CH && ((uintptr_t)a % 16) == 0 && ((uintptr_t)an % 16) == 0 &&
                     ((size_t)lda * esz) % 16 == 0 && ((size_t)ldn * esz) % 16 == 0;
    if (vec) {
        if (dt == DT::F16)
            hipLaunchKernelGGL(k_nag_rows<_Float16>, dim3((T + 3) / 4), dim3(256), 0, s, (_Float16*)a, lda,
                               (const _Float16*)an, ldn, T, dim, sc, tau, alpha);
        else
            hipLaunchKernelGGL(k_nag_rows<float>, dim3((T + 3) / 4), dim3(256), 0, s, (float*)a, lda, (const float*)an,
                               ldn, T, dim, sc, tau, alpha);
        return hipGetLastError();
    }
    if (dt == DT::F16)
        hipLaunchKernelGGL(k_nag<_Float16>, dim3(T), dim3(256), 0, s, (_Float16*)a, lda, (const _Float16*)an, ldn, dim,
                           sc, tau, alpha);
    else
        hipLaunchKernelGGL(k_nag<float>, dim3(T), dim3(256), 0, s, (float*)a, lda, (const float*)an, ldn, dim, sc, tau,
                           alpha);
    return hipGetLastError();
}

// ---- exact fp32 attention: one block per (query, head), keys in chunks with an online softmax ----
// Semantics of the reference's fp32 fallback (engine/src/kernels.cu:809-866): s = (q.k)/sqrt(Dh),
// causal limit key <= query, with npad the max starts at 0 and npad*exp(-m) joins the denominator.
constexpr int EX_CH = 256;
__global__ __launch_bounds__(256) void k_exact_attn(float* out, int ldo, const float* q, int ldq, const float* k,
                                                    int ldk, const float* v, int ldv, int Tk, int Dh, int causal,
                                                    int npad, float scale) {
    __shared__ float qs[256];
    __shared__ float ps[EX_CH];
    __shared__ float red[4];
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const float* qr = q + (size_t)t * ldq + (size_t)h * Dh;
    for (int d = tid; d < Dh; d += 256) qs[d] = qr[d];
    __syncthreads();
    const int lim = causal ? min(t + 1, Tk) : Tk;
    float m = npad ? 0.f : -INFINITY, l = 0.f, acc = 0.f;
    for (int c0 = 0; c0 < lim; c0 += EX_CH) {
        const int j = c0 + tid;
        float sj = -INFINITY;
        if (tid < EX_CH && j < lim) {
            const float* kr = k + (size_t)j * ldk + (size_t)h * Dh;
            float a = 0.f;
            for (int d = 0; d < Dh; d++) a += qs[d] * kr[d];
            sj = a * scale;
        }
        const float cm = block_max256(sj, red);
        const float mn = fmaxf(m, cm);
        const float corr = expf(m - mn);
        m = mn;
        const float pj = (j < lim) ? expf(sj - m) : 0.f;
        ps[tid] = pj;
        const float psum = block_sum256(pj, red);
        l = l * corr + psum;
        acc *= corr;
        __syncthreads();
        if (tid < Dh) {
            const int n = min(EX_CH, lim - c0);
            const float* vr = v + (size_t)c0 * ldv + (size_t)h * Dh + tid;
            for (int jj = 0; jj < n; jj++) acc += ps[jj] * vr[(size_t)jj * ldv];
        }
        __syncthreads();
    }
    if (npad) l += (float)npad * expf(-m);
    if (tid < Dh) out[(size_t)t * ldo + (size_t)h * Dh + tid] = acc / l;
}

// ---- the same for Dh = 128 on the fp32 matrix cores (v_mfma_f32_16x16x4_f32: fp32 products and sums, as the
// reference's cuBLAS SGEMM fallback computes them) with an online softmax over 32-key tiles ----
// Workgroup = 4 waves x 32 query rows of one head. Per 16-key block a wave computes S^T = K Q^T for its two 16-row
// query blocks (32 MFMAs each, over d = 32g + s in lane group g and step s) and O^T += V^T P^T (8 d blocks x 4
// steps): P^T comes straight out of the S^T accumulators (lane group g holds keys 4g + i, i = 0..3, of query
// lane & 15; step kk takes element kk, and the V^T operand of lane (g, dd) is row 4g + kk of the block at
// d = 8 dd + db, so the output accumulator db holds d = 32g + 8i + db). K/V tiles are staged in LDS as fp32 with
// 132-float rows (conflict-free operand reads), two stages.
constexpr int X_KT = 32, X_RS = 132, X_BM = 128;
constexpr int X_STAGE = 2 * X_KT * X_RS;  // floats: K then V

__global__ __launch_bounds__(256, 2) void k_exact_attn128(float* out, int ldo, const float* q, int ldq,
                                                          const float* k, int ldk, const float* v, int ldv, int Tq,
                                                          int Tk, int causal, int npad, float scale) {
    extern __shared__ __attribute__((aligned(16))) float xs[];  // 2 stages
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int g = lane >> 4, n = lane & 15;
    const int h = blockIdx.y, q0 = blockIdx.x * X_BM + wv * 32;
    // Q operands: query block qb, row q0 + 16 qb + n, d = 32 g .. 32 g + 31 (rows past Tq read row Tq - 1)
    float qo[2][32];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const float* qr = q + (size_t)min(q0 + 16 * qb + n, Tq - 1) * ldq + (size_t)h * 128 + 32 * g;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const floatx4 t = *reinterpret_cast<const floatx4*>(qr + 4 * c);
#pragma unroll
            for (int e = 0; e < 4; e++) qo[qb][4 * c + e] = t[e];
        }
    }
    // the tile loads of this thread: row tid / 8 of the tile, floats 16 (tid % 8) .. + 16, of K and of V
    const int lr = tid >> 3, lc = (tid & 7) * 16;
    floatx4 kr[4], vr[4];
    auto load = [&](int t) {  // keys past Tk read the last key and are zeroed (no divergent branch)
        const int key = t * X_KT + lr;
        const bool in = key < Tk;
        const float* kp = k + (size_t)min(key, Tk - 1) * ldk + (size_t)h * 128 + lc;
        const float* vp = v + (size_t)min(key, Tk - 1) * ldv + (size_t)h * 128 + lc;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const floatx4 a = *reinterpret_cast<const floatx4*>(kp + 4 * c);
            const floatx4 b = *reinterpret_cast<const floatx4*>(vp + 4 * c);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                kr[c][e] = in ? a[e] : 0.f;
                vr[c][e] = in ? b[e] : 0.f;
            }
        }
    };
    auto store = [&](int st) {
        float* ks = xs + st * X_STAGE;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            *reinterpret_cast<floatx4*>(ks + lr * X_RS + lc + 4 * c) = kr[c];
            *reinterpret_cast<floatx4*>(ks + X_KT * X_RS + lr * X_RS + lc + 4 * c) = vr[c];
        }
    };
    // causal: no key past the last query row of the workgroup
    const int kend = causal ? min(Tk, blockIdx.x * X_BM + X_BM) : Tk;
    const int nt = (kend + X_KT - 1) / X_KT;
    floatx4 o[2][8];
    float m[2], l[2];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
#pragma unroll
        for (int db = 0; db < 8; db++) o[qb][db] = floatx4{0.f, 0.f, 0.f, 0.f};
        m[qb] = npad ? 0.f : -INFINITY;  // with padding keys the max starts at their score, 0
        l[qb] = 0.f;
    }
    if (nt > 0) {
        load(0);
        store(0);
        if (nt > 1) load(1);
    }
    for (int t = 0; t < nt; t++) {
        __syncthreads();  // tile t stored by every thread
        const float* ks = xs + (t & 1) * X_STAGE;
        const float* vs = ks + X_KT * X_RS;
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            floatx4 sc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
            const float* krow = ks + (kb * 16 + n) * X_RS + 32 * g;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const floatx4 ka = *reinterpret_cast<const floatx4*>(krow + 4 * c);
#pragma unroll
                for (int e = 0; e < 4; e++)
#pragma unroll
                    for (int qb = 0; qb < 2; qb++)
                        sc[qb] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[e], qo[qb][4 * c + e], sc[qb], 0, 0, 0);
            }
            float pr[2][4];
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                const int row = q0 + 16 * qb + n;
                float bm = -INFINITY;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int key = t * X_KT + kb * 16 + 4 * g + i;
                    const bool in = key < Tk && (!causal || key <= row);
                    sc[qb][i] = in ? sc[qb][i] * scale : -INFINITY;
                    bm = fmaxf(bm, sc[qb][i]);
                }
                bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
                bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
                const float mn = fmaxf(m[qb], bm);
                const float corr = mn == -INFINITY ? 1.f : expf(m[qb] - mn);
                m[qb] = mn;
                l[qb] *= corr;
#pragma unroll
                for (int db = 0; db < 8; db++) o[qb][db] *= corr;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    pr[qb][i] = sc[qb][i] == -INFINITY ? 0.f : expf(sc[qb][i] - mn);
                    l[qb] += pr[qb][i];
                }
            }
            // O^T += V^T P^T: step kk takes key 4g + kk of the block in lane group g
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const float* vrow = vs + (kb * 16 + 4 * g + kk) * X_RS + 8 * n;
                const floatx4 va = *reinterpret_cast<const floatx4*>(vrow);
                const floatx4 vb = *reinterpret_cast<const floatx4*>(vrow + 4);
#pragma unroll
                for (int qb = 0; qb < 2; qb++)
#pragma unroll
                    for (int db = 0; db < 8; db++)
                        o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(db < 4 ? va[db] : vb[db - 4], pr[qb][kk],
                                                                         o[qb][db], 0, 0, 0);
            }
        }
        if (t + 1 < nt) {
            store((t + 1) & 1);  // its stage's tile t-1 was read before this iteration's barrier
            if (t + 2 < nt) load(t + 2);
        }
    }
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        float lt = l[qb] + __shfl_xor(l[qb], 16, 64);
        lt += __shfl_xor(lt, 32, 64);
        if (npad) lt += (float)npad * expf(-m[qb]);
        const float inv = 1.f / lt;
        const int row = q0 + 16 * qb + n;
        if (row >= Tq) continue;
        float* orow = out + (size_t)row * ldo + (size_t)h * 128 + 32 * g;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            floatx4 a, b;
#pragma unroll
            for (int db = 0; db < 4; db++) {
                a[db] = o[qb][db][i] * inv;
                b[db] = o[qb][db + 4][i] * inv;
            }
            *reinterpret_cast<floatx4*>(orow + 8 * i) = a;
            *reinterpret_cast<floatx4*>(orow + 8 * i + 4) = b;
        }
    }
}

hipError_t launch_exact_attn(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                             int ldv, int Tq, int Tk, int H, int Dh, bool causal, int npad, hipStream_t s) {
    if (Tq <= 0 || H <= 0) return hipSuccess;
    const auto a16 = [](const void* p) { return ((uintptr_t)p % 16) == 0; };
    if (Dh == 128 && Tk > 0 && a16(q) && a16(k) && a16(v) && a16(out) && ldq % 4 == 0 && ldk % 4 == 0 &&
        ldv % 4 == 0 && ldo % 4 == 0) {
        hipLaunchKernelGGL(k_exact_attn128, dim3((Tq + X_BM - 1) / X_BM, H), dim3(256),
                           (size_t)2 * X_STAGE * sizeof(float), s, out, ldo, q, ldq, k, ldk, v, ldv, Tq, Tk,
                           causal ? 1 : 0, npad, 1.f / sqrtf(128.f));
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_exact_attn, dim3(Tq, H), dim3(256), 0, s, out, ldo, q, ldq, k, ldk, v, ldv, Tk, Dh,
                       causal ? 1 : 0, npad, 1.f / sqrtf((float)Dh));
    return hipGetLastError();
}

// rows x cols 16-bit units of a strided matrix set to zero (the output of a call with only padding keys). A
// kernel rather than hipMemset2DAsync, so a call can be captured into a HIP graph.
__global__ void k_zero_rows(uint16_t* out, size_t ld, size_t cols, int rows) {
    const size_t n = cols * (size_t)rows;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[(i / cols) * ld + i % cols] = 0;
}

hipError_t launch_zero_rows(void* out, size_t ld_bytes, size_t row_bytes, int rows, hipStream_t s) {
    if (rows <= 0 || row_bytes == 0) return hipSuccess;
    if (ld_bytes % 2 || row_bytes % 2 || (uintptr_t)out % 2) return hipErrorInvalidValue;
    const size_t n = row_bytes / 2 * (size_t)rows;
    const int blocks = (int)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_zero_rows, dim3(blocks), dim3(256), 0, s, static_cast<uint16_t*>(out), ld_bytes / 2,
                       row_bytes / 2, rows);
    return hipGetLastError();
}

}  // namespace kiln
