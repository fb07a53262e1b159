// The DiT forward's small passes around the transformer blocks (gfx950): per-step modulation matvecs with bf16
// weights, SiLU, patch embedding layout (patchify / unpatchify), the fp32 linear layers with bf16 weights
// (x embedder, final layer) and the CFG combine. Each is HBM- or launch-bound; none is on the attention path.
//
// Contracts (the reference's, engine/src/kernels.cu and engine/src/dit.cu):
//   matvec       y[r] = sum_c W[r][c] x[c] (+ add[r]), W bf16 [rows, cols]        kernels.cu k_matvec
//   silu         y = v / (1 + exp(-v))                                               kernels.cu:735-739
//   patchify     tok [T, 68] from a 16-channel latent [16, Hl, Wl], 2x2 patches      dit.cu:174-182
//   unpatchify   latent [16, Hl, Wl] from tok [T, 64]                                dit.cu:184-191
//   linear_f32   y [T, rows] = x [T, cols] W^T, W bf16 [rows, cols], fp32 MFMA      kernels.cu:508-529 (linear)
//   cfg_combine  v = vn + cfg (v - vn)                                              kernels.cu:1058-1062
#include <algorithm>

#include "common.hpp"
#include "internal.hpp"

namespace kiln {

// One wave per row: 16-byte bf16 loads striding the row, fp32 partial sums, a wave reduction. Grouped form:
// rows [g*grows, (g+1)*grows) read input vector x + g*xstride and add[row - g*grows] (xstride = 0: one x).
__global__ __launch_bounds__(256) void k_matvec_bf16(float* __restrict__ y, const uint16_t* __restrict__ W,
                                                     const float* __restrict__ x, const float* __restrict__ add,
                                                     int rows, int cols, int grows, int xstride) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int grp = row / grows;
    x += (size_t)grp * xstride;
    const uint16_t* w = W + (size_t)row * cols;
    float s = 0.f;
    if ((cols & 7) == 0 && ((size_t)w & 15) == 0 && ((size_t)x & 15) == 0) {
        for (int c = lane * 8; c < cols; c += 64 * 8) {
            const u32x4 raw = *reinterpret_cast<const u32x4*>(w + c);
            const floatx4 xa = *reinterpret_cast<const floatx4*>(x + c);
            const floatx4 xb = *reinterpret_cast<const floatx4*>(x + c + 4);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                s += __uint_as_float(raw[e] << 16) * (e < 2 ? xa[2 * e] : xb[2 * e - 4]);
                s += __uint_as_float(raw[e] & 0xffff0000u) * (e < 2 ? xa[2 * e + 1] : xb[2 * e - 3]);
            }
        }
    } else {
        for (int c = lane; c < cols; c += 64) s += bf16_to_f32(w[c]) * x[c];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) y[row] = s + (add ? add[row - grp * grows] : 0.f);
}

// cols == 256 (the adaLN second layers): a row is 512 bytes, so a wave takes 8 rows, 4 per half wave, every load of
// the 4 rows in flight together (one row per wave would leave half the lanes idle and one load per lane in flight)
__global__ __launch_bounds__(256) void k_matvec_bf16_256(float* __restrict__ y, const uint16_t* __restrict__ W,
                                                         const float* __restrict__ x, const float* __restrict__ add,
                                                         int rows, int grows, int xstride) {
    const int lane = threadIdx.x & 63, half = lane >> 5, l32 = lane & 31;
    const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + half * 4;
    u32x4 raw[4];
    floatx4 xa[4], xb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = min(r0 + i, rows - 1);
        const float* xr = x + (size_t)(row / grows) * xstride + l32 * 8;
        raw[i] = *reinterpret_cast<const u32x4*>(W + (size_t)row * 256 + l32 * 8);
        xa[i] = *reinterpret_cast<const floatx4*>(xr);
        xb[i] = *reinterpret_cast<const floatx4*>(xr + 4);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            s += __uint_as_float(raw[i][e] << 16) * (e < 2 ? xa[i][2 * e] : xb[i][2 * e - 4]);
            s += __uint_as_float(raw[i][e] & 0xffff0000u) * (e < 2 ? xa[i][2 * e + 1] : xb[i][2 * e - 3]);
        }
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        const int row = r0 + i;
        if (l32 == 0 && row < rows) y[row] = s + (add ? add[row % grows] : 0.f);
    }
}

__global__ void k_silu(float* __restrict__ y, const float* __restrict__ x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float v = x[i];
        y[i] = v / (1.f + expf(-v));
    }
}

// tok[t][f], f = 4c + 2m + nn: channel c (< 16; channel 16 is the all-zero padding mask), patch row m, column nn
__global__ void k_patchify(float* __restrict__ tok, const float* __restrict__ lat, int Hl, int Wl) {
    const int Wp = Wl / 2, T = (Hl / 2) * Wp;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)T * 68) return;
    const int f = (int)(i % 68), t = (int)(i / 68);
    const int c = f >> 2, m = (f >> 1) & 1, nn = f & 1;
    const int yy = (t / Wp) * 2 + m, xx = (t % Wp) * 2 + nn;
    tok[i] = c < 16 ? lat[((size_t)c * Hl + yy) * Wl + xx] : 0.f;
}

// tok[t][f], f = 32 p1 + 16 p2 + c
__global__ void k_unpatchify(float* __restrict__ lat, const float* __restrict__ tok, int ldt, int Hl, int Wl) {
    const int Wp = Wl / 2, T = (Hl / 2) * Wp;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)T * 64) return;
    const int f = (int)(i & 63), t = (int)(i >> 6);
    const int p1 = f >> 5, p2 = (f >> 4) & 1, c = f & 15;
    const int yy = (t / Wp) * 2 + p1, xx = (t % Wp) * 2 + p2;
    lat[((size_t)c * Hl + yy) * Wl + xx] = tok[(size_t)t * ldt + f];
}

// y [T, rows] (row stride ldy) = x [T, cols] (row stride ldx) W^T on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32: fp32 products, fp32 accumulation). One wave per 16 rows x 64 output columns; k in
// chunks of 32: lane (i = lane % 16, g = lane / 16) holds x[i][k0 + 8g .. 8g + 8) and, for each of the 4 column
// blocks, W[j = i][k0 + 8g .. 8g + 8), and MFMA step s of the chunk takes element s of both (the same k on the
// A and the B side). Out-of-range rows and k read as 0.
__global__ __launch_bounds__(256) void k_linear_f32(float* __restrict__ y, int ldy, const float* __restrict__ x,
                                                    int ldx, const uint16_t* __restrict__ W, int T, int rows, int cols) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nt = (rows + 63) / 64;
    const int t0 = (wave / nt) * 16, n0 = (wave % nt) * 64;
    if (t0 >= T) return;
    const int i = lane & 15, g = lane >> 4;
    const int tr = t0 + i;
    const float* xr = x + (size_t)min(tr, T - 1) * ldx;
    floatx4 acc[4] = {};
    const uint16_t* wr[4];
    bool nin[4];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
        const int n = n0 + nb * 16 + i;
        nin[nb] = n < rows;
        wr[nb] = W + (size_t)min(n, rows - 1) * cols;
    }
    // vector loads (16 bytes of x, 16 bytes of W per lane and block) for whole chunks when rows are 16-byte
    // aligned; element loads with bounds for the tail chunk and unaligned rows
    const bool vec = ((cols & 7) == 0) && ((ldx & 3) == 0) && (((size_t)x & 15) == 0) && (((size_t)W & 15) == 0);
    const int kfull = vec ? cols / 32 * 32 : 0;
    float xa[2][8], wv[2][4][8];
    auto load = [&](int k0, float(&xo)[8], float(&wo)[4][8]) {
        const int kb = k0 + 8 * g;
        const floatx4 a0 = *reinterpret_cast<const floatx4*>(xr + kb);
        const floatx4 a1 = *reinterpret_cast<const floatx4*>(xr + kb + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            xo[e] = tr < T ? a0[e] : 0.f;
            xo[e + 4] = tr < T ? a1[e] : 0.f;
        }
#pragma unroll
        for (int nb = 0; nb < 4; nb++) {
            const u32x4 raw = *reinterpret_cast<const u32x4*>(wr[nb] + kb);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                wo[nb][2 * e] = nin[nb] ? __uint_as_float(raw[e] << 16) : 0.f;
                wo[nb][2 * e + 1] = nin[nb] ? __uint_as_float(raw[e] & 0xffff0000u) : 0.f;
            }
        }
    };
    auto mma = [&](const float(&xo)[8], const float(&wo)[4][8]) {
#pragma unroll
        for (int e = 0; e < 8; e++)
#pragma unroll
            for (int nb = 0; nb < 4; nb++) acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xo[e], wo[nb][e], acc[nb], 0, 0, 0);
    };
    int k0 = 0;
    if (kfull > 0) {
        load(0, xa[0], wv[0]);
        for (; k0 + 32 < kfull; k0 += 64) {  // the next chunk's loads in flight during this chunk's MFMAs
            load(k0 + 32, xa[1], wv[1]);
            mma(xa[0], wv[0]);
            if (k0 + 64 < kfull) load(k0 + 64, xa[0], wv[0]);
            mma(xa[1], wv[1]);
        }
        if (k0 < kfull) {
            mma(xa[0], wv[0]);
            k0 += 32;
        }
    }
    for (; k0 < cols; k0 += 32) {
        const int kb = k0 + 8 * g;
        float xo[8], wo[4][8];
#pragma unroll
        for (int e = 0; e < 8; e++) xo[e] = (tr < T && kb + e < cols) ? xr[kb + e] : 0.f;
#pragma unroll
        for (int nb = 0; nb < 4; nb++)
#pragma unroll
            for (int e = 0; e < 8; e++) wo[nb][e] = (nin[nb] && kb + e < cols) ? bf16_to_f32(wr[nb][kb + e]) : 0.f;
        mma(xo, wo);
    }
    // lane holds column n0 + nb*16 + i of rows t0 + 4g + r
#pragma unroll
    for (int nb = 0; nb < 4; nb++) {
        const int n = n0 + nb * 16 + i;
        if (n >= rows) continue;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int t = t0 + 4 * g + r;
            if (t < T) y[(size_t)t * ldy + n] = acc[nb][r];
        }
    }
}

__global__ void k_cfg_combine(float* __restrict__ v, const float* __restrict__ vn, float cfg, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) v[i] = vn[i] + cfg * (v[i] - vn[i]);
}

// flow-matching sampler (engine/src/pipeline.cu:304-331): the start x = s noise + (1 - s) init, and one Euler step
// of the velocity v in the reference's arithmetic: den = x - v s, then x + (x - den) / s (sn - s)
__global__ void k_flow_start(float* __restrict__ x, const float* __restrict__ noise, const float* __restrict__ init,
                             float s, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = s * noise[i] + (init ? (1.f - s) * init[i] : 0.f);
}
__global__ void k_flow_euler(float* __restrict__ x, const float* __restrict__ v, float s, float sn, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float xi = x[i], den = xi - v[i] * s;
        x[i] = xi + (xi - den) / s * (sn - s);
    }
}

// k_euler_step on a given denoised estimate (the masked path): the same expression as k_flow_euler
__global__ void k_flow_euler_den(float* __restrict__ x, const float* __restrict__ den, float s, float sn, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float xi = x[i];
        x[i] = xi + (xi - den[i]) / s * (sn - s);
    }
}

// latents [16, H, W] with an odd side go through the forward on the 2x2 patch grid: circular padding to
// [16, Hd, Wd] and a crop back (engine/src/dit.cu:342-370)
__global__ void k_pad_circular(float* __restrict__ dst, const float* __restrict__ src, int Hs, int Ws, int Hd, int Wd) {
    const size_t n = (size_t)16 * Hd * Wd;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int x = (int)(i % Wd), y = (int)((i / Wd) % Hd);
    const size_t c = i / ((size_t)Wd * Hd);
    dst[i] = src[(c * Hs + y % Hs) * Ws + x % Ws];
}
__global__ void k_crop(float* __restrict__ dst, const float* __restrict__ src, int Hs, int Ws, int Hd, int Wd) {
    const size_t n = (size_t)16 * Hd * Wd;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int x = (int)(i % Wd), y = (int)((i / Wd) % Hd);
    const size_t c = i / ((size_t)Wd * Hd);
    dst[i] = src[(c * Hs + y) * Ws + x];
}

// Synthetic weights: p[i] = bf16(lo + (hi - lo) u_i), u_i in [0, 1) from a counter-based hash of (seed, i)
// (SplitMix64's finalizer, a published 64-bit mixer), so a weight set is a pure function of its seed.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
__global__ void k_fill_uniform_bf16(uint16_t* __restrict__ p, size_t n, uint64_t seed, float lo, float hi) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const uint64_t h = mix64(seed * 0x9e3779b97f4a7c15ULL + i + 1);
        const float u = (float)(h >> 40) * (1.0f / 16777216.0f);
        const float v = lo + (hi - lo) * u;
        uint32_t bits = __float_as_uint(v);
        bits += 0x7FFF + ((bits >> 16) & 1);  // round to nearest even
        p[i] = (uint16_t)(bits >> 16);
    }
}

// first-block step cache (engine/src/dit.cu:327-340): y = a - b, and the relative L1 change sum|a - b| / sum|b|
// as two sums (acc[0], acc[1]) that the host divides
__global__ void k_sub(float* __restrict__ y, const float* __restrict__ a, const float* __restrict__ b, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = a[i] - b[i];
}
__global__ void k_zero2(float* acc) {
    if (threadIdx.x < 2) acc[threadIdx.x] = 0.f;
}
__global__ __launch_bounds__(256) void k_rel_l1(const float* __restrict__ a, const float* __restrict__ b, size_t n,
                                                float* acc) {
    float d = 0.f, r = 0.f;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        d += fabsf(a[i] - b[i]);
        r += fabsf(b[i]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        d += __shfl_xor(d, o, 64);
        r += __shfl_xor(r, o, 64);
    }
    if ((threadIdx.x & 63) == 0) {
        atomicAdd(acc, d);
        atomicAdd(acc + 1, r);
    }
}

// the sampler's denoised estimate without a mask (pipeline.cu:318-324) and the generic sampler step
// x <- a x + b den + c old (pipeline.cu:333-337, k_update; old may be null)
__global__ void k_flow_denoised(float* __restrict__ den, const float* __restrict__ x, const float* __restrict__ v,
                                float s, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) den[i] = x[i] - v[i] * s;
}
__global__ void k_flow_update(float* __restrict__ x, const float* __restrict__ den, const float* __restrict__ old,
                              float a, float b, float c, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = a * x[i] + b * den[i] + (old ? c * old[i] : 0.f);
}

// inpainting (pipeline.cu:309-324): the model input regenerates where m = 1 and is the init re-noised to this
// sigma where m = 0; the denoised estimate is pinned to the init outside the mask. mask [P] per pixel of the
// 16-channel latent [16, P].
__global__ void k_flow_inpaint_in(float* __restrict__ xin, const float* __restrict__ x, const float* __restrict__ noise,
                                  const float* __restrict__ init, const float* __restrict__ mask, float s, int P) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)16 * P) return;
    const float m = mask[i % P];
    xin[i] = m * x[i] + (1.f - m) * (s * noise[i] + (1.f - s) * init[i]);
}
__global__ void k_flow_denoised_masked(float* __restrict__ den, const float* __restrict__ xin,
                                       const float* __restrict__ v, const float* __restrict__ init,
                                       const float* __restrict__ mask, float s, int P) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)16 * P) return;
    const float d = xin[i] - v[i] * s, m = mask[i % P];
    den[i] = m * d + (1.f - m) * init[i];
}

// GELU in place, fp32 (kernels.cu:728-733, the fp32 branch's MLP activation): erf form with the device erff
__global__ void k_gelu(float* __restrict__ x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float v = x[i];
        x[i] = 0.5f * v * (1.f + erff(v * 0.70710678118654752f));
    }
}

// er_sde update of the latent (the per-element part of pipeline.cu:345-359; weights from the host): with the
// first divided difference D1 = (den - old) d1_inv, which is also kept for the next step, and the second
// D2 = (D1 - D1_prev) d2_inv,
//   x <- x_w x + den_w den [+ d1_w D1 [+ d2_w D2]] [+ noise_w noise]
// ORDER (1-3) selects the terms at compile time. Four elements per thread through 16-byte accesses; the
// launcher takes this form only when every array is 16-byte aligned, and a second launch covers n % 4.
struct ErSdeW {
    float x_w, den_w, d1_w, d1_inv, d2_w, d2_inv, noise_w;
};
template <int ORDER, bool NOISE, int V>
__global__ void k_flow_ersde(float* __restrict__ x, const float* __restrict__ den, const float* __restrict__ old,
                             float* __restrict__ d1_keep, const float* __restrict__ noise, const ErSdeW w, size_t nv) {
    typedef float vec __attribute__((ext_vector_type(V)));
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nv) return;
    const vec dv = reinterpret_cast<const vec*>(den)[t];
    vec acc = reinterpret_cast<const vec*>(x)[t] * w.x_w + dv * w.den_w;
    if constexpr (ORDER >= 2) {
        const vec d1 = (dv - reinterpret_cast<const vec*>(old)[t]) * w.d1_inv;
        acc += d1 * w.d1_w;
        if constexpr (ORDER >= 3) acc += ((d1 - reinterpret_cast<const vec*>(d1_keep)[t]) * w.d2_inv) * w.d2_w;
        reinterpret_cast<vec*>(d1_keep)[t] = d1;
    }
    if constexpr (NOISE) acc += reinterpret_cast<const vec*>(noise)[t] * w.noise_w;
    reinterpret_cast<vec*>(x)[t] = acc;
}

template <int ORDER, bool NOISE>
static void launch_ersde_order(float* x, const float* den, const float* old, float* d1, const float* noise,
                               const ErSdeW& w, size_t n, bool vec4, hipStream_t st) {
    size_t done = 0;
    if (vec4 && n >= 4) {
        const size_t nv = n / 4;
        hipLaunchKernelGGL((k_flow_ersde<ORDER, NOISE, 4>), dim3((unsigned)((nv + 255) / 256)), dim3(256), 0, st, x, den,
                           old, d1, noise, w, nv);
        done = nv * 4;
    }
    if (done < n) {
        auto off = [&](auto* p) { return p ? p + done : p; };
        hipLaunchKernelGGL((k_flow_ersde<ORDER, NOISE, 1>), dim3((unsigned)((n - done + 255) / 256)), dim3(256), 0, st,
                           x + done, den + done, off(old), off(d1), off(noise), w, n - done);
    }
}

static unsigned nblk(size_t n) { return (unsigned)((n + 255) / 256); }

hipError_t launch_matvec_bf16(float* y, const uint16_t* W, const float* x, const float* add, int rows, int cols,
                              int groups, hipStream_t s) {
    const int grows = rows, xstride = groups > 1 ? cols : 0;
    if (cols == 256 && ((size_t)W & 15) == 0 && ((size_t)x & 15) == 0) {
        const int total = rows * groups;
        hipLaunchKernelGGL(k_matvec_bf16_256, dim3((total + 31) / 32), dim3(256), 0, s, y, W, x, add, total, grows,
                           xstride);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_matvec_bf16, dim3((rows * groups + 3) / 4), dim3(256), 0, s, y, W, x, add, rows * groups,
                       cols, grows, xstride);
    return hipGetLastError();
}
hipError_t launch_silu(float* y, const float* x, size_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_silu, dim3(nblk(n)), dim3(256), 0, s, y, x, n);
    return hipGetLastError();
}
hipError_t launch_patchify(float* tok, const float* lat, int Hl, int Wl, hipStream_t s) {
    const size_t n = (size_t)(Hl / 2) * (Wl / 2) * 68;
    hipLaunchKernelGGL(k_patchify, dim3(nblk(n)), dim3(256), 0, s, tok, lat, Hl, Wl);
    return hipGetLastError();
}
hipError_t launch_unpatchify(float* lat, const float* tok, int ldt, int Hl, int Wl, hipStream_t s) {
    const size_t n = (size_t)(Hl / 2) * (Wl / 2) * 64;
    hipLaunchKernelGGL(k_unpatchify, dim3(nblk(n)), dim3(256), 0, s, lat, tok, ldt, Hl, Wl);
    return hipGetLastError();
}
// The same product for the DiT's large fp32 linears (K a multiple of 32, 16-byte aligned rows): workgroup tile 64
// rows x 128 output columns, k chunks of 32 staged in LDS (x as fp32, W as bf16, rows padded so the 16 rows of an
// operand read land in distinct banks), two stages, the next chunk's global loads in registers during the current
// chunk's MFMAs; 4 waves as 2 x 2, each 32 rows x 64 columns (2 x 4 blocks of v_mfma_f32_16x16x4_f32), the k
// mapping of k_linear_f32 (lane group g holds k 8g .. 8g + 8 of the chunk, step s takes element s).
constexpr int LF_BM = 64, LF_BN = 128, LF_BK = 32;
constexpr int LF_XS = 36;  // x row stride in LDS, floats (144 bytes)
constexpr int LF_WS = 40;  // W row stride in LDS, bf16 (80 bytes)
constexpr int LF_XB = LF_BM * LF_XS * 4, LF_STAGE = LF_XB + LF_BN * LF_WS * 2;

__global__ __launch_bounds__(256, 2) void k_linear_f32t(float* __restrict__ y, int ldy, const float* __restrict__ x,
                                                        int ldx, const uint16_t* __restrict__ W, int T, int rows,
                                                        int cols) {
    __shared__ __attribute__((aligned(16))) unsigned char sm[2 * LF_STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wr = wv >> 1, wc = wv & 1, i = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.x * LF_BM, n0 = blockIdx.y * LF_BN;
    // this thread's global pieces of a chunk: x rows f / 8 (f = tid + 256 r), 4 floats at 4 (f % 8); W rows f / 4,
    // 8 bf16 at 8 (f % 4); rows past the matrix read its last row (results unused)
    const float* xp[2];
    const uint16_t* wp[2];
    uint32_t xo_l[2], wo_l[2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int f = tid + 256 * r;
        xp[r] = x + (size_t)min(m0 + f / 8, T - 1) * ldx + 4 * (f % 8);
        xo_l[r] = (uint32_t)(((f / 8) * LF_XS + 4 * (f % 8)) * 4);
        wp[r] = W + (size_t)min(n0 + f / 4, rows - 1) * cols + 8 * (f % 4);
        wo_l[r] = (uint32_t)(LF_XB + ((f / 4) * LF_WS + 8 * (f % 4)) * 2);
    }
    floatx4 xr[2];
    u32x4 wr4[2];
    auto load = [&](int kc) {
#pragma unroll
        for (int r = 0; r < 2; r++) {
            xr[r] = *reinterpret_cast<const floatx4*>(xp[r] + kc * LF_BK);
            wr4[r] = *reinterpret_cast<const u32x4*>(wp[r] + kc * LF_BK);
        }
    };
    auto store = [&](int st) {
        unsigned char* b = sm + st * LF_STAGE;
#pragma unroll
        for (int r = 0; r < 2; r++) {
            *reinterpret_cast<floatx4*>(b + xo_l[r]) = xr[r];
            *reinterpret_cast<u32x4*>(b + wo_l[r]) = wr4[r];
        }
    };
    floatx4 acc[2][4] = {};
    const int nk = cols / LF_BK;
    load(0);
    store(0);
    __syncthreads();
    for (int kc = 0; kc < nk; kc++) {
        if (kc + 1 < nk) load(kc + 1);
        const unsigned char* b = sm + (kc & 1) * LF_STAGE;
        float xo[2][8], wo[4][8];
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
            const float* xs = reinterpret_cast<const float*>(b) + (32 * wr + 16 * rb + i) * LF_XS + 8 * g;
            const floatx4 a = *reinterpret_cast<const floatx4*>(xs), c = *reinterpret_cast<const floatx4*>(xs + 4);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                xo[rb][e] = a[e];
                xo[rb][e + 4] = c[e];
            }
        }
#pragma unroll
        for (int cb = 0; cb < 4; cb++) {
            const u32x4 raw = *reinterpret_cast<const u32x4*>(
                reinterpret_cast<const uint16_t*>(b + LF_XB) + (64 * wc + 16 * cb + i) * LF_WS + 8 * g);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                wo[cb][2 * e] = __uint_as_float(raw[e] << 16);
                wo[cb][2 * e + 1] = __uint_as_float(raw[e] & 0xffff0000u);
            }
        }
#pragma unroll
        for (int st = 0; st < 8; st++)
#pragma unroll
            for (int rb = 0; rb < 2; rb++)
#pragma unroll
                for (int cb = 0; cb < 4; cb++)
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xo[rb][st], wo[cb][st], acc[rb][cb], 0, 0, 0);
        if (kc + 1 < nk) store((kc + 1) & 1);  // its stage's chunk kc-1 was read before the last barrier
        __syncthreads();
    }
    // lane holds column n0 + 64 wc + 16 cb + i of rows m0 + 32 wr + 16 rb + 4 g + r
#pragma unroll
    for (int cb = 0; cb < 4; cb++) {
        const int n = n0 + 64 * wc + 16 * cb + i;
        if (n >= rows) continue;
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = m0 + 32 * wr + 16 * rb + 4 * g + r;
                if (t < T) y[(size_t)t * ldy + n] = acc[rb][cb][r];
            }
    }
}

hipError_t launch_linear_f32(float* y, int ldy, const float* x, int ldx, const uint16_t* W, int T, int rows, int cols,
                             hipStream_t s) {
    if (cols % LF_BK == 0 && ldx % 4 == 0 && ((size_t)x & 15) == 0 && ((size_t)W & 15) == 0 && T >= LF_BM &&
        rows >= LF_BN) {
        hipLaunchKernelGGL(k_linear_f32t, dim3((T + LF_BM - 1) / LF_BM, (rows + LF_BN - 1) / LF_BN), dim3(256), 0, s,
                           y, ldy, x, ldx, W, T, rows, cols);
        return hipGetLastError();
    }
    const long waves = (long)((T + 15) / 16) * ((rows + 63) / 64);
    hipLaunchKernelGGL(k_linear_f32, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, y, ldy, x, ldx, W, T, rows,
                       cols);
    return hipGetLastError();
}
hipError_t launch_cfg_combine(float* v, const float* vn, float cfg, size_t n, hipStream_t s) {
    hipLaunchKernelGGL(k_cfg_combine, dim3(nblk(n)), dim3(256), 0, s, v, vn, cfg, n);
    return hipGetLastError();
}

hipError_t launch_flow_start(float* x, const float* noise, const float* init, float s, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_flow_start, dim3(nblk(n)), dim3(256), 0, st, x, noise, init, s, n);
    return hipGetLastError();
}
hipError_t launch_flow_euler(float* x, const float* v, float s, float sn, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_flow_euler, dim3(nblk(n)), dim3(256), 0, st, x, v, s, sn, n);
    return hipGetLastError();
}

hipError_t launch_flow_euler_den(float* x, const float* den, float s, float sn, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_flow_euler_den, dim3(nblk(n)), dim3(256), 0, st, x, den, s, sn, n);
    return hipGetLastError();
}

hipError_t launch_pad_circular(float* dst, const float* src, int Hs, int Ws, int Hd, int Wd, hipStream_t st) {
    const size_t n = (size_t)16 * Hd * Wd;
    hipLaunchKernelGGL(k_pad_circular, dim3(nblk(n)), dim3(256), 0, st, dst, src, Hs, Ws, Hd, Wd);
    return hipGetLastError();
}
hipError_t launch_crop(float* dst, const float* src, int Hs, int Ws, int Hd, int Wd, hipStream_t st) {
    const size_t n = (size_t)16 * Hd * Wd;
    hipLaunchKernelGGL(k_crop, dim3(nblk(n)), dim3(256), 0, st, dst, src, Hs, Ws, Hd, Wd);
    return hipGetLastError();
}

hipError_t launch_fill_uniform_bf16(uint16_t* p, size_t n, uint64_t seed, float lo, float hi, hipStream_t st) {
    const int blocks = (int)std::min<size_t>((n + 255) / 256, 8192);
    hipLaunchKernelGGL(k_fill_uniform_bf16, dim3(blocks), dim3(256), 0, st, p, n, seed, lo, hi);
    return hipGetLastError();
}

hipError_t launch_sub(float* y, const float* a, const float* b, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_sub, dim3(nblk(n)), dim3(256), 0, st, y, a, b, n);
    return hipGetLastError();
}
hipError_t launch_rel_l1(const float* a, const float* b, size_t n, float* acc, hipStream_t st) {
    hipLaunchKernelGGL(k_zero2, dim3(1), dim3(64), 0, st, acc);
    hipLaunchKernelGGL(k_rel_l1, dim3(512), dim3(256), 0, st, a, b, n, acc);
    return hipGetLastError();
}

hipError_t launch_flow_ersde(float* x, const float* den, const float* old, float* oldd, const float* noise, float a,
                             float b, float c2, float inv2, float c3, float inv3, float cn, int stage, size_t n,
                             hipStream_t st) {
    const ErSdeW w{a, b, c2, inv2, c3, inv3, cn};
    bool vec4 = true;
    for (const void* p : {(const void*)x, (const void*)den, (const void*)old, (const void*)oldd, (const void*)noise})
        vec4 &= ((uintptr_t)p & 15) == 0;
    const bool nz = noise != nullptr;
    auto go = [&](auto order) {
        constexpr int O = decltype(order)::value;
        if (nz) launch_ersde_order<O, true>(x, den, old, oldd, noise, w, n, vec4, st);
        else launch_ersde_order<O, false>(x, den, old, oldd, noise, w, n, vec4, st);
    };
    if (stage >= 3) go(std::integral_constant<int, 3>{});
    else if (stage == 2) go(std::integral_constant<int, 2>{});
    else go(std::integral_constant<int, 1>{});
    return hipGetLastError();
}
hipError_t launch_gelu(float* x, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_gelu, dim3(nblk(n)), dim3(256), 0, st, x, n);
    return hipGetLastError();
}
hipError_t launch_flow_inpaint_in(float* xin, const float* x, const float* noise, const float* init, const float* mask,
                                  float s, int P, hipStream_t st) {
    hipLaunchKernelGGL(k_flow_inpaint_in, dim3(nblk((size_t)16 * P)), dim3(256), 0, st, xin, x, noise, init, mask, s, P);
    return hipGetLastError();
}
hipError_t launch_flow_denoised_masked(float* den, const float* xin, const float* v, const float* init,
                                      const float* mask, float s, int P, hipStream_t st) {
    hipLaunchKernelGGL(k_flow_denoised_masked, dim3(nblk((size_t)16 * P)), dim3(256), 0, st, den, xin, v, init, mask,
                       s, P);
    return hipGetLastError();
}
hipError_t launch_flow_denoised(float* den, const float* x, const float* v, float s, size_t n, hipStream_t st) {
    hipLaunchKernelGGL(k_flow_denoised, dim3(nblk(n)), dim3(256), 0, st, den, x, v, s, n);
    return hipGetLastError();
}
hipError_t launch_flow_update(float* x, const float* den, const float* old, float a, float b, float c, size_t n,
                              hipStream_t st) {
    hipLaunchKernelGGL(k_flow_update, dim3(nblk(n)), dim3(256), 0, st, x, den, old, a, b, c, n);
    return hipGetLastError();
}

}  // namespace kiln
