/*
 * CPU oracle for the fused attention path (DiT self-attention with QK-RMSNorm + 3D RoPE,
 * text cross-attention with zero-padded context keys, NAG blend).
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker: only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it. The product path (kiln_amd/libkiln_attn.so) never links,
 * loads or falls back to it.
 *
 * Every function restates the reference algorithm it names (paths relative to the reference
 * repository root). Pinning status of each function (what independent check fixes it) is stated
 * in its comment; the checks live in tests/test_oracle.py.
 *
 * Layout convention (same as the reference op layer, engine/src/gpu.h:149-153): row-major
 * [T, ld] matrices, head h occupies columns [h*Dh, (h+1)*Dh).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------ */
/* fp16 / bf16 helpers (IEEE binary16, round-to-nearest-even, as __floats2half2_rn)            */
/* ------------------------------------------------------------------------------------------ */

static inline float f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = s;
        else { /* subnormal: m * 2^-24 */
            float f = (float)m * 5.9604644775390625e-08f;
            memcpy(&bits, &f, 4);
            bits |= s;
        }
    } else if (e == 31) bits = s | 0x7f800000u | (m << 13);
    else bits = s | ((e + 112) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t s = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(s | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0)); /* inf/nan */
    if (ax >= 0x477ff000u) return (uint16_t)(s | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) { /* below 2^-14: subnormal or zero, RNE at 2^-24 */
        float a;
        memcpy(&a, &ax, 4);
        float q = a * 16777216.0f; /* exact scaling by 2^24 */
        float r = nearbyintf(q);   /* default rounding mode: nearest-even */
        return (uint16_t)(s | (uint16_t)r);
    }
    uint32_t mant = ax & 0x7fffffu, exp = (ax >> 23) - 112;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) h++;
    return (uint16_t)(s | h);
}

static inline float bf16_to_f32(uint16_t b) {
    uint32_t bits = (uint32_t)b << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float round_f16(float f) { return f16_to_f32(f32_to_f16(f)); }

void oracle_f32_to_f16(uint16_t* dst, const float* src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = f32_to_f16(src[i]);
}
void oracle_f16_to_f32(float* dst, const uint16_t* src, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = f16_to_f32(src[i]);
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------------------------ */
/* Attention                                                                                   */
/* ------------------------------------------------------------------------------------------ */

/*
 * The reference's fp32 ground truth, restated line for line from the one-thread-per-(query,
 * head) two-pass kernel ref_attn (bench/flash_test.cu:10-32, identical in bench/tfa_test.cu:11-33):
 *   m = npad ? 0 : -inf;  m = max over keys of (q.k)/sqrt(128)      (fp32 dot products)
 *   l = npad * exp(-m);   l += exp(s - m), acc += p * v               (fp32)
 *   out = acc / l
 * Dh is a parameter here (the reference hard-codes 128). Used as the CPU baseline of the bench
 * (kind "port"). Pinned by tests/test_oracle.py against torch float64 softmax attention and
 * against the appended-zero-key identity for npad.
 */
void oracle_ref_attn_f32(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                         int ldv, int Tq, int Tk, int H, int Dh, int npad) {
    const float rs = sqrtf((float)Dh);
    long n = (long)Tq * H;
#pragma omp parallel for schedule(dynamic, 16)
    for (long i = 0; i < n; i++) {
        int t = (int)(i / H), h = (int)(i % H);
        const float* qr = q + (size_t)t * ldq + (size_t)h * Dh;
        float m = npad ? 0.f : -INFINITY;
        for (int j = 0; j < Tk; j++) {
            const float* kr = k + (size_t)j * ldk + (size_t)h * Dh;
            float s = 0.f;
            for (int d = 0; d < Dh; d++) s += qr[d] * kr[d];
            m = fmaxf(m, s / rs);
        }
        float acc[512];
        for (int d = 0; d < Dh; d++) acc[d] = 0.f;
        float l = (float)npad * expf(-m);
        for (int j = 0; j < Tk; j++) {
            const float* kr = k + (size_t)j * ldk + (size_t)h * Dh;
            const float* vr = v + (size_t)j * ldv + (size_t)h * Dh;
            float s = 0.f;
            for (int d = 0; d < Dh; d++) s += qr[d] * kr[d];
            float p = expf(s / rs - m);
            l += p;
            for (int d = 0; d < Dh; d++) acc[d] += p * vr[d];
        }
        float* o = out + (size_t)t * ldo + (size_t)h * Dh;
        for (int d = 0; d < Dh; d++) o[d] = acc[d] / l;
    }
}

/*
 * Same algorithm with double accumulation: the golden "fp32 reference" every parity test measures
 * max-abs / mean-abs error against. Optional causal mask (key j visible to query t iff j <= t),
 * the reference's exact-mode fallback semantics (engine/src/kernels.cu:809-826: causal limit,
 * npad term with m = max(m, 0)). scale <= 0 selects 1/sqrt(Dh).
 */
void oracle_attn_f64(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v, int ldv,
                     int Tq, int Tk, int H, int Dh, int causal, int npad, double scale) {
    if (scale <= 0) scale = 1.0 / sqrt((double)Dh);
    long n = (long)Tq * H;
#pragma omp parallel for schedule(dynamic, 16)
    for (long i = 0; i < n; i++) {
        int t = (int)(i / H), h = (int)(i % H);
        int lim = causal ? (t + 1 < Tk ? t + 1 : Tk) : Tk;
        const float* qr = q + (size_t)t * ldq + (size_t)h * Dh;
        double* s = (double*)malloc(sizeof(double) * (size_t)(lim > 0 ? lim : 1));
        double m = npad ? 0.0 : -INFINITY;
        for (int j = 0; j < lim; j++) {
            const float* kr = k + (size_t)j * ldk + (size_t)h * Dh;
            double a = 0.0;
            for (int d = 0; d < Dh; d++) a += (double)qr[d] * (double)kr[d];
            s[j] = a * scale;
            if (s[j] > m) m = s[j];
        }
        double acc[512];
        for (int d = 0; d < Dh; d++) acc[d] = 0.0;
        double l = npad ? (double)npad * exp(-m) : 0.0;
        for (int j = 0; j < lim; j++) {
            const float* vr = v + (size_t)j * ldv + (size_t)h * Dh;
            double p = exp(s[j] - m);
            l += p;
            for (int d = 0; d < Dh; d++) acc[d] += p * (double)vr[d];
        }
        float* o = out + (size_t)t * ldo + (size_t)h * Dh;
        for (int d = 0; d < Dh; d++) o[d] = (float)(acc[d] / l);
        free(s);
    }
}

/*
 * Emulator of the reference's fp16 tensor-core semantics (engine/src/tcflash.cuh:33-156), Dh=128:
 *   - Q scaled by qscale = log2(e)/sqrt(128) in fp32, then rounded to fp16 (RN-even)  (:38)
 *   - K, V rounded to fp16                                                              (:62-63)
 *   - S = Q K^T with fp32 accumulation                                                  (:67-80)
 *   - keys streamed in tiles of 64; base-2 online softmax: m' = max(m, tile max),
 *     corr = 2^(m - m'), p = 2^(s - m'), P rounded to fp16, l = l*corr + sum(p) (fp32 p) (:82-115)
 *   - O = O*corr + P V. The reference accumulates PV in fp16 over 32 keys (a GeForce speed trick,
 *     :117-133); this emulator accumulates in fp32, which is what the MI355X build does.
 *   - epilogue npad term: m' = max(m, 0), l = l*2^(m-m') + npad*2^(-m'), out = O*2^(m-m')/l (:136-155)
 *   - out16 != 0: the output is rounded to fp16 (attention16).
 * Inputs are fp32 (already normed/roped); out is fp32 holding the (possibly fp16-rounded) values.
 * Pinned against oracle_attn_f64: its error must sit inside the fp16 rounding budget and its
 * per-element deviations must be explained by those roundings (tests/test_oracle.py).
 */
void oracle_attn_f16sem(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v, int ldv,
                        int Tq, int Tk, int H, int npad, int out16) {
    const int D = 128, BC = 64;
    const float qscale = 1.4426950408889634f / sqrtf((float)D);
    long n = (long)Tq * H;
#pragma omp parallel for schedule(dynamic, 16)
    for (long i = 0; i < n; i++) {
        int t = (int)(i / H), h = (int)(i % H);
        float qh[128];
        const float* qr = q + (size_t)t * ldq + (size_t)h * D;
        for (int d = 0; d < D; d++) qh[d] = round_f16(qr[d] * qscale);
        float o[128];
        for (int d = 0; d < D; d++) o[d] = 0.f;
        float m = -INFINITY, l = 0.f;
        for (int k0 = 0; k0 < Tk; k0 += BC) {
            int nk = Tk - k0 < BC ? Tk - k0 : BC;
            float s[64], mx = -INFINITY;
            for (int j = 0; j < nk; j++) {
                const float* kr = k + (size_t)(k0 + j) * ldk + (size_t)h * D;
                float a = 0.f;
                for (int d = 0; d < D; d++) a += qh[d] * round_f16(kr[d]);
                s[j] = a;
                mx = fmaxf(mx, a);
            }
            float mn = fmaxf(m, mx);
            float corr = exp2f(m - mn);
            m = mn;
            float sum = 0.f;
            for (int d = 0; d < D; d++) o[d] *= corr;
            for (int j = 0; j < nk; j++) {
                float p = exp2f(s[j] - m);
                sum += p;
                float ph = round_f16(p);
                const float* vr = v + (size_t)(k0 + j) * ldv + (size_t)h * D;
                for (int d = 0; d < D; d++) o[d] += ph * round_f16(vr[d]);
            }
            l = l * corr + sum;
        }
        float scale = 1.f;
        if (npad) {
            float mn = fmaxf(m, 0.f);
            scale = exp2f(m - mn);
            l = l * scale + (float)npad * exp2f(-mn);
        }
        float inv = scale / l;
        float* dst = out + (size_t)t * ldo + (size_t)h * D;
        for (int d = 0; d < D; d++) dst[d] = out16 ? round_f16(o[d] * inv) : o[d] * inv;
    }
}

/* ------------------------------------------------------------------------------------------ */
/* QK-RMSNorm, rotate-half RoPE, Cosmos 3D RoPE tables                                          */
/* ------------------------------------------------------------------------------------------ */

/*
 * Per-row RMSNorm with bf16 weights (engine/src/kernels.cu:656-666, k_rmsnorm_warp):
 *   r = rsqrt(sum(x^2)/dim + eps);  y = x * r * w   (w == NULL -> 1)
 * rows = T*H when applied per head (engine/src/dit.cu:464-465). In place allowed.
 * Pinned: w=1 gives unit RMS per row; matches torch.nn.functional.rms_norm (tests).
 */
void oracle_rmsnorm_rows(float* y, const float* x, const uint16_t* w_bf16, long rows, int dim, float eps) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * dim;
        float* yr = y + (size_t)r * dim;
        float s = 0.f;
        for (int i = 0; i < dim; i++) s += xr[i] * xr[i];
        float rr = 1.0f / sqrtf(s / (float)dim + eps);
        for (int i = 0; i < dim; i++) yr[i] = xr[i] * rr * (w_bf16 ? bf16_to_f32(w_bf16[i]) : 1.f);
    }
}

/*
 * Modulated LayerNorm of the DiT block (engine/src/kernels.cu:678-697, k_layernorm_mod; called as
 * layernorm_mod / layernorm_mod16 at engine/src/dit.cu:460,474,491), per row of `dim`:
 *   mean = sum(x)/dim;  var = sum((x - mean)^2)/dim;  y = (x - mean) * rsqrt(var + eps) * (1 + scale) + shift
 * scale/shift are per column. fp32 arithmetic in the reference's order (two passes).
 * Pinned: equals torch layer_norm (no affine) * (1 + scale) + shift in float64; scale = shift = 0 gives
 * rows of mean 0 and variance 1.
 */
void oracle_layernorm_mod(float* y, const float* x, const float* scale, const float* shift, long rows, int dim,
                          float eps) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * dim;
        float* yr = y + (size_t)r * dim;
        float s = 0.f;
        for (int i = 0; i < dim; i++) s += xr[i];
        const float mean = s / (float)dim;
        float v = 0.f;
        for (int i = 0; i < dim; i++) {
            const float d = xr[i] - mean;
            v += d * d;
        }
        const float rr = 1.0f / sqrtf(v / (float)dim + eps);
        for (int i = 0; i < dim; i++) yr[i] = (xr[i] - mean) * rr * (1.f + scale[i]) + shift[i];
    }
}

/*
 * Gated residual (engine/src/kernels.cu:700-708, k_add_gated): x[r][i] += (gate ? gate[i] : 1) * y[r][i].
 * Pinned: gate = NULL is plain addition; gate = 0 leaves x unchanged.
 */
void oracle_add_gated(float* x, const float* y, const float* gate, long rows, int dim) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < rows; r++)
        for (int i = 0; i < dim; i++) x[(size_t)r * dim + i] += (gate ? gate[i] : 1.f) * y[(size_t)r * dim + i];
}

/*
 * fp16 linear layer with fused epilogue (engine/src/kernels.cu:573-609 linear16, kernel tc16::k_gemm16 with its
 * epilogue at engine/src/tcgemm16.cuh:145-175):
 *   acc[t][n] = sum_k x16[t][k] w16[n][k] + sum_k a2[t][k] w2[n][k]      (k2 = 0: no second product)
 * accumulated in double over the exact fp16 values, then by epi:
 *   0 F32:    y32[t][n] = acc + beta * y32[t][n]
 *   1 F16:    y16[t][n] = fp16(acc)
 *   2 GELU16: y16[t][n] = fp16(acc/2 (1 + erf(acc/sqrt 2)))      (the erf form, tcgemm16.cuh:55)
 *   3 RESID:  y32[t][n] = y32[t][n] + (gate ? gate[n] : 1) * acc
 * y rows have ldy elements. The reference accumulates 32-wide k tiles in fp16 (tcgemm16.cuh:6-7); the oracle is
 * the exact sum, which both the reference and the GPU path approximate.
 * Pinned: equals numpy float64 x @ w.T (+ a2 @ w2.T) on the same fp16 values; the LoRA product equals one
 * product over the concatenated [x | a2] and [w | w2]; GELU equals math.erf's closed form, with GELU(0) = 0 and
 * GELU(v) -> v for large v; RESID with gate = 0 leaves y unchanged.
 */
void oracle_linear16(float* y32, uint16_t* y16, int ldy, const uint16_t* x16, int T, const uint16_t* w16, int rows,
                     int cols, const uint16_t* a2, const uint16_t* w2, int k2, int epi, const float* gate, float beta) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++) {
        double* xr = (double*)malloc(sizeof(double) * (size_t)(cols + k2));
        for (int k = 0; k < cols; k++) xr[k] = f16_to_f32(x16[(size_t)t * cols + k]);
        for (int k = 0; k < k2; k++) xr[cols + k] = f16_to_f32(a2[(size_t)t * k2 + k]);
        for (int n = 0; n < rows; n++) {
            double acc = 0.0;
            for (int k = 0; k < cols; k++) acc += xr[k] * f16_to_f32(w16[(size_t)n * cols + k]);
            for (int k = 0; k < k2; k++) acc += xr[cols + k] * f16_to_f32(w2[(size_t)n * k2 + k]);
            const size_t o = (size_t)t * ldy + n;
            switch (epi) {
                case 0: y32[o] = (float)(acc + (double)beta * y32[o]); break;
                case 1: y16[o] = f32_to_f16((float)acc); break;
                case 2: y16[o] = f32_to_f16((float)(0.5 * acc * (1.0 + erf(acc * 0.70710678118654752440)))); break;
                default: y32[o] = (float)((double)y32[o] + (gate ? (double)gate[n] : 1.0) * acc); break;
            }
        }
        free(xr);
    }
}

/*
 * matvec with bf16 weights (engine/src/kernels.cu k_matvec, matvec at gpu.h:122): y[r] = sum_c W[r][c] x[c] (+ add[r]),
 * accumulated in double. Pinned: equals numpy float64 W @ x on the bf16 values.
 */
void oracle_matvec_bf16(float* y, const uint16_t* W, const float* x, const float* add, int rows, int cols) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        double s = 0.0;
        for (int c = 0; c < cols; c++) s += (double)bf16_to_f32(W[(size_t)r * cols + c]) * x[c];
        y[r] = (float)(s + (add ? add[r] : 0.0));
    }
}

/*
 * 2x2 patch embedding layout (engine/src/dit.cu:174-191). patchify: tok[t][4c + 2m + n] = lat[c][2(t / Wp) + m]
 * [2(t % Wp) + n] for c < 16, 0 for the padding-mask channel c = 16. unpatchify: lat[c][2(t / Wp) + p1][2(t % Wp)
 * + p2] = tok[t][32 p1 + 16 p2 + c]. Pinned: hand-computed positions; unpatchify of a patchify with the feature
 * order mapped from (c, m, n) to (m, n, c) returns the latent.
 */
void oracle_patchify(float* tok, const float* lat, int Hl, int Wl) {
    const int Wp = Wl / 2, T = (Hl / 2) * Wp;
    for (int t = 0; t < T; t++)
        for (int f = 0; f < 68; f++) {
            const int c = f / 4, m = (f / 2) % 2, n = f % 2;
            tok[(size_t)t * 68 + f] = c < 16 ? lat[((size_t)c * Hl + (t / Wp) * 2 + m) * Wl + (t % Wp) * 2 + n] : 0.f;
        }
}
void oracle_unpatchify(float* lat, const float* tok, int Hl, int Wl) {
    const int Wp = Wl / 2, T = (Hl / 2) * Wp;
    for (int t = 0; t < T; t++)
        for (int f = 0; f < 64; f++) {
            const int p1 = f / 32, p2 = (f / 16) % 2, c = f % 16;
            lat[((size_t)c * Hl + (t / Wp) * 2 + p1) * Wl + (t % Wp) * 2 + p2] = tok[(size_t)t * 64 + f];
        }
}

/*
 * fp32 linear layer with bf16 weights (engine/src/kernels.cu:508-529 linear, used for the x embedder and the final
 * layer, dit.cu:417,542): y[t][n] = sum_k x[t][k] W[n][k], accumulated in double. Pinned: numpy float64 x @ W.T.
 */
void oracle_linear_f32(float* y, const float* x, const uint16_t* W, int T, int rows, int cols) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; t++)
        for (int n = 0; n < rows; n++) {
            double s = 0.0;
            for (int k = 0; k < cols; k++) s += (double)x[(size_t)t * cols + k] * bf16_to_f32(W[(size_t)n * cols + k]);
            y[(size_t)t * rows + n] = (float)s;
        }
}

/*
 * Rotate-half RoPE (engine/src/kernels.cu:759-772, k_rope_half), in place on x [T, H*Dh]
 * (row stride ld elements), tables [T, Dh/2]:
 *   a = p[i], b = p[i+half];  p[i] = a*c - b*s;  p[i+half] = b*c + a*s
 * Pinned: equals multiplying (a + i b) by exp(i*theta) (complex rotation); preserves pair norms.
 */
void oracle_rope_half(float* x, int ld, int T, int H, int Dh, const float* cos_t, const float* sin_t) {
    int half = Dh / 2;
#pragma omp parallel for schedule(static)
    for (long t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            float* p = x + (size_t)t * ld + (size_t)h * Dh;
            for (int i = 0; i < half; i++) {
                float c = cos_t[(size_t)t * half + i], s = sin_t[(size_t)t * half + i];
                float a = p[i], b = p[i + half];
                p[i] = a * c - b * s;
                p[i + half] = b * c + a * s;
            }
        }
}

/*
 * Cosmos-Predict2 3D RoPE tables for one image (T=1), head dim 128 (engine/src/dit.cu:196-215):
 * dim_h = 128/6*2 = 42, dim_t = 44; ntk = 4^(42/40); h_theta = 1e4*ntk; hf[j] = 1/h_theta^(2j/42).
 * Columns [0,22): temporal (identity for T=1), [22,43): height y*hf[j], [43,64): width x*hf[j],
 * for token t = y*Wp + x. cos/sin [Hp*Wp, 64], fp32 with float libm like the reference.
 * Pinned against an independent float64 restatement of the published Cosmos
 * VideoRopePosition3DEmb frequencies (tests).
 */
void oracle_cosmos_rope(float* cos_t, float* sin_t, int Hp, int Wp) {
    const int DH = 128, dim_h = DH / 6 * 2, dim_t = DH - 2 * dim_h, half = DH / 2;
    double ntk = pow(4.0, (double)dim_h / (dim_h - 2));
    float h_theta = (float)(10000.0 * ntk);
    float hf[64];
    for (int j = 0; j < dim_h / 2; j++) hf[j] = 1.0f / powf(h_theta, (float)(2 * j) / (float)dim_h);
    int T = Hp * Wp;
    for (int t = 0; t < T; t++) {
        int y = t / Wp, xx = t % Wp;
        for (int i = 0; i < half; i++) {
            cos_t[(size_t)t * half + i] = 1.f;
            sin_t[(size_t)t * half + i] = 0.f;
        }
        for (int j = 0; j < dim_h / 2; j++) {
            float ah = (float)y * hf[j], aw = (float)xx * hf[j];
            cos_t[(size_t)t * half + dim_t / 2 + j] = cosf(ah);
            sin_t[(size_t)t * half + dim_t / 2 + j] = sinf(ah);
            cos_t[(size_t)t * half + dim_t / 2 + dim_h / 2 + j] = cosf(aw);
            sin_t[(size_t)t * half + dim_t / 2 + dim_h / 2 + j] = sinf(aw);
        }
    }
}

/* ------------------------------------------------------------------------------------------ */
/* NAG combine                                                                                 */
/* ------------------------------------------------------------------------------------------ */

/*
 * Normalized Attention Guidance combine, one token row at a time over all dim columns
 * (engine/src/dit.cu:295-324, k_nag; arithmetic in fp32):
 *   g = z+ * s - z- * (s - 1);  ratio = sum|g| / max(sum|z+|, 1e-12);  k = ratio > tau ? tau/ratio : 1
 *   a = alpha * g * k + (1 - alpha) * z+
 * a (z+) is overwritten in place. Row stride lda / ldn elements.
 * Pinned by a hand-computed row and by the s=1, alpha=0 and no-clamp invariants (tests).
 */
void oracle_nag(float* a, int lda, const float* an, int ldn, int T, int dim, float s, float tau, float alpha) {
#pragma omp parallel for schedule(static)
    for (long t = 0; t < T; t++) {
        float* p = a + (size_t)t * lda;
        const float* n = an + (size_t)t * ldn;
        double lp = 0, lg = 0;
        for (int i = 0; i < dim; i++) {
            float g = p[i] * s - n[i] * (s - 1.f);
            lp += fabsf(p[i]);
            lg += fabsf(g);
        }
        float ratio = (float)lg / fmaxf((float)lp, 1e-12f);
        float kk = ratio > tau ? tau / ratio : 1.f;
        for (int i = 0; i < dim; i++) {
            float pi = p[i];
            float g = pi * s - n[i] * (s - 1.f);
            p[i] = alpha * g * kk + (1.f - alpha) * pi;
        }
    }
}

/* ------------------------------------------------------------------------------------------ */
/* torch-compatible CPU randn                                                                  */
/* ------------------------------------------------------------------------------------------ */

/*
 * Bit-exact torch.manual_seed(seed); torch.randn(n) on the CPU (engine/src/pipeline.cu:17-64):
 * MT19937 seeded with the low 32 bits; 24-bit uniforms u = (r & 0xffffff) * 2^-24; Box-Muller in
 * blocks of 16 (u1 = 1 - d[j], u2 = d[j+8]); a ragged tail redraws the last 16 values.
 * Requires n >= 16 (the reference's layout; torch uses another path below 16).
 * Pinned against torch.randn in this container (tests/golden/randn_seed*.json).
 */
typedef struct { uint32_t s[624]; int idx; } mt_t;
static void mt_seed(mt_t* g, uint64_t seed) {
    g->s[0] = (uint32_t)(seed & 0xffffffffu);
    for (int j = 1; j < 624; j++) g->s[j] = 1812433253u * (g->s[j - 1] ^ (g->s[j - 1] >> 30)) + (uint32_t)j;
    g->idx = 624;
}
static uint32_t mt_next(mt_t* g) {
    if (g->idx >= 624) {
        for (int k = 0; k < 624; k++) {
            uint32_t y = (g->s[k] & 0x80000000u) | (g->s[(k + 1) % 624] & 0x7fffffffu);
            g->s[k] = g->s[(k + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        }
        g->idx = 0;
    }
    uint32_t y = g->s[g->idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}
static float mt_uniform(mt_t* g) { return (float)(mt_next(g) & ((1u << 24) - 1)) * (1.0f / (float)(1u << 24)); }
static void normal_fill_16(float* d) {
    for (int j = 0; j < 8; j++) {
        float u1 = 1.f - d[j], u2 = d[j + 8];
        float radius = sqrtf(-2.f * logf(u1));
        float theta = 2.0f * 3.14159265358979323846f * u2;
        d[j] = radius * cosf(theta);
        d[j + 8] = radius * sinf(theta);
    }
}
int oracle_torch_randn(float* d, uint64_t seed, size_t n) {
    if (n < 16) return -1;
    mt_t* g = (mt_t*)malloc(sizeof(mt_t));
    mt_seed(g, seed);
    for (size_t i = 0; i < n; i++) d[i] = mt_uniform(g);
    for (size_t i = 0; i + 16 <= n; i += 16) normal_fill_16(d + i);
    if (n % 16) {
        float* t = d + n - 16;
        for (int i = 0; i < 16; i++) t[i] = mt_uniform(g);
        normal_fill_16(t);
    }
    free(g);
    return 0;
}
