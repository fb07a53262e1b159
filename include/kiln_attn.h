/*
 * kiln_attn.h - C ABI of the MI355X (gfx950) fused attention path of Kiln's diffusion engine.
 *
 * One shared library, kiln_amd/libkiln_attn.so. Every entry point:
 *   - takes plain device pointers, element strides and sizes (no framework types);
 *   - enqueues work on the given HIP stream (NULL = the default stream) and never synchronizes;
 *   - returns a kiln_status (0 = OK); kiln_attn_last_error() gives a detail message for the
 *     calling thread. The C++ header kiln_amd/host/kiln_gpu.hpp turns non-zero codes into
 *     std::runtime_error, the reference op layer's error behaviour (engine/src/gpu.h:15-16,
 *     engine/src/kernels.cu:870).
 *
 * Layout contract (the reference's, engine/src/gpu.h:149-153): row-major [T, ld] matrices with the
 * row stride ld in elements; head h occupies columns [h*Dh, (h+1)*Dh). Rows must be 16-byte
 * aligned. Keys beyond Tk are never read; npad extra all-zero keys (K = 0, V = 0) are accounted for
 * analytically (they add npad*exp(-max) to the softmax denominator and nothing to the output).
 * The Dh = 128 flash path takes up to 2^22 keys per head (KILN_EUNSUPPORTED above; the reference's
 * longest context is 6144).
 *
 * fp16 values cross the ABI as uint16_t bit patterns (IEEE binary16), bf16 norm weights likewise.
 */
#ifndef KILN_ATTN_H
#define KILN_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* kiln_stream_t; /* identical to hipStream_t */

typedef enum {
    KILN_OK = 0,
    KILN_EINVAL = 1,       /* bad argument (null pointer, negative size, ...) */
    KILN_EUNSUPPORTED = 2, /* shape/stride/alignment this path does not take (reference: attention16 throws) */
    KILN_EHIP = 3,         /* a HIP runtime call or kernel launch failed */
    KILN_ENOMEM = 4        /* workspace allocation failed or the given workspace is too small */
} kiln_status;

typedef enum { KILN_F32 = 0, KILN_F16 = 1 } kiln_dtype;

const char* kiln_attn_status_string(int status);
const char* kiln_attn_last_error(void);
/* gfx target of device `dev` as "gfx950" etc.; returns KILN_EHIP if no device. */
int kiln_attn_device_arch(int dev, char* buf, int buflen);

/* ------------------------------------------------------------------------------------------
 * Workspace of the entry points that take none (the drop-ins kiln_attn_fwd_f32out / _f16out and any
 * call passing workspace = NULL): the fp16 K/V tiles and key-split partials. The reference's flash
 * paths allocate nothing per call (they use the engine's arena, engine/src/gpu.h:51-59,
 * kernels.cu:293-301); to get the same, set the workspace up once per device:
 *   - kiln_attn_set_workspace(ptr, bytes): bind a caller-owned buffer (e.g. an arena slice,
 *     256-byte aligned) to the current device; NULL unbinds;
 *   - kiln_attn_workspace_reserve(bytes): the library allocates it now (synchronizes the device).
 * After either, no call allocates or synchronizes (so calls can be captured into a HIP graph);
 * a call needing more than the buffer returns KILN_ENOMEM. Without either, the first call that
 * needs more allocates (grow-only, outgrown buffers kept until kiln_attn_workspace_release).
 * Calls sharing one device's workspace must be ordered on one stream.
 * ------------------------------------------------------------------------------------------ */
/* Bytes one drop-in call (kiln_attn_fwd_f32out / _f16out, flash path) of this shape needs. */
size_t kiln_attn_dropin_workspace_bytes(int Tq, int Tk, int H);
int kiln_attn_workspace_reserve(size_t bytes);
int kiln_attn_set_workspace(void* ptr, size_t bytes);
/* Synchronizes the current device and frees the library-owned buffers (a bound buffer stays bound). */
int kiln_attn_workspace_release(void);

/* ------------------------------------------------------------------------------------------
 * Per-category GPU timing (replaces the reference's ProfScope / prof_enable / prof_report,
 * engine/src/kernels.cu:14-58, gpu.h:92-99). While enabled, every entry point records a hipEvent pair
 * on its stream under its category: attention (all attention entry points and the K/V prepare),
 * gemm_tc16 (linear16 and the projections of the fused DiT sections), gemm_fp32, matvec, norm,
 * layernorm, rope, nag, eltwise, w->f16. Not for use under HIP graph capture.
 * ------------------------------------------------------------------------------------------ */
/* on != 0 starts a new profile (clears the previous one); 0 stops recording. */
int kiln_prof_enable(int on);
/* Waits for the recorded events and writes one line per category ("name ms percent (calls)") and a sum line. */
int kiln_prof_report(char* buf, size_t buflen);
/* The summed milliseconds and call count of one category. */
int kiln_prof_category(const char* name, double* ms, int* calls);

/* ------------------------------------------------------------------------------------------
 * Drop-in replacements of the reference op layer
 * ------------------------------------------------------------------------------------------ */

/* Replaces attention() (engine/src/gpu.h:149-153, impl engine/src/kernels.cu:828-866).
 * fp32 Q/K/V/out. Dh == 128 and !causal run the fp16-MFMA flash kernel (the reference's
 * tfa::k_flash<float> path, engine/src/tcflash.cuh:20-157); any other Dh (<= 256) or causal runs
 * the exact fp32 kernel (the reference's cuBLAS fallback semantics, kernels.cu:809-866).
 * Uses the device's workspace (above) for the fp16 K/V tiles. */
int kiln_attn_fwd_f32out(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                         int ldv, int Tq, int Tk, int H, int Dh, int causal, int npad, kiln_stream_t stream);

/* Replaces attention16() (engine/src/gpu.h:155-156, impl engine/src/kernels.cu:868-873).
 * fp32 Q/K/V, fp16 out; Dh must be 128 (KILN_EUNSUPPORTED otherwise, where the reference throws). */
int kiln_attn_fwd_f16out(uint16_t* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                         int ldv, int Tq, int Tk, int H, int Dh, int npad, kiln_stream_t stream);

/* attention16 (kiln_attn_fwd_f16out, same arguments, results and errors) for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. No
 * counterpart in the reference. Its scratch (fp16 K/V tiles, key-split partials) is a fixed device array of
 * kiln_attn_noalloc_scratch_bytes() (64 MiB) per device, held until the process ends; a call whose K/V tiles
 * (kiln_kv_prepped_bytes(Tk, H)) exceed it returns KILN_ENOMEM. It calls no hipMalloc/hipFree and never
 * synchronizes the host. Every call on one device shares that device's scratch, so eager calls are ordered on it:
 * a call on another stream than the device's previous call first makes its stream wait for that call (one event
 * per device, created at the first call; calls from several host threads are serialized). Calls under HIP graph
 * capture skip that ordering: a replayed graph and calls on other streams must not overlap on one GPU (they would
 * race on the scratch). */
int kiln_attn_fwd_f16out_noalloc(uint16_t* out, int ldo, const float* q, int ldq, const float* k, int ldk,
                                 const float* v, int ldv, int Tq, int Tk, int H, int Dh, int npad,
                                 kiln_stream_t stream);
size_t kiln_attn_noalloc_scratch_bytes(void);

/* Exact fp32 attention (the reference's fallback when G.fp16 is off: --fp32 / "precision":"fp32",
 * engine/src/kernels.cu:840-865): any Dh <= 256, optional causal mask, npad. */
int kiln_attn_fwd_exact(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                        int ldv, int Tq, int Tk, int H, int Dh, int causal, int npad, kiln_stream_t stream);

/* Replaces the rmsnorm() calls of the DiT QK-norm (engine/src/gpu.h:133, kernels.cu:656-673):
 * per row of `dim`, y = x * rsqrt(mean(x^2) + eps) * w (w bf16, NULL = 1). In place allowed. */
int kiln_rmsnorm_rows(float* y, const float* x, const uint16_t* w_bf16, int rows, int dim, float eps,
                      kiln_stream_t stream);

/* Replaces rope_half() (engine/src/gpu.h:145, kernels.cu:759-777): rotate pairs (i, i+Dh/2) of every
 * head of x [T, H*Dh] (dense rows) with tables cos/sin [T, Dh/2], in place. */
int kiln_rope_half(float* x, int T, int H, int Dh, const float* cos_t, const float* sin_t, kiln_stream_t stream);

/* Replaces the k_nag<T><<<T,256>>> launch (engine/src/dit.cu:295-324, launched :486 / :524):
 * per row of `dim` columns, a <- alpha*clamp(g) + (1-alpha)*a, g = a*s - an*(s-1), the clamp limiting
 * |g|_1 to tau*|a|_1. dtype KILN_F16 (fp16 rows, fp32 math) or KILN_F32. */
int kiln_nag_combine(void* a, int lda, const void* an, int ldn, int dtype, int T, int dim, float s, float tau,
                     float alpha, kiln_stream_t stream);

/* Replaces layernorm_mod() (engine/src/gpu.h:134, impl engine/src/kernels.cu:678-692): the DiT block's
 * modulated LayerNorm, per row of `dim`: y = (x - mean) * rsqrt(var + eps) * (1 + scale) + shift, with
 * scale/shift per column (fp32 [dim]). x, y [rows, dim] dense fp32. */
int kiln_layernorm_mod(float* y, const float* x, const float* scale, const float* shift, int rows, int dim, float eps,
                       kiln_stream_t stream);

/* Replaces layernorm_mod16() (engine/src/gpu.h:135, impl engine/src/kernels.cu:693-697): the same with an fp16
 * output (the input of the fp16-activation projections, engine/src/dit.cu:460,474,491). */
int kiln_layernorm_mod16(uint16_t* y, const float* x, const float* scale, const float* shift, int rows, int dim,
                         float eps, kiln_stream_t stream);

/* Replaces add_gated() (engine/src/gpu.h:136, impl engine/src/kernels.cu:700-708): the gated residual
 * x += gate * y per row (gate fp32 [dim], NULL = 1). x, y [rows, dim] dense fp32. */
int kiln_add_gated(float* x, const float* y, const float* gate, int rows, int dim, kiln_stream_t stream);

/* Epilogues of kiln_linear16: the reference's Epi16 (engine/src/gpu.h:125, tcgemm16.cuh:20). */
typedef enum { KILN_EPI_F32 = 0, KILN_EPI_F16 = 1, KILN_EPI_GELU16 = 2, KILN_EPI_RESID = 3 } kiln_epi;

/* Replaces linear16() (engine/src/gpu.h:126, impl engine/src/kernels.cu:573-609 with tc16::k_gemm16,
 * engine/src/tcgemm16.cuh:1-200): acc = x16 W^T over x16 fp16 [T, cols] (dense rows) and the fp16 weight
 * W [rows, cols] (a weight after weight_to_f16), plus the folded LoRA product a2 w2^T (a2 fp16 [T, k2],
 * w2 fp16 [rows, k2], dense; k2 = 0: none), accumulated in fp32. Epilogue by `epi`:
 *   KILN_EPI_F32:    y fp32  = acc + beta*y
 *   KILN_EPI_F16:    y fp16  = acc
 *   KILN_EPI_GELU16: y fp16  = GELU(acc) = acc/2 (1 + erf(acc/sqrt 2))
 *   KILN_EPI_RESID:  y fp32 += gate[col] * acc   (gate fp32 [rows], NULL = 1)
 * y has rows of ldy >= rows elements. Requires rows % 128 == 0, cols % 32 == 0, k2 % 32 == 0 (the reference's
 * eligibility, tcgemm16.cuh:177) and 16-byte aligned x16/W/a2/w2 (KILN_EUNSUPPORTED otherwise, where the
 * reference throws); ldy even and y aligned to two elements. */
int kiln_linear16(void* y, int ldy, const uint16_t* x16, int T, const uint16_t* w16, int rows, int cols, int epi,
                  const float* gate, float beta, const uint16_t* a2, const uint16_t* w2, int k2, kiln_stream_t stream);

/* Bytes of the prepared form of a [rows, cols] linear16 weight: rows rounded up to 256, times cols, fp16. */
size_t kiln_linear16_prepped_weight_bytes(int rows, int cols);

/* Replaces weight_to_f16() for a linear16 weight (engine/src/kernels.cu:531-544, called at load,
 * engine/src/dit.cu:100): converts W [rows, cols] (fp16, or bf16 when src_bf16 != 0: clamped to +-65504 and
 * rounded to nearest even, as k_bf16_to_f16) into the prepared tile layout that kiln_linear16_prepped streams
 * with one contiguous 16 KB read per 256-row x 32-k tile. wp: kiln_linear16_prepped_weight_bytes(rows, cols)
 * bytes, 16-byte aligned, not overlapping w. Same eligibility as kiln_linear16. */
int kiln_linear16_prepare_weight(uint16_t* wp, const uint16_t* w, int rows, int cols, int src_bf16,
                                 kiln_stream_t stream);

/* kiln_linear16 with the weight in the prepared layout (wp from kiln_linear16_prepare_weight of the same rows
 * and cols). The LoRA product's w2 stays in plain [rows, k2] rows. Results equal kiln_linear16's on the
 * fp16 weight. */
int kiln_linear16_prepped(void* y, int ldy, const uint16_t* x16, int T, const uint16_t* wp, int rows, int cols,
                          int epi, const float* gate, float beta, const uint16_t* a2, const uint16_t* w2, int k2,
                          kiln_stream_t stream);

/* ---- the DiT forward's passes around the transformer blocks (engine/src/dit.cu:242-272, 414-417, 537-545) ---- */

/* Replaces matvec() (engine/src/gpu.h:122, kernels.cu k_matvec): y[r] = sum_c W[r][c] x[c] (+ add[r]), W bf16
 * [rows, cols] row-major, x fp32 [cols], add fp32 [rows] or NULL. The per-step modulation vectors. */
int kiln_matvec_bf16(float* y, const uint16_t* w_bf16, const float* x, const float* add, int rows, int cols,
                     kiln_stream_t stream);
/* groups matvecs in one launch (the per-block adaLN second layers of Dit::step_tables, engine/src/dit.cu:266-268):
 * y[g*rows + r] = sum_c W[g*rows + r][c] x[g*cols + c] (+ add[r]); W bf16 [groups*rows, cols] (the groups' weights
 * stacked), x fp32 [groups, cols], add fp32 [rows] shared by every group (the adaLN-LoRA vector) or NULL. */
int kiln_matvec_bf16_grouped(float* y, const uint16_t* w_bf16, const float* x, const float* add, int groups, int rows,
                             int cols, kiln_stream_t stream);
/* Replaces silu() (engine/src/gpu.h:142, kernels.cu:735-739): y = x / (1 + exp(-x)), n elements, in place
 * allowed. */
int kiln_silu(float* y, const float* x, size_t n, kiln_stream_t stream);
/* Replaces k_patchify (engine/src/dit.cu:174-182): a 16-channel latent [16, Hl, Wl] (Hl, Wl even) into
 * tokens [T = Hl/2 * Wl/2, 68], feature 4c + 2m + n = channel c of pixel (2ty + m, 2tx + n); features 64-67
 * (the padding-mask channel) are 0. */
int kiln_patchify(float* tok, const float* latent, int Hl, int Wl, kiln_stream_t stream);
/* Replaces k_unpatchify (engine/src/dit.cu:184-191): tokens [T, 64] (row stride ldt) into the latent
 * [16, Hl, Wl], feature 32 p1 + 16 p2 + c -> channel c of pixel (2ty + p1, 2tx + p2). */
int kiln_unpatchify(float* latent, const float* tok, int ldt, int Hl, int Wl, kiln_stream_t stream);
/* Replaces linear() for the DiT's small fp32 layers (engine/src/gpu.h:118, kernels.cu:508-529; the x embedder
 * and the final layer, dit.cu:417,542): y [T, rows] (row stride ldy) = x [T, cols] (row stride ldx) W^T with
 * W bf16 [rows, cols], fp32 arithmetic. */
int kiln_linear_f32(float* y, int ldy, const float* x, int ldx, const uint16_t* w_bf16, int T, int rows, int cols,
                    kiln_stream_t stream);
/* First-block step cache (engine/src/dit.cu:327-340, used at :404-433): y = a - b (k_sub), and the two sums of
 * the relative L1 change, acc[0] = sum |a - b|, acc[1] = sum |b| (device float[2], overwritten; k_rel_l1). */
/* Synthetic weights (no reference counterpart: the reference loads checkpoints): p[i] = bf16 of lo + (hi - lo) u_i,
 * u_i uniform in [0, 1) from a counter-based hash of (seed, i); lo == hi fills a constant. */
int kiln_fill_uniform_bf16(uint16_t* p, size_t n, uint64_t seed, float lo, float hi, kiln_stream_t stream);
/* Odd latent sides (engine/src/dit.cu:342-370): circular padding of a latent [16, Hs, Ws] to [16, Hd, Wd]
 * (k_pad_circular), and the crop of [16, Hs, Ws] to its top-left [16, Hd, Wd] (k_crop). */
int kiln_pad_circular(float* dst, const float* src, int Hs, int Ws, int Hd, int Wd, kiln_stream_t stream);
int kiln_crop(float* dst, const float* src, int Hs, int Ws, int Hd, int Wd, kiln_stream_t stream);
int kiln_sub(float* y, const float* a, const float* b, size_t n, kiln_stream_t stream);
int kiln_rel_l1(const float* a, const float* b, size_t n, float* acc, kiln_stream_t stream);
/* Replaces torch_randn() (engine/src/pipeline.cu:17-64): host memory out[n] = torch.manual_seed(seed);
 * torch.randn(n) on the CPU (MT19937, 24-bit uniforms, Box-Muller in blocks of 16). n >= 16. Host code: no
 * device, no stream. The sampler's initial noise (pipeline.cu:428-429). */
int kiln_torch_randn(float* host_out, uint64_t seed, size_t n);
/* Flow-matching sampler start (engine/src/pipeline.cu:304-307, k_start): x = sigma * noise + (1 - sigma) * init
 * (init NULL: 0), n elements. */
int kiln_flow_start(float* x, const float* noise, const float* init, float sigma, size_t n, kiln_stream_t stream);
/* One Euler step of the velocity v without a mask (engine/src/pipeline.cu:318-331, k_denoised then
 * k_euler_step): den = x - v * sigma; x = x + (x - den) / sigma * (sigma_next - sigma). sigma > 0. */
int kiln_flow_euler_step(float* x, const float* v, float sigma, float sigma_next, size_t n, kiln_stream_t stream);
/* k_euler_step (engine/src/pipeline.cu:326-331) on a given denoised estimate (the masked Euler path):
 * x = x + (x - den) / sigma * (sigma_next - sigma). sigma > 0. */
int kiln_flow_euler_den(float* x, const float* den, float sigma, float sigma_next, size_t n, kiln_stream_t stream);
/* The sampler's denoised estimate without a mask (engine/src/pipeline.cu:318-324): den = x - v * sigma. */
int kiln_flow_denoised(float* den, const float* x, const float* v, float sigma, size_t n, kiln_stream_t stream);
/* Inpainting (engine/src/pipeline.cu:309-324), latents [16, P] and mask [P]: the model input
 * xin = m x + (1 - m) (sigma noise + (1 - sigma) init) (k_inpaint_in), and the denoised estimate pinned to the
 * init outside the mask, den = m (xin - v sigma) + (1 - m) init (k_denoised with a mask). */
int kiln_flow_inpaint_in(float* xin, const float* x, const float* noise, const float* init, const float* mask,
                         float sigma, int P, kiln_stream_t stream);
int kiln_flow_denoised_masked(float* den, const float* xin, const float* v, const float* init, const float* mask,
                              float sigma, int P, kiln_stream_t stream);
/* The generic sampler step (engine/src/pipeline.cu:333-337, k_update): x = a x + b den + c old (old NULL: 0). */
int kiln_flow_update(float* x, const float* den, const float* old, float a, float b, float c, size_t n,
                     kiln_stream_t stream);
/* The er_sde sampler step (engine/src/pipeline.cu:345-359, coefficients :361-391): x = a x + b den; from stage 2
 * + c2 dd with dd = (den - old) * inv2 (stored into oldd); at stage 3 + c3 (dd - oldd_prev) * inv3; + cn noise
 * (noise NULL: none). */
int kiln_flow_ersde_step(float* x, const float* den, const float* old, float* oldd, const float* noise, float a,
                         float b, float c2, float inv2, float c3, float inv3, float cn, int stage, size_t n,
                         kiln_stream_t stream);
/* Replaces gelu() (engine/src/gpu.h:141, kernels.cu:728-733): x = x/2 (1 + erf(x / sqrt 2)) in place, fp32. */
int kiln_gelu(float* x, size_t n, kiln_stream_t stream);
/* Replaces cfg_combine() (engine/src/gpu.h:144, kernels.cu:1058-1062): v = vn + cfg * (v - vn), n elements. */
int kiln_cfg_combine(float* v, const float* vn, float cfg, size_t n, kiln_stream_t stream);

/* Host-side Cosmos 3D RoPE tables for an Hp x Wp patch grid (engine/src/dit.cu:196-215):
 * cos_t, sin_t are HOST arrays of Hp*Wp*64 floats. */
int kiln_cosmos_rope_tables(float* cos_t, float* sin_t, int Hp, int Wp);

/* ------------------------------------------------------------------------------------------
 * MI355X-native entry points of the same path (no counterpart with this signature in the
 * reference; they batch what the reference does per batch element, engine/src/dit.cu:466-487)
 * ------------------------------------------------------------------------------------------ */

/* Bytes of a prepared K/V buffer for Tk keys and H heads of dim 128: K and V in fp16, tiled
 * 64 keys at a time in the MFMA operand order the attention kernel reads, zero beyond Tk. */
size_t kiln_kv_prepped_bytes(int Tk, int H);

/* Prepare K/V once (e.g. the cross-attention context K/V cached per generation, the reference's
 * Dit::cache_context, engine/src/dit.cu:217-234). k, v: [Tk, ld] in_dtype rows, head h at column
 * h*128. Optional per-head RMSNorm of K (k_norm_w bf16 [128], eps) and RoPE of K (tables [Tk, 64]). */
int kiln_kv_prepare(uint16_t* kvp, const void* k, int ldk, const void* v, int ldv, int in_dtype, int Tk, int H,
                    const uint16_t* k_norm_w, float eps, const float* rope_cos, const float* rope_sin,
                    kiln_stream_t stream);

/* Attention of Q [Tq, ldq] (in_dtype) against a prepared K/V buffer. The Q tile load applies the
 * optional per-head RMSNorm (q_norm_w, eps) and RoPE (tables [Tq, 64]) before the fp16 rounding. */
int kiln_attn_fwd_prepped(void* out, int out_dtype, int ldo, const void* q, int in_dtype, int ldq,
                          const uint16_t* q_norm_w, float eps, const float* rope_cos, const float* rope_sin,
                          const uint16_t* kvp, int Tq, int Tk, int H, int npad, kiln_stream_t stream);

/* Batched form of kiln_attn_fwd_prepped: B independent query sets (q + b*bsq, out + b*bso, elements)
 * against prepared K/V buffers kvp[b] (host array of B device pointers), one launch. B <= 4. */
int kiln_attn_fwd_prepped_batch(void* out, int out_dtype, int ldo, long long bso, const void* q, int in_dtype, int ldq,
                                long long bsq, const uint16_t* q_norm_w, float eps, const float* rope_cos,
                                const float* rope_sin, const uint16_t* const* kvp, int B, int Tq, int Tk, int H,
                                int npad, kiln_stream_t stream);

/* Plain batched fp16 attention: B independent (Q, K, V) sets at batch strides bs* (elements).
 * workspace NULL = library-owned (sized for the key split of small grids too); a caller's workspace of
 * kiln_attn_fwd_f16in_workspace_bytes() runs unsplit. */
int kiln_attn_fwd_f16in(void* out, int out_dtype, int ldo, long long bso, const uint16_t* q, int ldq, long long bsq,
                        const uint16_t* k, int ldk, long long bsk, const uint16_t* v, int ldv, long long bsv, int B,
                        int Tq, int Tk, int H, int npad, void* workspace, size_t ws_bytes, kiln_stream_t stream);
size_t kiln_attn_fwd_f16in_workspace_bytes(int B, int Tk, int H);

/* Fused DiT self-attention of a CFG batch (engine/src/dit.cu:458-470): q, k, v are the raw
 * projections [B*T, ld] (batch b at rows b*T); QK-RMSNorm (bf16 weights, eps) and RoPE (tables
 * [T, 64]) are applied inside (K in the K/V prepare pass, Q in the attention kernel's tile load),
 * softmax scale 1/sqrt(128). out [B*T, ldo] in out_dtype. workspace NULL = library-owned. */
int kiln_dit_self_attn_fused(void* out, int out_dtype, int ldo, const void* q, const void* k, const void* v,
                             int in_dtype, int ld, const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps,
                             const float* rope_cos, const float* rope_sin, int B, int T, int H, void* workspace,
                             size_t ws_bytes, kiln_stream_t stream);
/* Workspace of kiln_dit_self_attn_fused on the current device: the prepared K/V of the B items, plus, when
 * the launch would fill under a third of the device's workgroup slots (few heads, e.g. one GPU's share of a
 * head-parallel run), the partial results of splitting every query tile's keys into ranges. A smaller
 * workspace that still holds the prepared K/V runs the same call unsplit. */
size_t kiln_dit_self_attn_workspace_bytes(int B, int T, int H);

/* The DiT self-attention section from the block's fp16 LayerNorm output (engine/src/dit.cu:460-469: linear16 of
 * sa_q, sa_k, sa_v, rmsnorm of Q and K per head, rope_half, attention16 per item) in two launches: one fp16 GEMM
 * of x16 [B*T, D] (D = 128 H) with the stacked [Wq; Wk; Wv] weight (kiln_linear16_prepare_weight of [3D, D])
 * whose epilogue applies the QK-RMSNorm (bf16 weights) and RoPE (tables [T, 64]) and writes fp16 Q and the
 * prepared K/V (no fp32 Q/K/V round trip, no K/V prepare pass), then the attention of the B items. H even,
 * B <= 4. workspace: kiln_dit_self_attn_x16_workspace_bytes (fp16 Q, prepared K/V, key-split partials),
 * 16-byte aligned (KILN_ENOMEM if smaller). out [B*T, ldo] fp32 or fp16. */
int kiln_dit_self_attn_x16(void* out, int out_dtype, int ldo, const uint16_t* x16, const uint16_t* wqkv_prepped,
                           const uint16_t* q_norm_w, const uint16_t* k_norm_w, float eps, const float* rope_cos,
                           const float* rope_sin, int B, int T, int H, void* workspace, size_t ws_bytes,
                           kiln_stream_t stream);
size_t kiln_dit_self_attn_x16_workspace_bytes(int B, int T, int H);

/* DiT cross-attention of a CFG batch plus NAG (engine/src/dit.cu:473-487): batch item b's queries
 * (rows b*T of q, RMS-normed inside with q_norm_w) attend to prepared context kvp[b] (Lk[b] real keys,
 * npad[b] zero keys). If kvp_neg is not NULL, item 0's queries also attend to kvp_neg into
 * out_neg [T, ldo] (caller scratch) and item 0's output is replaced by the NAG combine with
 * (nag_scale, nag_tau, nag_alpha). B <= 3. */
int kiln_cross_attn_nag(void* out, void* out_neg, int out_dtype, int ldo, const void* q, int in_dtype, int ldq,
                        const uint16_t* q_norm_w, float eps, int B, int T, int H, const uint16_t* const* kvp,
                        const int* Lk, const int* npad, const uint16_t* kvp_neg, int Lk_neg, int npad_neg,
                        float nag_scale, float nag_tau, float nag_alpha, kiln_stream_t stream);

/* The DiT cross-attention section from the block's fp16 LayerNorm output (engine/src/dit.cu:475-487): the cross
 * Q projection (wq_prepped: kiln_linear16_prepare_weight of ca_q [D, D]) with the Q RMSNorm fused into its
 * epilogue (fp16 Q, pre-scaled), then kiln_cross_attn_nag's attention and NAG with those Q. workspace: B*T*D*2
 * bytes (the fp16 Q), 16-byte aligned. Other arguments as kiln_cross_attn_nag. */
int kiln_dit_cross_attn_x16(void* out, void* out_neg, int out_dtype, int ldo, const uint16_t* x16,
                            const uint16_t* wq_prepped, const uint16_t* q_norm_w, float eps, int B, int T, int H,
                            const uint16_t* const* kvp, const int* Lk, const int* npad, const uint16_t* kvp_neg,
                            int Lk_neg, int npad_neg, float nag_scale, float nag_tau, float nag_alpha, void* workspace,
                            size_t ws_bytes, kiln_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* KILN_ATTN_H */
