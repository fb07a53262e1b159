/*
 * kiln_dit.h - C ABI of libkiln_dit.so: the DiT step driver of Kiln's diffusion engine on MI355X, host C++
 * (kiln_amd/host/dit.cpp, sampler.cpp) over libkiln_attn.so (include/kiln_attn.h).
 *
 *   - the Cosmos-Predict2 DiT: Dit::forward_batch (engine/src/dit.cu:357-546), Dit::step_tables
 *     (dit.cu:242-278), Dit::cache_context (dit.cu:217-234), the first-block step cache (models.h:66-76) and
 *     NAG (models.h:80), on the fp16-activation path or the fp32 path (the engine's --fp32);
 *   - sample() (engine/src/pipeline.cu:415-598) with its samplers and schedulers (pipeline.cu:66-411).
 *
 * Every function returns a kiln_status (include/kiln_attn.h), or KILN_ECANCELLED when a sampling run was
 * cancelled; kiln_dit_last_error() gives the calling thread's message. Pointers named as device memory are
 * device memory of the current device; all GPU work is ordered on the stream given at creation / per call.
 */
#ifndef KILN_DIT_H
#define KILN_DIT_H

#include <stddef.h>
#include <stdint.h>

#include "kiln_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define KILN_ECANCELLED 5

typedef struct kiln_dit kiln_dit;                   /* the model (weights, scratch, stream) */
typedef struct kiln_dit_context kiln_dit_context;   /* a text context cached for one generation */
typedef struct kiln_dit_step_cache kiln_dit_step_cache;

typedef struct {
    int blocks;  /* transformer blocks (28 in the 2B model) */
    int heads;   /* attention heads of dim 128 (16: D = 2048); even */
    int ctx_dim; /* text-context width (1024); multiple of 32 */
    int mlp;     /* MLP hidden width, 0 = 4 D; multiple of 256 */
    float eps;   /* norm epsilon (1e-6) */
} kiln_dit_dims;

/* One block's checkpoint weights: bf16 device arrays [out, in] (copied by kiln_dit_set_block). */
typedef struct {
    const uint16_t *sa_q, *sa_k, *sa_v, *sa_o; /* [D, D] */
    const uint16_t *ca_q, *ca_o;               /* [D, D] */
    const uint16_t *ca_k, *ca_v;               /* [D, ctx_dim] */
    const uint16_t *mlp1, *mlp2;               /* [F, D], [D, F] */
    const uint16_t *sa_qn, *sa_kn, *ca_qn, *ca_kn; /* [128] */
    const uint16_t *mod_sa1, *mod_sa2, *mod_ca1, *mod_ca2, *mod_mlp1, *mod_mlp2; /* [256, D] / [3D, 256] */
} kiln_dit_block_weights;

/* The weights outside the blocks: bf16 device arrays. */
typedef struct {
    const uint16_t *t_lin1, *t_lin2, *t_norm;  /* [D, D], [3D, D], [D] */
    const uint16_t *final_mod1, *final_mod2;   /* [256, D], [2D, 256] */
    const uint16_t *x_embed, *final_lin;       /* [D, 68], [64, D] */
} kiln_dit_step_weights;

/* NAG on batch item 0: neg NULL = off. */
typedef struct {
    const kiln_dit_context* neg;
    float scale, tau, alpha;
} kiln_dit_nag;

const char* kiln_dit_last_error(void);

int kiln_dit_create(const kiln_dit_dims* dims, kiln_stream_t stream, kiln_dit** out);
void kiln_dit_destroy(kiln_dit* dit);
int kiln_dit_set_step_weights(kiln_dit* dit, const kiln_dit_step_weights* w);
int kiln_dit_set_block(kiln_dit* dit, int i, const kiln_dit_block_weights* w);

/* Dit::cache_context: ctx [len, ctx_dim] fp32 device rows, the first `real` real (the rest zero padding, entering
 * attention as npad zero keys). fp32 != 0 also keeps fp32 K/V for the fp32 path. */
int kiln_dit_cache_context(kiln_dit* dit, const float* ctx, int real, int len, int fp32, kiln_dit_context** out);
void kiln_dit_context_destroy(kiln_dit_context* c);
/* The prepared K/V of block `block` of a cached context (the layout kiln_kv_prepare writes, `real` keys, the
 * other len - real rows as npad zero keys): what Dit::forward_batch hands kiln_cross_attn_nag /
 * kiln_dit_cross_attn_x16, for callers that drive a block's cross-attention themselves (Dit::kv_for,
 * engine/src/dit.cu:407-413). The pointer lives as long as the context. */
int kiln_dit_context_kv(const kiln_dit_context* c, int block, const uint16_t** kvp, int* real, int* len);

int kiln_dit_step_cache_create(float threshold, kiln_dit_step_cache** out);
void kiln_dit_step_cache_destroy(kiln_dit_step_cache* sc);
/* allow: the next forward may skip blocks 1.. (set per step by a sampler) */
int kiln_dit_step_cache_set_allow(kiln_dit_step_cache* sc, int allow);
/* state after a forward: skipped (0/1), valid (0/1), the last relative L1 change */
int kiln_dit_step_cache_state(const kiln_dit_step_cache* sc, int* skipped, int* valid, float* last_change);

/* Dit::forward_batch: B (1..3) items from one latent [16, Hl, Wl] (device fp32) at timestep t; outs: host array of B
 * device pointers [16, Hl, Wl] (the velocities); cs: host array of B contexts; nag and sc may be NULL. */
int kiln_dit_forward(kiln_dit* dit, float* const* outs, const float* latent, int Hl, int Wl, float t,
                     const kiln_dit_context* const* cs, int B, const kiln_dit_nag* nag, kiln_dit_step_cache* sc,
                     int fp32);
/* Dit::step_tables' modulation vectors: mods [blocks * 9D + 2D] fp32 device (per block: shift, scale, gate of
 * self-attention, cross-attention, MLP; then the final layer's shift, scale). */
int kiln_dit_step_tables(kiln_dit* dit, float t, float* mods);
/* One block on X [B*T, D] fp32 device (in place), T = Hp Wp, with modulation mods [9D]: the block loop body of
 * forward_batch. */
int kiln_dit_run_block(kiln_dit* dit, int i, float* X, const float* mods, int Hp, int Wp,
                       const kiln_dit_context* const* cs, int B, const kiln_dit_nag* nag, int fp32);

/* ---- schedules and sampler coefficients (host arithmetic) ---- */

/* schedule_sigmas / flow_sigmas (pipeline.cu:66-78, 188-277) in flow space: writes up to cap sigmas into out
 * (host) and returns their count (>= 0), or -KILN_EINVAL for an unknown scheduler or bad arguments. */
int kiln_schedule_sigmas(const char* scheduler, int steps, float shift, float denoise, float* out, int cap);
/* (a, b, c) of x <- a x + b den + c old (pipeline.cu:396-411) */
int kiln_step_coef(const char* sampler, const float* sig, int nsig, int i, int have_old, float* abc);
/* er_sde coefficients (pipeline.cu:361-391): c7 = (a, b, c2, inv2, c3, inv3, cn), *stage */
int kiln_ersde_coef(const float* sig, int nsig, int i, float* c7, int* stage);
/* The Beta(a, b) quantile of the "beta" scheduler. */
double kiln_beta_quantile(double p, double a, double b);

/* ---- sampling ---- */

typedef struct {
    int steps;
    float cfg, shift, denoise;
    uint64_t seed;
    float cfg_until;
    const char* sampler;   /* euler | euler_ancestral | dpmpp_2m | res_multistep | er_sde */
    const char* scheduler; /* see kiln_schedule_sigmas */
    const float* sigmas;   /* host; nsigmas > 0 overrides the scheduler */
    int nsigmas;
    int add_noise;         /* 0: zero noise */
    const float* noise;    /* host [16 Hl Wl] or NULL: torch_randn(seed) */
    float timestep_mult;
    float cache_threshold, cache_start, cache_end;
    int cache_max_hits;
} kiln_sample_params;
void kiln_sample_params_default(kiln_sample_params* p);

/* A velocity model: writes the prompt's velocity into outs[0] and, when cfg_now, the negative context's into
 * outs[1] (device [16 Hl Wl]) for x at timestep t; may skip blocks when cache_allow and report *cache_skipped.
 * Returns 0, or non-zero to abort the run. */
typedef int (*kiln_velocity_fn)(void* user, float* const* outs, const float* x, float t, int cfg_now, int cache_allow,
                                int* cache_skipped);
/* Called after each step's model pass (the stream synchronized): step (1-based), steps, sigma, x, v (device). */
typedef void (*kiln_step_fn)(void* user, int step, int steps, float sigma, const float* x, const float* v, double ms);

/* sample() with any velocity model: x [16, Hl, Wl] device (overwritten); negative: a negative context exists;
 * init (img2img start) and mask [Hl Wl] (inpainting, 1 = regenerate) device or NULL; cancel: polled between
 * steps (non-zero: stop with KILN_ECANCELLED) or NULL; *cache_skips (or NULL): steps the model skipped. */
int kiln_sample(kiln_velocity_fn model, void* model_user, float* x, int Hl, int Wl, int negative,
                const kiln_sample_params* sp, const float* init, const float* mask, kiln_step_fn on_step,
                void* step_user, const volatile int* cancel, int* cache_skips, kiln_stream_t stream);

/* sample() with the DiT: CFG against neg (NULL: none) in one batched forward when batch_cfg, else two passes;
 * NAG on the prompt while sigma >= nag_sigma_end; the step cache when sp->cache_threshold > 0. */
int kiln_dit_sample(kiln_dit* dit, float* x, int Hl, int Wl, const kiln_dit_context* pos, const kiln_dit_context* neg,
                    const kiln_dit_nag* nag, float nag_sigma_end, int batch_cfg, int fp32, const kiln_sample_params* sp,
                    const float* init, const float* mask, kiln_step_fn on_step, void* step_user,
                    const volatile int* cancel, int* cache_skips);

#ifdef __cplusplus
}
#endif
#endif
