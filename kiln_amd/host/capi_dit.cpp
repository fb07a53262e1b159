// capi_dit.cpp - the C ABI of libkiln_dit.so (include/kiln_dit.h) over the C++ driver (dit.hpp, sampler.hpp):
// argument checks, exception -> status mapping, handles.
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "../../include/kiln_dit.h"
#include "dit.hpp"
#include "sampler.hpp"

struct kiln_dit {
    kiln::Dit dit;
    kiln_dit(const kiln::DitDims& d, hipStream_t s) : dit(d, s) {}
};
struct kiln_dit_context {
    std::unique_ptr<kiln::CachedContext> c;
};
struct kiln_dit_step_cache {
    kiln::StepCache sc;
};

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

// runs f, mapping exceptions to status codes: a kiln::Error keeps its own (HIP failure, device memory, a failed
// library call), anything else is a bad argument
template <typename F>
int guarded(F&& f) {
    try {
        f();
        return KILN_OK;
    } catch (const kiln::Cancelled&) {
        return fail(KILN_ECANCELLED, "cancelled");
    } catch (const kiln::Error& e) {
        return fail(e.status, e.what());
    } catch (const std::bad_alloc&) {
        return fail(KILN_ENOMEM, "host out of memory");
    } catch (const std::exception& e) {
        return fail(KILN_EINVAL, e.what());
    }
}

kiln::NagParams nag_of(const kiln_dit_nag* n) {
    kiln::NagParams p;
    if (n && n->neg) {
        p.neg = n->neg->c.get();
        p.scale = n->scale, p.tau = n->tau, p.alpha = n->alpha;
    }
    return p;
}

int contexts(const kiln_dit_context* const* cs, int B, const kiln::CachedContext** out) {
    if (!cs || B < 1 || B > 3) return fail(KILN_EINVAL, "contexts: B outside 1..3");
    for (int b = 0; b < B; b++) {
        if (!cs[b] || !cs[b]->c) return fail(KILN_EINVAL, "contexts: null context");
        out[b] = cs[b]->c.get();
    }
    return KILN_OK;
}

kiln::SampleParams params_of(const kiln_sample_params* p) {
    kiln::SampleParams sp;
    sp.steps = p->steps;
    sp.cfg = p->cfg, sp.shift = p->shift, sp.denoise = p->denoise;
    sp.seed = p->seed;
    sp.cfg_until = p->cfg_until;
    if (p->sampler) sp.sampler = p->sampler;
    if (p->scheduler) sp.scheduler = p->scheduler;
    if (p->sigmas && p->nsigmas > 0) sp.sigmas.assign(p->sigmas, p->sigmas + p->nsigmas);
    sp.add_noise = p->add_noise != 0;
    sp.noise = p->noise;
    sp.timestep_mult = p->timestep_mult;
    sp.cache_threshold = p->cache_threshold, sp.cache_start = p->cache_start, sp.cache_end = p->cache_end;
    sp.cache_max_hits = p->cache_max_hits;
    return sp;
}

// a C velocity callback as the sampler's model
class CallbackModel : public kiln::VelocityModel {
   public:
    CallbackModel(kiln_velocity_fn fn, void* user) : fn_(fn), user_(user) {}
    void forward(float* const* outs, const float* x, float sigma, float t, bool cfg_now, bool cache_allow,
                 bool* cache_skipped) override {
        int skipped = 0;
        if (fn_(user_, outs, x, t, cfg_now ? 1 : 0, cache_allow ? 1 : 0, &skipped) != 0)
            throw std::runtime_error("velocity model callback failed");
        *cache_skipped = skipped != 0;
    }

   private:
    kiln_velocity_fn fn_;
    void* user_;
};

kiln::StepFn step_fn(kiln_step_fn f, void* user) {
    if (!f) return {};
    return [f, user](int step, int steps, float s, const float* x, const float* v, double ms) {
        f(user, step, steps, s, x, v, ms);
    };
}

std::function<bool()> cancel_fn(const volatile int* c) {
    if (!c) return {};
    return [c]() { return *c != 0; };
}

}  // namespace

extern "C" {

const char* kiln_dit_last_error(void) { return g_err.c_str(); }

int kiln_dit_create(const kiln_dit_dims* dims, kiln_stream_t stream, kiln_dit** out) {
    if (!dims || !out) return fail(KILN_EINVAL, "dit_create: null argument");
    *out = nullptr;
    return guarded([&] {
        kiln::DitDims d;
        d.blocks = dims->blocks, d.heads = dims->heads, d.ctx_dim = dims->ctx_dim, d.mlp = dims->mlp;
        d.eps = dims->eps > 0.f ? dims->eps : 1e-6f;
        *out = new kiln_dit(d, (hipStream_t)stream);
    });
}

void kiln_dit_destroy(kiln_dit* dit) {
    if (dit) {
        (void)hipStreamSynchronize(dit->dit.stream());
        delete dit;
    }
}

int kiln_dit_set_step_weights(kiln_dit* dit, const kiln_dit_step_weights* w) {
    if (!dit || !w) return fail(KILN_EINVAL, "set_step_weights: null argument");
    return guarded([&] {
        kiln::StepWeights s{w->t_lin1, w->t_lin2, w->t_norm, w->final_mod1, w->final_mod2, w->x_embed, w->final_lin};
        dit->dit.set_step_weights(s);
    });
}

int kiln_dit_set_block(kiln_dit* dit, int i, const kiln_dit_block_weights* w) {
    if (!dit || !w) return fail(KILN_EINVAL, "set_block: null argument");
    return guarded([&] {
        kiln::BlockWeights b{w->sa_q,  w->sa_k,  w->sa_v,  w->sa_o,    w->ca_q,    w->ca_o,    w->ca_k,
                             w->ca_v,  w->mlp1,  w->mlp2,  w->sa_qn,   w->sa_kn,   w->ca_qn,   w->ca_kn,
                             w->mod_sa1, w->mod_sa2, w->mod_ca1, w->mod_ca2, w->mod_mlp1, w->mod_mlp2};
        dit->dit.set_block(i, b);
    });
}

int kiln_dit_cache_context(kiln_dit* dit, const float* ctx, int real, int len, int fp32, kiln_dit_context** out) {
    if (!dit || !ctx || !out) return fail(KILN_EINVAL, "cache_context: null argument");
    *out = nullptr;
    return guarded([&] {
        auto c = new kiln_dit_context;
        try {
            c->c = dit->dit.cache_context(ctx, real, len, fp32 != 0);
        } catch (...) {
            delete c;
            throw;
        }
        *out = c;
    });
}

void kiln_dit_context_destroy(kiln_dit_context* c) { delete c; }

int kiln_dit_context_kv(const kiln_dit_context* c, int block, const uint16_t** kvp, int* real, int* len) {
    if (!c || !c->c || !kvp || !real || !len) return fail(KILN_EINVAL, "context_kv: null argument");
    const kiln::CachedContext& cc = *c->c;
    const size_t blocks = cc.kv_per_block ? cc.kv16.bytes() / cc.kv_per_block : 0;
    if (block < 0 || (size_t)block >= blocks) 
        return fail(KILN_EINVAL, "context_kv: block " + std::to_string(block) + " outside the context's " +
                                     std::to_string(blocks) + " blocks");
    *kvp = cc.kv(block);
    *real = cc.real;
    *len = cc.len;
    return KILN_OK;
}

int kiln_dit_step_cache_create(float threshold, kiln_dit_step_cache** out) {
    if (!out) return fail(KILN_EINVAL, "step_cache_create: null argument");
    return guarded([&] {
        *out = new kiln_dit_step_cache;
        (*out)->sc.threshold = threshold;
    });
}

void kiln_dit_step_cache_destroy(kiln_dit_step_cache* sc) { delete sc; }

int kiln_dit_step_cache_set_allow(kiln_dit_step_cache* sc, int allow) {
    if (!sc) return fail(KILN_EINVAL, "step_cache: null");
    sc->sc.allow = allow != 0;
    return KILN_OK;
}

int kiln_dit_step_cache_state(const kiln_dit_step_cache* sc, int* skipped, int* valid, float* last_change) {
    if (!sc) return fail(KILN_EINVAL, "step_cache: null");
    if (skipped) *skipped = sc->sc.skipped;
    if (valid) *valid = sc->sc.valid;
    if (last_change) *last_change = sc->sc.last_change;
    return KILN_OK;
}

int kiln_dit_forward(kiln_dit* dit, float* const* outs, const float* latent, int Hl, int Wl, float t,
                     const kiln_dit_context* const* cs, int B, const kiln_dit_nag* nag, kiln_dit_step_cache* sc,
                     int fp32) {
    if (!dit || !outs || !latent) return fail(KILN_EINVAL, "forward: null argument");
    const kiln::CachedContext* c[3];
    if (int r = contexts(cs, B, c)) return r;
    for (int b = 0; b < B; b++)
        if (!outs[b]) return fail(KILN_EINVAL, "forward: null output");
    return guarded([&] {
        dit->dit.forward_batch(outs, latent, Hl, Wl, t, c, B, nag_of(nag), sc ? &sc->sc : nullptr, fp32 != 0);
    });
}

int kiln_dit_step_tables(kiln_dit* dit, float t, float* mods) {
    if (!dit || !mods) return fail(KILN_EINVAL, "step_tables: null argument");
    return guarded([&] { dit->dit.step_tables(t, mods); });
}

int kiln_dit_run_block(kiln_dit* dit, int i, float* X, const float* mods, int Hp, int Wp,
                       const kiln_dit_context* const* cs, int B, const kiln_dit_nag* nag, int fp32) {
    if (!dit || !X || !mods) return fail(KILN_EINVAL, "run_block: null argument");
    if (Hp <= 0 || Wp <= 0) return fail(KILN_EINVAL, "run_block: bad grid");
    const kiln::CachedContext* c[3];
    if (int r = contexts(cs, B, c)) return r;
    return guarded([&] { dit->dit.run_block(i, X, mods, Hp, Wp, B, c, nag_of(nag), fp32 != 0); });
}

int kiln_schedule_sigmas(const char* scheduler, int steps, float shift, float denoise, float* out, int cap) {
    if (!scheduler || (!out && cap > 0) || cap < 0) return -fail(KILN_EINVAL, "schedule_sigmas: bad arguments");
    std::vector<float> s;
    const int r = guarded([&] {
        s = kiln::schedule_sigmas(scheduler, steps, shift, denoise);
    });
    if (r) return -r;
    for (int k = 0; k < (int)s.size() && k < cap; k++) out[k] = s[k];
    return (int)s.size();
}

int kiln_step_coef(const char* sampler, const float* sig, int nsig, int i, int have_old, float* abc) {
    if (!sampler || !sig || !abc || i < 0 || i + 1 >= nsig || (have_old && i < 1))
        return fail(KILN_EINVAL, "step_coef: bad arguments");
    return guarded([&] {
        const kiln::LinearStep w = kiln::linear_step(sampler, std::vector<float>(sig, sig + nsig), i, have_old != 0);
        abc[0] = w.x_w, abc[1] = w.den_w, abc[2] = w.old_w;
    });
}

int kiln_ersde_coef(const float* sig, int nsig, int i, float* c7, int* stage) {
    if (!sig || !c7 || !stage || i < 0 || i + 1 >= nsig) return fail(KILN_EINVAL, "ersde_coef: bad arguments");
    return guarded([&] {
        const kiln::ErSdeStep e = kiln::ersde_step(std::vector<float>(sig, sig + nsig), i);
        const float v[7] = {e.x_w, e.den_w, e.d1_w, e.d1_inv, e.d2_w, e.d2_inv, e.noise_w};
        for (int k = 0; k < 7; k++) c7[k] = v[k];
        *stage = e.order;
    });
}

double kiln_beta_quantile(double p, double a, double b) { return kiln::beta_quantile(p, a, b); }

void kiln_sample_params_default(kiln_sample_params* p) {
    if (!p) return;
    const kiln::SampleParams d;
    *p = kiln_sample_params{};
    p->steps = d.steps;
    p->cfg = d.cfg, p->shift = d.shift, p->denoise = d.denoise;
    p->seed = d.seed;
    p->cfg_until = d.cfg_until;
    p->sampler = "euler";
    p->scheduler = "simple";
    p->add_noise = 1;
    p->timestep_mult = d.timestep_mult;
    p->cache_threshold = d.cache_threshold, p->cache_start = d.cache_start, p->cache_end = d.cache_end;
    p->cache_max_hits = d.cache_max_hits;
}

int kiln_sample(kiln_velocity_fn model, void* model_user, float* x, int Hl, int Wl, int negative,
                const kiln_sample_params* sp, const float* init, const float* mask, kiln_step_fn on_step,
                void* step_user, const volatile int* cancel, int* cache_skips, kiln_stream_t stream) {
    if (!model || !x || !sp || Hl <= 0 || Wl <= 0) return fail(KILN_EINVAL, "sample: bad arguments");
    return guarded([&] {
        CallbackModel m(model, model_user);
        const kiln::SampleResult r = kiln::sample(m, x, Hl, Wl, negative != 0, params_of(sp), init, mask,
                                                  step_fn(on_step, step_user), cancel_fn(cancel), (hipStream_t)stream);
        if (cache_skips) *cache_skips = r.cache_skips;
    });
}

int kiln_dit_sample(kiln_dit* dit, float* x, int Hl, int Wl, const kiln_dit_context* pos, const kiln_dit_context* neg,
                    const kiln_dit_nag* nag, float nag_sigma_end, int batch_cfg, int fp32, const kiln_sample_params* sp,
                    const float* init, const float* mask, kiln_step_fn on_step, void* step_user,
                    const volatile int* cancel, int* cache_skips) {
    if (!dit || !x || !sp || !pos || !pos->c || Hl <= 0 || Wl <= 0) return fail(KILN_EINVAL, "dit_sample: bad arguments");
    if (neg && !neg->c) return fail(KILN_EINVAL, "dit_sample: null negative context");
    return guarded([&] {
        const kiln::SampleParams p = params_of(sp);
        kiln::DitVelocity m(dit->dit, Hl, Wl, pos->c.get(), neg ? neg->c.get() : nullptr, nag_of(nag), nag_sigma_end,
                            p.cache_threshold, batch_cfg != 0, fp32 != 0);
        const kiln::SampleResult r = kiln::sample(m, x, Hl, Wl, neg != nullptr, p, init, mask,
                                                  step_fn(on_step, step_user), cancel_fn(cancel), dit->dit.stream());
        if (cache_skips) *cache_skips = r.cache_skips;
    });
}

}  // extern "C"
