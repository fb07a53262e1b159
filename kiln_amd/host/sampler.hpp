// sampler.hpp - flow-matching sampling of the DiT (the reference's sample(), engine/src/pipeline.cu:415-598),
// its schedulers (pipeline.cu:66-78, 188-277) and step coefficients (pipeline.cu:361-411), in C++ over the C ABI
// of libkiln_attn.so. Every array operation runs on the GPU; the schedules and coefficients are host arithmetic.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <functional>
#include <string>
#include <vector>

#include "dit.hpp"

namespace kiln {

// "simple" schedule (flow_sigmas, pipeline.cu:66-78): steps + 1 sigmas ending in 0.
std::vector<float> flow_sigmas(int steps, float shift, float denoise);
// The flow-space schedulers (schedule_sigmas, pipeline.cu:188-277): simple, normal, sgm_uniform, karras,
// exponential, ddim_uniform, beta, linear_quadratic, kl_optimal. Throws on an unknown name.
std::vector<float> schedule_sigmas(const std::string& name, int steps, float shift, float denoise);
bool known_scheduler(const std::string& name);
bool known_sampler(const std::string& name);
// The Beta(a, b) quantile by bisection on the regularized incomplete beta function (the beta scheduler's ppf).
double beta_quantile(double p, double a, double b);
double beta_cdf(double x, double a, double b);

// One deterministic step from sigma_i to sigma_{i+1}: x <- x_w x + den_w den + old_w old (the samplers of
// pipeline.cu:396-411)
struct LinearStep {
    float x_w, den_w, old_w;
};
LinearStep linear_step(const std::string& sampler, const std::vector<float>& sig, int i, bool have_old);

// One er_sde step (pipeline.cu:361-391): x <- x_w x + den_w den + d1_w D1 + d2_w D2 + noise_w noise, with
// D1 = (den - old) d1_inv and D2 = (D1 - D1_prev) d2_inv; `order` terms are active (1: the first two).
struct ErSdeStep {
    float x_w, den_w, d1_w, d1_inv, d2_w, d2_inv, noise_w;
    int order;
};
ErSdeStep ersde_step(const std::vector<float>& sig, int i);

// The velocity model the sampler drives. forward() writes the prompt's velocity into outs[0] and, when cfg_now,
// the negative context's into outs[1], for the latent x at noise level sigma, whose model timestep is t (sigma times
// the model's timestep multiplier). cache_allow tells a model with a step
// cache whether it may skip this step; it reports a skip through *cache_skipped.
class VelocityModel {
   public:
    virtual ~VelocityModel() = default;
    virtual void forward(float* const* outs, const float* x, float sigma, float t, bool cfg_now, bool cache_allow,
                         bool* cache_skipped) = 0;
};

struct SampleParams {
    int steps = 8;
    float cfg = 1.f, shift = 3.f, denoise = 1.f;
    uint64_t seed = 0;
    float cfg_until = 1.f;
    std::string sampler = "euler", scheduler = "simple";
    std::vector<float> sigmas;    // overrides the scheduler when not empty
    bool add_noise = true;
    const float* noise = nullptr;  // host [16 P]; null: torch_randn(seed, 16 P)
    float timestep_mult = 1.f;     // the model sees sigma * timestep_mult
    float cache_threshold = 0.f;   // > 0: the first-block step cache is on
    float cache_start = 0.15f, cache_end = 0.9f;
    int cache_max_hits = 2;
};

// Per-step report: step (1-based), steps, sigma, x and v (device [16 P]), milliseconds of the step.
using StepFn = std::function<void(int, int, float, const float*, const float*, double)>;

struct SampleResult {
    int steps = 0, cache_skips = 0;
};

// sample() (pipeline.cu:415-598) on a latent x [16, Hl, Wl] (device, overwritten with the result). negative:
// a negative context exists (CFG runs for the first ceil(cfg_until * steps) steps). init: img2img start
// [16 P] or null; mask [P] (1 = regenerate) with init: inpainting. cancelled: polled between steps (a true
// result throws Cancelled). All work on `stream`.
struct Cancelled : std::runtime_error {
    Cancelled() : std::runtime_error("cancelled") {}
};
SampleResult sample(VelocityModel& model, float* x, int Hl, int Wl, bool negative, const SampleParams& sp,
                    const float* init, const float* mask, const StepFn& on_step,
                    const std::function<bool()>& cancelled, hipStream_t stream);

// The DiT as the sampler's model (the batching of pipeline.cu:436-504): the CFG pair in one forward_batch when
// `batch`, else the prompt pass (with NAG and the step cache) and the negative pass (without either); NAG off
// below nag_sigma_end.
class DitVelocity : public VelocityModel {
   public:
    DitVelocity(Dit& dit, int Hl, int Wl, const CachedContext* pos, const CachedContext* neg, const NagParams& nag,
                float nag_sigma_end, float cache_threshold, bool batch, bool fp32);
    void forward(float* const* outs, const float* x, float sigma, float t, bool cfg_now, bool cache_allow,
                 bool* cache_skipped) override;

   private:
    Dit& dit_;
    int Hl_, Wl_;
    const CachedContext *pos_, *neg_;
    NagParams nag_;
    float nag_end_;
    StepCache sc_;
    bool batch_, fp32_;
};

}  // namespace kiln
