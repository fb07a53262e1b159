// sampler.cpp - schedules, step coefficients and the sampling loop (declarations in sampler.hpp).
#include "sampler.hpp"

#include <math.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <stdexcept>

namespace kiln {

namespace {

kiln_stream_t ks(hipStream_t s) { return (kiln_stream_t)s; }

// ModelSamplingDiscreteFlow(shift): sigma(t) = shift t / (1 + (shift - 1) t); the 1000-entry table holds
// sigma((i + 1) / 1000) in float32 (pipeline.cu:66-78, 100-107).
double shifted(double shift, double t) { return shift == 1.0 ? t : shift * t / (1.0 + (shift - 1.0) * t); }

std::vector<float> sigma_table(float shift) {
    std::vector<float> tab(1000);
    for (int i = 0; i < 1000; i++) {
        const float t = (float)(i + 1) / 1000.f;
        tab[i] = shift == 1.f ? t : shift * t / (1.f + (shift - 1.f) * t);
    }
    return tab;
}

// Each scheduler returns its whole schedule of `steps` steps (steps + 1 sigmas, or fewer where the scheduler
// merges duplicates), ending in 0. smin / smax are the table's ends; in flow space timestep(sigma) = sigma.
using Schedule = std::vector<float>;

Schedule sched_simple(int steps, const std::vector<float>& tab) {
    Schedule s;
    const double stride = 1000.0 / steps;
    for (int k = 0; k < steps; k++) s.push_back(tab[999 - (int)(k * stride)]);
    s.push_back(0.f);
    return s;
}

// linspace in timestep space between smax and smin, mapped back through the shift
Schedule sched_uniform_t(int steps, double shift, double smin, double smax, bool sgm) {
    Schedule s;
    if (sgm) {  // steps + 1 points, the last dropped, then 0
        for (int k = 0; k < steps; k++) s.push_back((float)shifted(shift, smax + (smin - smax) * k / steps));
        s.push_back(0.f);
        return s;
    }
    int n = steps;
    const bool ends_at_zero = std::fabs(shifted(shift, smin)) < 1e-5;
    if (ends_at_zero) n++;
    for (int k = 0; k < n; k++) s.push_back((float)shifted(shift, n == 1 ? smax : smax + (smin - smax) * k / (n - 1)));
    if (!ends_at_zero) s.push_back(0.f);
    return s;
}

Schedule sched_karras(int steps, double smin, double smax) {
    const double rho = 7.0, hi = std::pow(smax, 1.0 / rho), lo = std::pow(smin, 1.0 / rho);
    Schedule s;
    for (int k = 0; k < steps; k++) {
        const double f = steps == 1 ? 0.0 : (double)k / (steps - 1);
        s.push_back((float)std::pow(hi + f * (lo - hi), rho));
    }
    s.push_back(0.f);
    return s;
}

Schedule sched_exponential(int steps, double smin, double smax) {
    const double lhi = std::log(smax), llo = std::log(smin);
    Schedule s;
    for (int k = 0; k < steps; k++) s.push_back((float)std::exp(steps == 1 ? lhi : lhi + (llo - lhi) * k / (steps - 1)));
    s.push_back(0.f);
    return s;
}

Schedule sched_ddim_uniform(int steps, const std::vector<float>& tab) {
    Schedule up;  // ascending, then reversed
    int n = steps;
    if (std::fabs(tab[1]) < 1e-5) n++;
    else up.push_back(0.f);
    const int stride = std::max(1000 / n, 1);
    for (int x = 1; x < 1000; x += stride) up.push_back(tab[x]);
    return Schedule(up.rbegin(), up.rend());
}

Schedule sched_beta(int steps, const std::vector<float>& tab) {
    Schedule s;
    int prev = -1;
    for (int k = 0; k < steps; k++) {
        const int t = (int)std::nearbyint(beta_quantile(1.0 - (double)k / steps, 0.6, 0.6) * 999.0);
        if (t != prev) s.push_back(tab[t]);
        prev = t;
    }
    s.push_back(0.f);
    return s;
}

Schedule sched_linear_quadratic(int steps, double smax) {
    if (steps == 1) return {1.f, 0.f};
    const double thr = 0.025;
    const int lin = steps / 2, quad = steps - lin;
    const double diff = lin - thr * steps;
    const double qa = diff / (lin * (double)quad * quad), qb = thr / lin - 2 * diff / ((double)quad * quad),
                 qc = qa * lin * lin;
    Schedule s;
    auto put = [&](double v) { s.push_back((float)((1.0 - v) * smax)); };
    for (int k = 0; k < lin; k++) put(k * thr / lin);
    for (int k = lin; k < steps; k++) put(qa * k * k + qb * k + qc);
    put(1.0);
    return s;
}

Schedule sched_kl_optimal(int steps, double smin, double smax) {
    Schedule s;
    const double amin = std::atan(smin), amax = std::atan(smax);
    for (int k = 0; k < steps; k++) {
        const double f = steps == 1 ? 0.0 : (double)k / (steps - 1);
        s.push_back((float)std::tan(f * amin + (1 - f) * amax));
    }
    s.push_back(0.f);
    return s;
}

Schedule full_schedule(const std::string& name, int steps, float shift) {
    const std::vector<float> tab = sigma_table(shift);
    const double smin = tab[0], smax = tab[999];
    if (name == "simple") return sched_simple(steps, tab);
    if (name == "normal") return sched_uniform_t(steps, shift, smin, smax, false);
    if (name == "sgm_uniform") return sched_uniform_t(steps, shift, smin, smax, true);
    if (name == "karras") return sched_karras(steps, smin, smax);
    if (name == "exponential") return sched_exponential(steps, smin, smax);
    if (name == "ddim_uniform") return sched_ddim_uniform(steps, tab);
    if (name == "beta") return sched_beta(steps, tab);
    if (name == "linear_quadratic") return sched_linear_quadratic(steps, smax);
    if (name == "kl_optimal") return sched_kl_optimal(steps, smin, smax);
    throw std::runtime_error("unknown scheduler " + name);
}

// partial denoise: the last steps + 1 sigmas of the schedule of (int)(steps / denoise) steps, with the reference's
// float denoise and its double division (pipeline.cu:67, 265-272)
bool partial(float denoise) { return !(denoise > 0.9999f); }
int partial_total(int steps, float denoise) { return (int)((double)steps / (double)denoise); }

Schedule tail(Schedule s, int steps) {
    if ((int)s.size() < steps + 1) return s;
    return Schedule(s.end() - (steps + 1), s.end());
}

}  // namespace

std::vector<float> flow_sigmas(int steps, float shift, float denoise) {
    if (steps < 1) throw std::runtime_error("flow_sigmas: steps < 1");
    if (denoise <= 0.f) return {};
    const int total = partial(denoise) ? partial_total(steps, denoise) : steps;
    if (total < steps) throw std::runtime_error("flow_sigmas: denoise must be in (0, 1]");
    return tail(sched_simple(total, sigma_table(shift)), steps);
}

std::vector<float> schedule_sigmas(const std::string& name, int steps, float shift, float denoise) {
    if (steps < 1) throw std::runtime_error("schedule_sigmas: steps < 1");
    if (!known_scheduler(name)) throw std::runtime_error("unknown scheduler " + name);
    if (!partial(denoise)) return full_schedule(name, steps, shift);
    if (denoise <= 0.f) return {};
    return tail(full_schedule(name, partial_total(steps, denoise), shift), steps);
}

bool known_scheduler(const std::string& n) {
    static const char* names[] = {"simple", "normal", "sgm_uniform", "karras", "exponential", "ddim_uniform",
                                  "beta", "linear_quadratic", "kl_optimal"};
    for (const char* k : names)
        if (n == k) return true;
    return false;
}

bool known_sampler(const std::string& n) {
    return n == "euler" || n == "euler_ancestral" || n == "dpmpp_2m" || n == "res_multistep" || n == "er_sde";
}

// The regularized incomplete beta function I_x(a, b) from its continued fraction (DLMF 8.17.22), evaluated
// with the modified Lentz algorithm, on the side of the symmetry I_x(a, b) = 1 - I_{1-x}(b, a) where the
// fraction converges fast (x < (a + 1) / (a + b + 2)).
double beta_cdf(double x, double a, double b) {
    if (x <= 0.0) return 0.0;
    if (x >= 1.0) return 1.0;
    if (x > (a + 1.0) / (a + b + 2.0)) return 1.0 - beta_cdf(1.0 - x, b, a);
    const double tiny = 1e-300;
    // prefactor x^a (1 - x)^b / (a B(a, b))
    const double lbeta = std::lgamma(a) + std::lgamma(b) - std::lgamma(a + b);
    const double front = std::exp(a * std::log(x) + b * std::log1p(-x) - lbeta) / a;
    // 1 / (1 + d1 / (1 + d2 / (1 + ...))): d_{2m+1} = -(a + m)(a + b + m) x / ((a + 2m)(a + 2m + 1)),
    // d_{2m} = m (b - m) x / ((a + 2m - 1)(a + 2m))
    auto coef = [&](int k) {
        const int m = k / 2;
        if (k % 2) return -(a + m) * (a + b + m) * x / ((a + 2 * m) * (a + 2 * m + 1));
        return m * (b - m) * x / ((a + 2 * m - 1) * (a + 2 * m));
    };
    double f = tiny, C = f, Dv = 0.0;
    for (int k = 0; k < 600; k++) {
        const double num = k == 0 ? 1.0 : coef(k);
        Dv = 1.0 + num * Dv;
        if (std::fabs(Dv) < tiny) Dv = tiny;
        C = 1.0 + num / C;
        if (std::fabs(C) < tiny) C = tiny;
        Dv = 1.0 / Dv;
        const double delta = C * Dv;
        f *= delta;
        if (k > 0 && std::fabs(delta - 1.0) < 1e-16) break;
    }
    // the loop's first term (num = 1) seeds f = 1 / (1 + d1 / ...) with a leading 0 + 1 / ..., so f is the fraction
    return front * f;
}

double beta_quantile(double p, double a, double b) {
    if (p <= 0.0) return 0.0;
    if (p >= 1.0) return 1.0;
    double lo = 0.0, hi = 1.0;
    for (int it = 0; it < 200 && hi - lo > 0.0; it++) {
        const double mid = 0.5 * (lo + hi);
        if (mid <= lo || mid >= hi) break;
        (beta_cdf(mid, a, b) < p ? lo : hi) = mid;
    }
    return 0.5 * (lo + hi);
}

StepCoef step_coef(const std::string& sampler, const std::vector<float>& sig, int i, bool have_old) {
    const double s = sig[i], sn = sig[i + 1];
    if (sampler == "euler" || !have_old || sn == 0.0) return {(float)(sn / s), (float)(1.0 - sn / s), 0.f};
    // log-sigma time t = -log sigma, step h = t_{i+1} - t_i (ComfyUI's k-diffusion, deterministic variants)
    const double t = -std::log(s), tn = -std::log(sn), tp = -std::log((double)sig[i - 1]), h = tn - t;
    if (sampler == "dpmpp_2m") {
        const double r = (t - tp) / h, em = -std::expm1(-h);
        return {(float)(sn / s), (float)(em * (1.0 + 1.0 / (2.0 * r))), (float)(-em / (2.0 * r))};
    }
    // res_multistep with eta 0: phi functions of -h, c2 = (t_prev - t) / h
    const double c2 = (tp - t) / h, phi1 = std::expm1(-h) / (-h), phi2 = (phi1 - 1.0) / (-h);
    return {(float)std::exp(-h), (float)(h * (phi1 - phi2 / c2)), (float)(h * (phi2 / c2))};
}

ErSdeCoef ersde_coef(const std::vector<float>& sig, int i) {
    // lambda = sigma / (1 - sigma), alpha = 1 - sigma, noise scaler f(l) = l (exp(l^0.3) + 10)
    auto lam = [&](int k) { const double v = sig[k]; return v / (1.0 - v); };
    auto f = [](double l) { return l * (std::exp(std::pow(l, 0.3)) + 10.0); };
    const double ls = lam(i), lt = lam(i + 1);
    const double al_s = sig[i] / ls, al_t = sig[i + 1] / lt;
    const double r = f(lt) / f(ls);
    ErSdeCoef c{};
    c.stage = std::min(3, i + 1);
    c.a = (float)(al_t / al_s * r);
    c.b = (float)(al_t * (1.0 - r));
    if (c.stage >= 2) {
        // integrals of 1/f and (l - l_i)/f over [l_{i+1}, l_i]: 200-point left sums from l_{i+1}
        const double dl = lt - ls, h = -dl / 200.0;
        double s1 = 0.0, s2 = 0.0;
        for (int k = 0; k < 200; k++) {
            const double l = lt + k * h, fl = f(l);
            s1 += 1.0 / fl;
            s2 += (l - ls) / fl;
        }
        s1 *= h;
        s2 *= h;
        c.c2 = (float)(al_t * (dl + s1 * f(lt)));
        c.inv2 = (float)(1.0 / (ls - lam(i - 1)));
        if (c.stage >= 3) {
            c.c3 = (float)(al_t * (dl * dl / 2.0 + s2 * f(lt)));
            c.inv3 = (float)(2.0 / (ls - lam(i - 2)));
        }
    }
    c.cn = (float)(al_t * std::sqrt(std::max(0.0, lt * lt - ls * ls * r * r)));
    return c;
}

// ---- sample() ----

SampleResult sample(VelocityModel& model, float* x, int Hl, int Wl, bool negative, const SampleParams& sp,
                    const float* init, const float* mask, const StepFn& on_step,
                    const std::function<bool()>& cancelled, hipStream_t stream) {
    const int P = Hl * Wl;
    const size_t n = (size_t)16 * P;
    const kiln_stream_t st = ks(stream);
    if (!known_sampler(sp.sampler)) throw std::runtime_error("unknown sampler " + sp.sampler);
    if (mask && !init) throw std::runtime_error("an inpainting mask needs init");
    std::vector<float> sig =
        !sp.sigmas.empty() ? sp.sigmas : schedule_sigmas(sp.scheduler, sp.steps, sp.shift, sp.denoise);
    const int steps = (int)sig.size() - 1;
    SampleResult res;
    res.steps = std::max(steps, 0);
    if (steps < 1) {  // nothing to do (denoise 0): the result is the input
        if (init) ck_hip(hipMemcpyAsync(x, init, n * 4, hipMemcpyDeviceToDevice, stream), "copy init");
        return res;
    }
    // host noise: none, given, or torch_randn(seed, n) (pipeline.cu:428-429)
    std::vector<float> nh(n, 0.f);
    if (sp.add_noise) {
        if (sp.noise) std::copy(sp.noise, sp.noise + n, nh.begin());
        else ck(kiln_torch_randn(nh.data(), sp.seed, n), "torch_randn");
    }
    const bool ersde = sp.sampler == "er_sde", ancestral = sp.sampler == "euler_ancestral";
    const int nbuf = 4 + (mask ? 1 : 0) + (negative ? 1 : 0) + (ersde || ancestral ? 1 : 0) + (ersde ? 1 : 0);
    DeviceBuffer buf(n * 4 * nbuf);
    float* p = buf.get<float>();
    float* noise = p;
    float* v = p + n;
    float* den = p + 2 * n;
    float* old = p + 3 * n;
    int k = 4;
    float* vn = negative ? p + n * k++ : nullptr;
    float* xin = mask ? p + n * k++ : x;
    float* anoise = ersde || ancestral ? p + n * k++ : nullptr;
    float* oldd = ersde ? p + n * k++ : nullptr;
    ck_hip(hipMemcpyAsync(noise, nh.data(), n * 4, hipMemcpyHostToDevice, stream), "noise upload");
    ck_hip(hipStreamSynchronize(stream), "noise upload");

    const int cfg_steps = negative ? (int)std::ceil(sp.cfg_until * steps - 1e-4f) : 0;
    const bool use_cache = sp.cache_threshold > 0.f;
    const int warm = std::max(2, (int)std::ceil(sp.cache_start * steps));
    const int tailn = std::max(1, (int)std::ceil((1.f - sp.cache_end) * steps));
    const int max_hits = sp.cache_max_hits < 0 ? steps : sp.cache_max_hits;
    int run = 0;
    bool have_old = false;
    ck(kiln_flow_start(x, noise, init, sig[0], n, st), "flow_start");
    if (ersde && sig[0] >= 1.f) sig[0] = 1.f - 1e-4f;  // lambda = sigma / (1 - sigma) needs sigma < 1

    std::vector<float> nz(ersde || ancestral ? n : 0);
    for (int i = 0; i < steps; i++) {
        if (cancelled && cancelled()) throw Cancelled();
        const auto t0 = std::chrono::steady_clock::now();
        const float s = sig[i], sn = sig[i + 1];
        if (mask) ck(kiln_flow_inpaint_in(xin, x, noise, init, mask, s, P, st), "inpaint input");
        const bool allow = use_cache && i >= warm && i < steps - tailn && run < max_hits;
        const bool cfg_now = negative && i < cfg_steps;
        bool skipped = false;
        float* outs[2] = {v, vn};
        model.forward(outs, xin, s * sp.timestep_mult, cfg_now, allow, &skipped);
        if (cfg_now) ck(kiln_cfg_combine(v, vn, sp.cfg, n, st), "cfg_combine");
        if (use_cache) {
            if (skipped) res.cache_skips++, run++;
            else run = 0;
        }
        if (on_step) {
            ck_hip(hipStreamSynchronize(stream), "step");
            on_step(i + 1, steps, s, x, v,
                    std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
        }
        if (mask) ck(kiln_flow_denoised_masked(den, xin, v, init, mask, s, P, st), "denoised");
        else ck(kiln_flow_denoised(den, xin, v, s, n, st), "denoised");
        if (sp.sampler == "euler") {
            ck(kiln_flow_euler_den(x, den, s, sn, n, st), "euler step");
        } else if (ancestral) {
            // the rectified-flow ancestral step with eta 1 and fresh noise torch_randn(seed + 1 + i)
            if (sn == 0.f) {
                ck(kiln_flow_update(x, den, nullptr, 0.f, 1.f, 0.f, n, st), "final step");
            } else {
                const double dsn = sn, sd = dsn * (1.0 + (dsn / s - 1.0)), aip1 = 1.0 - dsn, ad = 1.0 - sd;
                const double renoise = std::sqrt(std::max(0.0, dsn * dsn - sd * sd * aip1 * aip1 / (ad * ad)));
                const double r = sd / s, a = aip1 / ad;
                ck(kiln_torch_randn(nz.data(), sp.seed + 1 + i, n), "torch_randn");
                ck_hip(hipMemcpyAsync(anoise, nz.data(), n * 4, hipMemcpyHostToDevice, stream), "noise upload");
                ck(kiln_flow_update(x, den, nullptr, (float)(a * r), (float)(a * (1.0 - r)), 0.f, n, st), "ancestral");
                ck(kiln_flow_update(x, anoise, nullptr, 1.f, (float)renoise, 0.f, n, st), "renoise");
                ck_hip(hipStreamSynchronize(stream), "noise upload");  // nz is rewritten next step
            }
        } else if (ersde) {
            if (sn == 0.f) {
                ck(kiln_flow_update(x, den, nullptr, 0.f, 1.f, 0.f, n, st), "final step");
            } else {
                const ErSdeCoef c = ersde_coef(sig, i);
                ck(kiln_torch_randn(nz.data(), sp.seed + 1 + i, n), "torch_randn");
                ck_hip(hipMemcpyAsync(anoise, nz.data(), n * 4, hipMemcpyHostToDevice, stream), "noise upload");
                ck(kiln_flow_ersde_step(x, den, old, oldd, anoise, c.a, c.b, c.c2, c.inv2, c.c3, c.inv3, c.cn, c.stage,
                                        n, st),
                   "er_sde step");
                ck_hip(hipStreamSynchronize(stream), "noise upload");
            }
        } else {
            const StepCoef co = step_coef(sp.sampler, sig, i, have_old);
            ck(kiln_flow_update(x, den, have_old ? old : nullptr, co.a, co.b, co.c, n, st), "sampler step");
        }
        std::swap(den, old);
        have_old = true;
    }
    // stopped above sigma 0 (leftover noise for a second pass): x / (1 - sigma_last) (pipeline.cu:583-588)
    if (sig.back() > 0.f && sig.back() < 1.f)
        ck(kiln_flow_update(x, x, nullptr, 1.f / (1.f - sig.back()), 0.f, 0.f, n, st), "inverse noise scaling");
    ck_hip(hipStreamSynchronize(stream), "sample");
    return res;
}

// ---- the DiT as the sampler's model ----

DitVelocity::DitVelocity(Dit& dit, int Hl, int Wl, const CachedContext* pos, const CachedContext* neg,
                         const NagParams& nag, float nag_sigma_end, float cache_threshold, bool batch, bool fp32)
    : dit_(dit), Hl_(Hl), Wl_(Wl), pos_(pos), neg_(neg), nag_(nag), nag_end_(nag_sigma_end), batch_(batch),
      fp32_(fp32) {
    sc_.threshold = cache_threshold;
}

void DitVelocity::forward(float* const* outs, const float* x, float t, bool cfg_now, bool cache_allow,
                          bool* cache_skipped) {
    NagParams nag = nag_;
    if (nag.neg && t / tmult_ < nag_end_) nag.neg = nullptr;  // NAG only while sigma >= nag_sigma_end
    sc_.allow = cache_allow;
    StepCache* sc = sc_.threshold > 0.f ? &sc_ : nullptr;
    if (cfg_now && batch_) {
        const CachedContext* cs[2] = {pos_, neg_};
        dit_.forward_batch(outs, x, Hl_, Wl_, t, cs, 2, nag, sc, fp32_);
    } else {
        // an unbatched CFG run would skip the prompt pass but not the negative one: no cache there
        StepCache* use = (!neg_ || batch_) ? sc : nullptr;
        const CachedContext* cs[1] = {pos_};
        dit_.forward_batch(outs, x, Hl_, Wl_, t, cs, 1, nag, use, fp32_);
        if (cfg_now) {  // the negative pass never gets NAG
            const CachedContext* cn[1] = {neg_};
            float* on[1] = {outs[1]};
            dit_.forward_batch(on, x, Hl_, Wl_, t, cn, 1, NagParams(), nullptr, fp32_);
        }
    }
    *cache_skipped = sc && sc_.skipped;
}

}  // namespace kiln
