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

// Flow-space model sampling (ComfyUI's ModelSamplingDiscreteFlow with shift s): sigma(t) = s t / (1 + (s - 1) t),
// and the model's discrete table holds sigma((i + 1) / 1000) in float32 (pipeline.cu:66-78, 100-107). A flow
// model's timestep is its sigma, so the schedulers that work in timestep space apply only the shift.
struct FlowSpace {
    double shift;
    std::vector<float> table;  // ascending: table[0] = sigma_min, table[999] = sigma_max

    explicit FlowSpace(float s) : shift(s), table(1000) {
        for (int i = 0; i < 1000; i++) {
            const float t = (float)(i + 1) / 1000.f;
            table[i] = s == 1.f ? t : s * t / (1.f + (s - 1.f) * t);
        }
    }
    double lo() const { return table.front(); }
    double hi() const { return table.back(); }
    double sigma(double t) const { return shift == 1.0 ? t : shift * t / (1.0 + (shift - 1.0) * t); }
};

// Schedules have `steps` steps (steps + 1 sigmas, or fewer where a scheduler drops repeats) and end in 0.
using Schedule = std::vector<float>;

// The fraction k / (n - 1) of n evenly spaced points (the single point of n = 1 sits at 0).
double frac(int k, int n) { return n == 1 ? 0.0 : (double)k / (n - 1); }

// Schedulers that space the steps evenly in a warped coordinate w(sigma) between w(sigma_max) and w(sigma_min)
// and map back: karras (w = sigma^(1/7), Karras et al. 2022, eq. 5), exponential (w = log sigma) and
// kl_optimal (w = atan sigma, Sabour et al. 2024).
template <class W, class Winv>
Schedule warped(const FlowSpace& fs, int steps, W w, Winv winv) {
    const double top = w(fs.hi()), bottom = w(fs.lo());
    Schedule s(steps + 1, 0.f);
    for (int k = 0; k < steps; k++) s[k] = (float)winv(top + frac(k, steps) * (bottom - top));
    return s;
}

// Schedulers that space timesteps evenly: normal (steps points from sigma_max to sigma_min; if the last
// one maps to 0 it becomes an extra step instead of the appended 0) and sgm_uniform (steps + 1 points, the last
// replaced by 0). ComfyUI's normal_scheduler.
Schedule timestep_uniform(const FlowSpace& fs, int steps, bool sgm) {
    const double t0 = fs.hi(), t1 = fs.lo();
    const bool extra = !sgm && std::fabs(fs.sigma(t1)) < 1e-5;
    const int n = extra ? steps + 1 : steps;
    Schedule s;
    for (int k = 0; k < n; k++) {
        const double u = sgm ? (double)k / steps : frac(k, n);
        s.push_back((float)fs.sigma(t0 + u * (t1 - t0)));
    }
    if (!extra) s.push_back(0.f);
    return s;
}

// Schedulers that pick entries of the model's table by index (ComfyUI's simple, ddim_uniform and beta
// schedulers). Repeated indices are dropped where the scheduler asks for it.
Schedule from_table(const FlowSpace& fs, const std::vector<int>& idx, bool drop_repeats) {
    Schedule s;
    for (size_t k = 0; k < idx.size(); k++)
        if (!drop_repeats || k == 0 || idx[k] != idx[k - 1]) s.push_back(fs.table[idx[k]]);
    s.push_back(0.f);
    return s;
}

std::vector<int> idx_simple(int steps) {  // every 1000/steps-th entry from the top
    std::vector<int> idx(steps);
    const double stride = 1000.0 / steps;
    for (int k = 0; k < steps; k++) idx[k] = 999 - (int)(k * stride);
    return idx;
}

std::vector<int> idx_beta(int steps) {  // the Beta(0.6, 0.6) quantiles of 1 - k/steps, rounded to the table
    std::vector<int> idx(steps);
    for (int k = 0; k < steps; k++) idx[k] = (int)std::nearbyint(beta_quantile(1.0 - (double)k / steps, 0.6, 0.6) * 999.0);
    return idx;
}

// ddim_uniform: entries 1, 1 + c, 1 + 2c, ... (c = 1000 / steps) from the bottom of the table, reversed, after a 0
// unless entry 1 is itself ~0 (then one more step). The 0 comes first in ascending order, so it ends the schedule.
Schedule ddim_uniform(const FlowSpace& fs, int steps) {
    const bool zero_at_1 = std::fabs(fs.table[1]) < 1e-5;
    const int c = std::max(1000 / (zero_at_1 ? steps + 1 : steps), 1);
    Schedule s;
    for (int x = 1; x < 1000; x += c) s.push_back(fs.table[x]);
    std::reverse(s.begin(), s.end());
    if (!zero_at_1) s.push_back(0.f);
    return s;
}

// linear_quadratic (ComfyUI, from Movie Gen): the noise level nu rises linearly to 0.025 over the first half of
// the steps, then along the quadratic that meets it there and reaches 1 at the end; sigma = (1 - nu) sigma_max.
Schedule linear_quadratic(const FlowSpace& fs, int steps) {
    if (steps == 1) return {1.f, 0.f};
    const double th = 0.025;
    const int nl = steps / 2, nq = steps - nl;
    const double excess = nl - th * steps;  // what the quadratic part must add above a straight continuation
    const double q2 = excess / (nl * (double)nq * nq), q1 = th / nl - 2 * excess / ((double)nq * nq), q0 = q2 * nl * nl;
    auto nu = [&](int k) { return k < nl ? k * th / nl : q2 * k * k + q1 * k + q0; };
    Schedule s(steps + 1);
    for (int k = 0; k < steps; k++) s[k] = (float)((1.0 - nu(k)) * fs.hi());
    s[steps] = 0.f;  // nu = 1
    return s;
}

Schedule full_schedule(const std::string& name, int steps, float shift) {
    const FlowSpace fs(shift);
    if (name == "simple") return from_table(fs, idx_simple(steps), false);
    if (name == "beta") return from_table(fs, idx_beta(steps), true);
    if (name == "ddim_uniform") return ddim_uniform(fs, steps);
    if (name == "normal" || name == "sgm_uniform") return timestep_uniform(fs, steps, name == "sgm_uniform");
    if (name == "karras")
        return warped(fs, steps, [](double v) { return std::pow(v, 1.0 / 7.0); }, [](double w) { return std::pow(w, 7.0); });
    if (name == "exponential")
        return warped(fs, steps, [](double v) { return std::log(v); }, [](double w) { return std::exp(w); });
    if (name == "kl_optimal")
        return warped(fs, steps, [](double v) { return std::atan(v); }, [](double w) { return std::tan(w); });
    if (name == "linear_quadratic") return linear_quadratic(fs, steps);
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
    return tail(full_schedule("simple", total, shift), steps);
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

namespace {
// phi_1(z) = (e^z - 1) / z and phi_2(z) = (phi_1(z) - 1) / z, the weights of exponential integrators.
double phi1(double z) { return std::expm1(z) / z; }
double phi2(double z) { return (phi1(z) - 1.0) / z; }
}  // namespace

// The deterministic samplers in exponential-integrator form (ComfyUI's sample_euler, sample_dpmpp_2m and
// sample_res_multistep with eta 0, in the data-prediction parameterization of Lu et al., DPM-Solver++): with the
// log-sigma time lambda = -log sigma and the step h = lambda_{i+1} - lambda_i, the latent keeps the share
// e^-h = sigma_{i+1} / sigma_i and the remaining 1 - e^-h = h phi_1(-h) goes to a combination of the current and
// the previous data estimates, which the second-order methods extrapolate over the previous step h_prev.
LinearStep linear_step(const std::string& sampler, const std::vector<float>& sig, int i, bool have_old) {
    const double s_now = sig[i], s_next = sig[i + 1];
    LinearStep w{(float)(s_next / s_now), (float)(1.0 - s_next / s_now), 0.f};  // first order: Euler = DDIM
    if (sampler == "euler" || !have_old || s_next == 0.0) return w;
    const double lam = -std::log(s_now), lam_next = -std::log(s_next), lam_prev = -std::log((double)sig[i - 1]);
    const double h = lam_next - lam, h_prev = lam - lam_prev;
    if (sampler == "dpmpp_2m") {
        // data estimate extrapolated to the middle of the step: (1 + 1/2r) den - 1/2r old, r = h_prev / h
        const double share = -std::expm1(-h), half_inv_r = h / (2.0 * h_prev);
        w.den_w = (float)(share * (1.0 + half_inv_r));
        w.old_w = (float)(-share * half_inv_r);
        return w;
    }
    // res_multistep: second-order Adams-type weights through the previous node at c = -h_prev / h
    const double c = -h_prev / h, p1 = phi1(-h), p2 = phi2(-h);
    w.x_w = (float)std::exp(-h);
    w.den_w = (float)(h * (p1 - p2 / c));
    w.old_w = (float)(h * (p2 / c));
    return w;
}

namespace {
// The left Riemann sum of g over [lo, hi] with n points (ComfyUI's er_sde integrates with 200 of them).
template <class G>
double left_sum(G g, double lo, double hi, int n) {
    const double dx = (hi - lo) / n;
    double acc = 0.0;
    for (int k = 0; k < n; k++) acc += g(lo + k * dx);
    return acc * dx;
}
}  // namespace

// er_sde (Cui et al. 2025, "Elucidating the solution space of extended reverse-time SDEs"; ComfyUI's
// sample_er_sde with max_stage 3 and its default noise scaler), for a flow model: the SDE runs in
// lambda = sigma / alpha with alpha = 1 - sigma, and the noise scaler is f(lambda) = lambda (e^(lambda^0.3) + 10).
// From lambda_i to lambda_{i+1} = lambda_i + dl:
//   x' = (alpha'/alpha) r x + alpha' (1 - r) den                                    r = f(lambda') / f(lambda)
//      + alpha' (dl + f(lambda') int 1/f) D1                   from the 2nd step,  D1 = (den - old) / (lambda - lambda_{i-1})
//      + alpha' (dl^2 / 2 + f(lambda') int (l - lambda)/f) D2  from the 3rd step,  D2 = (D1 - D1_prev) 2 / (lambda - lambda_{i-2})
//      + alpha' sqrt(lambda'^2 - lambda^2 r^2) noise
// with both integrals over [lambda', lambda].
ErSdeStep ersde_step(const std::vector<float>& sig, int i) {
    auto lambda = [&](int k) { return (double)sig[k] / (1.0 - (double)sig[k]); };
    auto f = [](double l) { return l * (std::exp(std::pow(l, 0.3)) + 10.0); };
    const double l_now = lambda(i), l_next = lambda(i + 1), dl = l_next - l_now;
    const double alpha_now = sig[i] / l_now, alpha_next = sig[i + 1] / l_next;  // = 1 - sigma, as ComfyUI forms it
    const double r = f(l_next) / f(l_now);
    ErSdeStep e{};
    e.order = std::min(3, i + 1);
    e.x_w = (float)(alpha_next / alpha_now * r);
    e.den_w = (float)(alpha_next * (1.0 - r));
    e.noise_w = (float)(alpha_next * std::sqrt(std::max(0.0, l_next * l_next - l_now * l_now * r * r)));
    if (e.order < 2) return e;
    const double i1 = left_sum([&](double l) { return 1.0 / f(l); }, l_next, l_now, 200);
    e.d1_w = (float)(alpha_next * (dl + i1 * f(l_next)));
    e.d1_inv = (float)(1.0 / (l_now - lambda(i - 1)));
    if (e.order < 3) return e;
    const double i2 = left_sum([&](double l) { return (l - l_now) / f(l); }, l_next, l_now, 200);
    e.d2_w = (float)(alpha_next * (dl * dl / 2.0 + i2 * f(l_next)));
    e.d2_inv = (float)(2.0 / (l_now - lambda(i - 2)));
    return e;
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
        model.forward(outs, xin, s, s * sp.timestep_mult, cfg_now, allow, &skipped);
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
                const ErSdeStep e = ersde_step(sig, i);
                ck(kiln_torch_randn(nz.data(), sp.seed + 1 + i, n), "torch_randn");
                ck_hip(hipMemcpyAsync(anoise, nz.data(), n * 4, hipMemcpyHostToDevice, stream), "noise upload");
                ck(kiln_flow_ersde_step(x, den, old, oldd, anoise, e.x_w, e.den_w, e.d1_w, e.d1_inv, e.d2_w, e.d2_inv, e.noise_w, e.order,
                                        n, st),
                   "er_sde step");
                ck_hip(hipStreamSynchronize(stream), "noise upload");
            }
        } else {
            const LinearStep w = linear_step(sp.sampler, sig, i, have_old);
            ck(kiln_flow_update(x, den, have_old ? old : nullptr, w.x_w, w.den_w, w.old_w, n, st), "sampler step");
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

void DitVelocity::forward(float* const* outs, const float* x, float sigma, float t, bool cfg_now, bool cache_allow,
                          bool* cache_skipped) {
    NagParams nag = nag_;
    if (nag.neg && !(sigma >= nag_end_)) nag.neg = nullptr;  // NAG only while sigma >= nag_sigma_end
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
