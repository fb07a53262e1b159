// engine_main.cpp - kiln_engine: the engine process of Kiln's JSON-lines protocol (the reference's
// engine/src/main.cpp:620-801, parse_job :562-600, Engine::generate engine.h:672-792) on MI355X, driving the DiT
// through the C++ step driver (dit.hpp, sampler.hpp).
//
// stdin: one JSON request per line (generate, cancel, info; graph / train / tag / ext_* are answered with an
// error: those subsystems are not part of this build). stdout: one JSON event per line (ready, loading, encoded,
// step, decoded, done, error, cancelled, info, log). A reader thread takes requests and one worker thread runs
// generate jobs from a queue; cancel stops the running job between steps or removes a queued one.
//
// This build has no checkpoint loader, text encoder or VAE (outside the attention path it was built for): the
// DiT has 2B-shaped random-init weights (torch Linear's default U(+-1/sqrt(in)), norm weights 1, --weights-seed),
// the text context of a prompt is a fixed pseudo-random embedding per Qwen token id (N(0,1)-like rows, one per
// id, padded to max(512, ids)), and "decoding" maps the final latent to RGB through the latent preview factors,
// upsampled 8x. Everything between (conditioning contexts -> sampling with CFG / NAG / step cache -> latent) is
// the real DiT path.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <fstream>
#include <iostream>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#include "dit.hpp"
#include "json.hpp"
#include "sampler.hpp"

namespace {

using Clock = std::chrono::steady_clock;
double ms_since(Clock::time_point t) { return std::chrono::duration<double, std::milli>(Clock::now() - t).count(); }

std::mutex g_out_mu;
void emit(const std::string& line) {
    std::lock_guard<std::mutex> lk(g_out_mu);
    fwrite(line.data(), 1, line.size(), stdout);
    fputc('\n', stdout);
    fflush(stdout);
}
void log_msg(const std::string& m) { emit("{\"ev\":\"log\",\"msg\":" + kiln::json::quote(m) + "}"); }
std::string ev(const std::string& id, const std::string& name) {
    return "{\"id\":" + kiln::json::quote(id) + ",\"ev\":\"" + name + "\"";
}

std::string base64(const uint8_t* p, size_t n) {
    static const char A[] = "ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz0123456789+/";
    std::string o;
    o.reserve((n + 2) / 3 * 4);
    size_t i = 0;
    for (; i + 3 <= n; i += 3) {
        const uint32_t v = (uint32_t)p[i] << 16 | (uint32_t)p[i + 1] << 8 | p[i + 2];
        o += A[v >> 18], o += A[(v >> 12) & 63], o += A[(v >> 6) & 63], o += A[v & 63];
    }
    if (i < n) {
        const uint32_t v = (uint32_t)p[i] << 16 | (i + 1 < n ? (uint32_t)p[i + 1] << 8 : 0);
        o += A[v >> 18], o += A[(v >> 12) & 63];
        o += i + 1 < n ? A[(v >> 6) & 63] : '=';
        o += '=';
    }
    return o;
}

// latent -> RGB approximation of the 16-channel latent space (ComfyUI's latent_rgb_factors for the Wan2.1 VAE,
// the table the reference's previews use, engine.h:64-70): rgb = bias + sum_c latent_c * F[c]
const float PREVIEW_F[16][3] = {
    {-0.1299f, -0.1692f, 0.2932f}, {0.0671f, 0.0406f, 0.0442f},   {0.3568f, 0.2548f, 0.1747f},
    {0.0372f, 0.2344f, 0.1420f},   {0.0313f, 0.0189f, -0.0328f},  {0.0296f, -0.0956f, -0.0665f},
    {-0.3477f, -0.4059f, -0.2925f}, {0.0166f, 0.1902f, 0.1975f},  {-0.0412f, 0.0267f, -0.1364f},
    {-0.1293f, 0.0740f, 0.1636f},  {0.0680f, 0.3019f, 0.1128f},   {0.0032f, 0.0581f, 0.0639f},
    {-0.1251f, 0.0927f, 0.1699f},  {0.0060f, -0.0633f, 0.0005f},  {0.3477f, 0.2275f, 0.2950f},
    {0.1984f, 0.0913f, 0.1861f}};
const float PREVIEW_B[3] = {-0.1835f, -0.0868f, -0.3360f};

uint8_t to8(float v) { return (uint8_t)(std::min(1.f, std::max(0.f, (v + 1.f) / 2.f)) * 255.f); }

// RGB8 [Hl * up, Wl * up, 3] of the latent lat [16, Hl, Wl] (host), each latent pixel an up x up block
std::vector<uint8_t> latent_rgb(const std::vector<float>& lat, int Hl, int Wl, int up) {
    const size_t P = (size_t)Hl * Wl;
    std::vector<uint8_t> px(P * 3);
    for (size_t p = 0; p < P; p++)
        for (int k = 0; k < 3; k++) {
            float v = PREVIEW_B[k];
            for (int c = 0; c < 16; c++) v += lat[c * P + p] * PREVIEW_F[c][k];
            px[p * 3 + k] = to8(v);
        }
    if (up == 1) return px;
    const int W = Wl * up;
    std::vector<uint8_t> out((size_t)Hl * up * W * 3);
    for (int y = 0; y < Hl * up; y++)
        for (int x = 0; x < W; x++)
            memcpy(&out[((size_t)y * W + x) * 3], &px[((size_t)(y / up) * Wl + x / up) * 3], 3);
    return out;
}

struct Job {
    std::string id, family, sampler, scheduler, out;
    std::vector<int> pos_ids, neg_ids;
    int width = 512, height = 768, steps = 8;
    float cfg = 1.f, cfg_until = 1.f, shift = 3.f, cache = 0.f;
    uint64_t seed = 0;
    bool preview = true, fp32 = false, skip_decode = false;
    struct {
        bool on = false;
        float scale = 5.f, tau = 2.5f, alpha = 0.25f;
    } nag;
    std::vector<std::string> ignored;  // requested features this build does not run (hires, face, ...)
};

std::vector<int> token_ids(const kiln::json::Value& v) {
    std::vector<int> ids;
    for (auto& x : v["qwen_ids"].items()) ids.push_back((int)x.i64());
    if (ids.empty()) ids.push_back(151643);  // the reference's empty-prompt token (main.cpp:537)
    return ids;
}

// parse_job (main.cpp:562-600): the same fields, defaults and clamps
Job parse_job(const kiln::json::Value& r) {
    Job j;
    j.family = r["family"].str("anima");
    j.id = r["id"].str();
    j.scheduler = r["scheduler"].str(j.family == "sdxl" ? "karras" : "simple");
    j.pos_ids = token_ids(r);
    j.neg_ids = token_ids(r["neg"]);
    const int align = j.family == "sdxl" ? 32 : 16;
    j.width = std::max(align, (int)r["width"].i64(512) / align * align);
    j.height = std::max(align, (int)r["height"].i64(768) / align * align);
    j.steps = std::max(1, (int)r["steps"].i64(8));
    j.cfg = (float)r["cfg"].num(1.0);
    j.cfg_until = std::min(1.f, std::max(0.f, (float)r["cfg_cutoff"].num(1.0)));
    j.sampler = r["sampler"].str("euler");
    j.cache = std::max(0.f, (float)r["step_cache"].num(0.0));
    if (r.has("nag")) {
        const auto& n = r["nag"];
        j.nag.on = n["enabled"].is_null() ? true : n["enabled"].boolean();
        j.nag.scale = std::max(1.f, (float)n["scale"].num(5.0));
        j.nag.tau = std::max(1.f, (float)n["tau"].num(2.5));
        j.nag.alpha = std::min(1.f, std::max(0.f, (float)n["alpha"].num(0.25)));
    }
    j.shift = (float)r["shift"].num(3.0);
    j.seed = (uint64_t)r["seed"].num(0);
    j.preview = r["preview"].is_null() ? true : r["preview"].boolean();
    j.out = r["out"].str();
    j.fp32 = r["precision"].str() == "fp32";
    j.skip_decode = r["skip_decode"].boolean();
    for (const char* k : {"hires", "face", "upscale"})
        if (r.has(k)) j.ignored.push_back(k);
    if (!r["loras"].items().empty()) j.ignored.push_back("loras");
    return j;
}

// splitmix64 (a published 64-bit mixer) -> a pseudo-random embedding row per token id
uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

class Engine {
   public:
    std::atomic<bool> cancel{false};

    Engine(const kiln::DitDims& dims, uint64_t wseed, hipStream_t s) : dims_(dims), s_(s), dit_(dims, s) {
        init_weights(wseed);
    }
    std::string gpu_name() const { return gpu_; }
    void set_gpu_name(const std::string& n) { gpu_ = n; }

    void generate(const Job& j);
    int bench(int W, int H);

   private:
    kiln::DitDims dims_;
    hipStream_t s_;
    kiln::Dit dit_;
    std::string gpu_;

    void fill(kiln::DeviceBuffer& b, size_t n, uint64_t seed, float bound) {
        b.resize(n * 2);
        kiln::ck(kiln_fill_uniform_bf16(b.get<uint16_t>(), n, seed, -bound, bound, (kiln_stream_t)s_), "init");
    }
    void init_weights(uint64_t seed);
    std::unique_ptr<kiln::CachedContext> condition(const std::vector<int>& ids, bool fp32);
};

void Engine::init_weights(uint64_t seed) {
    const size_t D = dims_.D(), F = dims_.F(), C = dims_.ctx_dim;
    uint64_t k = seed * 1000003ULL;
    kiln::DeviceBuffer ones;
    ones.resize(std::max<size_t>(D, 128) * 2);
    kiln::ck(kiln_fill_uniform_bf16(ones.get<uint16_t>(), std::max<size_t>(D, 128), 0, 1.f, 1.f, (kiln_stream_t)s_),
             "init");
    auto lin = [&](kiln::DeviceBuffer& b, size_t out, size_t in) { fill(b, out * in, ++k, 1.f / sqrtf((float)in)); };
    for (int i = 0; i < dims_.blocks; i++) {
        kiln::DeviceBuffer w[20];
        lin(w[0], D, D), lin(w[1], D, D), lin(w[2], D, D), lin(w[3], D, D);  // sa q k v o
        lin(w[4], D, D), lin(w[5], D, D);                                    // ca q o
        lin(w[6], D, C), lin(w[7], D, C);                                    // ca k v
        lin(w[8], F, D), lin(w[9], D, F);                                    // mlp
        for (int m = 0; m < 3; m++) lin(w[10 + 2 * m], 256, D), lin(w[11 + 2 * m], 3 * D, 256);
        const uint16_t* one = ones.get<uint16_t>();
        kiln::BlockWeights bw{w[0].get<uint16_t>(),  w[1].get<uint16_t>(),  w[2].get<uint16_t>(),  w[3].get<uint16_t>(),
                              w[4].get<uint16_t>(),  w[5].get<uint16_t>(),  w[6].get<uint16_t>(),  w[7].get<uint16_t>(),
                              w[8].get<uint16_t>(),  w[9].get<uint16_t>(),  one, one, one, one,
                              w[10].get<uint16_t>(), w[11].get<uint16_t>(), w[12].get<uint16_t>(),
                              w[13].get<uint16_t>(), w[14].get<uint16_t>(), w[15].get<uint16_t>()};
        dit_.set_block(i, bw);  // copies (and synchronizes), so the buffers can go
    }
    kiln::DeviceBuffer t1, t2, f1, f2, xe, fl;
    lin(t1, D, D), lin(t2, 3 * D, D), lin(f1, 256, D), lin(f2, 2 * D, 256), lin(xe, D, 68), lin(fl, 64, D);
    dit_.set_step_weights({t1.get<uint16_t>(), t2.get<uint16_t>(), ones.get<uint16_t>(), f1.get<uint16_t>(),
                           f2.get<uint16_t>(), xe.get<uint16_t>(), fl.get<uint16_t>()});
    kiln::ck_hip(hipStreamSynchronize(s_), "weights");
}

std::unique_ptr<kiln::CachedContext> Engine::condition(const std::vector<int>& ids, bool fp32) {
    const int C = dims_.ctx_dim, real = (int)ids.size(), len = std::max(512, real);
    std::vector<float> h((size_t)real * C);
    for (int r = 0; r < real; r++)
        for (int c = 0; c < C; c++) {
            // Irwin-Hall sum of 4 uniforms: mean 0, variance 1
            const uint64_t z = mix64(((uint64_t)(uint32_t)ids[r] << 20) ^ (uint64_t)c);
            float s = 0.f;
            for (int q = 0; q < 4; q++) s += (float)((z >> (16 * q)) & 0xFFFF) / 65536.f;
            h[(size_t)r * C + c] = (s - 2.f) * sqrtf(3.f);
        }
    kiln::DeviceBuffer d(h.size() * 4);
    kiln::ck_hip(hipMemcpyAsync(d.get(), h.data(), h.size() * 4, hipMemcpyHostToDevice, s_), "context upload");
    auto c = dit_.cache_context(d.get<float>(), real, len, fp32);  // synchronizes
    return c;
}

void Engine::generate(const Job& j) {
    const auto t0 = Clock::now();
    std::ostringstream tm;
    try {
        if (j.family != "anima") throw std::runtime_error("family " + j.family + " is not supported by this engine");
        if (!kiln::known_sampler(j.sampler)) throw std::runtime_error("unknown sampler " + j.sampler);
        if (!kiln::known_scheduler(j.scheduler)) throw std::runtime_error("unknown scheduler " + j.scheduler);
        if (!j.skip_decode && j.out.empty()) throw std::runtime_error("missing out path");
        for (auto& f : j.ignored) log_msg(f + " is not supported by this engine build; rendering without it");
        const auto te = Clock::now();
        auto pos = condition(j.pos_ids, j.fp32);
        const bool use_neg = j.cfg > 1.f;
        const bool use_nag = !use_neg && j.nag.on;  // NAG is the negative prompt's route when CFG is off
        std::unique_ptr<kiln::CachedContext> nctx;
        if (use_neg || use_nag) nctx = condition(j.neg_ids, j.fp32);
        const double enc_ms = ms_since(te);
        emit(ev(j.id, "encoded") + ",\"ms\":" + std::to_string((int)enc_ms) + "}");
        tm << "\"encode_ms\":" << (int)enc_ms;

        const int H = j.height, W = j.width, Hl = H / 8, Wl = W / 8;
        const size_t n = (size_t)16 * Hl * Wl;
        kiln::DeviceBuffer xb(n * 4);
        kiln::SampleParams sp;
        sp.steps = j.steps, sp.cfg = j.cfg, sp.shift = j.shift, sp.seed = j.seed, sp.cfg_until = j.cfg_until;
        sp.sampler = j.sampler, sp.scheduler = j.scheduler, sp.cache_threshold = j.cache;
        kiln::NagParams nag;
        if (use_nag) nag.neg = nctx.get(), nag.scale = j.nag.scale, nag.tau = j.nag.tau, nag.alpha = j.nag.alpha;
        kiln::DitVelocity model(dit_, Hl, Wl, pos.get(), use_neg ? nctx.get() : nullptr, nag, 0.f, j.cache, true,
                                j.fp32);
        double sample_ms = 0;
        std::vector<float> hx(n), hv(n), x0(n);
        auto on_step = [&](int step, int steps, float s, const float* x, const float* v, double ms) {
            sample_ms += ms;
            std::string pv;
            if (j.preview) {  // the denoised estimate x - v s through the preview factors, at latent size
                kiln::ck_hip(hipMemcpy(hx.data(), x, n * 4, hipMemcpyDeviceToHost), "preview");
                kiln::ck_hip(hipMemcpy(hv.data(), v, n * 4, hipMemcpyDeviceToHost), "preview");
                for (size_t i = 0; i < n; i++) x0[i] = hx[i] - hv[i] * s;
                const std::vector<uint8_t> px = latent_rgb(x0, Hl, Wl, 1);
                pv = ",\"preview\":{\"w\":" + std::to_string(Wl) + ",\"h\":" + std::to_string(Hl) + ",\"rgb\":\"" +
                     base64(px.data(), px.size()) + "\"}";
            }
            emit(ev(j.id, "step") + ",\"stage\":\"base\",\"step\":" + std::to_string(step) + ",\"of\":" +
                 std::to_string(steps) + ",\"ms\":" + std::to_string((int)ms) + pv + "}");
        };
        const kiln::SampleResult r = kiln::sample(model, xb.get<float>(), Hl, Wl, use_neg, sp, nullptr, nullptr, on_step,
                                                  [this]() { return cancel.load(); }, s_);
        tm << ",\"sample_ms\":" << (int)sample_ms;
        if (j.cache > 0.f) tm << ",\"cache_skips\":" << r.cache_skips;
        if (j.skip_decode) {
            emit(ev(j.id, "done") + ",\"skipped_decode\":true}");
            return;
        }
        const auto td = Clock::now();
        kiln::ck_hip(hipMemcpy(hx.data(), xb.get(), n * 4, hipMemcpyDeviceToHost), "latent");
        const std::vector<uint8_t> img = latent_rgb(hx, Hl, Wl, 8);
        const double dec_ms = ms_since(td);
        emit(ev(j.id, "decoded") + ",\"ms\":" + std::to_string((int)dec_ms) + "}");
        tm << ",\"decode_ms\":" << (int)dec_ms << ",\"arena_peak_mb\":" << (dit_.arena_peak() >> 20);
        std::ofstream f(j.out, std::ios::binary);
        if (!f) throw std::runtime_error("cannot write " + j.out);
        f.write(reinterpret_cast<const char*>(img.data()), (std::streamsize)img.size());
        f.close();
        if (!f) throw std::runtime_error("cannot write " + j.out);
        emit(ev(j.id, "done") + ",\"out\":" + kiln::json::quote(j.out) + ",\"w\":" + std::to_string(W) + ",\"h\":" +
             std::to_string(H) + ",\"total_ms\":" + std::to_string((int)ms_since(t0)) + ",\"timings\":{" + tm.str() +
             "}}");
    } catch (const kiln::Cancelled&) {
        (void)hipStreamSynchronize(s_);
        emit(ev(j.id, "cancelled") + "}");
    } catch (const std::exception& e) {
        (void)hipStreamSynchronize(s_);
        (void)hipGetLastError();
        emit(ev(j.id, "error") + ",\"msg\":" + kiln::json::quote(e.what()) + "}");
    }
}

// --bench WxH (main.cpp:110-150): the warm time of one DiT forward of the CFG pair at W x H with NAG on the prompt
// item, then its per-category GPU profile (kiln_prof_*), as log events
int Engine::bench(int W, int H) {
    const int Hl = H / 8, Wl = W / 8;
    const size_t n = (size_t)16 * Hl * Wl;
    std::vector<int> ids(24);
    for (int i = 0; i < 24; i++) ids[i] = 1000 + 37 * i;
    auto pos = condition(ids, false);
    auto neg = condition({151643}, false);
    auto nagc = condition({9, 8, 7}, false);
    kiln::DeviceBuffer x(n * 4), o(2 * n * 4);
    std::vector<float> h(n);
    for (size_t i = 0; i < n; i++) h[i] = (float)((mix64(i) >> 40) * (1.0 / 16777216.0)) * 2.f - 1.f;
    kiln::ck_hip(hipMemcpy(x.get(), h.data(), n * 4, hipMemcpyHostToDevice), "latent");
    float* outs[2] = {o.get<float>(), o.get<float>() + n};
    const kiln::CachedContext* cs[2] = {pos.get(), neg.get()};
    kiln::NagParams nag;
    nag.neg = nagc.get();
    auto fwd = [&] { dit_.forward_batch(outs, x.get<float>(), Hl, Wl, 0.9f, cs, 2, nag); };
    fwd();  // warm-up (arena, RoPE tables, code objects)
    kiln::ck_hip(hipStreamSynchronize(s_), "bench");
    const auto t0 = Clock::now();
    for (int i = 0; i < 3; i++) fwd();
    kiln::ck_hip(hipStreamSynchronize(s_), "bench");
    char b[200];
    snprintf(b, sizeof b, "DiT forward of the CFG pair at %dx%d (latent %dx%d): %.2f ms", W, H, Wl, Hl, ms_since(t0) / 3);
    log_msg(b);
    kiln::ck(kiln_prof_enable(1), "prof");
    fwd();
    std::vector<char> rep(1 << 14);
    kiln::ck(kiln_prof_report(rep.data(), rep.size()), "prof report");
    kiln::ck(kiln_prof_enable(0), "prof");
    std::istringstream ss(rep.data());
    std::string line;
    while (std::getline(ss, line)) log_msg(line);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    int device = 0;
    uint64_t wseed = 1;
    int bench_w = 0, bench_h = 0;
    kiln::DitDims dims;  // the 2B model: 28 blocks, 16 heads, 1024-wide contexts
    for (int i = 1; i < argc; i++) {
        const std::string a = argv[i];
        auto next = [&]() { return i + 1 < argc ? std::string(argv[++i]) : std::string(); };
        try {
            if (a == "--device") device = std::stoi(next());
            else if (a == "--blocks") dims.blocks = std::stoi(next());
            else if (a == "--heads") dims.heads = std::stoi(next());
            else if (a == "--ctx-dim") dims.ctx_dim = std::stoi(next());
            else if (a == "--weights-seed") wseed = std::stoull(next());
            else if (a == "--bench") {
                const std::string wh = next();
                bench_w = std::stoi(wh);
                bench_h = std::stoi(wh.substr(wh.find('x') + 1));
            }
            else if (a == "--help") {
                printf("kiln_engine [--device N] [--blocks 28] [--heads 16] [--ctx-dim 1024] [--weights-seed S] "
                       "[--bench WxH]\n");
                return 0;
            }
        } catch (const std::exception&) {
            emit("{\"ev\":\"fatal\",\"msg\":" + kiln::json::quote("bad value for " + a) + "}");
            return 1;
        }
    }
    std::unique_ptr<Engine> E;
    hipStream_t stream = nullptr;
    try {
        kiln::ck_hip(hipSetDevice(device), "hipSetDevice");
        hipDeviceProp_t prop;
        kiln::ck_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
        kiln::ck_hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
        log_msg(std::string("GPU: ") + (prop.name[0] ? prop.name : "AMD Instinct") + " (" + prop.gcnArchName + ", " +
                std::to_string(prop.totalGlobalMem >> 30) + " GB): fp16 MFMA path ON");
        emit("{\"ev\":\"loading\",\"what\":\"dit\"}");
        E = std::make_unique<Engine>(dims, wseed, stream);
        E->set_gpu_name(prop.name[0] ? std::string(prop.name) : std::string("AMD ") + prop.gcnArchName);
        log_msg("DiT: " + std::to_string(dims.blocks) + " blocks x " + std::to_string(dims.heads) +
                " heads, random-init weights (seed " + std::to_string(wseed) + "); text encoder and VAE: stand-ins");
    } catch (const std::exception& e) {
        emit(std::string("{\"ev\":\"fatal\",\"msg\":") + kiln::json::quote(e.what()) + "}");
        return 1;
    }
    if (bench_w > 0 && bench_h > 0) {
        try {
            return E->bench(bench_w / 16 * 16, bench_h / 16 * 16);
        } catch (const std::exception& e) {
            log_msg(std::string("bench failed: ") + e.what());
            return 1;
        }
    }
    emit("{\"ev\":\"ready\",\"gpu\":" + kiln::json::quote(E->gpu_name()) + ",\"tc\":true,\"tc16\":true}");

    std::mutex mu;
    std::condition_variable cv;
    struct Work {
        std::string id;
        Job job;
    };
    std::deque<Work> queue;
    std::string running;
    bool quit = false;

    std::thread worker([&] {
        kiln::ck_hip(hipSetDevice(device), "hipSetDevice");
        for (;;) {
            Work w;
            {
                std::unique_lock<std::mutex> lk(mu);
                cv.wait(lk, [&] { return quit || !queue.empty(); });
                if (queue.empty()) return;
                w = std::move(queue.front());
                queue.pop_front();
                running = w.id;
                E->cancel = false;
            }
            E->generate(w.job);
            std::lock_guard<std::mutex> lk(mu);
            running.clear();
        }
    });

    std::string line;
    while (std::getline(std::cin, line)) {
        if (line.size() >= 3 && (uint8_t)line[0] == 0xEF && (uint8_t)line[1] == 0xBB && (uint8_t)line[2] == 0xBF)
            line.erase(0, 3);
        while (!line.empty() && (line.back() == '\r' || line.back() == ' ')) line.pop_back();
        if (line.empty()) continue;
        kiln::json::Value r;
        try {
            r = kiln::json::parse(line);
        } catch (const std::exception& e) {
            log_msg(std::string("bad request: ") + e.what());
            continue;
        }
        const std::string cmd = r["cmd"].str(), id = r["id"].str();
        if (cmd == "generate") {
            Work w{id, parse_job(r)};
            std::lock_guard<std::mutex> lk(mu);
            queue.push_back(std::move(w));
            cv.notify_one();
        } else if (cmd == "cancel") {
            std::lock_guard<std::mutex> lk(mu);
            if (running == id) E->cancel = true;
            for (auto it = queue.begin(); it != queue.end(); ++it)
                if (it->id == id) {
                    queue.erase(it);
                    emit(ev(id, "cancelled") + "}");
                    break;
                }
        } else if (cmd == "info") {
            size_t fr = 0, tot = 0;
            (void)hipMemGetInfo(&fr, &tot);
            emit(ev(id, "info") + ",\"gpu\":" + kiln::json::quote(E->gpu_name()) + ",\"vram_free_mb\":" +
                 std::to_string(fr >> 20) + ",\"family\":\"anima\",\"tc\":true,\"features\":{\"ext\":false," +
                 "\"train\":false,\"tag\":false,\"face\":false}}");
        } else if (cmd == "graph" || cmd == "train" || cmd == "tag" || cmd == "ext_result" || cmd == "ext_op") {
            emit(ev(id, "error") + ",\"msg\":" + kiln::json::quote("command " + cmd + " is not supported by this engine") +
                 "}");
        } else {
            log_msg("unknown cmd " + cmd);
        }
    }
    {  // stdin closed: finish what is queued, then exit
        std::lock_guard<std::mutex> lk(mu);
        quit = true;
    }
    cv.notify_one();
    worker.join();
    E.reset();
    (void)hipStreamDestroy(stream);
    return 0;
}
