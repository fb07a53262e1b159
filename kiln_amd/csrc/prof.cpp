// Per-category GPU timing of the library's entry points (the reference's ProfScope / prof_report,
// engine/src/kernels.cu:14-58): while enabled, every entry point records a hipEvent pair around its launches on the
// caller's stream; the report waits for the events and sums them per category. Disabled (the default) a scope
// costs one flag test.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/kiln_attn.h"
#include "capi_util.hpp"

namespace kiln::prof {

namespace {
struct Pair {
    const char* name;
    hipEvent_t a = nullptr, b = nullptr;
};
std::atomic<bool> g_on{false};
std::mutex g_mu;
std::vector<Pair> g_pairs;  // the event pool; [0, g_used) hold this profile's scopes
size_t g_used = 0;
unsigned g_gen = 0;            // bumped by kiln_prof_enable: scopes of an earlier profile record nothing more
thread_local int t_depth = 0;  // a scope inside another one (an entry point calling another) is not timed
}  // namespace

// The thread's depth counts every scope that was entered while profiling was on, timed or not, so that a failed
// event call cannot leave the depth raised (which would make every later scope look nested).
Scope::Scope(const char* name, hipStream_t s) {
    if (!g_on.load(std::memory_order_relaxed)) return;
    counted_ = true;
    if (t_depth++ > 0) return;
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_used == g_pairs.size()) {
        Pair p{name};
        if (hipEventCreate(&p.a) != hipSuccess) return;
        if (hipEventCreate(&p.b) != hipSuccess) {
            (void)hipEventDestroy(p.a);
            return;
        }
        g_pairs.push_back(p);
    }
    if (hipEventRecord(g_pairs[g_used].a, s) != hipSuccess) return;
    slot_ = (int)g_used++;
    g_pairs[slot_].name = name;
    gen_ = g_gen;
    s_ = s;
}

Scope::~Scope() {
    if (counted_) t_depth--;
    if (slot_ < 0) return;
    std::lock_guard<std::mutex> lk(g_mu);
    if (gen_ == g_gen) (void)hipEventRecord(g_pairs[slot_].b, s_);  // a re-enabled profile may own the slot now
}

}  // namespace kiln::prof

extern "C" {

int kiln_prof_enable(int on) {
    std::lock_guard<std::mutex> lk(kiln::prof::g_mu);
    kiln::prof::g_used = 0;
    kiln::prof::g_gen++;
    kiln::prof::g_on = on != 0;
    return KILN_OK;
}

int kiln_prof_category(const char* name, double* ms, int* calls) {
    using namespace kiln::prof;
    if (!name || !ms || !calls) return kiln::capi::fail(KILN_EINVAL, "prof_category: null argument");
    std::lock_guard<std::mutex> lk(g_mu);
    double t = 0.0;
    int n = 0;
    for (size_t i = 0; i < g_used; i++) {
        if (strcmp(g_pairs[i].name, name) != 0) continue;
        if (hipEventSynchronize(g_pairs[i].b) != hipSuccess) return kiln::capi::fail(KILN_EHIP, "prof: event wait");
        float e = 0.f;
        if (hipEventElapsedTime(&e, g_pairs[i].a, g_pairs[i].b) != hipSuccess)
            return kiln::capi::fail(KILN_EHIP, "prof: elapsed time");
        t += e, n++;
    }
    *ms = t, *calls = n;
    return KILN_OK;
}

int kiln_prof_report(char* buf, size_t buflen) {
    using namespace kiln::prof;
    if (!buf || !buflen) return kiln::capi::fail(KILN_EINVAL, "prof_report: no buffer");
    std::map<std::string, std::pair<double, int>> acc;
    double total = 0.0;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        for (size_t i = 0; i < g_used; i++) {
            if (hipEventSynchronize(g_pairs[i].b) != hipSuccess) return kiln::capi::fail(KILN_EHIP, "prof: event wait");
            float e = 0.f;
            if (hipEventElapsedTime(&e, g_pairs[i].a, g_pairs[i].b) != hipSuccess)
                return kiln::capi::fail(KILN_EHIP, "prof: elapsed time");
            acc[g_pairs[i].name].first += e;
            acc[g_pairs[i].name].second++;
            total += e;
        }
    }
    std::string out;
    char line[160];
    for (auto& [n, v] : acc) {
        snprintf(line, sizeof line, "%-14s %8.2f ms %5.1f%% (%d calls)\n", n.c_str(), v.first,
                 total > 0 ? 100.0 * v.first / total : 0.0, v.second);
        out += line;
    }
    snprintf(line, sizeof line, "%-14s %8.2f ms\n", "sum", total);
    out += line;
    snprintf(buf, buflen, "%s", out.c_str());
    return out.size() < buflen ? KILN_OK : kiln::capi::fail(KILN_ENOMEM, "prof_report: buffer too small");
}

}  // extern "C"
