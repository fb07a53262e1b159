// C++ harness of the DiT block attention section (engine/src/dit.cu:458-488) through the reference-named host
// mirror (kiln_amd/host/kiln_gpu.hpp): a CFG batch of 2 on an 8x12 patch grid, 4 heads, fp32 activations (the
// reference engine's `big` buffers), two blocks, three contexts with zero padding (ContextKV: prompt 40 of 64
// rows real, unconditional 64 of 64, NAG negative 33 of 64), self-attention with QK-RMSNorm + Cosmos RoPE, and
// cross-attention with NAG on item 0. A host reference in double precision restates the same steps
// (kernels.cu:656-666 RMSNorm, 759-772 RoPE, 809-826 attention with npad zero keys, dit.cu:295-324 NAG).
// Then the block's linear layers: a bf16 weight prepared at load (kiln::Linear16Weight, weight_to_f16) and
// linear16 with the GELU16 and gated-residual epilogues (kernels.cu:573-609) against a double restatement.
// Exit status 1 if any output leaves max-abs 2e-3 / mean-abs 2e-4.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "../../kiln_amd/host/kiln_gpu.hpp"

#define CK(x)                                                                                   \
    do {                                                                                        \
        hipError_t e_ = (x);                                                                    \
        if (e_ != hipSuccess) {                                                                 \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            std::exit(2);                                                                       \
        }                                                                                       \
    } while (0)

static const int H = 4, D = 128, LD = H * D, Hp = 8, Wp = 12, T = Hp * Wp, B = 2, NBLK = 2, LEN = 64;
static const float EPS = 1e-6f;

static float bf16f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
static float h2f(uint16_t h) {
    _Float16 x;
    std::memcpy(&x, &h, 2);
    return (float)x;
}

// per-head RMSNorm in place over rows [rows, LD]
static void rmsnorm(std::vector<double>& x, int rows, const std::vector<uint16_t>& w) {
    for (int r = 0; r < rows; r++)
        for (int h = 0; h < H; h++) {
            double* p = &x[(size_t)r * LD + h * D];
            double ss = 0;
            for (int d = 0; d < D; d++) ss += p[d] * p[d];
            const double inv = 1.0 / std::sqrt(ss / D + EPS);
            for (int d = 0; d < D; d++) p[d] = p[d] * inv * bf16f(w[d]);
        }
}
static void rope(std::vector<double>& x, const std::vector<float>& c, const std::vector<float>& s) {
    for (int t = 0; t < T; t++)
        for (int h = 0; h < H; h++) {
            double* p = &x[(size_t)t * LD + h * D];
            for (int i = 0; i < 64; i++) {
                const double a = p[i], b = p[i + 64], cc = c[t * 64 + i], ss = s[t * 64 + i];
                p[i] = a * cc - b * ss;
                p[i + 64] = b * cc + a * ss;
            }
        }
}
// softmax(q k^T / sqrt(D)) v per head with npad implicit zero keys
static std::vector<double> attn(const std::vector<double>& q, int Tq, const std::vector<double>& k,
                                const std::vector<double>& v, int Tk, int npad) {
    std::vector<double> o((size_t)Tq * LD);
    std::vector<double> sc(Tk);
    for (int t = 0; t < Tq; t++)
        for (int h = 0; h < H; h++) {
            double m = npad ? 0.0 : -INFINITY;
            for (int j = 0; j < Tk; j++) {
                double a = 0;
                for (int d = 0; d < D; d++) a += q[(size_t)t * LD + h * D + d] * k[(size_t)j * LD + h * D + d];
                sc[j] = a / std::sqrt((double)D);
                m = std::max(m, sc[j]);
            }
            double l = npad * std::exp(-m);
            std::vector<double> acc(D, 0.0);
            for (int j = 0; j < Tk; j++) {
                const double p = std::exp(sc[j] - m);
                l += p;
                for (int d = 0; d < D; d++) acc[d] += p * v[(size_t)j * LD + h * D + d];
            }
            for (int d = 0; d < D; d++) o[(size_t)t * LD + h * D + d] = acc[d] / l;
        }
    return o;
}
static void nag(std::vector<double>& a, const std::vector<double>& an, float s, float tau, float alpha) {
    for (int t = 0; t < T; t++) {
        double lp = 0, lg = 0;
        for (int i = 0; i < LD; i++) {
            const double p = a[(size_t)t * LD + i], g = p * s - an[(size_t)t * LD + i] * (s - 1);
            lp += std::fabs(p);
            lg += std::fabs(g);
        }
        const double ratio = lg / std::max(lp, 1e-12), kk = ratio > tau ? tau / ratio : 1.0;
        for (int i = 0; i < LD; i++) {
            const double p = a[(size_t)t * LD + i], g = p * s - an[(size_t)t * LD + i] * (s - 1);
            a[(size_t)t * LD + i] = alpha * g * kk + (1 - alpha) * p;
        }
    }
}

static bool compare(const char* what, const std::vector<uint16_t>& got, const std::vector<double>& ref, size_t off) {
    double mx = 0, mean = 0;
    const size_t n = ref.size();
    for (size_t i = 0; i < n; i++) {
        const double d = std::fabs((double)h2f(got[off + i]) - ref[i]);
        mx = std::max(mx, d);
        mean += d;
    }
    mean /= (double)n;
    const bool ok = mx <= 2e-3 && mean <= 2e-4 && std::isfinite(mx);
    printf("%-40s max-abs %.3e  mean-abs %.3e  %s\n", what, mx, mean, ok ? "ok" : "FAIL");
    return ok;
}

template <typename Tv>
static Tv* to_dev(const std::vector<Tv>& h) {
    Tv* d;
    CK(hipMalloc(&d, h.size() * sizeof(Tv)));
    CK(hipMemcpy(d, h.data(), h.size() * sizeof(Tv), hipMemcpyHostToDevice));
    return d;
}

int main() {
    std::mt19937 rng(11);
    std::normal_distribution<float> nd(0.f, 1.f);
    std::uniform_real_distribution<float> ud(0.75f, 1.25f);
    auto randv = [&](size_t n) {
        std::vector<float> v(n);
        for (auto& x : v) x = nd(rng);
        return v;
    };
    auto bf16w = [&]() {
        std::vector<uint16_t> w(D);
        for (auto& x : w) {
            const float f = ud(rng);
            uint32_t u;
            std::memcpy(&u, &f, 4);
            x = (uint16_t)(u >> 16);  // truncation: the weight IS this bf16 value
        }
        return w;
    };
    std::vector<float> rc(T * 64), rs(T * 64);
    kiln::check(kiln_cosmos_rope_tables(rc.data(), rs.data(), Hp, Wp), "rope tables");
    float* d_rc = to_dev(rc);
    float* d_rs = to_dev(rs);

    // contexts: rows [real, LEN) of each context are padding; only the real rows are projected and stored
    const int reals[3] = {40, 64, 33};
    kiln::ContextKV pos(NBLK, LEN, reals[0], H), unc(NBLK, LEN, reals[1], H), neg(NBLK, LEN, reals[2], H);
    kiln::ContextKV* ctx[3] = {&pos, &unc, &neg};
    std::vector<std::vector<float>> ck[3], cv[3];
    std::vector<std::vector<uint16_t>> ckn(NBLK);
    for (int blk = 0; blk < NBLK; blk++) ckn[blk] = bf16w();
    for (int c = 0; c < 3; c++)
        for (int blk = 0; blk < NBLK; blk++) {
            ck[c].push_back(randv((size_t)reals[c] * LD));
            cv[c].push_back(randv((size_t)reals[c] * LD));
            float* dk = to_dev(ck[c][blk]);
            float* dv = to_dev(cv[c][blk]);
            uint16_t* dw = to_dev(ckn[blk]);
            ctx[c]->prepare(blk, dk, dv, LD, KILN_F32, dw, EPS);
            CK(hipDeviceSynchronize());
            CK(hipFree(dk));
            CK(hipFree(dv));
            CK(hipFree(dw));
        }

    bool ok = true;
    std::vector<uint16_t> out((size_t)B * T * LD);
    uint16_t *d_out, *d_neg;
    CK(hipMalloc(&d_out, out.size() * 2));
    CK(hipMalloc(&d_neg, (size_t)T * LD * 2));
    kiln::Nag nagp;
    nagp.neg = &neg;
    for (int blk = 0; blk < NBLK; blk++) {
        // ---- self-attention ----
        auto q = randv((size_t)B * T * LD), k = randv((size_t)B * T * LD), v = randv((size_t)B * T * LD);
        auto qn = bf16w(), kn = bf16w();
        float *dq = to_dev(q), *dk = to_dev(k), *dv = to_dev(v);
        uint16_t *dqn = to_dev(qn), *dkn = to_dev(kn);
        kiln::dit_self_attention(d_out, LD, dq, dk, dv, KILN_F32, LD, dqn, dkn, EPS, d_rc, d_rs, B, T, H);
        CK(hipMemcpy(out.data(), d_out, out.size() * 2, hipMemcpyDeviceToHost));
        for (int b = 0; b < B; b++) {
            std::vector<double> Q(q.begin() + (size_t)b * T * LD, q.begin() + (size_t)(b + 1) * T * LD);
            std::vector<double> K(k.begin() + (size_t)b * T * LD, k.begin() + (size_t)(b + 1) * T * LD);
            std::vector<double> V(v.begin() + (size_t)b * T * LD, v.begin() + (size_t)(b + 1) * T * LD);
            rmsnorm(Q, T, qn);
            rmsnorm(K, T, kn);
            rope(Q, rc, rs);
            rope(K, rc, rs);
            char what[64];
            snprintf(what, sizeof what, "block %d self-attention item %d", blk, b);
            ok &= compare(what, out, attn(Q, T, K, V, T, 0), (size_t)b * T * LD);
        }
        // ---- cross-attention with NAG on item 0 ----
        auto qc = randv((size_t)B * T * LD);
        auto qcn = bf16w();
        float* dqc = to_dev(qc);
        uint16_t* dqcn = to_dev(qcn);
        const kiln::ContextKV* cs[2] = {&pos, &unc};
        kiln::dit_cross_attention(d_out, d_neg, LD, dqc, KILN_F32, LD, dqcn, EPS, B, T, H, blk, cs, nagp);
        CK(hipMemcpy(out.data(), d_out, out.size() * 2, hipMemcpyDeviceToHost));
        auto ctx_ref = [&](int c) {
            std::vector<double> K(ck[c][blk].begin(), ck[c][blk].end()), V(cv[c][blk].begin(), cv[c][blk].end());
            rmsnorm(K, reals[c], ckn[blk]);
            return std::make_pair(K, V);
        };
        for (int b = 0; b < B; b++) {
            std::vector<double> Q(qc.begin() + (size_t)b * T * LD, qc.begin() + (size_t)(b + 1) * T * LD);
            rmsnorm(Q, T, qcn);
            auto kv = ctx_ref(b);
            auto o = attn(Q, T, kv.first, kv.second, reals[b], LEN - reals[b]);
            if (b == 0) {
                auto kvn = ctx_ref(2);
                nag(o, attn(Q, T, kvn.first, kvn.second, reals[2], LEN - reals[2]), nagp.scale, nagp.tau, nagp.alpha);
            }
            char what[64];
            snprintf(what, sizeof what, "block %d cross-attention item %d%s", blk, b, b == 0 ? " + NAG" : "");
            ok &= compare(what, out, o, (size_t)b * T * LD);
        }
        for (void* p : {(void*)dq, (void*)dk, (void*)dv, (void*)dqn, (void*)dkn, (void*)dqc, (void*)dqcn}) CK(hipFree(p));
    }
    // ---- the block's linear layers through kiln::Linear16Weight (prepared at load from bf16) ----
    {
        const int R = B * T, IN = LD, OUT = 2 * LD;
        std::vector<uint16_t> xh((size_t)R * IN), wb((size_t)OUT * IN);
        std::vector<double> xd(xh.size()), wd(wb.size());
        for (size_t i = 0; i < xh.size(); i++) {
            const _Float16 h = (_Float16)nd(rng);
            std::memcpy(&xh[i], &h, 2);
            xd[i] = (double)h;
        }
        for (size_t i = 0; i < wb.size(); i++) {
            const float f = nd(rng) * 0.05f;
            uint32_t u;
            std::memcpy(&u, &f, 4);
            wb[i] = (uint16_t)(u >> 16);
            wd[i] = (double)(_Float16)bf16f(wb[i]);  // bf16 -> fp16 (round to nearest even), as weight_to_f16
        }
        std::vector<float> gate(OUT), res((size_t)R * OUT);
        for (auto& g : gate) g = nd(rng);
        for (auto& r : res) r = nd(rng);
        uint16_t *dx = to_dev(xh), *dwb = to_dev(wb), *dh;
        float *dg = to_dev(gate), *dr = to_dev(res);
        CK(hipMalloc(&dh, (size_t)R * OUT * 2));
        kiln::Linear16Weight W(dwb, OUT, IN, true);
        kiln::linear16(dh, OUT, dx, R, W, kiln::Epi16::Gelu16);
        kiln::linear16(dr, OUT, dx, R, W, kiln::Epi16::Resid, dg);
        std::vector<uint16_t> gh((size_t)R * OUT);
        std::vector<float> rr((size_t)R * OUT);
        CK(hipMemcpy(gh.data(), dh, gh.size() * 2, hipMemcpyDeviceToHost));
        CK(hipMemcpy(rr.data(), dr, rr.size() * 4, hipMemcpyDeviceToHost));
        double emg = 0, emr = 0;
        bool lok = true;
        for (int r = 0; r < R; r++)
            for (int n = 0; n < OUT; n++) {
                double acc = 0, aabs = 0;
                for (int k = 0; k < IN; k++) {
                    acc += xd[(size_t)r * IN + k] * wd[(size_t)n * IN + k];
                    aabs += std::fabs(xd[(size_t)r * IN + k] * wd[(size_t)n * IN + k]);
                }
                const double bar = std::sqrt((double)IN) * std::ldexp(1.0, -21) * aabs + 1e-7;
                const double gl = 0.5 * acc * (1.0 + std::erf(acc / std::sqrt(2.0)));
                const double eg = std::fabs((double)h2f(gh[(size_t)r * OUT + n]) - gl);
                const double ulp = std::ldexp(1.0, (int)std::floor(std::log2(std::max(std::fabs(gl), 6.1e-5))) - 10);
                const double rf = (double)res[(size_t)r * OUT + n] + (double)gate[n] * acc;
                const double er = std::fabs((double)rr[(size_t)r * OUT + n] - rf);
                lok &= eg <= bar + ulp && er <= bar * std::fabs(gate[n]) + std::fabs(rf) * std::ldexp(1.0, -23);
                emg = std::max(emg, eg);
                emr = std::max(emr, er);
            }
        printf("%-40s max-abs %.3e (GELU16) %.3e (RESID)  %s\n", "linear16 (prepared bf16 weight)", emg, emr,
               lok ? "ok" : "FAIL");
        ok &= lok;
        for (void* p : {(void*)dx, (void*)dwb, (void*)dh, (void*)dg, (void*)dr}) CK(hipFree(p));
    }
    printf("%s\n", ok ? "dit_section_test: all ok" : "dit_section_test: FAILED");
    return ok ? 0 : 1;
}
