// dit.cpp - the DiT forward over the C ABI of libkiln_attn.so (declarations in dit.hpp).
#include "dit.hpp"

#include <math.h>
#include <string.h>

#include <algorithm>

namespace kiln {

namespace {
constexpr int HD = 128;
constexpr int TOK = 68;  // patch tokens: 16 channels x 2 x 2 + 4 mask channels (dit.cu:174-182)

kiln_stream_t ks(hipStream_t s) { return (kiln_stream_t)s; }
}  // namespace

void ck(int rc, const char* what) {
    if (rc != KILN_OK)
        throw Error(rc, std::string(what) + ": " + kiln_attn_status_string(rc) + " (" + kiln_attn_last_error() + ")");
}

void ck_hip(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw Error(e == hipErrorOutOfMemory ? KILN_ENOMEM : KILN_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

void DeviceBuffer::reserve(size_t bytes) {
    if (bytes > n_) resize(bytes);
}

void DeviceBuffer::resize(size_t bytes) {
    release();
    if (!bytes) return;
    ck_hip(hipMalloc(&p_, bytes), "hipMalloc");
    n_ = bytes;
}

void DeviceBuffer::release() {
    if (p_) (void)hipFree(p_);
    p_ = nullptr;
    n_ = 0;
}

void Arena::reserve(size_t bytes) {
    if (bytes <= buf_.bytes()) return;
    if (top_ != 0) throw std::logic_error("arena: grown while slices are live");
    // the old buffer may still be read by queued work
    ck_hip(hipDeviceSynchronize(), "arena grow");
    buf_.resize(bytes);
}

void* Arena::take(size_t bytes) {
    const size_t off = (top_ + 255) / 256 * 256;
    if (off + bytes > buf_.bytes())
        throw Error(KILN_ENOMEM, "arena: " + std::to_string(off + bytes) + " bytes needed, " +
                                 std::to_string(buf_.bytes()) + " reserved");
    top_ = off + bytes;
    peak_ = std::max(peak_, top_);
    return buf_.get<char>() + off;
}

// ---- weights ----

// a bf16 copy of a device array of n elements
static DeviceBuffer copy_bf16(const uint16_t* src, size_t n, hipStream_t s, const char* what) {
    if (!src) throw std::runtime_error(std::string("missing weight ") + what);
    DeviceBuffer b(n * 2);
    ck_hip(hipMemcpyAsync(b.get(), src, n * 2, hipMemcpyDeviceToDevice, s), what);
    return b;
}

// a linear16 weight [rows, cols] converted from bf16 into the prepared fp16 layout
static DeviceBuffer prep16(const uint16_t* src_bf16, int rows, int cols, hipStream_t s, const char* what) {
    DeviceBuffer b(kiln_linear16_prepped_weight_bytes(rows, cols));
    ck(kiln_linear16_prepare_weight(b.get<uint16_t>(), src_bf16, rows, cols, 1, ks(s)), what);
    return b;
}

struct Dit::Block {
    // fp16 path: prepared fp16 weights
    DeviceBuffer qkv16, sa_o16, ca_q16, ca_o16, mlp1_16, mlp2_16;
    // bf16 copies: the fp32 path's linears, the context projections, the norm and modulation weights
    DeviceBuffer sa_q, sa_k, sa_v, sa_o, ca_q, ca_o, ca_k, ca_v, mlp1, mlp2;
    DeviceBuffer sa_qn, sa_kn, ca_qn, ca_kn;
    DeviceBuffer mod[6];
};

struct Dit::Rope {
    int Hp, Wp;
    DeviceBuffer cs;  // cos [T, 64] then sin [T, 64]
    const float* c() const { return cs.get<float>(); }
    const float* s() const { return cs.get<float>() + (size_t)Hp * Wp * 64; }
};

Dit::Dit(const DitDims& dims, hipStream_t stream) : d_(dims), s_(stream) {
    if (d_.blocks <= 0 || d_.heads <= 0 || d_.heads % 2 || d_.ctx_dim <= 0 || d_.ctx_dim % 32 || d_.F() % 256)
        throw std::runtime_error("Dit: unsupported dimensions (heads even, ctx_dim % 32 == 0, mlp % 256 == 0)");
    blocks_.resize(d_.blocks);
}

Dit::~Dit() = default;

void Dit::set_step_weights(const StepWeights& w) {
    const size_t D = d_.D();
    t_lin1_ = copy_bf16(w.t_lin1, D * D, s_, "t_lin1");
    t_lin2_ = copy_bf16(w.t_lin2, 3 * D * D, s_, "t_lin2");
    t_norm_ = copy_bf16(w.t_norm, D, s_, "t_norm");
    fmod1_ = copy_bf16(w.final_mod1, 256 * D, s_, "final_mod1");
    fmod2_ = copy_bf16(w.final_mod2, 2 * D * 256, s_, "final_mod2");
    x_embed_ = copy_bf16(w.x_embed, D * TOK, s_, "x_embed");
    final_lin_ = copy_bf16(w.final_lin, 64 * D, s_, "final_lin");
}

void Dit::set_block(int i, const BlockWeights& w) {
    if (i < 0 || i >= d_.blocks) throw std::runtime_error("set_block: index out of range");
    const int D = d_.D(), F = d_.F(), C = d_.ctx_dim;
    const size_t DD = (size_t)D * D;
    auto b = std::make_unique<Block>();
    b->sa_q = copy_bf16(w.sa_q, DD, s_, "sa_q");
    b->sa_k = copy_bf16(w.sa_k, DD, s_, "sa_k");
    b->sa_v = copy_bf16(w.sa_v, DD, s_, "sa_v");
    b->sa_o = copy_bf16(w.sa_o, DD, s_, "sa_o");
    b->ca_q = copy_bf16(w.ca_q, DD, s_, "ca_q");
    b->ca_o = copy_bf16(w.ca_o, DD, s_, "ca_o");
    b->ca_k = copy_bf16(w.ca_k, (size_t)D * C, s_, "ca_k");
    b->ca_v = copy_bf16(w.ca_v, (size_t)D * C, s_, "ca_v");
    b->mlp1 = copy_bf16(w.mlp1, (size_t)F * D, s_, "mlp1");
    b->mlp2 = copy_bf16(w.mlp2, (size_t)D * F, s_, "mlp2");
    b->sa_qn = copy_bf16(w.sa_qn, HD, s_, "sa_qn");
    b->sa_kn = copy_bf16(w.sa_kn, HD, s_, "sa_kn");
    b->ca_qn = copy_bf16(w.ca_qn, HD, s_, "ca_qn");
    b->ca_kn = copy_bf16(w.ca_kn, HD, s_, "ca_kn");
    const uint16_t* mods[6] = {w.mod_sa1, w.mod_sa2, w.mod_ca1, w.mod_ca2, w.mod_mlp1, w.mod_mlp2};
    for (int j = 0; j < 6; j++) b->mod[j] = copy_bf16(mods[j], (j % 2 ? 3 * (size_t)D * 256 : 256 * (size_t)D), s_, "mod");
    // the stacked self-attention projection [Wq; Wk; Wv] (one GEMM whose epilogue splits Q, K, V)
    DeviceBuffer qkv(3 * DD * 2);
    for (int j = 0; j < 3; j++) {
        const DeviceBuffer& src = j == 0 ? b->sa_q : j == 1 ? b->sa_k : b->sa_v;
        ck_hip(hipMemcpyAsync(qkv.get<char>() + j * DD * 2, src.get(), DD * 2, hipMemcpyDeviceToDevice, s_), "stack qkv");
    }
    b->qkv16 = prep16(qkv.get<uint16_t>(), 3 * D, D, s_, "sa_qkv");
    b->sa_o16 = prep16(b->sa_o.get<uint16_t>(), D, D, s_, "sa_o");
    b->ca_q16 = prep16(b->ca_q.get<uint16_t>(), D, D, s_, "ca_q");
    b->ca_o16 = prep16(b->ca_o.get<uint16_t>(), D, D, s_, "ca_o");
    b->mlp1_16 = prep16(b->mlp1.get<uint16_t>(), F, D, s_, "mlp1");
    b->mlp2_16 = prep16(b->mlp2.get<uint16_t>(), D, F, s_, "mlp2");
    ck_hip(hipStreamSynchronize(s_), "set_block");  // the stacking buffer goes out of scope
    blocks_[i] = std::move(b);
    mods_stacked_ = false;
}

const Dit::Rope& Dit::rope(int Hp, int Wp) {
    for (auto& r : ropes_)
        if (r->Hp == Hp && r->Wp == Wp) return *r;
    auto r = std::make_unique<Rope>();
    r->Hp = Hp, r->Wp = Wp;
    const size_t n = (size_t)Hp * Wp * 64;
    std::vector<float> h(2 * n);
    ck(kiln_cosmos_rope_tables(h.data(), h.data() + n, Hp, Wp), "cosmos_rope_tables");
    r->cs.resize(2 * n * 4);
    ck_hip(hipMemcpyAsync(r->cs.get(), h.data(), 2 * n * 4, hipMemcpyHostToDevice, s_), "rope upload");
    ck_hip(hipStreamSynchronize(s_), "rope upload");  // the host table goes out of scope (dit.cu:277)
    ropes_.push_back(std::move(r));
    return *ropes_.back();
}

std::unique_ptr<CachedContext> Dit::cache_context(const float* ctx, int real, int len, bool fp32) {
    if (real <= 0 || len < real || !ctx) throw std::runtime_error("cache_context: bad context");
    const int D = d_.D(), H = d_.heads, C = d_.ctx_dim;
    auto c = std::make_unique<CachedContext>();
    c->real = real, c->len = len;
    c->kv_per_block = kiln_kv_prepped_bytes(real, H);
    c->kv16.resize(c->kv_per_block * d_.blocks);
    if (fp32) {
        c->k32.resize((size_t)d_.blocks * real * D * 4);
        c->v32.resize((size_t)d_.blocks * real * D * 4);
    }
    const size_t m = arena_.mark();
    arena_.reserve(std::max(arena_.capacity(), (size_t)2 * real * D * 4 + 4096));
    float* k = arena_.f((size_t)real * D);
    float* v = arena_.f((size_t)real * D);
    for (int i = 0; i < d_.blocks; i++) {
        const Block& b = *blocks_.at(i);
        // K = rmsnorm(ctx W_k^T; ca_kn), V = ctx W_v^T (fp32 products of the bf16 weights)
        ck(kiln_linear_f32(k, D, ctx, C, b.ca_k.get<uint16_t>(), real, D, C, ks(s_)), "ctx K");
        ck(kiln_rmsnorm_rows(k, k, b.ca_kn.get<uint16_t>(), real * H, HD, d_.eps, ks(s_)), "ctx K norm");
        ck(kiln_linear_f32(v, D, ctx, C, b.ca_v.get<uint16_t>(), real, D, C, ks(s_)), "ctx V");
        ck(kiln_kv_prepare(const_cast<uint16_t*>(c->kv(i)), k, D, v, D, KILN_F32, real, H, nullptr, d_.eps, nullptr,
                           nullptr, ks(s_)),
           "ctx K/V prepare");
        if (fp32) {
            const size_t n = (size_t)real * D * 4;
            ck_hip(hipMemcpyAsync(c->k32.get<char>() + n * i, k, n, hipMemcpyDeviceToDevice, s_), "ctx K copy");
            ck_hip(hipMemcpyAsync(c->v32.get<char>() + n * i, v, n, hipMemcpyDeviceToDevice, s_), "ctx V copy");
        }
    }
    ck_hip(hipStreamSynchronize(s_), "cache_context");
    arena_.release(m);
    return c;
}

// ---- step tables (dit.cu:242-272) ----

static size_t step_tables_bytes(const DitDims& d) { return ((size_t)3 * d.blocks * 256 + 8 * (size_t)d.D()) * 4 + 8 * 256; }

void Dit::step_tables(float t, float* mods) {
    const int D = d_.D(), nb = d_.blocks;
    for (int i = 0; i < nb; i++)
        if (!blocks_[i]) throw std::runtime_error("step_tables: block " + std::to_string(i) + " has no weights");
    if (!t_lin1_.get()) throw std::runtime_error("step_tables: no step weights");
    if (!mods_stacked_) {  // every block's first modulation layers, then the second ones, contiguous
        const size_t n1 = 256 * (size_t)D * 2, n2 = 3 * (size_t)D * 256 * 2;
        mod1_all_.resize(3 * nb * n1);
        mod2_all_.resize(3 * nb * n2);
        for (int i = 0; i < nb; i++)
            for (int j = 0; j < 3; j++) {
                ck_hip(hipMemcpyAsync(mod1_all_.get<char>() + (3 * i + j) * n1, blocks_[i]->mod[2 * j].get(), n1,
                                      hipMemcpyDeviceToDevice, s_),
                       "stack mod1");
                ck_hip(hipMemcpyAsync(mod2_all_.get<char>() + (3 * i + j) * n2, blocks_[i]->mod[2 * j + 1].get(), n2,
                                      hipMemcpyDeviceToDevice, s_),
                       "stack mod2");
            }
        mods_stacked_ = true;
    }
    // the timestep sinusoid on the host, fp32 arithmetic: cos(t e_i), sin(t e_i), e_i = exp(-i ln(10000) / (D/2))
    std::vector<float> sh(D);
    const float lg = -logf(10000.f);
    for (int i = 0; i < D / 2; i++) {
        const float e = expf((float)i * lg / (float)(D / 2));
        sh[i] = cosf(t * e);
        sh[i + D / 2] = sinf(t * e);
    }
    if (arena_.mark() == 0) arena_.reserve(step_tables_bytes(d_));
    const size_t m = arena_.mark();
    float* s = arena_.f(D);
    float* s1 = arena_.f(D);
    float* lora = arena_.f(3 * (size_t)D);
    float* temb = arena_.f(D);
    float* hid = arena_.f((size_t)3 * nb * 256);
    float* h256 = arena_.f(256);
    ck_hip(hipMemcpyAsync(s, sh.data(), (size_t)D * 4, hipMemcpyHostToDevice, s_), "sinusoid upload");
    ck(kiln_matvec_bf16(s1, t_lin1_.get<uint16_t>(), s, nullptr, D, D, ks(s_)), "t_lin1");
    ck(kiln_silu(s1, s1, D, ks(s_)), "silu");
    ck(kiln_matvec_bf16(lora, t_lin2_.get<uint16_t>(), s1, nullptr, 3 * D, D, ks(s_)), "t_lin2");
    ck(kiln_rmsnorm_rows(temb, s, t_norm_.get<uint16_t>(), 1, D, d_.eps, ks(s_)), "t_norm");
    ck(kiln_silu(temb, temb, D, ks(s_)), "silu");  // every modulation MLP starts with SiLU
    // every block's three modulation MLPs in two launches (the reference: six matvecs per block)
    ck(kiln_matvec_bf16(hid, mod1_all_.get<uint16_t>(), temb, nullptr, 3 * nb * 256, D, ks(s_)), "mod first layers");
    ck(kiln_matvec_bf16_grouped(mods, mod2_all_.get<uint16_t>(), hid, lora, 3 * nb, 3 * D, 256, ks(s_)),
       "mod second layers");
    float* fmod = mods + (size_t)nb * 9 * D;
    ck(kiln_matvec_bf16(h256, fmod1_.get<uint16_t>(), temb, nullptr, 256, D, ks(s_)), "final_mod1");
    ck(kiln_matvec_bf16(fmod, fmod2_.get<uint16_t>(), h256, lora, 2 * D, 256, ks(s_)), "final_mod2");
    ck_hip(hipStreamSynchronize(s_), "step tables");  // the host sinusoid goes out of scope (dit.cu:277)
    arena_.release(m);
}

// ---- the block loop body ----

void Dit::block16(int i, float* X, const float* mods, int T, int B, const Rope& rp, const CachedContext* const* cs,
                  const NagParams& nag) {
    const Block& bl = *blocks_[i];
    const int D = d_.D(), F = d_.F(), H = d_.heads, R = B * T;
    const float eps = d_.eps;
    const float *mo = mods, *mc = mods + 3 * D, *mm = mods + 6 * D;
    const size_t m = arena_.mark();
    uint16_t* n16 = arena_.h((size_t)R * D);
    uint16_t* a16 = arena_.h((size_t)R * D);
    const size_t ws_bytes = std::max(kiln_dit_self_attn_x16_workspace_bytes(B, T, H), (size_t)R * D * 2);
    void* ws = arena_.take(ws_bytes);
    // self-attention: LN16 -> [Wq; Wk; Wv] GEMM whose epilogue applies the QK-RMSNorm and RoPE and writes fp16 Q and
    // the prepared K/V -> attention of the B items -> O projection added into X (dit.cu:460-471)
    ck(kiln_layernorm_mod16(n16, X, mo + D, mo, R, D, eps, ks(s_)), "LN16 self");
    ck(kiln_dit_self_attn_x16(a16, KILN_F16, D, n16, bl.qkv16.get<uint16_t>(), bl.sa_qn.get<uint16_t>(),
                              bl.sa_kn.get<uint16_t>(), eps, rp.c(), rp.s(), B, T, H, ws, ws_bytes, ks(s_)),
       "self-attention");
    ck(kiln_linear16_prepped(X, D, a16, R, bl.sa_o16.get<uint16_t>(), D, D, KILN_EPI_RESID, mo + 2 * D, 0.f, nullptr,
                             nullptr, 0, ks(s_)),
       "self O");
    // cross-attention: each item against its own context, NAG on item 0 (dit.cu:473-488)
    ck(kiln_layernorm_mod16(n16, X, mc + D, mc, R, D, eps, ks(s_)), "LN16 cross");
    const uint16_t* kvp[3];
    int Lk[3], np[3];
    for (int b = 0; b < B; b++) kvp[b] = cs[b]->kv(i), Lk[b] = cs[b]->real, np[b] = cs[b]->len - cs[b]->real;
    uint16_t* an16 = nag.neg ? arena_.h((size_t)T * D) : nullptr;
    const CachedContext* ng = nag.neg;
    ck(kiln_dit_cross_attn_x16(a16, an16, KILN_F16, D, n16, bl.ca_q16.get<uint16_t>(), bl.ca_qn.get<uint16_t>(), eps,
                               B, T, H, kvp, Lk, np, ng ? ng->kv(i) : nullptr, ng ? ng->real : 0,
                               ng ? ng->len - ng->real : 0, nag.scale, nag.tau, nag.alpha, ws, ws_bytes, ks(s_)),
       "cross-attention");
    ck(kiln_linear16_prepped(X, D, a16, R, bl.ca_o16.get<uint16_t>(), D, D, KILN_EPI_RESID, mc + 2 * D, 0.f, nullptr,
                             nullptr, 0, ks(s_)),
       "cross O");
    // MLP: GELU in the first GEMM's epilogue, the second adds into X (dit.cu:489-493)
    ck(kiln_layernorm_mod16(n16, X, mm + D, mm, R, D, eps, ks(s_)), "LN16 mlp");
    uint16_t* h16 = arena_.h((size_t)R * F);
    ck(kiln_linear16_prepped(h16, F, n16, R, bl.mlp1_16.get<uint16_t>(), F, D, KILN_EPI_GELU16, nullptr, 0.f, nullptr,
                             nullptr, 0, ks(s_)),
       "mlp1");
    ck(kiln_linear16_prepped(X, D, h16, R, bl.mlp2_16.get<uint16_t>(), D, F, KILN_EPI_RESID, mm + 2 * D, 0.f, nullptr,
                             nullptr, 0, ks(s_)),
       "mlp2");
    arena_.release(m);
}

void Dit::block32(int i, float* X, const float* mods, int T, int B, const Rope& rp, const CachedContext* const* cs,
                  const NagParams& nag) {
    const Block& bl = *blocks_[i];
    const int D = d_.D(), F = d_.F(), H = d_.heads, R = B * T;
    const float eps = d_.eps;
    const float *mo = mods, *mc = mods + 3 * D, *mm = mods + 6 * D;
    for (int b = 0; b < B; b++)
        if (!cs[b]->k32.get()) throw std::runtime_error("fp32 forward: context cached without fp32 K/V");
    if (nag.neg && !nag.neg->k32.get()) throw std::runtime_error("fp32 forward: NAG context cached without fp32 K/V");
    const size_t m = arena_.mark();
    const size_t RD = (size_t)R * D;
    float *N = arena_.f(RD), *Q = arena_.f(RD), *K = arena_.f(RD), *V = arena_.f(RD), *A = arena_.f(RD),
          *Y = arena_.f(RD);
    auto lin = [&](float* y, const float* x, int rows_in, const DeviceBuffer& w, int out, int in, const char* what) {
        ck(kiln_linear_f32(y, out, x, in, w.get<uint16_t>(), rows_in, out, in, ks(s_)), what);
    };
    // self-attention (dit.cu:497-509)
    ck(kiln_layernorm_mod(N, X, mo + D, mo, R, D, eps, ks(s_)), "LN self");
    lin(Q, N, R, bl.sa_q, D, D, "sa_q");
    lin(K, N, R, bl.sa_k, D, D, "sa_k");
    lin(V, N, R, bl.sa_v, D, D, "sa_v");
    ck(kiln_rmsnorm_rows(Q, Q, bl.sa_qn.get<uint16_t>(), R * H, HD, eps, ks(s_)), "q norm");
    ck(kiln_rmsnorm_rows(K, K, bl.sa_kn.get<uint16_t>(), R * H, HD, eps, ks(s_)), "k norm");
    for (int b = 0; b < B; b++) {
        const size_t o = (size_t)b * T * D;
        ck(kiln_rope_half(Q + o, T, H, HD, rp.c(), rp.s(), ks(s_)), "rope q");
        ck(kiln_rope_half(K + o, T, H, HD, rp.c(), rp.s(), ks(s_)), "rope k");
        ck(kiln_attn_fwd_exact(A + o, D, Q + o, D, K + o, D, V + o, D, T, T, H, HD, 0, 0, ks(s_)), "self attention");
    }
    lin(Y, A, R, bl.sa_o, D, D, "sa_o");
    ck(kiln_add_gated(X, Y, mo + 2 * D, R, D, ks(s_)), "gated residual");
    // cross-attention (dit.cu:511-527)
    ck(kiln_layernorm_mod(N, X, mc + D, mc, R, D, eps, ks(s_)), "LN cross");
    lin(Q, N, R, bl.ca_q, D, D, "ca_q");
    ck(kiln_rmsnorm_rows(Q, Q, bl.ca_qn.get<uint16_t>(), R * H, HD, eps, ks(s_)), "cross q norm");
    auto ctx_k = [&](const CachedContext* c) { return c->k32.get<float>() + (size_t)i * c->real * D; };
    auto ctx_v = [&](const CachedContext* c) { return c->v32.get<float>() + (size_t)i * c->real * D; };
    for (int b = 0; b < B; b++) {
        const size_t o = (size_t)b * T * D;
        ck(kiln_attn_fwd_exact(A + o, D, Q + o, D, ctx_k(cs[b]), D, ctx_v(cs[b]), D, T, cs[b]->real, H, HD, 0,
                               cs[b]->len - cs[b]->real, ks(s_)),
           "cross attention");
    }
    if (nag.neg) {
        float* An = arena_.f((size_t)T * D);
        const CachedContext* n = nag.neg;
        ck(kiln_attn_fwd_exact(An, D, Q, D, ctx_k(n), D, ctx_v(n), D, T, n->real, H, HD, 0, n->len - n->real, ks(s_)),
           "NAG attention");
        ck(kiln_nag_combine(A, D, An, D, KILN_F32, T, D, nag.scale, nag.tau, nag.alpha, ks(s_)), "NAG combine");
    }
    lin(Y, A, R, bl.ca_o, D, D, "ca_o");
    ck(kiln_add_gated(X, Y, mc + 2 * D, R, D, ks(s_)), "gated residual");
    // MLP (dit.cu:529-534)
    ck(kiln_layernorm_mod(N, X, mm + D, mm, R, D, eps, ks(s_)), "LN mlp");
    float* Hd = arena_.f((size_t)R * F);
    lin(Hd, N, R, bl.mlp1, F, D, "mlp1");
    ck(kiln_gelu(Hd, (size_t)R * F, ks(s_)), "gelu");
    lin(Y, Hd, R, bl.mlp2, D, F, "mlp2");
    ck(kiln_add_gated(X, Y, mm + 2 * D, R, D, ks(s_)), "gated residual");
    arena_.release(m);
}

static size_t block_scratch_bytes(const DitDims& d, int B, int T) {
    const size_t R = (size_t)B * T, D = d.D(), F = d.F();
    const size_t h16 = 2 * R * D * 2 + std::max(kiln_dit_self_attn_x16_workspace_bytes(B, T, d.heads), R * D * 2) +
                       T * D * 2 + R * F * 2;
    const size_t f32 = (6 * R * D + T * D + R * F) * 4;
    return std::max(h16, f32) + 16 * 256;
}

void Dit::run_block(int i, float* X, const float* mods, int Hp, int Wp, int B, const CachedContext* const* cs,
                    const NagParams& nag, bool fp32) {
    if (i < 0 || i >= d_.blocks || !blocks_[i]) throw std::runtime_error("run_block: no such block");
    if (B < 1 || B > 3) throw std::runtime_error("run_block: B outside 1..3");
    const int T = Hp * Wp;
    const Rope& rp = rope(Hp, Wp);
    arena_.reserve(block_scratch_bytes(d_, B, T));  // run_block is a top-level call: no live slices
    if (fp32) block32(i, X, mods, T, B, rp, cs, nag);
    else block16(i, X, mods, T, B, rp, cs, nag);
}

// ---- forward_batch (dit.cu:357-546) ----

static size_t forward_bytes(const DitDims& d, int Hl, int Wl, int B) {
    const size_t T = (size_t)(Hl / 2) * (Wl / 2), R = B * T, D = d.D();
    return ((size_t)d.blocks * 9 * D + 2 * D) * 4 + R * TOK * 4 + 3 * R * D * 4 + step_tables_bytes(d) +
           block_scratch_bytes(d, B, (int)T) + 32 * 256;
}

void Dit::forward_batch(float* const* outs, const float* latent, int Hl, int Wl, float t, const CachedContext* const* cs,
                        int B, const NagParams& nag, StepCache* sc, bool fp32) {
    if (B < 1 || B > 3) throw std::runtime_error("forward_batch: B outside 1..3");
    if (Hl < 2 || Wl < 2) throw std::runtime_error("forward_batch: latent too small");
    for (int b = 0; b < B; b++)
        if (!cs[b]) throw std::runtime_error("forward_batch: missing context");
    if (Hl % 2 == 0 && Wl % 2 == 0) {
        forward_even(outs, latent, Hl, Wl, t, cs, B, nag, sc, fp32);
        return;
    }
    // odd side: pad to the 2x2 patch grid (circular), run, crop back (dit.cu:359-371)
    const int H2 = Hl + Hl % 2, W2 = Wl + Wl % 2;
    const size_t n2 = (size_t)16 * H2 * W2;
    arena_.reserve(forward_bytes(d_, H2, W2, B) + (B + 1) * (n2 * 4 + 256));
    const size_t m = arena_.mark();
    float* pin = arena_.f(n2);
    float* po[3];
    for (int b = 0; b < B; b++) po[b] = arena_.f(n2);
    ck(kiln_pad_circular(pin, latent, Hl, Wl, H2, W2, ks(s_)), "pad");
    forward_even(po, pin, H2, W2, t, cs, B, nag, sc, fp32);
    for (int b = 0; b < B; b++) ck(kiln_crop(outs[b], po[b], H2, W2, Hl, Wl, ks(s_)), "crop");
    arena_.release(m);
}

void Dit::forward_even(float* const* outs, const float* latent, int Hl, int Wl, float t,
                       const CachedContext* const* cs, int B, const NagParams& nag, StepCache* sc, bool fp32) {
    const int Hp = Hl / 2, Wp = Wl / 2, T = Hp * Wp, R = B * T, D = d_.D(), nb = d_.blocks;
    const size_t TD = (size_t)T * D, RD = (size_t)R * D;
    const Rope& rp = rope(Hp, Wp);
    if (arena_.mark() == 0) arena_.reserve(forward_bytes(d_, Hl, Wl, B));
    const size_t m = arena_.mark();
    float* mods = arena_.f((size_t)nb * 9 * D + 2 * D);
    step_tables(t, mods);
    const float* fmod = mods + (size_t)nb * 9 * D;
    float* tok = arena_.f((size_t)R * TOK);
    float* X = arena_.f(RD);
    // every batch item starts from the same latent
    ck(kiln_patchify(tok, latent, Hl, Wl, ks(s_)), "patchify");
    ck(kiln_linear_f32(X, D, tok, TOK, x_embed_.get<uint16_t>(), T, D, TOK, ks(s_)), "x_embed");
    for (int b = 1; b < B; b++)
        ck_hip(hipMemcpyAsync(X + b * TD, X, TD * 4, hipMemcpyDeviceToDevice, s_), "replicate tokens");

    const bool use_cache = sc && sc->threshold > 0.f;
    float* X0 = nullptr;
    if (use_cache) {
        if (sc->R != R || !sc->r0.get()) {
            sc->valid = false;
            sc->R = R;
            sc->r0.resize(RD * 4);
            sc->resid.resize(RD * 4);
            sc->acc.resize(256);
        }
        X0 = arena_.f(RD);
        ck_hip(hipMemcpyAsync(X0, X, RD * 4, hipMemcpyDeviceToDevice, s_), "block-0 input");
        sc->skipped = false;
    }
    for (int i = 0; i < nb; i++) {
        if (use_cache && i == 1) {
            ck(kiln_sub(X0, X, X0, RD, ks(s_)), "block-0 residual");
            if (sc->valid) {
                ck(kiln_rel_l1(X0, sc->r0.get<float>(), RD, sc->acc.get<float>(), ks(s_)), "rel_l1");
                float h[2];
                // the reference reads the two sums back here (dit.cu:414-416)
                ck_hip(hipMemcpyAsync(h, sc->acc.get(), 8, hipMemcpyDeviceToHost, s_), "rel_l1 readback");
                ck_hip(hipStreamSynchronize(s_), "rel_l1 readback");
                sc->last_change = h[1] > 0.f ? h[0] / h[1] : 1.f;
                if (sc->allow && sc->last_change < sc->threshold) {
                    // X = block-0 output + the cached residual of blocks 1..N-1
                    ck(kiln_add_gated(X, sc->resid.get<float>(), nullptr, R, D, ks(s_)), "cached residual");
                    sc->skipped = true;
                    break;
                }
            }
            ck_hip(hipMemcpyAsync(sc->r0.get(), X0, RD * 4, hipMemcpyDeviceToDevice, s_), "cache r0");
            ck_hip(hipMemcpyAsync(sc->resid.get(), X, RD * 4, hipMemcpyDeviceToDevice, s_), "cache resid");
        }
        const float* mo = mods + (size_t)i * 9 * D;
        if (fp32) block32(i, X, mo, T, B, rp, cs, nag);
        else block16(i, X, mo, T, B, rp, cs, nag);
    }
    if (use_cache && !sc->skipped) {
        // resid holds block 0's output: turn it into the residual of blocks 1..N-1
        ck(kiln_sub(sc->resid.get<float>(), X, sc->resid.get<float>(), RD, ks(s_)), "cache residual");
        sc->valid = true;
    }
    // final layer: modulated LayerNorm, linear to 64 = 16 channels x 2 x 2, unpatchify per item
    float* N = arena_.f(RD);
    ck(kiln_layernorm_mod(N, X, fmod + D, fmod, R, D, d_.eps, ks(s_)), "final LN");
    ck(kiln_linear_f32(tok, 64, N, D, final_lin_.get<uint16_t>(), R, 64, D, ks(s_)), "final linear");
    for (int b = 0; b < B; b++)
        ck(kiln_unpatchify(outs[b], tok + (size_t)b * T * 64, 64, Hl, Wl, ks(s_)), "unpatchify");
    arena_.release(m);
}

}  // namespace kiln
