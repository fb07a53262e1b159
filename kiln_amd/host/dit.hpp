// dit.hpp - the Cosmos-Predict2 DiT forward and its per-generation state, in C++ over the C ABI of
// libkiln_attn.so (include/kiln_attn.h). The reference's Dit (engine/src/models.h:20-90, engine/src/dit.cu):
//   * Dit::forward_batch on the fp16-activation path (dit.cu:357-494, 532-546) and the fp32 path (dit.cu:495-530);
//   * Dit::step_tables (dit.cu:242-278), Dit::cache_context (dit.cu:217-234), the first-block StepCache
//     (models.h:66-76, dit.cu:404-433, 532-536) and NAG (models.h:80).
// Weights arrive as bf16 device arrays in the checkpoint's [out, in] layout and are copied: the linear16 weights
// are converted to fp16 in the prepared tile layout at load (the reference's weight_to_f16, kernels.cu:531-544),
// with the self-attention Q/K/V stacked into one [3D, D] weight; bf16 copies stay for the fp32 path, the context
// projections and the modulation matvecs.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/kiln_attn.h"

namespace kiln {

// A failure that carries its kiln_status (KILN_EHIP for a HIP error, KILN_ENOMEM for device memory or an arena
// that is too small, the library's own code for a failed C-ABI call), so the C ABI can hand it back unchanged.
struct Error : std::runtime_error {
    int status;
    Error(int st, const std::string& msg) : std::runtime_error(msg), status(st) {}
};

// Throw kiln::Error with the library's message when a C-ABI call or a HIP call fails.
void ck(int rc, const char* what);
void ck_hip(hipError_t e, const char* what);

// An owned device allocation.
class DeviceBuffer {
   public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) { resize(bytes); }
    ~DeviceBuffer() { release(); }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) { o.p_ = nullptr, o.n_ = 0; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            release();
            p_ = o.p_, n_ = o.n_;
            o.p_ = nullptr, o.n_ = 0;
        }
        return *this;
    }
    // reallocates (contents lost) when bytes exceeds the current size
    void reserve(size_t bytes);
    void resize(size_t bytes);
    void release();
    template <typename T = void>
    T* get() const {
        return static_cast<T*>(p_);
    }
    size_t bytes() const { return n_; }

   private:
    void* p_ = nullptr;
    size_t n_ = 0;
};

// A bump allocator over one device buffer, like the reference's arena (engine/src/gpu.h:51-59): mark() and
// release() bracket the scratch of one call; slices are 256-byte aligned.
class Arena {
   public:
    // grows the buffer (synchronizing the device first) when no slice is live
    void reserve(size_t bytes);
    size_t mark() const { return top_; }
    void release(size_t m) { top_ = m; }
    void* take(size_t bytes);
    float* f(size_t n) { return static_cast<float*>(take(n * 4)); }
    uint16_t* h(size_t n) { return static_cast<uint16_t*>(take(n * 2)); }
    size_t capacity() const { return buf_.bytes(); }
    size_t peak() const { return peak_; }

   private:
    DeviceBuffer buf_;
    size_t top_ = 0, peak_ = 0;
};

struct DitDims {
    int blocks = 28;      // transformer blocks
    int heads = 16;       // attention heads of dim 128: D = 128 * heads
    int ctx_dim = 1024;   // text-context width (the LLM adapter's output)
    int mlp = 0;          // MLP hidden width; 0 = 4 D
    float eps = 1e-6f;
    int D() const { return 128 * heads; }
    int F() const { return mlp > 0 ? mlp : 4 * D(); }
};

// One block's checkpoint weights: bf16 device arrays [out, in].
struct BlockWeights {
    const uint16_t *sa_q, *sa_k, *sa_v, *sa_o;   // [D, D]
    const uint16_t *ca_q, *ca_o;                 // [D, D]
    const uint16_t *ca_k, *ca_v;                 // [D, ctx_dim]
    const uint16_t *mlp1, *mlp2;                 // [F, D], [D, F]
    const uint16_t *sa_qn, *sa_kn, *ca_qn, *ca_kn;  // [128] per-head RMSNorm weights
    // adaLN modulation MLPs (dit.cu:266-268): self-attention, cross-attention, MLP; each [256, D] then [3D, 256]
    const uint16_t *mod_sa1, *mod_sa2, *mod_ca1, *mod_ca2, *mod_mlp1, *mod_mlp2;
};

// The weights outside the blocks (dit.cu:53-59, 242-272): bf16 device arrays.
struct StepWeights {
    const uint16_t *t_lin1, *t_lin2, *t_norm;  // [D, D], [3D, D], [D]
    const uint16_t *final_mod1, *final_mod2;   // [256, D], [2D, 256]
    const uint16_t *x_embed, *final_lin;       // [D, 68], [64, D]
};

// A text context prepared for one generation (the reference's Context + KVCache, models.h:26, 56-58): every
// block's cross-attention K (RMS-normed) and V from the real rows; rows [real, len) are zero padding and enter
// the softmax as npad = len - real zero keys. The fp16 path reads the prepared (tiled fp16) K/V; the fp32 path
// the fp32 K/V, kept only when the context was cached with fp32 = true.
struct CachedContext {
    int real = 0, len = 0;
    size_t kv_per_block = 0;
    DeviceBuffer kv16;        // blocks x kiln_kv_prepped_bytes(real, H)
    DeviceBuffer k32, v32;    // blocks x [real, D] fp32 (fp32 path)
    const uint16_t* kv(int block) const {
        return reinterpret_cast<const uint16_t*>(kv16.get<char>() + kv_per_block * block);
    }
};

// NAG (Dit::Nag, models.h:80): batch item 0's cross-attention becomes the blend of its positive and negative
// attentions; neg == nullptr turns it off.
struct NagParams {
    const CachedContext* neg = nullptr;
    float scale = 5.f, tau = 2.5f, alpha = 0.25f;
};

// The first-block step cache (Dit::StepCache, models.h:66-76).
struct StepCache {
    float threshold = 0.f;  // relative L1 change of block 0's residual below which blocks 1.. are skipped
    bool allow = false;     // set per step by the sampler
    bool valid = false, skipped = false;
    int R = 0;
    float last_change = 0.f;
    DeviceBuffer r0, resid, acc;
};

class Dit {
   public:
    Dit(const DitDims& dims, hipStream_t stream);
    ~Dit();
    Dit(const Dit&) = delete;
    Dit& operator=(const Dit&) = delete;
    const DitDims& dims() const { return d_; }
    hipStream_t stream() const { return s_; }

    void set_step_weights(const StepWeights& w);
    void set_block(int i, const BlockWeights& w);

    // Dit::cache_context (dit.cu:217-234): ctx [len, ctx_dim] fp32 device rows, the first `real` of them real.
    std::unique_ptr<CachedContext> cache_context(const float* ctx, int real, int len, bool fp32 = false);

    // Dit::forward_batch: B items (B <= 3) from one latent [16, Hl, Wl]; outs[b] [16, Hl, Wl] fp32 velocity of
    // item b against context cs[b]. nag applies to item 0. fp32 selects the fp32 block (the engine's --fp32).
    void forward_batch(float* const* outs, const float* latent, int Hl, int Wl, float t, const CachedContext* const* cs,
                       int B, const NagParams& nag = NagParams(), StepCache* sc = nullptr, bool fp32 = false);

    // The modulation vectors of every block ([9D] each) and of the final layer ([2D]) for timestep t, into
    // mods [blocks * 9D + 2D] (device); Dit::step_tables without the RoPE tables.
    void step_tables(float t, float* mods);

    // One block on X [B*T, D] (in place) with modulation mods [9D]: the block loop body of forward_batch.
    void run_block(int i, float* X, const float* mods, int Hp, int Wp, int B, const CachedContext* const* cs,
                   const NagParams& nag, bool fp32);

    size_t arena_peak() const { return arena_.peak(); }

   private:
    struct Block;
    struct Rope;
    const Rope& rope(int Hp, int Wp);
    void block16(int i, float* X, const float* mods, int T, int B, const Rope& rp, const CachedContext* const* cs,
                 const NagParams& nag);
    void block32(int i, float* X, const float* mods, int T, int B, const Rope& rp, const CachedContext* const* cs,
                 const NagParams& nag);
    void forward_even(float* const* outs, const float* latent, int Hl, int Wl, float t, const CachedContext* const* cs,
                      int B, const NagParams& nag, StepCache* sc, bool fp32);

    DitDims d_;
    hipStream_t s_;
    std::vector<std::unique_ptr<Block>> blocks_;
    DeviceBuffer t_lin1_, t_lin2_, t_norm_, fmod1_, fmod2_, x_embed_, final_lin_;
    DeviceBuffer mod1_all_, mod2_all_;  // every block's modulation layers stacked (two launches per step)
    bool mods_stacked_ = false;
    std::vector<std::unique_ptr<Rope>> ropes_;
    Arena arena_;
};

}  // namespace kiln
