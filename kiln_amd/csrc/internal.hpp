// Host-side launchers shared between the kernel translation units and the C ABI layer.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kiln_attn.h"

namespace kiln {

enum class DT { F32 = 0, F16 = 1 };

// One attention problem of a batched launch: queries q (rows [0, Tq), row stride ldq, head h at
// column h*128) against the prepared K/V buffer kv (Tk real keys, npad analytic zero keys).
struct AttnJob {
    const void* q;
    const uint16_t* kv;
    void* o;
    int Tk;
    int npad;
};
constexpr int MAX_JOBS = 4;

struct AttnLaunch {
    AttnJob job[MAX_JOBS];
    int njobs;
    int Tq, H, ldq, ldo;
    DT in, out;
    const uint16_t* qw;  // bf16 [128] q RMSNorm weight or null (no norm)
    float eps;
    const float* rcos;   // [Tq, 64] RoPE tables for Q or null
    const float* rsin;
    int ksplit;          // > 1: split every unit's keys into ksplit ranges (partials in `part`, then a merge)
    float* part;         // attn_split_bytes(ksplit, njobs, Tq, H) bytes of device scratch
    bool q_prescaled;    // fp16 Q already holds q * log2(e)/sqrt(128) (no norm, no RoPE): scale 1
    bool chain;          // context chain: one unit per (query tile, head) runs the jobs in order (jobs sharing a Q
                         // pointer next to each other keep the Q tile in registers); no key split
};

// Key ranges per unit for a launch of njobs x H heads x Tq queries against Tk keys: > 1 only when the grid
// would fill under a third of the resident workgroup slots (small head counts, one GPU's share of a
// head-parallel run) and every range keeps at least 16 32-key half tiles.
int attn_key_split(int njobs, int Tq, int Tk, int H);
size_t attn_split_bytes(int ksplit, int njobs, int Tq, int H);

hipError_t launch_attn_fwd(const AttnLaunch& a, hipStream_t s);

// One K/V context to prepare: raw K and V rows (row strides ldk, ldv; head h at column h*128) into the
// tiled fp16 buffer kvp.
struct KVPrepJob {
    uint16_t* kvp;
    const void* k;
    const void* v;
    int ldk, ldv;
};
// Prepares njobs (<= MAX_JOBS) contexts of Tk keys and H heads in one launch (K RMSNorm with kw, RoPE).
hipError_t launch_kv_prep(const KVPrepJob* jobs, int njobs, DT in, int Tk, int H, const uint16_t* kw, float eps,
                          const float* rcos, const float* rsin, hipStream_t s);

// acc = a [M,K] w[N,K]^T (+ a2 [M,K2] w2[N,K2]^T), all fp16 dense rows; epilogue `epi` (kiln_epi) into c (row
// stride ldc). N % 128 == 0, K % 32 == 0, K2 % 32 == 0, 16-byte aligned operand bases.
struct GemmLaunch {
    const uint16_t* a;
    const uint16_t* w;
    int K;
    const uint16_t* a2;
    const uint16_t* w2;
    int K2;
    void* c;
    int ldc;
    const float* gate;
    float beta;
    int M, N;
    int epi;
    bool wprep;  // w in the prepared layout of launch_gemm_wprep
    // epi == 4 (the DiT self-attention projection, N = 3 * 128 * H, H even): Q rows and prepared K/V per item
    uint16_t* q16;
    uint16_t* kvp[MAX_JOBS];
    int T, H;
    const uint16_t* qw;
    const uint16_t* kw;
    float eps;
    const float* rcos;
    const float* rsin;
};
// zero the last (partial) 64-key tile of each item's and head's prepared K/V before a projection writes the keys
hipError_t launch_kv_zero_tail(uint16_t* const* kvp, int njobs, int T, int H, hipStream_t s);
hipError_t launch_gemm16(const GemmLaunch& g, hipStream_t s);
// Weight [N, K] (fp16, or bf16 converted as the reference's weight_to_f16) into the prepared tile layout.
size_t gemm16_prepped_bytes(int N, int K);
hipError_t launch_gemm_wprep(uint16_t* wp, const uint16_t* w, int N, int K, bool src_bf16, hipStream_t s);

// the DiT forward's passes around the blocks (dit_aux.hip)
// groups > 1: W is groups stacked [rows, cols] matrices, x groups stacked [cols] vectors, y [groups * rows],
// add [rows] shared by every group
hipError_t launch_matvec_bf16(float* y, const uint16_t* W, const float* x, const float* add, int rows, int cols,
                              int groups, hipStream_t s);
hipError_t launch_silu(float* y, const float* x, size_t n, hipStream_t s);
hipError_t launch_patchify(float* tok, const float* lat, int Hl, int Wl, hipStream_t s);
hipError_t launch_unpatchify(float* lat, const float* tok, int ldt, int Hl, int Wl, hipStream_t s);
hipError_t launch_linear_f32(float* y, int ldy, const float* x, int ldx, const uint16_t* W, int T, int rows, int cols,
                             hipStream_t s);
hipError_t launch_cfg_combine(float* v, const float* vn, float cfg, size_t n, hipStream_t s);
hipError_t launch_sub(float* y, const float* a, const float* b, size_t n, hipStream_t st);
hipError_t launch_rel_l1(const float* a, const float* b, size_t n, float* acc, hipStream_t st);
hipError_t launch_flow_start(float* x, const float* noise, const float* init, float s, size_t n, hipStream_t st);
hipError_t launch_gelu(float* x, size_t n, hipStream_t st);
hipError_t launch_flow_ersde(float* x, const float* den, const float* old, float* oldd, const float* noise, float a,
                             float b, float c2, float inv2, float c3, float inv3, float cn, int stage, size_t n,
                             hipStream_t st);
hipError_t launch_flow_inpaint_in(float* xin, const float* x, const float* noise, const float* init, const float* mask,
                                  float s, int P, hipStream_t st);
hipError_t launch_flow_denoised_masked(float* den, const float* xin, const float* v, const float* init,
                                      const float* mask, float s, int P, hipStream_t st);
hipError_t launch_flow_denoised(float* den, const float* x, const float* v, float s, size_t n, hipStream_t st);
hipError_t launch_flow_update(float* x, const float* den, const float* old, float a, float b, float c, size_t n,
                              hipStream_t st);
hipError_t launch_flow_euler(float* x, const float* v, float s, float sn, size_t n, hipStream_t st);
hipError_t launch_pad_circular(float* dst, const float* src, int Hs, int Ws, int Hd, int Wd, hipStream_t st);
hipError_t launch_crop(float* dst, const float* src, int Hs, int Ws, int Hd, int Wd, hipStream_t st);
hipError_t launch_fill_uniform_bf16(uint16_t* p, size_t n, uint64_t seed, float lo, float hi, hipStream_t st);
hipError_t launch_zero_rows(void* out, size_t ld_bytes, size_t row_bytes, int rows, hipStream_t s);
hipError_t launch_flow_euler_den(float* x, const float* den, float s, float sn, size_t n, hipStream_t st);

// torch.manual_seed(seed); torch.randn(n) on the host (host_rng.cpp); false if n < 16
bool host_torch_randn(float* out, uint64_t seed, size_t n);

hipError_t launch_exact_attn(float* out, int ldo, const float* q, int ldq, const float* k, int ldk, const float* v,
                             int ldv, int Tq, int Tk, int H, int Dh, bool causal, int npad, hipStream_t s);

hipError_t launch_rmsnorm_rows(float* y, const float* x, const uint16_t* w, int rows, int dim, float eps, hipStream_t s);
hipError_t launch_rope_half(float* x, int T, int H, int Dh, const float* c, const float* sn, hipStream_t s);
hipError_t launch_layernorm_mod(void* y, DT out, const float* x, const float* scale, const float* shift, int rows,
                                int dim, float eps, hipStream_t s);
hipError_t launch_add_gated(float* x, const float* y, const float* gate, int rows, int dim, hipStream_t s);
hipError_t launch_nag(void* a, int lda, const void* an, int ldn, DT dt, int T, int dim, float sc, float tau,
                      float alpha, hipStream_t s);

}  // namespace kiln
