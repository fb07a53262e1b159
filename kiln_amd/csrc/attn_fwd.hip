// Flash-attention forward for head_dim 128 on gfx950 (CDNA4) fp16 MFMA with fp32 accumulation.
//
// Contract: the reference's tfa::k_flash (engine/src/tcflash.cuh:20-157): O = softmax(Q K^T / sqrt(128)) V
// per head, Q pre-scaled by log2(e)/sqrt(128) and rounded to fp16, base-2 online softmax, P rounded to
// fp16, analytic npad zero keys (tcflash.cuh:136-147). PV accumulates in fp32 (the MFMA's native
// accumulator) instead of the reference's GeForce-specific fp16 partial sums.
//
// Design (gfx950, wave64):
//  * workgroup = 4 waves x 32 query rows (BM = 128); K/V stream in tiles of 64 keys.
//  * scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_f16: each lane then owns ONE
//    query column and 32 of the tile's 64 keys, so the row max needs one v_permlane32_swap and the row
//    sum none until the epilogue.
//  * O^T = V^T P^T: P^T comes straight out of the S^T accumulator (no LDS round trip); V^T is the A
//    operand, pre-permuted by the K/V prepare pass so that every LDS operand read of a wave is one
//    contiguous, conflict-free 1 KB ds_read_b128.
//  * K/V tiles (32 KB each) are double-buffered in LDS: tile j+1 is fetched from HBM/L2 into registers
//    (coalesced 16-byte loads) while tile j is computed, then stored to the other LDS stage.
//  * Q's RMSNorm and RoPE are applied in the Q tile load, in fp32, before the single fp16 rounding.
//  * the softmax rescale of O is lazy: the running max only moves (and O/l are only rescaled) when a
//    tile's max exceeds it by more than 8 (log2 units), so P <= 2^8 stays far inside fp16 range.
//  * 1-D grid with an XCD-aware block -> work mapping: consecutive work items (the query tiles of one
//    head) land on the same XCD and share its L2.
#include "common.hpp"
#include "internal.hpp"

namespace kiln {

constexpr int BM = 128;
constexpr int NTHR = 256;
constexpr float RESCALE_TH = 8.0f;

struct AttnParams {
    AttnJob job[MAX_JOBS];
    int njobs, Tq, H, ldq, ldo, qtiles, total, per;
    int store_pairs;  // ldo or an output base not 8/16-byte aligned: store element pairs
    const uint16_t* qw;
    float eps, qscale;
    const float* rcos;
    const float* rsin;
};

template <typename OutT>
__device__ __forceinline__ void store4(OutT* dst, float a, float b, float c, float d, bool pairs);
template <>
__device__ __forceinline__ void store4<_Float16>(_Float16* dst, float a, float b, float c, float d, bool pairs) {
    if (!pairs) {
        half4 h = {(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
        *reinterpret_cast<half4*>(dst) = h;
    } else {
        half2v h0 = {(_Float16)a, (_Float16)b}, h1 = {(_Float16)c, (_Float16)d};
        reinterpret_cast<half2v*>(dst)[0] = h0;
        reinterpret_cast<half2v*>(dst)[1] = h1;
    }
}
template <>
__device__ __forceinline__ void store4<float>(float* dst, float a, float b, float c, float d, bool pairs) {
    if (!pairs) {
        floatx4 f = {a, b, c, d};
        *reinterpret_cast<floatx4*>(dst) = f;
    } else {
        typedef float f2 __attribute__((ext_vector_type(2)));
        f2 f0 = {a, b}, f1 = {c, d};
        reinterpret_cast<f2*>(dst)[0] = f0;
        reinterpret_cast<f2*>(dst)[1] = f1;
    }
}

template <typename InT, typename OutT, bool QNORM, bool ROPE>
__global__ __launch_bounds__(NTHR, 2) void k_attn_fwd(const AttnParams p) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[2 * KV_TILE_H];  // 2 stages x (K 16 KB + V 16 KB)

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int l32 = lane & 31, hh = lane >> 5;

    // blocks are dispatched round-robin over the 8 XCDs (block b -> XCD b % 8): give each XCD a
    // contiguous range of work items so the query tiles of one head share that XCD's L2.
    const int w = (int)(blockIdx.x & 7) * p.per + (int)(blockIdx.x >> 3);
    if (w >= p.total) return;
    const int qt = w % p.qtiles;
    const int rest = w / p.qtiles;
    const int h = rest % p.H;
    const int jb = rest / p.H;
    const AttnJob J = p.job[jb];

    // ---- Q tile: this lane's query row, d chunks {16s + 8hh .. +8}, s = 0..7 -> B operands ----
    const int row = qt * BM + wv * 32 + l32;
    const bool qin = row < p.Tq;
    half8 qreg[8];
    {
        float x[8][8];
        const InT* qr = reinterpret_cast<const InT*>(J.q) + (size_t)(qin ? row : 0) * p.ldq + h * HD + 8 * hh;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            if (qin) load8(qr + 16 * s, x[s]);
            else {
#pragma unroll
                for (int e = 0; e < 8; e++) x[s][e] = 0.f;
            }
        }
        if constexpr (QNORM) {
            float ss = 0.f;
#pragma unroll
            for (int s = 0; s < 8; s++)
#pragma unroll
                for (int e = 0; e < 8; e++) ss += x[s][e] * x[s][e];
            ss = pair_sum(ss);
            const float r = rsqrtf(ss * (1.0f / HD) + p.eps);
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const uint16_t* wp = p.qw + 16 * s + 8 * hh;
#pragma unroll
                for (int e = 0; e < 8; e++) x[s][e] = x[s][e] * r * bf16_to_f32(wp[e]);
            }
        }
        if constexpr (ROPE) {
            if (qin) {
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    float c[8], sn[8];
                    load8(p.rcos + (size_t)row * 64 + 16 * s + 8 * hh, c);
                    load8(p.rsin + (size_t)row * 64 + 16 * s + 8 * hh, sn);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float a = x[s][e], b = x[s + 4][e];
                        x[s][e] = a * c[e] - b * sn[e];
                        x[s + 4][e] = b * c[e] + a * sn[e];
                    }
                }
            }
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
#pragma unroll
            for (int e = 0; e < 8; e++) x[s][e] *= p.qscale;
            qreg[s] = to_half8(x[s]);
        }
    }

    const int Tk = J.Tk;
    const int nt = kv_tiles(Tk);
    const uint16_t* kvh = J.kv + (size_t)h * kv_head_stride(Tk);

    u32x4 pre[8];
    auto gload = [&](int j) {
        const u32x4* src = reinterpret_cast<const u32x4*>(kvh + (size_t)j * KV_TILE_H);
#pragma unroll
        for (int i = 0; i < 8; i++) pre[i] = src[tid + NTHR * i];
    };
    auto lstore = [&](int stage) {
        u32x4* dst = reinterpret_cast<u32x4*>(lds + stage * KV_TILE_H);
#pragma unroll
        for (int i = 0; i < 8; i++) dst[tid + NTHR * i] = pre[i];
    };

    gload(0);
    lstore(0);
    __syncthreads();

    floatx16 o[4];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[db][i] = 0.f;
    float m = -INFINITY, l = 0.f;

    for (int j = 0; j < nt; j++) {
        if (j + 1 < nt) gload(j + 1);
        const _Float16* ks = lds + (j & 1) * KV_TILE_H;
        const _Float16* vs = ks + TILE_H;

        // S^T[key][query] for the tile's two 32-key blocks
        floatx16 s0, s1;
#pragma unroll
        for (int i = 0; i < 16; i++) { s0[i] = 0.f; s1[i] = 0.f; }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const half8 a0 = *reinterpret_cast<const half8*>(ks + ((0 * 8 + s) * 64 + lane) * 8);
            const half8 a1 = *reinterpret_cast<const half8*>(ks + ((1 * 8 + s) * 64 + lane) * 8);
            s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qreg[s], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, qreg[s], s1, 0, 0, 0);
        }
        // accumulator item i of key block kb holds key j*64 + kb*32 + 8*(i/4) + 4*hh + i%4
        if ((j + 1) * KT > Tk) {
            const int kbase = j * KT + 4 * hh;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int key = kbase + 8 * (i / 4) + (i % 4);
                if (key >= Tk) s0[i] = -INFINITY;
                if (key + 32 >= Tk) s1[i] = -INFINITY;
            }
        }

        float mx = fmaxf(s0[0], s1[0]);
#pragma unroll
        for (int i = 1; i < 16; i++) mx = fmaxf(mx, fmaxf(s0[i], s1[i]));
        mx = pair_max(mx);
        const float mnew = fmaxf(m, mx);
        if (__builtin_amdgcn_ballot_w64(mnew > m + RESCALE_TH)) {
            const float corr = __builtin_amdgcn_exp2f(m - mnew);
#pragma unroll
            for (int db = 0; db < 4; db++)
#pragma unroll
                for (int i = 0; i < 16; i++) o[db][i] *= corr;
            l *= corr;
            m = mnew;
        }

        half8 pb[4];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float e0 = __builtin_amdgcn_exp2f(s0[i] - m);
            const float e1 = __builtin_amdgcn_exp2f(s1[i] - m);
            l += e0 + e1;
            pb[i / 8][i % 8] = (_Float16)e0;
            pb[2 + i / 8][i % 8] = (_Float16)e1;
        }

#pragma unroll
        for (int db = 0; db < 4; db++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const half8 a = *reinterpret_cast<const half8*>(vs + ((db * 4 + t) * 64 + lane) * 8);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[t], o[db], 0, 0, 0);
            }

        if (j + 1 < nt) lstore((j + 1) & 1);
        __syncthreads();
    }

    // epilogue: full row sum (lane pair), npad zero keys, normalize, store
    float lt = pair_sum(l);
    float sc = 1.f;
    if (J.npad) {
        const float mn = fmaxf(m, 0.f);
        sc = __builtin_amdgcn_exp2f(m - mn);
        lt = lt * sc + (float)J.npad * __builtin_amdgcn_exp2f(-mn);
    }
    const float inv = sc / lt;
    if (!qin) return;
    OutT* orow = reinterpret_cast<OutT*>(J.o) + (size_t)row * p.ldo + h * HD + 4 * hh;
    const bool pairs = p.store_pairs != 0;
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
        for (int g = 0; g < 4; g++)
            store4<OutT>(orow + db * 32 + 8 * g, o[db][4 * g] * inv, o[db][4 * g + 1] * inv, o[db][4 * g + 2] * inv,
                         o[db][4 * g + 3] * inv, pairs);
}

// ------------------------------------------------------------------------------------------------
// K/V prepare: fp16 conversion (+ K RMSNorm, + K RoPE) into the tiled MFMA operand order.
// One block per (64-key tile, head). Bandwidth-bound; runs once per K/V, not once per query tile.
// ------------------------------------------------------------------------------------------------
template <typename InT, bool KNORM, bool ROPE>
__global__ __launch_bounds__(256) void k_kv_prep(uint16_t* __restrict__ kvp, const InT* __restrict__ k, int ldk,
                                                 const InT* __restrict__ v, int ldv, int Tk,
                                                 const uint16_t* __restrict__ kw, float eps,
                                                 const float* __restrict__ rcos, const float* __restrict__ rsin) {
    __shared__ _Float16 vt[KT][HD + 8];
    const int tid = threadIdx.x, j = blockIdx.x, h = blockIdx.y;
    _Float16* dstK = reinterpret_cast<_Float16*>(kvp) + (size_t)h * kv_head_stride(Tk) + (size_t)j * KV_TILE_H;
    _Float16* dstV = dstK + TILE_H;

    const int kk = tid >> 2, qd = tid & 3;  // key within the tile, quarter of the row
    const int key = j * KT + kk;
    const bool valid = key < Tk;

    // K: chunks c in {2qd, 2qd+1, 2qd+8, 2qd+9} (8 elements each); (c, c+8) are RoPE partners
    {
        float x[4][8];
        const int cs[4] = {2 * qd, 2 * qd + 1, 2 * qd + 8, 2 * qd + 9};
        const InT* kr = k + (size_t)(valid ? key : 0) * ldk + h * HD;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            if (valid) load8(kr + 8 * cs[c], x[c]);
            else {
#pragma unroll
                for (int e = 0; e < 8; e++) x[c][e] = 0.f;
            }
        }
        if constexpr (KNORM) {
            float ss = 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int e = 0; e < 8; e++) ss += x[c][e] * x[c][e];
            ss += __shfl_xor(ss, 1);
            ss += __shfl_xor(ss, 2);
            const float r = rsqrtf(ss * (1.0f / HD) + eps);
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int e = 0; e < 8; e++) x[c][e] = x[c][e] * r * bf16_to_f32(kw[8 * cs[c] + e]);
        }
        if constexpr (ROPE) {
            if (valid) {
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    float cc[8], sn[8];
                    load8(rcos + (size_t)key * 64 + 8 * cs[c], cc);
                    load8(rsin + (size_t)key * 64 + 8 * cs[c], sn);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float a = x[c][e], b = x[c + 2][e];
                        x[c][e] = a * cc[e] - b * sn[e];
                        x[c + 2][e] = b * cc[e] + a * sn[e];
                    }
                }
            }
        }
        const int kb = kk >> 5, kl = kk & 31;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int s = cs[c] >> 1, hb = cs[c] & 1;
            const int off = ((kb * 8 + s) * 64 + kl + 32 * hb) * 8;
            *reinterpret_cast<half8*>(dstK + off) = to_half8(x[c]);
        }
    }
    // V: tile -> LDS (fp16), then gather the permuted-transposed operand order
    {
        const InT* vr = v + (size_t)(valid ? key : 0) * ldv + h * HD + 32 * qd;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float x[8];
            if (valid) load8(vr + 8 * c, x);
            else {
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] = 0.f;
            }
            *reinterpret_cast<half8*>(&vt[kk][32 * qd + 8 * c]) = to_half8(x);
        }
    }
    __syncthreads();
    {
        const int t = tid >> 6, ln = tid & 63;
        const int kbase = 16 * t + 4 * (ln >> 5);
#pragma unroll
        for (int db = 0; db < 4; db++) {
            const int d = db * 32 + (ln & 31);
            half8 o;
#pragma unroll
            for (int jj = 0; jj < 8; jj++) o[jj] = vt[kbase + 8 * (jj >> 2) + (jj & 3)][d];
            *reinterpret_cast<half8*>(dstV + ((db * 4 + t) * 64 + ln) * 8) = o;
        }
    }
}

// ------------------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------------------
template <typename InT, typename OutT>
static hipError_t dispatch_attn(const AttnParams& p, int nblocks, bool qnorm, bool rope, hipStream_t s) {
    dim3 grid(nblocks), block(NTHR);
    if (qnorm && rope) hipLaunchKernelGGL((k_attn_fwd<InT, OutT, true, true>), grid, block, 0, s, p);
    else if (qnorm) hipLaunchKernelGGL((k_attn_fwd<InT, OutT, true, false>), grid, block, 0, s, p);
    else if (rope) hipLaunchKernelGGL((k_attn_fwd<InT, OutT, false, true>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((k_attn_fwd<InT, OutT, false, false>), grid, block, 0, s, p);
    return hipGetLastError();
}

hipError_t launch_attn_fwd(const AttnLaunch& a, hipStream_t s) {
    AttnParams p{};
    for (int i = 0; i < a.njobs; i++) p.job[i] = a.job[i];
    p.njobs = a.njobs;
    p.Tq = a.Tq;
    p.H = a.H;
    p.ldq = a.ldq;
    p.ldo = a.ldo;
    p.qtiles = (a.Tq + BM - 1) / BM;
    p.total = p.qtiles * a.H * a.njobs;
    const int nblocks = (p.total + 7) / 8 * 8;
    p.per = nblocks / 8;
    const size_t osz = a.out == DT::F16 ? 2 : 4;
    bool pairs = (a.ldo * osz) % (4 * osz) != 0;
    for (int i = 0; i < a.njobs; i++) pairs |= ((uintptr_t)a.job[i].o % (4 * osz)) != 0;
    p.store_pairs = pairs;
    p.qw = a.qw;
    p.eps = a.eps;
    p.qscale = LOG2E / sqrtf((float)HD);
    p.rcos = a.rcos;
    p.rsin = a.rsin;
    const bool qn = a.qw != nullptr, rp = a.rcos != nullptr;
    if (p.total == 0) return hipSuccess;
    if (a.in == DT::F16) {
        if (a.out == DT::F16) return dispatch_attn<_Float16, _Float16>(p, nblocks, qn, rp, s);
        return dispatch_attn<_Float16, float>(p, nblocks, qn, rp, s);
    }
    if (a.out == DT::F16) return dispatch_attn<float, _Float16>(p, nblocks, qn, rp, s);
    return dispatch_attn<float, float>(p, nblocks, qn, rp, s);
}

template <typename InT>
static hipError_t dispatch_prep(uint16_t* kvp, const void* k, int ldk, const void* v, int ldv, int Tk, int H,
                                const uint16_t* kw, float eps, const float* rc, const float* rs, hipStream_t s) {
    dim3 grid(kv_tiles(Tk), H), block(256);
    const InT* kk = reinterpret_cast<const InT*>(k);
    const InT* vv = reinterpret_cast<const InT*>(v);
    if (kw && rc) hipLaunchKernelGGL((k_kv_prep<InT, true, true>), grid, block, 0, s, kvp, kk, ldk, vv, ldv, Tk, kw, eps, rc, rs);
    else if (kw) hipLaunchKernelGGL((k_kv_prep<InT, true, false>), grid, block, 0, s, kvp, kk, ldk, vv, ldv, Tk, kw, eps, rc, rs);
    else if (rc) hipLaunchKernelGGL((k_kv_prep<InT, false, true>), grid, block, 0, s, kvp, kk, ldk, vv, ldv, Tk, kw, eps, rc, rs);
    else hipLaunchKernelGGL((k_kv_prep<InT, false, false>), grid, block, 0, s, kvp, kk, ldk, vv, ldv, Tk, kw, eps, rc, rs);
    return hipGetLastError();
}

hipError_t launch_kv_prep(uint16_t* kvp, const void* k, int ldk, const void* v, int ldv, DT in, int Tk, int H,
                          const uint16_t* kw, float eps, const float* rcos, const float* rsin, hipStream_t s) {
    if (Tk <= 0 || H <= 0) return hipSuccess;
    if (in == DT::F16) return dispatch_prep<_Float16>(kvp, k, ldk, v, ldv, Tk, H, kw, eps, rcos, rsin, s);
    return dispatch_prep<float>(kvp, k, ldk, v, ldv, Tk, H, kw, eps, rcos, rsin, s);
}

}  // namespace kiln
