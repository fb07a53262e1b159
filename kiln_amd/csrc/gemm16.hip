// fp16 GEMM with fused epilogues for the DiT's linear layers on gfx950 (CDNA4) MFMA, fp32 accumulation.
//
// Contract: the reference's linear16 / tc16::k_gemm16 (engine/src/kernels.cu:559-609,
// engine/src/tcgemm16.cuh:1-200):
//   acc = A[M,K] W[N,K]^T (+ A2[M,K2] W2[N,K2]^T, the folded LoRA product), all fp16, row-major, K innermost;
//   epilogue F32:    C (fp32)  = acc + beta*C
//            F16:    C (fp16)  = acc
//            GELU16: C (fp16)  = GELU(acc), GELU(v) = v/2 (1 + erf(v/sqrt 2))
//            RESID:  C (fp32) += gate[col] * acc   (gate null: 1)
// The reference accumulates each 32-wide k tile in fp16 and flushes it into fp32 (tcgemm16.cuh:6-7); here
// every product accumulates in fp32 (the MFMA's native accumulator): more accurate, same inputs.
//
// Design (gfx950, wave64):
//  * workgroup tile 256 weight rows (n) x 256 activation rows (m), k tiles of 32; 8 waves in 2 (n) x 4 (m),
//    each wave 128 n x 64 m = 8 x 4 blocks of v_mfma_f32_16x16x32_f16 (the shape that sustains the higher
//    rate on a power-limited MI355X), 128 fp32 accumulators per lane, two waves per SIMD.
//  * the product is computed transposed, C^T = W A^T: the MFMA's A operand is a 16-row block of W, its B
//    operand a 16-row block of A, and each lane ends with 4 consecutive output columns of one output row
//    (one 16-byte fp32 / 8-byte fp16 store per block).
//  * both tiles stream global -> LDS through a 4-stage ring of buffer-form DMA (buffer_load ... lds), three
//    k tiles ahead; one barrier per k tile. LDS rows are 64 bytes (32 fp16 of k) holding four 16-byte
//    chunks, chunk c of row r at position c ^ ((r >> 1) & 3): the DMA reads whole row segments (coalesced)
//    and the MFMA operand reads (16 rows x one chunk per 16 lanes) are bank-conflict free.
//  * the operands of k tile t+1 are read from LDS while the MFMAs of k tile t run.
//  * each workgroup starts its k loop at its own offset (wrapping around): rows of one k tile are a 4 KB
//    multiple apart, and an unstaggered grid would hit one L2 channel at a time.
//  * 1-D grid, XCD-aware: workgroup b runs on XCD b % 8, and each XCD takes a contiguous range of tiles in
//    groups of 4 row tiles, so the workgroups resident on one XCD share A and W tiles in its L2.
#include "common.hpp"
#include "internal.hpp"

namespace kiln {

namespace {

constexpr int GBM = 256;             // activation rows (m) per workgroup
constexpr int GBN = 256;             // weight rows (n) per workgroup
constexpr int GBK = 32;              // k per tile: one 64-byte LDS row segment
constexpr int GNS = 4;               // LDS ring stages
constexpr int GTHR = 512;            // 8 waves
constexpr int GROUP_M = 4;           // row tiles per raster group
constexpr int REG_H = GBN * GBK;     // halves in one operand region of a stage (16 KB)
constexpr int STAGE_H = 2 * REG_H;   // W region, then A region
constexpr int DMA_PER_REG = REG_H * 2 / (GTHR * 16);  // 16-byte pieces per thread per region and k tile

typedef __attribute__((address_space(3))) half8 lds_half8;
typedef float f2v __attribute__((ext_vector_type(2)));

#define GEMM_WAIT_VMCNT(N) __builtin_amdgcn_s_waitcnt(((N) & 0xF) | (0x7 << 4) | (0xF << 8) | (((N) >> 4) << 14))

struct GemmParams {
    const _Float16* a;
    const _Float16* w;
    const _Float16* a2;
    const _Float16* w2;
    int K, K2, M, N;
    void* c;
    int ldc;
    const float* gate;
    float beta;
    int tiles_m, tiles_n, total, per;
    int pairs;  // output rows or base not 16-byte (fp32) / 8-byte (fp16) aligned: store element pairs
};

__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float gelu_erf(float v) { return 0.5f * v * (1.f + erff(v * 0.70710678118654752f)); }

template <int EPI>
__global__ __launch_bounds__(GTHR, 1) void k_gemm16(const GemmParams p) {
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];  // GNS x 32 KB
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wv >> 2, wm = wv & 3;

    // tile of this workgroup: XCD b % 8 takes the contiguous range [xcd * per, (xcd + 1) * per)
    const int i = (int)(blockIdx.x & 7) * p.per + (int)(blockIdx.x >> 3);
    if (i >= p.total) return;
    const int per_group = GROUP_M * p.tiles_n;
    const int g0 = (i / per_group) * GROUP_M;
    const int gsz = min(GROUP_M, p.tiles_m - g0);
    const int tm = g0 + (i % per_group) % gsz, tn = (i % per_group) / gsz;
    const int m0 = tm * GBM, n0 = tn * GBN;
    const int mrows = min(GBM, p.M - m0), nrows = min(GBN, p.N - n0);

    // DMA: this thread's 16-byte pieces q = tid + GTHR*r of a region: row q >> 2, LDS position q & 3 holding
    // k chunk (q & 3) ^ ((row >> 1) & 3). Rows past the matrix re-read its last row (results unused). Per
    // thread the byte offsets within the tile's rows are constants; the k tile goes in the scalar offset.
    uint32_t voff_w[DMA_PER_REG], voff_a[DMA_PER_REG];
    auto voffs = [&](int ld, uint32_t(&vw)[DMA_PER_REG], uint32_t(&va)[DMA_PER_REG]) {
#pragma unroll
        for (int r = 0; r < DMA_PER_REG; r++) {
            const int q = tid + GTHR * r, row = q >> 2, c = (q & 3) ^ ((row >> 1) & 3);
            vw[r] = (uint32_t)(min(row, nrows - 1) * ld + c * 8) * 2;
            va[r] = (uint32_t)(min(row, mrows - 1) * ld + c * 8) * 2;
        }
    };
    voffs(p.K, voff_w, voff_a);
    auto rsrc = [](const _Float16* base, size_t bytes) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(base), (short)0,
                                                 (int)min(bytes, (size_t)0x7fffffff), 0x00020000 /* raw, CDNA */);
    };
    const __amdgpu_buffer_rsrc_t rw1 = rsrc(p.w + (size_t)n0 * p.K, (size_t)nrows * p.K * 2);
    const __amdgpu_buffer_rsrc_t ra1 = rsrc(p.a + (size_t)m0 * p.K, (size_t)mrows * p.K * 2);
    const __amdgpu_buffer_rsrc_t rw2 = rsrc(p.w2 + (size_t)n0 * p.K2, (size_t)nrows * p.K2 * 2);
    const __amdgpu_buffer_rsrc_t ra2 = rsrc(p.a2 + (size_t)m0 * p.K2, (size_t)mrows * p.K2 * 2);
    const int KT1 = p.K / GBK, KTT = KT1 + p.K2 / GBK;
    // Staggered k order: rows of the same k tile sit one row stride apart (a multiple of 4 KB for the DiT's
    // widths), so tiles at the same k of every workgroup would fall into the same L2 channel. Workgroup i
    // starts its k loop (i % 16) x 256 bytes further along the row and wraps around.
    const int kstag = ((i & 15) * 4) % KT1;

    auto dma = [&](int kt, int stage) {
        _Float16* dw = lds + stage * STAGE_H + wv * 512;
        _Float16* da = dw + REG_H;
        if (kt < KT1) {
            const int kk = kt + kstag < KT1 ? kt + kstag : kt + kstag - KT1;
            const int so = kk * GBK * 2;
#pragma unroll
            for (int r = 0; r < DMA_PER_REG; r++) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rw1, (__attribute__((address_space(3))) void*)(dw + r * GTHR * 8), 16, voff_w[r], so, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra1, (__attribute__((address_space(3))) void*)(da + r * GTHR * 8), 16, voff_a[r], so, 0, 0);
            }
        } else {
            const int so = (kt - KT1) * GBK * 2;
            uint32_t voff_w2[DMA_PER_REG], voff_a2[DMA_PER_REG];  // the LoRA tiles (few): offsets recomputed
            voffs(p.K2, voff_w2, voff_a2);
#pragma unroll
            for (int r = 0; r < DMA_PER_REG; r++) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rw2, (__attribute__((address_space(3))) void*)(dw + r * GTHR * 8), 16, voff_w2[r], so, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    ra2, (__attribute__((address_space(3))) void*)(da + r * GTHR * 8), 16, voff_a2[r], so, 0, 0);
            }
        }
    };
    constexpr int DMA_PER_TILE = 2 * DMA_PER_REG;

    // operand reads: lane reads row (lane & 15) of a 16-row block, k chunk lane >> 4; blocks of one wave are
    // 1 KB apart, so they fold into ds_read_b128 immediate offsets.
    const uint32_t lds_base = (uint32_t)(size_t)(__attribute__((address_space(3))) _Float16*)lds;
    const int rl = lane & 15;
    const uint32_t swz = (uint32_t)((((lane >> 4) ^ ((rl >> 1) & 3))) * 16);
    const uint32_t wbase = lds_base + (uint32_t)((wn * 128 + rl) * 64) + swz;
    const uint32_t abase = lds_base + (uint32_t)(REG_H * 2 + (wm * 64 + rl) * 64) + swz;
    auto wfrag = [&](int stage, int nb) {
        return reinterpret_cast<const lds_half8*>((size_t)(wbase + stage * STAGE_H * 2))[nb * 64];
    };
    auto afrag = [&](int stage, int mb) {
        return reinterpret_cast<const lds_half8*>((size_t)(abase + stage * STAGE_H * 2))[mb * 64];
    };

    floatx4 acc[8][4];
#pragma unroll
    for (int nb = 0; nb < 8; nb++)
#pragma unroll
        for (int mb = 0; mb < 4; mb++) acc[nb][mb] = floatx4{0.f, 0.f, 0.f, 0.f};

    // prologue: k tiles 0..3 in flight; wait for tile 0 and read its operands
#pragma unroll
    for (int s = 0; s < GNS; s++)
        if (s < KTT) dma(s, s);
    if (KTT >= GNS) GEMM_WAIT_VMCNT((GNS - 1) * DMA_PER_TILE);
    else GEMM_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
    // Operands in registers: the W blocks of the current k tile (each replaced by the next tile's block as soon
    // as its four MFMAs are issued) and the A blocks of the current and the next tile (the loop alternates them).
    half8 fw[8], fa[4], ga[4];
#pragma unroll
    for (int b = 0; b < 8; b++) fw[b] = wfrag(0, b);
#pragma unroll
    for (int b = 0; b < 4; b++) fa[b] = afrag(0, b);
    __builtin_amdgcn_sched_barrier(0);

    auto step = [&](int kt, half8(&ca)[4], half8(&na)[4]) {
        // tile kt+1 landed in every wave, and every wave has read tile kt's operands (stage kt is free):
        // refill it with tile kt+4. Only tiles kt+2 and kt+3 may stay in flight.
        const int ahead = KTT - 1 - kt;
        if (ahead >= 3) GEMM_WAIT_VMCNT(2 * DMA_PER_TILE);
        else if (ahead == 2) GEMM_WAIT_VMCNT(DMA_PER_TILE);
        else GEMM_WAIT_VMCNT(0);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of stage kt are complete
        __builtin_amdgcn_s_barrier();
        if (kt + GNS < KTT) dma(kt + GNS, kt % GNS);
        __builtin_amdgcn_sched_barrier(0);
        const int nst = (kt + 1) % GNS;
        if (ahead >= 1) {
#pragma unroll
            for (int b = 0; b < 4; b++) na[b] = afrag(nst, b);
        }
#pragma unroll
        for (int nb = 0; nb < 8; nb++) {
#pragma unroll
            for (int mb = 0; mb < 4; mb++) acc[nb][mb] = mfma16(fw[nb], ca[mb], acc[nb][mb]);
            if (ahead >= 1) fw[nb] = wfrag(nst, nb);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    int kt = 0;
    for (; kt + 1 < KTT; kt += 2) {
        step(kt, fa, ga);
        step(kt + 1, ga, fa);
    }
    if (kt < KTT) step(kt, fa, ga);

    // epilogue: lane holds rows m0 + wm*64 + mb*16 + (lane & 15), columns n0 + wn*128 + nb*16 + 4*(lane >> 4) + e
    const int mrow = m0 + wm * 64 + rl;
    const int ncol = n0 + wn * 128 + 4 * (lane >> 4);
    if (ncol >= p.N) return;  // a 128-column half of the last tile past N (N % 256 == 128)
    floatx4 gv[8];
    if constexpr (EPI == KILN_EPI_RESID) {
#pragma unroll
        for (int nb = 0; nb < 8; nb++) {
            if (p.gate) {
                const float* g = p.gate + ncol + nb * 16;
                gv[nb] = floatx4{g[0], g[1], g[2], g[3]};
            } else {
                gv[nb] = floatx4{1.f, 1.f, 1.f, 1.f};
            }
        }
    }
#pragma unroll
    for (int mb = 0; mb < 4; mb++) {
        const int m = mrow + mb * 16;
        if (m >= p.M) break;
#pragma unroll
        for (int nb = 0; nb < 8; nb++) {
            const int n = ncol + nb * 16;
            const size_t off = (size_t)m * p.ldc + n;
            const floatx4 v = acc[nb][mb];
            if constexpr (EPI == KILN_EPI_F32 || EPI == KILN_EPI_RESID) {
                float* dst = static_cast<float*>(p.c) + off;
                floatx4 o;
                const bool need_old = EPI == KILN_EPI_RESID || p.beta != 0.f;
                if (need_old) {
                    if (!p.pairs) {
                        o = *reinterpret_cast<const floatx4*>(dst);
                    } else {
                        const f2v o0 = reinterpret_cast<const f2v*>(dst)[0], o1 = reinterpret_cast<const f2v*>(dst)[1];
                        o = floatx4{o0[0], o0[1], o1[0], o1[1]};
                    }
                }
                floatx4 r;
                if constexpr (EPI == KILN_EPI_RESID) {
#pragma unroll
                    for (int e = 0; e < 4; e++) r[e] = o[e] + gv[nb][e] * v[e];
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) r[e] = need_old ? v[e] + p.beta * o[e] : v[e];
                }
                if (!p.pairs) {
                    *reinterpret_cast<floatx4*>(dst) = r;
                } else {
                    reinterpret_cast<f2v*>(dst)[0] = f2v{r[0], r[1]};
                    reinterpret_cast<f2v*>(dst)[1] = f2v{r[2], r[3]};
                }
            } else {
                _Float16* dst = static_cast<_Float16*>(p.c) + off;
                floatx4 r = v;
                if constexpr (EPI == KILN_EPI_GELU16) {
#pragma unroll
                    for (int e = 0; e < 4; e++) r[e] = gelu_erf(v[e]);
                }
                if (!p.pairs) {
                    *reinterpret_cast<half4*>(dst) = half4{(_Float16)r[0], (_Float16)r[1], (_Float16)r[2], (_Float16)r[3]};
                } else {
                    reinterpret_cast<half2v*>(dst)[0] = half2v{(_Float16)r[0], (_Float16)r[1]};
                    reinterpret_cast<half2v*>(dst)[1] = half2v{(_Float16)r[2], (_Float16)r[3]};
                }
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm16(const GemmLaunch& g, hipStream_t s) {
    GemmParams p;
    p.a = reinterpret_cast<const _Float16*>(g.a);
    p.w = reinterpret_cast<const _Float16*>(g.w);
    p.a2 = reinterpret_cast<const _Float16*>(g.K2 > 0 ? g.a2 : g.a);
    p.w2 = reinterpret_cast<const _Float16*>(g.K2 > 0 ? g.w2 : g.w);
    p.K = g.K;
    p.K2 = g.K2;
    p.M = g.M;
    p.N = g.N;
    p.c = g.c;
    p.ldc = g.ldc;
    p.gate = g.gate;
    p.beta = g.beta;
    const size_t esz = (g.epi == KILN_EPI_F32 || g.epi == KILN_EPI_RESID) ? 4 : 2;
    p.pairs = ((size_t)g.c % (4 * esz) != 0) || (g.ldc % 4 != 0);
    p.tiles_m = (g.M + GBM - 1) / GBM;
    p.tiles_n = (g.N + GBN - 1) / GBN;
    p.total = p.tiles_m * p.tiles_n;
    const int nb = (p.total + 7) / 8 * 8;
    p.per = nb / 8;
    const size_t lds = (size_t)GNS * STAGE_H * sizeof(_Float16);
    switch (g.epi) {
        case KILN_EPI_F32: hipLaunchKernelGGL(k_gemm16<KILN_EPI_F32>, dim3(nb), dim3(GTHR), lds, s, p); break;
        case KILN_EPI_F16: hipLaunchKernelGGL(k_gemm16<KILN_EPI_F16>, dim3(nb), dim3(GTHR), lds, s, p); break;
        case KILN_EPI_GELU16: hipLaunchKernelGGL(k_gemm16<KILN_EPI_GELU16>, dim3(nb), dim3(GTHR), lds, s, p); break;
        case KILN_EPI_RESID: hipLaunchKernelGGL(k_gemm16<KILN_EPI_RESID>, dim3(nb), dim3(GTHR), lds, s, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace kiln
