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
//  * workgroup tile 256 weight rows (n) x 32*MB activation rows (m, MB = 8 or 7, whichever leaves the fewest
//    idle CUs in the last round), k tiles of 32; 8 waves in 4 (n) x 2 (m), each wave 64 n x 16*MB m =
//    4 x MB blocks of v_mfma_f32_16x16x32_f16 (the shape that sustains the higher rate on a power-limited
//    MI355X), up to 128 fp32 accumulators per lane, two waves per SIMD.
//  * the product is computed transposed, C^T = W A^T: the MFMA's A operand is a 16-row block of W, its B
//    operand a 16-row block of A, and each lane ends with 4 consecutive output columns of one output row
//    (one 16-byte fp32 / 8-byte fp16 store per block).
//  * both tiles stream global -> LDS through a 4-stage ring of buffer-form DMA (buffer_load ... lds), three
//    k tiles ahead; one barrier per k tile. LDS rows are 64 bytes (32 fp16 of k) holding four 16-byte
//    chunks, chunk c of row r at position c ^ ((r >> 1) & 3): the DMA reads whole row segments (coalesced)
//    and the MFMA operand reads (16 rows x one chunk per 16 lanes) are bank-conflict free.
//  * the operands of k tile t+1 are read from LDS while the MFMAs of k tile t run.
//  * 1-D grid, XCD-aware: workgroup b runs on XCD b % 8, and each XCD takes a contiguous range of tiles in
//    groups of 4 row tiles, so the workgroups resident on one XCD share A and W tiles in its L2.
#include <type_traits>

#include "common.hpp"
#include "internal.hpp"

namespace kiln {


constexpr int GBN = 256;             // weight rows (n) per workgroup
constexpr int GBK = 32;              // k per tile: one 64-byte LDS row segment
constexpr int GNS = 4;               // LDS ring stages
constexpr int WAVES_N = 4;                   // waves along n; 2 along m
constexpr int WAVES_M = 2;
constexpr int NBW = GBN / 16 / WAVES_N;      // 16-row W blocks per wave
constexpr int GTHR = 64 * WAVES_N * WAVES_M;
constexpr int GROUP_M = 4;           // row tiles per raster group
constexpr int W_REG_H = GBN * GBK;   // halves in the W region of a stage (16 KB)
constexpr int W_DMA = W_REG_H * 2 / (GTHR * 16);  // 16-byte W pieces per thread per k tile

// MB: 16-row activation blocks per wave; the workgroup's activation tile is 32*MB rows
template <int MB>
struct Tile {
    static constexpr int BM = 32 * MB;
    static constexpr int A_REG_H = BM * GBK;
    static constexpr int STAGE_H = W_REG_H + A_REG_H;
};
// 16-byte A pieces per thread per k tile (the same for every tile height used, so that no array size in the
// kernel depends on the template argument)
constexpr int A_DMA = Tile<8>::A_REG_H * 2 / (GTHR * 16);
constexpr int DMA_PER_TILE = W_DMA + A_DMA;
static_assert(Tile<8>::A_REG_H * 2 == A_DMA * GTHR * 16 && Tile<7>::A_REG_H * 2 > (A_DMA - 1) * GTHR * 16, "A pieces");

typedef __attribute__((address_space(3))) half8 lds_half8;
typedef float f2v __attribute__((ext_vector_type(2)));

// s_waitcnt vmcnt(N) (lgkmcnt and expcnt left alone). A device function, so that the host pass never checks
// the builtin's constant argument inside the kernel template (where it depends on the tile height).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

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
    int wprep;  // w is in the prepared tile layout (kiln_linear16_prepare_weight), not [N, K] rows
    // EPI_QKV (the DiT self-attention projection with its QK-RMSNorm, RoPE and fp16 K/V preparation fused):
    // columns [0, D) are Q, [D, 2D) K, [2D, 3D) V of H heads; row r is token r % T of item r / T
    _Float16* q16;      // [M, D]: fp16(rope(rmsnorm(q)) * qscale)
    uint16_t* kvp[MAX_JOBS];  // prepared K/V per item (common.hpp layout), K = rope(rmsnorm(k))
    int T, H;
    const uint16_t* qw;  // bf16 [128] norm weights
    const uint16_t* kw;
    float eps, qscale;
    const float* rcos;  // [T, 64]
    const float* rsin;
};
constexpr int EPI_QKV = 4;
struct KvTailJobs {
    uint16_t* kvp[MAX_JOBS];
};

__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// GELU(v) = v Phi(v) = v (1 + erf(v / sqrt 2)) / 2, with Phi from erfc, which keeps its relative accuracy in the
// negative tail: Phi(v) = erfc(z) / 2 for v < 0 and 1 - erfc(z) / 2 for v >= 0, z = |v| / sqrt 2. erfc(z) for
// z >= 0 is the Chebyshev approximation "erfcc" of Numerical Recipes in C (Press et al., 2nd ed., section 6.2),
// fractional error below 1.2e-7 everywhere: ~17 VALU operations and no branches, about half of a library erff,
// and far below the fp16 output's rounding.
__device__ __forceinline__ float gelu_erf(float v) {
    const float z = fabsf(v) * 0.70710678118654752f;
    const float t = __builtin_amdgcn_rcpf(1.f + 0.5f * z);
    float r = 0.17087277f;
    r = fmaf(t, r, -0.82215223f);
    r = fmaf(t, r, 1.48851587f);
    r = fmaf(t, r, -1.13520398f);
    r = fmaf(t, r, 0.27886807f);
    r = fmaf(t, r, -0.18628806f);
    r = fmaf(t, r, 0.09678418f);
    r = fmaf(t, r, 0.37409196f);
    r = fmaf(t, r, 1.00002368f);
    r = fmaf(t, r, -1.26551223f);
    const float half_erfc = 0.5f * t * __expf(r - z * z);
    return v * (v >= 0.f ? 1.f - half_erfc : half_erfc);
}

// EPI_QKV epilogue. The workgroup's 256 columns are two heads of one region (Q, K or V: D is a multiple of 256).
// A wave holds 64 columns = half a head; its partner wave (wv ^ 2, the same rows) holds the other half. In the Q and
// K regions the k loop read the wave's W blocks so that block nb holds head dims dq(nb) + 0..15, dq(nb) =
// 32*(wn & 1) + 16*(nb & 1) + 64*(nb >> 1): each RoPE pair (i, i + 64) is element (nb, e) and (nb + 2, e) of one
// lane. Q/K: per-row sum of squares over the head (own half + partner's, through LDS), scale by rsqrt(mean + eps)
// and the bf16 weight, then RoPE in registers. Q is stored as fp16(q * qscale) rows, K and V in the prepared K/V
// layout of their item (kv_k_el / kv_v_el).
template <int MB>
__device__ __forceinline__ void qkv_epilogue(const GemmParams& p, floatx4 (&acc)[NBW][MB], _Float16* lds, int m0,
                                             int n0, int wv, int wn, int wm, int lane) {
    const int D = p.H * HD;
    const int region = n0 / D, c0 = n0 - region * D;
    const int hd = (c0 + (wn >> 1) * HD) / HD, half = wn & 1;
    const int rl = lane & 15, cq = 4 * (lane >> 4);  // column within a 16-column block: cq + e
    const int rbase = m0 + wm * 16 * MB + rl;
    auto dq = [&](int nb) { return 32 * half + 16 * (nb & 1) + 64 * (nb >> 1); };  // Q/K head dim of block nb
    float* lf = reinterpret_cast<float*>(lds);
    __syncthreads();  // every wave is done with the k loop's LDS stages
    if (region < 2) {
        const uint16_t* w = region == 0 ? p.qw : p.kw;
        float wt[NBW][4];
#pragma unroll
        for (int nb = 0; nb < NBW; nb++)
#pragma unroll
            for (int e = 0; e < 4; e++) wt[nb][e] = bf16_to_f32(w[dq(nb) + cq + e]);  // any alignment of w
        float r[MB];
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            float ss = 0.f;
#pragma unroll
            for (int nb = 0; nb < NBW; nb++)
#pragma unroll
                for (int e = 0; e < 4; e++) ss += acc[nb][mb][e] * acc[nb][mb][e];
            ss += __shfl_xor(ss, 16, 64);
            ss += __shfl_xor(ss, 32, 64);
            if (lane < 16) lf[wv * 16 * MB + mb * 16 + rl] = ss;
            r[mb] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int mb = 0; mb < MB; mb++) r[mb] = rsqrtf((r[mb] + lf[(wv ^ 2) * 16 * MB + mb * 16 + rl]) * (1.0f / HD) + p.eps);
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int nb = 0; nb < NBW; nb++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[nb][mb][e] *= r[mb] * wt[nb][e];
        if (p.rcos) {  // RoPE (none for the cross-attention Q projection)
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
                const int row = rbase + mb * 16;
                const int t = (row < p.M ? row : 0) % p.T;
#pragma unroll
                for (int nb = 0; nb < 2; nb++) {
                    const floatx4 cs = *reinterpret_cast<const floatx4*>(p.rcos + (size_t)t * 64 + dq(nb) + cq);
                    const floatx4 sn = *reinterpret_cast<const floatx4*>(p.rsin + (size_t)t * 64 + dq(nb) + cq);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float a = acc[nb][mb][e], b = acc[nb + 2][mb][e];
                        acc[nb][mb][e] = a * cs[e] - b * sn[e];
                        acc[nb + 2][mb][e] = b * cs[e] + a * sn[e];
                    }
                }
            }
        }
    }
    if (region == 2 && p.T % 32 == 0) {
        // V through LDS, one head (128 columns) per pass: the wave pairs of that head write their fp16 values
        // row-major (rows padded to 288 bytes), then every wave assembles whole 16-byte V^T operand units (8 keys of
        // one d) with transposing reads, as the K/V prepare pass does, instead of 2-byte scatters. With T a
        // multiple of 32 (and the tile's first row one too) no 32-key half tile straddles two items.
        constexpr int VRS = HD + 16, BM = 32 * MB;
        static_assert(BM * VRS <= GNS * Tile<MB>::STAGE_H, "the staged V tile fits in the ring's LDS");
        const int i = lane & 15, gq = lane >> 4;
        typedef short s4 __attribute__((ext_vector_type(4)));
        typedef short s8 __attribute__((ext_vector_type(8)));
        typedef __attribute__((address_space(3))) s4 lds_s4;
#pragma unroll
        for (int pass = 0; pass < 2; pass++) {
            if ((wn >> 1) == pass) {
#pragma unroll
                for (int mb = 0; mb < MB; mb++)
#pragma unroll
                    for (int nb = 0; nb < NBW; nb++) {
                        const floatx4 v = acc[nb][mb];
                        *reinterpret_cast<half4*>(lds + (wm * 16 * MB + mb * 16 + rl) * VRS + half * 64 + nb * 16 + cq) =
                            half4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
                    }
            }
            __syncthreads();
            const int hdp = (c0 + pass * HD) / HD;
            for (int op = wv; op < (BM / 32) * 8; op += WAVES_N * WAVES_M) {
                const int ht = op >> 3, db = op & 7, row0 = m0 + ht * 32;
                if (row0 >= p.M) break;  // ops ascend with ht: every later one is past the matrix too
                const int b = row0 / p.T, key0 = row0 - b * p.T;
                const _Float16* src = lds + (ht * 32 + 4 * gq + (i >> 2)) * VRS + 16 * db + 4 * (i & 3);
                const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)src);
                const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(src + 16 * VRS));
                _Float16* kv = reinterpret_cast<_Float16*>(p.kvp[b]) + (size_t)hdp * kv_head_stride(p.T) +
                               (size_t)(key0 / KT) * KV_TILE_H;
                *reinterpret_cast<s8*>(kv + kv_v_off((key0 % KT) / 32, db, lane)) =
                    s8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
            __syncthreads();  // every read of this head's values precedes the next pass's writes
        }
        return;
    }
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const int row = rbase + mb * 16;
        if (row >= p.M) continue;
        const int b = row / p.T, key = row - b * p.T;
        _Float16* kv = reinterpret_cast<_Float16*>(p.kvp[b]) + (size_t)hd * kv_head_stride(p.T) +
                       (size_t)(key / KT) * KV_TILE_H;
        const int kc = (key % KT) / 32, k32 = key % 32;
#pragma unroll
        for (int nb = 0; nb < NBW; nb++) {
            // 4 consecutive d, inside one 8-element chunk (Q/K: the permuted head dims; V: the plain ones)
            const int d = (region < 2 ? dq(nb) : half * 64 + nb * 16) + cq;
            const floatx4 v = acc[nb][mb];
            if (region == 0) {
                *reinterpret_cast<half4*>(p.q16 + (size_t)row * D + hd * HD + d) =
                    half4{(_Float16)(v[0] * p.qscale), (_Float16)(v[1] * p.qscale), (_Float16)(v[2] * p.qscale),
                          (_Float16)(v[3] * p.qscale)};
            } else if (region == 1) {
                *reinterpret_cast<half4*>(kv + kv_k_el(kc, k32, d)) =
                    half4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) kv[kv_v_el(kc, k32, d + e)] = (_Float16)v[e];
            }
        }
    }
}

// LATE (prepared weights): in steady steps the refill DMA leaves the barrier's shadow and the two waves of a SIMD
// issue it at different points of the MFMA stream: waves 0-3 after the first activation block's MFMAs, waves 4-7
// after the fourth. Waves w and w + 4 share a SIMD; with both refills issued together right after the barrier,
// the DMA issue stalls of the two waves coincide and the matrix core idles through them. Measured on the DiT
// shapes (A/B on one box): the block's four GEMMs -1.4% with waves 4-7 moved, -1.0 to -1.9% more with waves 0-3
// moved as well; the split slows plain-weight launches (whose W rows arrive as 64-byte row pieces) by ~2%, which
// keep the refill after the barrier.
constexpr int EARLY_MB = 1, LATE_MB = 3;
template <int EPI, int MB, bool LATE>
__global__ __launch_bounds__(GTHR, 1) void k_gemm16(const GemmParams p) {
    using TL = Tile<MB>;
    constexpr int BM = TL::BM, STAGE_H = TL::STAGE_H;
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];  // GNS stages of [W 256 rows | A BM rows]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wv / WAVES_M, wm = wv % WAVES_M;

    // tile of this workgroup: XCD b % 8 takes the contiguous range [xcd * per, (xcd + 1) * per)
    const int i = (int)(blockIdx.x & 7) * p.per + (int)(blockIdx.x >> 3);
    if (i >= p.total) return;
    const int per_group = GROUP_M * p.tiles_n;
    const int g0 = (i / per_group) * GROUP_M;
    const int gsz = min(GROUP_M, p.tiles_m - g0);
    const int tm = g0 + (i % per_group) % gsz, tn = (i % per_group) / gsz;
    const int m0 = tm * BM, n0 = tn * GBN;
    const int mrows = min(BM, p.M - m0), nrows = min(GBN, p.N - n0);

    // DMA: this thread's 16-byte pieces q = tid + GTHR*r of a region: row q >> 2, LDS position q & 3 holding
    // k chunk (q & 3) ^ ((row >> 1) & 3). Rows past the matrix re-read its last row (results unused); pieces
    // past a region's end repeat the piece one round earlier (same source, same LDS bytes), so every wave
    // issues the same number of DMA operations. The k tile goes in the scalar offset.
    uint32_t voff_w[W_DMA], voff_a[A_DMA];
    auto voffs = [&](int ld, bool prep, uint32_t(&vw)[W_DMA], uint32_t(&va)[A_DMA]) {
#pragma unroll
        for (int r = 0; r < W_DMA; r++) {
            const int q = tid + GTHR * r, row = q >> 2, c = (q & 3) ^ ((row >> 1) & 3);
            // prepared W (main product only): the k tile's 16 KB block is already in LDS order
            vw[r] = prep ? (uint32_t)q * 16 : (uint32_t)(min(row, nrows - 1) * ld + c * 8) * 2;
        }
#pragma unroll
        for (int r = 0; r < A_DMA; r++) {
            int q = tid + GTHR * r;
            if (q >= BM * 4) q -= GTHR;
            const int row = q >> 2, c = (q & 3) ^ ((row >> 1) & 3);
            va[r] = (uint32_t)(min(row, mrows - 1) * ld + c * 8) * 2;
        }
    };
    voffs(p.K, p.wprep != 0, voff_w, voff_a);
#define GEMM_RSRC(base, bytes)                                                                             \
    __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(base), (short)0, (int)min((size_t)(bytes), (size_t)0x7fffffff), \
                                      0x00020000 /* raw, CDNA */)
    const __amdgpu_buffer_rsrc_t rw1 =
        p.wprep ? GEMM_RSRC(p.w + (size_t)tn * GBN * p.K, (size_t)GBN * p.K * 2)
                : GEMM_RSRC(p.w + (size_t)n0 * p.K, (size_t)nrows * p.K * 2);
    const __amdgpu_buffer_rsrc_t ra1 = GEMM_RSRC(p.a + (size_t)m0 * p.K, (size_t)mrows * p.K * 2);
    const __amdgpu_buffer_rsrc_t rw2 = GEMM_RSRC(p.w2 + (size_t)n0 * p.K2, (size_t)nrows * p.K2 * 2);
    const __amdgpu_buffer_rsrc_t ra2 = GEMM_RSRC(p.a2 + (size_t)m0 * p.K2, (size_t)mrows * p.K2 * 2);
    const int KT1 = p.K / GBK, KTT = KT1 + p.K2 / GBK;
    // the wave's 64 lanes write 1 KB of contiguous LDS at the wave-uniform base the DMA takes from M0
    auto dma = [&](int kt, int stage) {
        _Float16* base = lds + stage * STAGE_H;
        _Float16* aq0[A_DMA];
#pragma unroll
        for (int r = 0; r < A_DMA; r++) {
            int q0 = GTHR * r + wv * 64;
            if (q0 >= BM * 4) q0 -= GTHR;
            aq0[r] = base + W_REG_H + q0 * 8;
        }
        if (kt < KT1) {
            const int so = kt * GBK * 2;
            const int sow = p.wprep ? kt * W_REG_H * 2 : so;
#pragma unroll
            for (int r = 0; r < W_DMA; r++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rw1, (__attribute__((address_space(3))) void*)(base + (GTHR * r + wv * 64) * 8), 16, voff_w[r], sow, 0, 0);
#pragma unroll
            for (int r = 0; r < A_DMA; r++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra1, (__attribute__((address_space(3))) void*)aq0[r], 16,
                                                         voff_a[r], so, 0, 0);
        } else {
            const int so = (kt - KT1) * GBK * 2;
            uint32_t vw2[W_DMA], va2[A_DMA];  // the LoRA tiles (few): offsets recomputed
            voffs(p.K2, false, vw2, va2);
#pragma unroll
            for (int r = 0; r < W_DMA; r++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rw2, (__attribute__((address_space(3))) void*)(base + (GTHR * r + wv * 64) * 8), 16, vw2[r], so, 0, 0);
#pragma unroll
            for (int r = 0; r < A_DMA; r++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra2, (__attribute__((address_space(3))) void*)aq0[r], 16,
                                                         va2[r], so, 0, 0);
        }
    };

    // operand reads: lane reads row (lane & 15) of a 16-row block, k chunk lane >> 4; blocks of one wave are
    // 1 KB apart, so they fold into ds_read_b128 immediate offsets.
    const uint32_t lds_base = (uint32_t)(size_t)(__attribute__((address_space(3))) _Float16*)lds;
    const int rl = lane & 15;
    const uint32_t swz = (uint32_t)((((lane >> 4) ^ ((rl >> 1) & 3))) * 16);
    // EPI_QKV, Q and K regions: the wave's W blocks are the head rows 32*(wn & 1) + {0, 16, 64, 80} instead of
    // 64*(wn & 1) + {0, 16, 32, 48}, so that each RoPE pair (d, d + 64) lands in one lane (blocks nb and nb + 2)
    const bool qkperm = EPI == EPI_QKV && n0 / (p.H * HD) < 2;
    const uint32_t wbase = lds_base + (uint32_t)((((wn >> 1) * 128 + (wn & 1) * (qkperm ? 32 : 64)) + rl) * 64) + swz;
    const uint32_t wbase_hi = wbase + (qkperm ? 2048u : 0u);  // blocks nb >= 2
    const uint32_t abase = lds_base + (uint32_t)(W_REG_H * 2 + (wm * MB * 16 + rl) * 64) + swz;
    auto wfrag = [&](int stage, int nb) {
        return reinterpret_cast<const lds_half8*>((size_t)((nb < 2 ? wbase : wbase_hi) + stage * STAGE_H * 2))[nb * 64];
    };
    auto afrag = [&](int stage, int mb) {
        return reinterpret_cast<const lds_half8*>((size_t)(abase + stage * STAGE_H * 2))[mb * 64];
    };

    floatx4 acc[NBW][MB];
#pragma unroll
    for (int nb = 0; nb < NBW; nb++)
#pragma unroll
        for (int mb = 0; mb < MB; mb++) acc[nb][mb] = floatx4{0.f, 0.f, 0.f, 0.f};

    // prologue: k tiles 0..3 in flight; wait for tile 0 and read its operands
#pragma unroll
    for (int s = 0; s < GNS; s++)
        if (s < KTT) dma(s, s);
    if (KTT >= GNS) wait_vmcnt<(GNS - 1) * DMA_PER_TILE>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    // Operands in registers: the activation blocks of the current k tile (each replaced by the next tile's
    // block as soon as its four MFMAs are issued) and the W blocks of the current and the next tile (the loop
    // alternates them).
    half8 fa[MB], fw[NBW], gw[NBW];
#pragma unroll
    for (int b = 0; b < MB; b++) fa[b] = afrag(0, b);
#pragma unroll
    for (int b = 0; b < NBW; b++) fw[b] = wfrag(0, b);
    __builtin_amdgcn_sched_barrier(0);

    // STEADY: kt + GNS < KTT (a refill to issue, the next tile's operands to read, GNS - 2 tiles in flight)
    auto step = [&](auto steady_tag, int kt, half8(&cw)[NBW], half8(&nw)[NBW]) {
        constexpr bool STEADY = decltype(steady_tag)::value;
        // tile kt+1 landed in every wave, and every wave has read tile kt's operands (stage kt is free):
        // refill it with tile kt+GNS. Only tiles kt+2 .. kt+GNS-1 may stay in flight.
        const int ahead = KTT - 1 - kt;
        static_assert(GNS == 4, "the waits below assume a 4-stage ring");
        if (STEADY || ahead >= 3) wait_vmcnt<2 * DMA_PER_TILE>();
        else if (ahead == 3) wait_vmcnt<2 * DMA_PER_TILE>();
        else if (ahead == 2) wait_vmcnt<DMA_PER_TILE>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of stage kt are complete
        __builtin_amdgcn_s_barrier();
        const bool split = LATE && STEADY;  // the refill moves into the MFMA stream (position by wave)
        if (!split && (STEADY || kt + GNS < KTT)) dma(kt + GNS, kt % GNS);
        __builtin_amdgcn_sched_barrier(0);
        const int nst = (kt + 1) % GNS;
        const bool more = STEADY || ahead >= 1;
        if (more) {
#pragma unroll
            for (int b = 0; b < NBW; b++) nw[b] = wfrag(nst, b);
        }
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
#pragma unroll
            for (int nb = 0; nb < NBW; nb++) acc[nb][mb] = mfma16(cw[nb], fa[mb], acc[nb][mb]);
            if (more) fa[mb] = afrag(nst, mb);
            if (split && mb == (wv >= 4 ? LATE_MB : EARLY_MB)) {
                __builtin_amdgcn_sched_barrier(0);
                dma(kt + GNS, kt % GNS);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // steady steps: one operand read, then two MFMAs, in turn (the backend otherwise clusters the reads;
        // +1-1.5% on the DiT shapes)
        if constexpr (STEADY) {
#pragma unroll
            for (int i = 0; i < NBW + MB; i++) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using True = std::true_type;
    using False = std::false_type;
    int kt = 0;
    for (; kt + 1 + GNS < KTT; kt += 2) {
        step(True{}, kt, fw, gw);
        step(True{}, kt + 1, gw, fw);
    }
    for (; kt + 1 < KTT; kt += 2) {
        step(False{}, kt, fw, gw);
        step(False{}, kt + 1, gw, fw);
    }
    if (kt < KTT) step(False{}, kt, fw, gw);

    if constexpr (EPI == EPI_QKV) {
        qkv_epilogue<MB>(p, acc, lds, m0, n0, wv, wn, wm, lane);
        return;
    }
    // epilogue: lane holds rows m0 + wm*16*MB + mb*16 + (lane & 15), columns n0 + wn*64 + nb*16 + 4*(lane >> 4) + e
    const int mrow = m0 + wm * 16 * MB + rl;
    const int ncol = n0 + wn * NBW * 16 + 4 * (lane >> 4);
    if (ncol >= p.N) return;  // a column range of the last tile past N (N % 256 == 128)
    floatx4 gv[NBW];
    if constexpr (EPI == KILN_EPI_RESID) {
#pragma unroll
        for (int nb = 0; nb < NBW; nb++) {
            if (p.gate) {
                const float* g = p.gate + ncol + nb * 16;
                gv[nb] = floatx4{g[0], g[1], g[2], g[3]};
            } else {
                gv[nb] = floatx4{1.f, 1.f, 1.f, 1.f};
            }
        }
    }
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const int m = mrow + mb * 16;
        if (m >= p.M) break;
#pragma unroll
        for (int nb = 0; nb < NBW; nb++) {
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

// Prepared weight layout: [ceil(N/256) column tiles][K/32 k tiles][16 KB block], the block holding the 256 rows
// x 32 k of the tile in the kernel's LDS order (16-byte piece q: row q >> 2, k chunk (q & 3) ^ ((row >> 1) & 3));
// rows past N are zero. The k loop's W DMA then reads one contiguous 16 KB block per k tile instead of 256 row
// segments 2 KB or more apart (measured 14-17% faster on the DiT shapes). The source is fp16 or bf16; bf16 is
// clamped to the fp16 range and rounded to nearest even (the reference's weight_to_f16, kernels.cu:531-544).
__global__ void k_gemm_wprep(_Float16* __restrict__ wp, const uint16_t* __restrict__ w, int N, int K, int src_bf16,
                             long total) {
    const long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= total) return;
    const int q = (int)(g & 1023);
    const long blk = g >> 10;
    const int KT = K / GBK;
    const int kt = (int)(blk % KT), tn = (int)(blk / KT);
    const int row = q >> 2, c = (q & 3) ^ ((row >> 1) & 3);
    const int n = tn * GBN + row;
    half8 v = {};
    if (n < N) {
        const uint16_t* src = w + (size_t)n * K + kt * GBK + c * 8;
        if (src_bf16) {
            const u32x4 raw = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint16_t b = (uint16_t)(raw[e / 2] >> (16 * (e & 1)));
                v[e] = (_Float16)fminf(fmaxf(bf16_to_f32(b), -65504.f), 65504.f);
            }
        } else {
            v = *reinterpret_cast<const half8*>(src);
        }
    }
    *reinterpret_cast<half8*>(wp + g * 8) = v;
}

size_t gemm16_prepped_bytes(int N, int K) { return (size_t)((N + GBN - 1) / GBN) * GBN * K * sizeof(_Float16); }

hipError_t launch_gemm_wprep(uint16_t* wp, const uint16_t* w, int N, int K, bool src_bf16, hipStream_t s) {
    const long total = (long)((N + GBN - 1) / GBN) * (K / GBK) * 1024;
    hipLaunchKernelGGL(k_gemm_wprep, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       reinterpret_cast<_Float16*>(wp), w, N, K, src_bf16 ? 1 : 0, total);
    return hipGetLastError();
}

__global__ void k_kv_zero_tail(KvTailJobs j, size_t head_stride, size_t tail_off) {
    // block (item, head): 32 KB of the last tile, 16 bytes per thread and step
    _Float16* base = reinterpret_cast<_Float16*>(j.kvp[blockIdx.y]) + blockIdx.x * head_stride + tail_off;
    for (int i = threadIdx.x; i < KV_TILE_H / 8; i += blockDim.x) reinterpret_cast<half8*>(base)[i] = half8{};
}

hipError_t launch_kv_zero_tail(uint16_t* const* kvp, int njobs, int T, int H, hipStream_t s) {
    if (T % KT == 0 || njobs <= 0) return hipSuccess;
    KvTailJobs j{};
    for (int b = 0; b < njobs && b < MAX_JOBS; b++) j.kvp[b] = kvp[b];
    hipLaunchKernelGGL(k_kv_zero_tail, dim3(H, njobs), dim3(256), 0, s, j, kv_head_stride(T),
                       (size_t)(kv_tiles(T) - 1) * KV_TILE_H);
    return hipGetLastError();
}

static int cu_count() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus[dev] = 256;
    return cus[dev];
}

template <int MB>
static hipError_t launch_mb(GemmParams p, int epi, hipStream_t s) {
    constexpr int BM = Tile<MB>::BM;
    p.tiles_m = (p.M + BM - 1) / BM;
    p.tiles_n = (p.N + GBN - 1) / GBN;
    p.total = p.tiles_m * p.tiles_n;
    const int nb = (p.total + 7) / 8 * 8;
    p.per = nb / 8;
    const size_t lds = (size_t)GNS * Tile<MB>::STAGE_H * sizeof(_Float16);
    void (*kern)(GemmParams) = nullptr;
    const bool late = p.wprep != 0;
    switch (epi) {
        case KILN_EPI_F32: kern = late ? k_gemm16<KILN_EPI_F32, MB, true> : k_gemm16<KILN_EPI_F32, MB, false>; break;
        case KILN_EPI_F16: kern = late ? k_gemm16<KILN_EPI_F16, MB, true> : k_gemm16<KILN_EPI_F16, MB, false>; break;
        case KILN_EPI_GELU16:
            kern = late ? k_gemm16<KILN_EPI_GELU16, MB, true> : k_gemm16<KILN_EPI_GELU16, MB, false>;
            break;
        case KILN_EPI_RESID:
            kern = late ? k_gemm16<KILN_EPI_RESID, MB, true> : k_gemm16<KILN_EPI_RESID, MB, false>;
            break;
        case EPI_QKV: kern = late ? k_gemm16<EPI_QKV, MB, true> : k_gemm16<EPI_QKV, MB, false>; break;
        default: return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(kern, dim3(nb), dim3(GTHR), lds, s, p);
    return hipGetLastError();
}


// Activation tile height (32*MB rows, MB in {8, 7}): the one with the fewest CU rounds x rows per tile, one
// workgroup per CU. M = 6912 (the DiT's CFG batch) is 27 tiles of 256 rows, so every grid of 256-row tiles
// leaves 5/32 of the last round idle; 224-row tiles give 31 per column and fill 97%.
int gemm16_mb(int M, int N) {
    const int cus = cu_count(), tn = (N + GBN - 1) / GBN;
    int best = 8;
    long best_cost = -1;
    for (int mb : {8, 7}) {
        const long tiles = (long)((M + 32 * mb - 1) / (32 * mb)) * tn;
        const long cost = (tiles + cus - 1) / cus * mb;
        if (best_cost < 0 || cost < best_cost) {
            best = mb;
            best_cost = cost;
        }
    }
    return best;
}

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
    p.wprep = g.wprep ? 1 : 0;
    if (g.epi == EPI_QKV) {
        p.q16 = reinterpret_cast<_Float16*>(g.q16);
        for (int b = 0; b < MAX_JOBS; b++) p.kvp[b] = g.kvp[b];
        p.T = g.T;
        p.H = g.H;
        p.qw = g.qw;
        p.kw = g.kw;
        p.eps = g.eps;
        p.qscale = LOG2E / sqrtf((float)HD);
        p.rcos = g.rcos;
        p.rsin = g.rsin;
    }
    if (gemm16_mb(g.M, g.N) == 7) return launch_mb<7>(p, g.epi, s);
    return launch_mb<8>(p, g.epi, s);
}

}  // namespace kiln
