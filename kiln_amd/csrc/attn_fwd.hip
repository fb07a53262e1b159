// Flash-attention forward for head_dim 128 on gfx950 (CDNA4) fp16 MFMA with fp32 accumulation.
//
// Contract: the reference's tfa::k_flash (engine/src/tcflash.cuh:20-157): O = softmax(Q K^T / sqrt(128)) V
// per head, Q pre-scaled by log2(e)/sqrt(128) and rounded to fp16, base-2 online softmax, P rounded to
// fp16, analytic npad zero keys (tcflash.cuh:136-147). PV accumulates in fp32 (the MFMA's native
// accumulator) instead of the reference's GeForce-specific fp16 partial sums.
//
// Design (gfx950, wave64):
//  * workgroup = 4 waves x 32 query rows (BM = 128, two workgroups per CU), or 8 waves x 32 rows (one per CU,
//    for grids whose 256-row tiles fill whole rounds of CUs, or at least one round of units with >= 2048 keys);
//    K/V stream in half tiles of 32 keys.
//  * scores are computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_f16 (under the chip's power limit
//    this shape sustains more flop/s than 32x32x16): a wave's 32 rows are two 16-column query blocks, and
//    the four lanes n, n+16, n+32, n+48 of a column hold 8 of each half tile's 32 keys, so the row max needs
//    a cross-lane step only when the running max moves; the row sum comes from the matrix core (P^T times an
//    all-ones block).
//  * O^T = V^T P^T: P^T comes straight out of the two S^T accumulators of a query block (no LDS round trip);
//    V^T is the A operand, pre-permuted by the K/V prepare pass so that every LDS operand read of a wave is
//    one contiguous, conflict-free 1 KB ds_read_b128, and each read feeds both query blocks.
//  * K/V stream through a ring of LDS stages filled by buffer-form global->LDS DMA, several tiles ahead.
//  * the VALU, not the matrix core, is the tighter budget (MFMA and VALU work of a step barely overlap), so
//    per-step vector work is cut to the softmax itself: the QK accumulator starts from -m (no subtraction
//    before the exp), the loop is unrolled by two (no register copies of S), and DMA addressing is scalar.
//  * Q's RMSNorm and RoPE are applied in the Q tile load, in fp32, before the single fp16 rounding.
//  * the softmax rescale of O is lazy: the running max only moves (and O/l are only rescaled) when a
//    tile's max exceeds it by more than 8 (log2 units), so P <= 2^8 stays far inside fp16 range.
//  * 1-D grid with an XCD-aware block -> work mapping: consecutive work items (the query tiles of one
//    head) land on the same XCD and share its L2.
//  * grids that would fill under a third of the resident workgroup slots split every query tile's keys into
//    ranges; each range writes a partial (unnormalized O, m, l) and k_attn_merge combines them.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "internal.hpp"

namespace kiln {

constexpr float RESCALE_TH = 8.0f;

struct AttnParams {
    AttnJob job[MAX_JOBS];
    int njobs, Tq, H, ldq, ldo, qtiles, total, per;
    int ksplit;   // key ranges per (query tile, head, job): > 1 writes partial (m, l, O) for k_attn_merge
    int chain;    // context chain: a unit is a (query tile, head) and runs every job's keys in turn
    float* part;  // partials: [unit][ksplit] x (O [128 rows][128] fp32, then (m, l) per row)
    int store_pairs;  // ldo or an output base not 8/16-byte aligned: store element pairs
    int store_rows;   // ldo and every output base 16-byte aligned: output rows staged through LDS
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

__device__ __forceinline__ floatx4 mfma16(half8 a, half8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---- shared pieces of the two kernels ----

// Work item of block b. Blocks are dispatched round-robin over the 8 XCDs (block b -> XCD b % 8):
// each XCD gets a contiguous range of work items, so the query tiles of one head share its L2.
struct Work {
    int qt, h, jb, ks;
};
__device__ __forceinline__ bool decode_work(const AttnParams& p, Work& w) {
    const int i = (int)(blockIdx.x & 7) * p.per + (int)(blockIdx.x >> 3);
    if (i >= p.total) return false;
    w.qt = i % p.qtiles;
    int rest = i / p.qtiles;
    w.ks = rest % p.ksplit;  // the key ranges of one query tile sit in one XCD's range, next to each other
    rest /= p.ksplit;
    w.h = rest % p.H;
    w.jb = rest / p.H;
    return true;
}

// 8 consecutive input elements as loaded (16 B of fp16 or 32 B of fp32)
template <typename InT>
struct Chunk8;
template <>
struct Chunk8<_Float16> {
    half8 v;
    __device__ __forceinline__ void load(const _Float16* p) { v = *reinterpret_cast<const half8*>(p); }
    __device__ __forceinline__ void zero() { v = half8{}; }
    __device__ __forceinline__ float operator[](int e) const { return (float)v[e]; }
};
template <>
struct Chunk8<float> {
    floatx4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = *reinterpret_cast<const floatx4*>(p);
        b = *reinterpret_cast<const floatx4*>(p + 4);
    }
    __device__ __forceinline__ void zero() { a = b = floatx4{}; }
    __device__ __forceinline__ float operator[](int e) const { return e < 4 ? a[e] : b[e - 4]; }
};

// Q tile of one lane: query rows row[qb] (qb = 0, 1: the wave's two 16-row blocks), d chunks {32c + 8g .. +8}
// for c = 0..3 (the B operands of S^T = K Q^T), RMSNorm and RoPE applied in fp32, pre-scaled by
// log2(e)/sqrt(128), rounded once to fp16. The four lanes g = 0..3 of a query column hold its 128 dims.
template <typename InT, bool QNORM, bool ROPE>
__device__ __forceinline__ void load_q(const AttnParams& p, const void* q, const int (&row)[2], const bool (&qin)[2],
                                       int h, int g, half8 (&qreg)[2][4]) {
    // Every load (Q rows, RoPE rows, norm weights) is issued before any of them is used, unconditionally (rows
    // past Tq read row 0 and are zeroed afterwards): one memory round trip for the whole tile. A per-lane
    // branch around a load, or a conversion scheduled between loads, serializes them.
    int rr[2];
    Chunk8<InT> raw[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        rr[qb] = qin[qb] ? row[qb] : 0;
        const InT* qr = reinterpret_cast<const InT*>(q) + (size_t)rr[qb] * p.ldq + h * HD + 8 * g;
#pragma unroll
        for (int c = 0; c < 4; c++) raw[qb][c].load(qr + 32 * c);
    }
    floatx4 cr[2][2][2], sr[2][2][2];  // [qb][c < 2][4-element half]: RoPE pairs (d, d + 64) = chunks (c, c + 2)
    if constexpr (ROPE) {
#pragma unroll
        for (int qb = 0; qb < 2; qb++)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const float* cp = p.rcos + (size_t)rr[qb] * 64 + 32 * c + 8 * g;
                const float* sp = p.rsin + (size_t)rr[qb] * 64 + 32 * c + 8 * g;
                cr[qb][c][0] = *reinterpret_cast<const floatx4*>(cp);
                cr[qb][c][1] = *reinterpret_cast<const floatx4*>(cp + 4);
                sr[qb][c][0] = *reinterpret_cast<const floatx4*>(sp);
                sr[qb][c][1] = *reinterpret_cast<const floatx4*>(sp + 4);
            }
    }
    uint16_t wb[4][8];
    if constexpr (QNORM) {
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) wb[c][e] = p.qw[32 * c + 8 * g + e];
    }
    __builtin_amdgcn_sched_barrier(0);

    // Rows past Tq (which read row 0) are zeroed by the final multiplier; the norm's per-row factor r joins the
    // pre-scale there: q' = RoPE(x * w) * (r * qscale), the same mathematics as RoPE(x * r * w) * qscale.
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        float x[4][8];
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) x[c][e] = raw[qb][c][e];
        float sc = p.qscale;
        if constexpr (QNORM) {
            float ss = 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int e = 0; e < 8; e++) ss += x[c][e] * x[c][e];
            ss = quad_sum(ss);
            sc *= rsqrtf(ss * (1.0f / HD) + p.eps);
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int e = 0; e < 8; e++) x[c][e] *= bf16_to_f32(wb[c][e]);
        }
        sc = qin[qb] ? sc : 0.f;
        if constexpr (ROPE) {
#pragma unroll
            for (int c = 0; c < 2; c++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float cs = cr[qb][c][e / 4][e % 4], sn = sr[qb][c][e / 4][e % 4];
                    const float a = x[c][e], b = x[c + 2][e];
                    x[c][e] = a * cs - b * sn;
                    x[c + 2][e] = b * cs + a * sn;
                }
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
#pragma unroll
            for (int e = 0; e < 8; e++) x[c][e] *= sc;
            qreg[qb][c] = to_half8(x[c]);
        }
    }
}

// accumulator item i of key block kb of a 32-key half tile holds key 32*jh + 16*kb + 4*g + i
__device__ __forceinline__ void mask_half(int jh, int Tk, int g, floatx4 (&a)[2][2]) {
    const int kbase = jh * 32 + 4 * g;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int qb = 0; qb < 2; qb++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (kbase + 16 * kb + i >= Tk) a[kb][qb][i] = -INFINITY;
}

// full row sum (four lanes), npad zero keys (tcflash.cuh:136-147), normalize, store this lane's 32 dims of
// the row: O^T accumulator db holds d = 16*db + 4*g + i
template <typename OutT>
__device__ __forceinline__ void epilogue(const AttnParams& p, const AttnJob& J, int row, bool qin, int h, int g,
                                         float m, float l, const floatx4 (&o)[8]) {
    float lt = quad_sum(l);
    float sc = 1.f;
    if (J.npad) {
        const float mn = fmaxf(m, 0.f);
        sc = __builtin_amdgcn_exp2f(m - mn);
        lt = lt * sc + (float)J.npad * __builtin_amdgcn_exp2f(-mn);
    }
    const float inv = sc / lt;
    if (!qin) return;
    OutT* orow = reinterpret_cast<OutT*>(J.o) + (size_t)row * p.ldo + h * HD + 4 * g;
    const bool pairs = p.store_pairs != 0;
#pragma unroll
    for (int db = 0; db < 8; db++)
        store4<OutT>(orow + 16 * db, o[db][0] * inv, o[db][1] * inv, o[db][2] * inv, o[db][3] * inv, pairs);
}

// The same through LDS, for aligned outputs: the wave's 16 normalized rows of one query block go row-major into
// its LDS region (rows padded by 16 bytes: the 16 rows of a write land in different banks), then leave as whole
// rows, 16 bytes per lane (a 256-byte fp16 row from 16 lanes, a 512-byte fp32 row from 32), instead of 8-byte
// pieces of 16 rows per store instruction.
template <typename OutT>
constexpr int ORS = HD + 16 / (int)sizeof(OutT);  // LDS row stride of the staged output, elements
template <typename OutT>
__device__ __forceinline__ void epilogue_rows(const AttnParams& p, const AttnJob& J, int row0, int h, int g, int lane,
                                              float m, float l, const floatx4 (&o)[8], OutT* stg) {
    float lt = quad_sum(l);
    float sc = 1.f;
    if (J.npad) {
        const float mn = fmaxf(m, 0.f);
        sc = __builtin_amdgcn_exp2f(m - mn);
        lt = lt * sc + (float)J.npad * __builtin_amdgcn_exp2f(-mn);
    }
    const float inv = sc / lt;
    OutT* srow = stg + (lane & 15) * ORS<OutT> + 4 * g;
#pragma unroll
    for (int db = 0; db < 8; db++) {
        if constexpr (std::is_same<OutT, _Float16>::value)
            *reinterpret_cast<half4*>(srow + 16 * db) = half4{(_Float16)(o[db][0] * inv), (_Float16)(o[db][1] * inv),
                                                              (_Float16)(o[db][2] * inv), (_Float16)(o[db][3] * inv)};
        else
            *reinterpret_cast<floatx4*>(srow + 16 * db) = o[db] * inv;
    }
    __builtin_amdgcn_wave_barrier();  // the wave's LDS writes precede its reads (one wave, in-order LDS queue)
    constexpr int RPI = 64 * 16 / (HD * (int)sizeof(OutT));  // rows per 16-byte-per-lane instruction: 4 or 2
    constexpr int LPR = 64 / RPI;                              // lanes per row
#pragma unroll
    for (int i = 0; i < 16 / RPI; i++) {
        const int r = RPI * i + lane / LPR, col = (lane % LPR) * (16 / (int)sizeof(OutT));
        const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * ORS<OutT> + col);
        if (row0 + r < p.Tq)
            *reinterpret_cast<u32x4*>(reinterpret_cast<OutT*>(J.o) + (size_t)(row0 + r) * p.ldo + h * HD + col) = v;
    }
    __builtin_amdgcn_wave_barrier();  // reads done before the next block's writes reuse the region
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt[3:0] | expcnt 7 << 4 | lgkmcnt 15 << 8 | vmcnt[5:4] << 14)
#define KILN_WAIT_VMCNT(N) __builtin_amdgcn_s_waitcnt(((N) & 0xF) | (0x7 << 4) | (0xF << 8) | (((N) >> 4) << 14))

// ------------------------------------------------------------------------------------------------
// The kernel. A wave owns two query blocks of 16 rows (32 rows), a workgroup NW = 4 waves (BM = 128 rows), two
// workgroups per CU (two waves per SIMD), NS = 4 ring stages (64 KB of LDS per workgroup; five measured the same
// on long units and slower on short ones, whose prologue fills the ring); or 8 waves (256 rows), one workgroup per
// CU, NS8 = 8 stages (128 KB). All products on v_mfma_f32_16x16x32_f16.
//
// Keys stream in 32-key half tiles (16 KB: K 8 KB + V 8 KB) through an NS-stage LDS ring filled by
// direct global->LDS DMA (buffer_load_dwordx4 ... lds: no staging registers, no ds_write), NS-2 half
// tiles ahead of use. Per half tile a wave issues 16 QK MFMAs (2 key blocks x 2 query blocks x 4 d chunks) and
// 16 PV MFMAs (8 d blocks x 2 query blocks); each 1 KB K or V operand read from LDS feeds both query blocks.
//
// Software pipeline, per half tile j (S_j - m and max(S_j) - m in registers, K_{j+1} d chunks 0-1 in
// registers, half tiles j .. j+NS-3 resident or in flight):
//   [rare: rescale O, l, m]                                         (the only branch)
//   K_{j+1} chunks 2-3, V_j[db 0-3] reads | QK_{j+1} MFMAs interleaved with exp/cvt of S_j |
//   wait tile j+2, barrier | DMA tile j+NS-1 into the stage of tile j-1 | K_{j+2} chunks 0-1, V_j[db 4-7] reads |
//   PV_j and row-sum MFMAs interleaved with max(S_{j+1})
// (one-job 4-wave workgroups issue the DMA between the two halves of the PV MFMAs instead)
// Every read of a stage completes before the barrier that precedes its refill.
// ------------------------------------------------------------------------------------------------
// a scheduling fence: keeps the phases of a step in the order written and bounds the live registers
#define KILN_FENCE() __builtin_amdgcn_sched_barrier(0)
typedef __attribute__((address_space(3))) half8 lds_half8;
constexpr int NW = 4, BM = NW * 32, NS = 4, NS8 = 8;  // the 4-wave form's geometry (key-split partials use BM)
constexpr int PART_FLOATS = BM * HD + 2 * BM;      // one key range's partial result of a query tile
static_assert(NS == 4, "ring: tiles j-1 (refilled), j, j+1 and j+2 (read this iteration); half tile j in stage j % 4");

// NWT waves per workgroup: 4 (two workgroups per CU, a 4-stage ring each) or 8 (one workgroup per CU, 256 query
// rows sharing one 8-stage ring: half the K/V DMA, L2 reads and LDS writes per flop, which the power-limited
// chip turns into clock).
// CHAIN: a context chain (one unit per query tile and head, every job in turn); a separate instantiation, so
// the one-job kernels compile exactly as without the job loop (the loop costs them ~1.5%).
template <typename InT, typename OutT, bool QNORM, bool ROPE, int NWT, bool CHAIN>
__global__ __launch_bounds__(NWT * 64, 8 / NWT) void k_attn_fwd(const AttnParams p) {  // 2nd: workgroups per CU
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];  // NS x 16 KB
    constexpr int KBM = NWT * 32;                          // query rows of the workgroup
    constexpr int KDMA = HT_H * 2 / 16 / (NWT * 64);      // 16-byte DMA pieces per thread per half tile
    static_assert(NWT == 4 || NWT == 8, "4 or 8 waves");
    constexpr int KNS = NWT == 8 ? NS8 : NS;               // ring stages (half tile j in stage j % KNS)
    static_assert(KNS == 4 || KNS == 8, "a power of two: stage = j & (KNS - 1)");
    const int tid = threadIdx.x, lane_in = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g_in = lane_in >> 4;  // 16-lane row of the wave: keys 4g..4g+3 of a key block, dims 8g.. of a d chunk
    Work W;
    if (!decode_work(p, W)) return;
    half8 qreg[2][4];  // the Q tile (B operands); a context chain keeps it for consecutive jobs of one Q
    // one job of the unit: the keys of p.job[jb] for this query tile and head, with its epilogue; qload: load the
    // Q tile (a chain skips it when the job shares the previous job's queries)
    auto run_job = [&](int jb, int lane, int g, bool qload) {
    const AttnJob J = p.job[jb];

    const int Tk = J.Tk;
    const int nhall = (Tk + 31) / 32;  // half tiles holding real keys
    // this unit's key range: half tiles [h0, h0 + nh) (all of them unless the launch splits the keys)
    const int h0 = W.ks * nhall / p.ksplit;
    const int nh = (W.ks + 1) * nhall / p.ksplit - h0;
    const _Float16* kvh = reinterpret_cast<const _Float16*>(J.kv) + (size_t)W.h * kv_head_stride(Tk);
    const uint32_t lds_base = (uint32_t)(size_t)(__attribute__((address_space(3))) _Float16*)lds;

    // half tile jh -> stage: each wave copies KDMA 16-byte pieces per lane; the wave's 64 lanes write 1 KB
    // of contiguous LDS at the wave-uniform base the DMA takes from M0.
    // Buffer-form DMA: the lane offset tid*16 is a constant VGPR; the half tile and piece offsets go in the
    // SGPR soffset, so a refill costs no vector instructions. The descriptor's range is the head's K/V block.
    const __amdgpu_buffer_rsrc_t kv_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(kvh), (short)0, (int)(kv_head_stride(Tk) * 2), 0x00020000 /* raw, CDNA */);
    // Wave w copies the contiguous KDMA KB [KDMA w, KDMA (w + 1)) KB of the half tile (4 KB with 4 waves, 2 KB with
    // 8) in 1 KB pieces: one M0 (LDS base) and one soffset serve all of them, the piece offset is the instruction's
    // immediate (it applies to the global and the LDS address alike).
    const uint32_t dma_off = (uint32_t)wv * (KDMA * 1024) + lane * 16;
    auto dma = [&](int jh, int stage) {
        auto* dst = (__attribute__((address_space(3))) void*)(lds + stage * HT_H + wv * (KDMA * 512));
        const int so = (h0 + jh) * (HT_H * 2);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kv_rsrc, dst, 16, dma_off, so, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kv_rsrc, dst, 16, dma_off, so, 1024, 0);
        if constexpr (KDMA == 4) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(kv_rsrc, dst, 16, dma_off, so, 2048, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(kv_rsrc, dst, 16, dma_off, so, 3072, 0);
        }
    };
    // operand reads through 32-bit LDS byte addresses: base + immediate offsets fold into ds_read_b128
    auto kptr = [&](int stage) {
        return reinterpret_cast<const lds_half8*>((size_t)(lds_base + stage * HT_H * 2 + lane * 16));
    };
    // max over this lane's 8 keys of one query column (its two key-block accumulators)
    auto max8 = [](const floatx4& a, const floatx4& b) {
        const float x0 = fmaxf(fmaxf(a[0], a[1]), a[2]), x1 = fmaxf(fmaxf(a[3], b[0]), b[1]);
        return fmaxf(fmaxf(x0, x1), fmaxf(b[2], b[3]));
    };

    // prologue: half tiles 0 .. 2 in flight, then the Q tile loads (their latencies overlap), then the rest of a
    // deeper ring (after the Q math, which waits for every vector memory operation issued before its loads);
    // wait for tiles 0 and 1
#pragma unroll
    for (int i = 0; i < 3; i++) dma(min(i, nh - 1), i);
    __builtin_amdgcn_sched_barrier(0);
    int row[2];
    bool qin[2];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        row[qb] = W.qt * KBM + wv * 32 + 16 * qb + (lane & 15);
        qin[qb] = row[qb] < p.Tq;
    }
    if (qload) load_q<InT, QNORM, ROPE>(p, J.q, row, qin, W.h, g, qreg);
#pragma unroll
    for (int i = 3; i < KNS - 1; i++) dma(min(i, nh - 1), i);
    KILN_WAIT_VMCNT((KNS - 3) * KDMA);
    __builtin_amdgcn_s_barrier();

    floatx4 o[2][8];  // O^T per query block: d block db holds d = 16*db + 4g + i
    float m[2], l[2], mx[2];
    floatx4 sc[2][2], sc2[2][2];  // [key block][query block]: S_j - m and S_{j+1} - m; the unrolled loop
                                  // alternates their roles
    floatx4 mneg[2];              // -m in every item: the first QK MFMA of a chain starts from it
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
#pragma unroll
        for (int db = 0; db < 8; db++) o[qb][db] = floatx4{0.f, 0.f, 0.f, 0.f};
        l[qb] = 0.f;
    }
    // Row sums on the matrix core: P^T times a 9th V^T block of ones (constant registers, no LDS read), whose
    // accumulator holds the row's sum of the fp16-rounded P values the PV MFMAs consume in every one of its rows:
    // two MFMAs per half tile instead of eight v_dot2c_f32_f16 on the VALU, which bounds the loop.
    const half8 ones8 = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f,
                         (_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};
    floatx4 lsum[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};

    half8 ka[8];  // K operands s = 2c + kb: d chunks 0-1 (s < 4) of the next QK chains are read a phase ahead
#pragma unroll
    for (int s = 0; s < 8; s++) ka[s] = kptr(0)[s * 64];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int qb = 0; qb < 2; qb++) sc[kb][qb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; s++)
#pragma unroll
        for (int qb = 0; qb < 2; qb++) sc[s & 1][qb] = mfma16(ka[s], qreg[qb][s >> 1], sc[s & 1][qb]);
    if (Tk < 32) mask_half(0, Tk, g, sc);
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        m[qb] = quad_max(max8(sc[0][qb], sc[1][qb]));  // the first half tile sets the running max of the row
        mx[qb] = 0.f;  // max(S_j) - m over this lane's 8 keys of the row (three other lanes hold the rest)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            sc[0][qb][i] -= m[qb];
            sc[1][qb][i] -= m[qb];
            mneg[qb][i] = -m[qb];
        }
    }
#pragma unroll
    for (int s = 0; s < 4; s++) ka[s] = kptr(1)[s * 64];
    // Enter the loop with no LDS read in flight: the loop body's first MFMA then waits only for the reads
    // of the previous iteration, and the waitcnt pass keeps the step's own new reads in flight.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)

    // the running max moves up by d: O and l scale by 2^-d, and S_j - m (cur) shifts by -d
    auto rescale = [&](floatx4(&cur)[2][2]) {
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            // the rescale decision is wave-uniform (a ballot over every lane's own maximum), so the row's
            // common maximum over its four lanes is formed only here, on the rare path
            const float d = fmaxf(quad_max(mx[qb]), 0.f);
            const float corr = __builtin_amdgcn_exp2f(-d);
#pragma unroll
            for (int db = 0; db < 8; db++) o[qb][db] *= corr;
            lsum[qb] *= corr;
            m[qb] += d;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                cur[0][qb][i] -= d;
                cur[1][qb][i] -= d;
                mneg[qb][i] -= d;
            }
        }
    };
    auto need_rescale = [&]() {
        const bool need = fmaxf(mx[0], mx[1]) > RESCALE_TH;
        return __builtin_amdgcn_ballot_w64(need) != 0;
    };

    auto stage = [](int jh) { return jh & (KNS - 1); };  // LDS stage of half tile jh
    // Tile j+2 landed in every wave; every wave is done with tile j-1, whose stage is refilled. Only tiles
    // j+3 .. j+KNS-2 may be in flight; the peeled masking step (whose register spills, if any, are vector memory
    // operations too) waits for everything.
    // One-job 4-wave workgroups issue the plain steps' refill between the two halves of the PV MFMAs instead of
    // right after the barrier, where it delays the K_{j+2} / V_j operand reads that the PV MFMAs wait for (the two
    // workgroups of a CU run in step with each other, and their issue stalls add up there): config 2 kernel
    // -1.5%, config 3 -1%; at the end of the step: config 2 -1.2%. Context chains keep it after the barrier
    // (their short jobs measured +5% with it at the end of the step), and so do 8-wave workgroups (no change).
    constexpr bool REFILL_LATE = NWT == 4 && !CHAIN;
    auto sync_refill = [&](auto maskn_tag, int j) {
        if constexpr (decltype(maskn_tag)::value) KILN_WAIT_VMCNT(0);
        else KILN_WAIT_VMCNT((KNS - 4) * KDMA);
        __builtin_amdgcn_s_barrier();
        if constexpr (!REFILL_LATE || decltype(maskn_tag)::value)
            dma(min(j + KNS - 1, nh - 1), stage(j + KNS - 1));  // into the stage of tile j-1
    };
    // One half tile j with a successor. MASKN: the successor is the last half tile and ragged.
    auto step = [&](auto maskn_tag, int j, floatx4 (&cur)[2][2], floatx4 (&sn)[2][2]) {
        constexpr bool MASKN = decltype(maskn_tag)::value;
        if (need_rescale()) rescale(cur);  // lazy rescale (rare)
        const int st = stage(j), st1 = stage(j + 1);
        half8 va[4];
        {
            const lds_half8* kp = kptr(st1);
#pragma unroll
            for (int s = 4; s < 8; s++) ka[s] = kp[s * 64];
            const lds_half8* vp = kptr(st) + 32 * HD / 8;
#pragma unroll
            for (int db = 0; db < 4; db++) va[db] = vp[db * 64];
        }
        KILN_FENCE();

        // the softmax phase issues at a raised wave priority: when both waves of a SIMD are ready, the one with
        // exp/convert work to interleave goes first
        __builtin_amdgcn_s_setprio(1);
        // S_{j+1} on the matrix cores while the VALU turns S_j into P_j: MFMA pair s (d chunk s/2, key block
        // s%2, both query blocks) with P values 2s, 2s+1 (query block s/4, B-operand elements (2s)%8, +1)
        half8 pb[2];
#pragma unroll
        for (int s = 0; s < 8; s++) {
#pragma unroll
            for (int qb = 0; qb < 2; qb++)
                sn[s & 1][qb] = mfma16(ka[s], qreg[qb][s >> 1], s < 2 ? mneg[qb] : sn[s & 1][qb]);
            const int qb = s >> 2, e = (2 * s) % 8, kb = e / 4, i = e % 4;
            pb[qb][e] = (_Float16)__builtin_amdgcn_exp2f(cur[kb][qb][i]);
            pb[qb][e + 1] = (_Float16)__builtin_amdgcn_exp2f(cur[kb][qb][i + 1]);
        }
        KILN_FENCE();

        sync_refill(maskn_tag, j);
        half8 vb[4];
        {
            const lds_half8* kp = kptr(stage(j + 2));  // K_{j+2}; past the end: stale, unused
#pragma unroll
            for (int s = 0; s < 4; s++) ka[s] = kp[s * 64];
            const lds_half8* vp = kptr(st) + 32 * HD / 8 + 4 * 64;
#pragma unroll
            for (int db = 0; db < 4; db++) vb[db] = vp[db * 64];
        }
        KILN_FENCE();

        if constexpr (MASKN) mask_half(h0 + j + 1, Tk, g, sn);
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int db = 0; db < 4; db++)
#pragma unroll
            for (int qb = 0; qb < 2; qb++) o[qb][db] = mfma16(va[db], pb[qb], o[qb][db]);
        if constexpr (REFILL_LATE && !MASKN) {
            KILN_FENCE();
            dma(min(j + KNS - 1, nh - 1), stage(j + KNS - 1));
            KILN_FENCE();
        }
#pragma unroll
        for (int db = 0; db < 4; db++)
#pragma unroll
            for (int qb = 0; qb < 2; qb++) o[qb][db + 4] = mfma16(vb[db], pb[qb], o[qb][db + 4]);
#pragma unroll
        for (int qb = 0; qb < 2; qb++) lsum[qb] = mfma16(ones8, pb[qb], lsum[qb]);
#pragma unroll
        for (int qb = 0; qb < 2; qb++) mx[qb] = max8(sn[0][qb], sn[1][qb]);
        KILN_FENCE();
    };

    using True = std::true_type;
    using False = std::false_type;
    // Steps j = 0 .. nh-2 (each with a successor), then the last half tile. Only a ragged last half tile of the
    // keys needs the masking step; every other step runs one of the two copies below (the unrolled pair or the
    // single step), so no third copy of the step body, with its own register allocation, is inlined.
    const bool ragged = (Tk & 31) != 0 && h0 + nh == nhall;
    const int nplain = nh - 1 - (ragged && nh >= 2 ? 1 : 0);  // steps without masking: j = 0 .. nplain-1
    auto copy_s = [&]() {
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int qb = 0; qb < 2; qb++) sc[kb][qb] = sc2[kb][qb];
    };
    int j = 0;
    for (; j + 1 < nplain; j += 2) {
        step(False{}, j, sc, sc2);
        step(False{}, j + 1, sc2, sc);
    }
    if (j < nplain) {
        step(False{}, j, sc, sc2);
        j++;
        copy_s();
    }
    if (ragged && nh >= 2) {
        step(True{}, j, sc, sc2);
        j++;
        copy_s();
    }
    // last half tile: no successor
    if (need_rescale()) rescale(sc);
    {
        half8 va[8];
        const lds_half8* vp = kptr(stage(j)) + 32 * HD / 8;
#pragma unroll
        for (int db = 0; db < 8; db++) va[db] = vp[db * 64];
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            half8 pb;
#pragma unroll
            for (int e = 0; e < 8; e++) pb[e] = (_Float16)__builtin_amdgcn_exp2f(sc[e / 4][qb][e % 4]);
            lsum[qb] = mfma16(ones8, pb, lsum[qb]);
#pragma unroll
            for (int db = 0; db < 8; db++) o[qb][db] = mfma16(va[db], pb, o[qb][db]);
        }
    }
    // every row of the ones block holds the full sum: a quarter in each of the four lanes the epilogue adds (exact)
#pragma unroll
    for (int qb = 0; qb < 2; qb++) l[qb] = lsum[qb][0] * 0.25f;
    KILN_WAIT_VMCNT(0);  // drain the re-fetch DMAs before the workgroup's LDS is reused or released
    if (p.ksplit <= 1 && p.store_rows) {
        __builtin_amdgcn_s_barrier();  // every wave is done with the ring: its LDS now stages the output rows
        OutT* stg = reinterpret_cast<OutT*>(lds) + wv * 16 * ORS<OutT>;
#pragma unroll
        for (int qb = 0; qb < 2; qb++)
            epilogue_rows<OutT>(p, J, W.qt * KBM + wv * 32 + 16 * qb, W.h, g, lane, m[qb], l[qb], o[qb], stg);
        return;
    }
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        if (NWT == 4 && p.ksplit > 1) {  // partial result of this key range: unnormalized O, running max m, row sum l
            const int unit = (W.jb * p.H + W.h) * p.qtiles + W.qt;
            float* po = p.part + (size_t)(unit * p.ksplit + W.ks) * PART_FLOATS;
            const int r = wv * 32 + 16 * qb + (lane & 15);
            float* prow = po + r * HD + 4 * g;
#pragma unroll
            for (int db = 0; db < 8; db++) *reinterpret_cast<floatx4*>(prow + 16 * db) = o[qb][db];
            const float lt = quad_sum(l[qb]);
            if (g == 0) *reinterpret_cast<float2*>(po + BM * HD + 2 * r) = make_float2(m[qb], lt);
        } else {
            epilogue<OutT>(p, J, row[qb], qin[qb], W.h, g, m[qb], l[qb], o[qb]);
        }
    }
    };  // run_job

    if constexpr (!CHAIN) {
        run_job(W.jb, lane_in, g_in, true);
    } else {
        const void* qcur = nullptr;
        for (int jb = 0; jb < p.njobs; jb++) {
            if (jb) __syncthreads();  // the previous job's output staging reads of the ring are done
            // per-lane indices enter each job through an empty asm: otherwise the compiler hoists the job's
            // lane-dependent addresses out of the job loop and keeps them live across the key loop
            int lane = lane_in, g = g_in;
            asm volatile("" : "+v"(lane), "+v"(g));
            run_job(jb, lane, g, p.job[jb].q != qcur);
            qcur = p.job[jb].q;
        }
    }
}

// ------------------------------------------------------------------------------------------------
// K/V prepare: fp16 conversion (+ K RMSNorm, + K RoPE) into the tiled MFMA operand order.
// One block per (64-key tile, head). Bandwidth-bound; runs once per K/V, not once per query tile.
// ------------------------------------------------------------------------------------------------
struct PrepParams {
    KVPrepJob job[MAX_JOBS];  // blockIdx.z selects the job
    int Tk, tpb;              // keys; 32-key half tiles per block
    const uint16_t* kw;
    float eps;
    const float* rcos;
    const float* rsin;
};

// All global loads of one 32-key half tile for one thread (8 threads per key): K chunks q8 and q8+8 of key
// kk (RoPE partners: d and d+64), V chunks 2q8 and 2q8+1, and the key's RoPE cos/sin for K chunk q8.
// Loaded a half tile ahead of use, so a block's reads of the next half tile overlap its stores.
template <typename InT, bool ROPE>
struct PrepHalf {
    Chunk8<InT> k[2], v[2];
    floatx4 rc[2], rs[2];
};

template <typename InT, bool KNORM, bool ROPE>
__global__ __launch_bounds__(256) void k_kv_prep(const PrepParams p) {
    // V half tile in fp16, rows padded to 288 bytes: the transposing reads of one 16-lane group touch 4 rows
    // 8 banks apart, conflict-free
    __shared__ __attribute__((aligned(16))) _Float16 vt[32][HD + 16];
    const int tid = threadIdx.x, h = blockIdx.y;
    const KVPrepJob& jb = p.job[blockIdx.z];
    const int Tk = p.Tk, nhalf = 2 * kv_tiles(Tk);
    const int t0 = blockIdx.x * p.tpb, t1 = min(t0 + p.tpb, nhalf);
    if (t0 >= t1) return;
    const InT* __restrict__ k = reinterpret_cast<const InT*>(jb.k);
    const InT* __restrict__ v = reinterpret_cast<const InT*>(jb.v);
    _Float16* dst_h = reinterpret_cast<_Float16*>(jb.kvp) + (size_t)h * kv_head_stride(Tk);
    const int kk = tid >> 3, q8 = tid & 7;  // key within the half tile, eighth of the row
    float kwf[2][8];
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
        for (int e = 0; e < 8; e++) kwf[c][e] = KNORM ? bf16_to_f32(p.kw[8 * (q8 + 8 * c) + e]) : 1.f;

    auto load_half = [&](int jh, PrepHalf<InT, ROPE>& t) {
        const int key = jh * 32 + kk;
        if (key < Tk) {
            const InT* kr = k + (size_t)key * jb.ldk + h * HD + 8 * q8;
            const InT* vr = v + (size_t)key * jb.ldv + h * HD + 16 * q8;
            t.k[0].load(kr);
            t.k[1].load(kr + 64);
            t.v[0].load(vr);
            t.v[1].load(vr + 8);
            if constexpr (ROPE) {
                const float* cp = p.rcos + (size_t)key * 64 + 8 * q8;
                const float* sp = p.rsin + (size_t)key * 64 + 8 * q8;
                t.rc[0] = *reinterpret_cast<const floatx4*>(cp);
                t.rc[1] = *reinterpret_cast<const floatx4*>(cp + 4);
                t.rs[0] = *reinterpret_cast<const floatx4*>(sp);
                t.rs[1] = *reinterpret_cast<const floatx4*>(sp + 4);
            }
        } else {  // keys past Tk: zeros (the attention kernel relies on a zero-padded last tile)
#pragma unroll
            for (int c = 0; c < 2; c++) {
                t.k[c].zero();
                t.v[c].zero();
            }
            if constexpr (ROPE) t.rc[0] = t.rc[1] = t.rs[0] = t.rs[1] = floatx4{};
        }
    };

    PrepHalf<InT, ROPE> cur, nxt;
    load_half(t0, cur);
    for (int jh = t0; jh < t1; jh++) {
        if (jh + 1 < t1) load_half(jh + 1, nxt);
        // half tile jh of the prepared buffer: [K_c 8 KB | V_c 8 KB] (K_c and V_c orders in common.hpp)
        _Float16* dst = dst_h + (size_t)(jh >> 1) * KV_TILE_H;
        const int c = jh & 1;
        // V: half tile -> LDS (fp16)
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
            half8 hv;
#pragma unroll
            for (int e = 0; e < 8; e++) hv[e] = (_Float16)cur.v[cc][e];
            *reinterpret_cast<half8*>(&vt[kk][16 * q8 + 8 * cc]) = hv;
        }
        // K: RMSNorm (8 threads per key), RoPE, fp16, into the K_c operand order
        {
            float x[2][8];
#pragma unroll
            for (int cc = 0; cc < 2; cc++)
#pragma unroll
                for (int e = 0; e < 8; e++) x[cc][e] = cur.k[cc][e];
            if constexpr (KNORM) {
                float ss = 0.f;
#pragma unroll
                for (int cc = 0; cc < 2; cc++)
#pragma unroll
                    for (int e = 0; e < 8; e++) ss += x[cc][e] * x[cc][e];
                // sum over the key's 8 consecutive lanes: DPP quad swaps, then the half-row mirror
                ss += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0xB1, 0xF, 0xF, false));
                ss += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x4E, 0xF, 0xF, false));
                ss += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x141, 0xF, 0xF, false));
                const float r = rsqrtf(ss * (1.0f / HD) + p.eps);
#pragma unroll
                for (int cc = 0; cc < 2; cc++)
#pragma unroll
                    for (int e = 0; e < 8; e++) x[cc][e] = x[cc][e] * r * kwf[cc][e];
            }
            if constexpr (ROPE) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const float cs = cur.rc[e / 4][e % 4], sn = cur.rs[e / 4][e % 4];
                    const float a = x[0][e], b = x[1][e];
                    x[0][e] = a * cs - b * sn;
                    x[1][e] = b * cs + a * sn;
                }
            }
#pragma unroll
            for (int cc = 0; cc < 2; cc++) {
                const int ch = q8 + 8 * cc;  // 8-element chunk of the row: d = 8 ch
                *reinterpret_cast<half8*>(dst + kv_k_el(c, kk, 8 * ch)) = to_half8(x[cc]);
            }
        }
        __syncthreads();
        // V^T operand units (db, lane): 8 keys of one d. ds_read_b64_tr_b16 (gfx950) transposes within each
        // group of 16 lanes: source lane r supplies 4 halves of row r/4, and lane i receives element e of row
        // 4e + i/4, column i%4. Lane r pointing at vt[key0 + r/4][d0 + 4(r%4)] therefore leaves lane i holding
        // vt[key0 + e][d0 + i], e = 0..3: four consecutive keys of its own d. Lane group g takes keys 4g.. of
        // both key blocks (key0 = 4g and 16 + 4g); wave w the d blocks 2w and 2w + 1.
        {
            const int w = tid >> 6, ln = tid & 63;
            const int g = ln >> 4, i = ln & 15;
            typedef short s4 __attribute__((ext_vector_type(4)));
            typedef short s8 __attribute__((ext_vector_type(8)));
            typedef __attribute__((address_space(3))) s4 lds_s4;
#pragma unroll
            for (int dd = 0; dd < 2; dd++) {
                const int db = 2 * w + dd;
                const int d0 = 16 * db + 4 * (i & 3);
                const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)&vt[4 * g + (i >> 2)][d0]);
                const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)&vt[16 + 4 * g + (i >> 2)][d0]);
                const s8 o = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                *reinterpret_cast<s8*>(dst + kv_v_off(c, db, ln)) = o;
            }
        }
        if (jh + 1 < t1) {
            __syncthreads();  // vt is rewritten by the next half tile
            cur = nxt;
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Merge of key-split partials (launches whose grid would fill under a quarter of the resident workgroup
// slots split each unit's keys into ksplit ranges): per query row, O = sum_i O_i 2^(m_i - m) / sum_i l_i
// 2^(m_i - m) with m = max_i m_i, then the npad zero keys and the output rounding of the epilogue.
// ------------------------------------------------------------------------------------------------
template <typename OutT>
__global__ __launch_bounds__(256) void k_attn_merge(const AttnParams p) {
    // block = 32 rows of one unit (four blocks per unit); thread = 16 columns of one row
    const int unit = blockIdx.x >> 2, qt = unit % p.qtiles, rest = unit / p.qtiles, h = rest % p.H, jb = rest / p.H;
    const AttnJob& J = p.job[jb];
    const int r = (blockIdx.x & 3) * 32 + (threadIdx.x >> 3), c0 = 16 * (threadIdx.x & 7);
    const int row = qt * BM + r;
    if (row >= p.Tq) return;
    const float* base = p.part + (size_t)unit * p.ksplit * PART_FLOATS;
    float mx = -INFINITY;
    for (int ks = 0; ks < p.ksplit; ks++) mx = fmaxf(mx, base[ks * PART_FLOATS + BM * HD + 2 * r]);
    float lt = 0.f;
    floatx4 acc[4] = {};
    for (int ks = 0; ks < p.ksplit; ks++) {
        const float* pk = base + ks * PART_FLOATS;
        const float w = __builtin_amdgcn_exp2f(pk[BM * HD + 2 * r] - mx);
        lt += pk[BM * HD + 2 * r + 1] * w;
        const floatx4* src = reinterpret_cast<const floatx4*>(pk + r * HD + c0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] += src[i] * w;
    }
    float sc = 1.f;
    if (J.npad) {
        const float mn = fmaxf(mx, 0.f);
        sc = __builtin_amdgcn_exp2f(mx - mn);
        lt = lt * sc + (float)J.npad * __builtin_amdgcn_exp2f(-mn);
    }
    const float inv = sc / lt;
    OutT* orow = reinterpret_cast<OutT*>(J.o) + (size_t)row * p.ldo + h * HD + c0;
    const bool pairs = p.store_pairs != 0;
#pragma unroll
    for (int i = 0; i < 4; i++)
        store4<OutT>(orow + 4 * i, acc[i][0] * inv, acc[i][1] * inv, acc[i][2] * inv, acc[i][3] * inv, pairs);
}

// ------------------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------------------
// resident workgroup slots of the current device (two per CU); 0 if there is no device
static int resident_slots() {
    static int slots[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (!slots[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        slots[dev] = 2 * cus;
    }
    return slots[dev];
}

int attn_key_split(int njobs, int Tq, int Tk, int H) {
    const long units = (long)((Tq + BM - 1) / BM) * H * njobs;
    const int slots = resident_slots();
    if (units <= 0 || slots <= 0) return 1;
    long ks = slots / units;
    ks = std::min<long>(ks, 8);
    ks = std::min<long>(ks, ((Tk + 31) / 32) / 16);  // every range keeps at least 16 half tiles
    return ks >= 3 ? (int)ks : 1;  // below 3 ranges the extra prologues and the merge cost more than they save
}

size_t attn_split_bytes(int ksplit, int njobs, int Tq, int H) {
    if (ksplit <= 1) return 0;
    return (size_t)((Tq + BM - 1) / BM) * H * njobs * ksplit * PART_FLOATS * sizeof(float);
}
template <typename InT, typename OutT, bool QN, bool RP, int NWT, bool CHAIN = false>
static hipError_t launch_nw(AttnParams& p, int Tq, int units, hipStream_t s) {
    constexpr int KBM = NWT * 32;
    p.qtiles = (Tq + KBM - 1) / KBM;
    p.total = p.qtiles * units * p.ksplit;
    const int nb = (p.total + 7) / 8 * 8;
    p.per = nb / 8;
    auto kern = k_attn_fwd<InT, OutT, QN, RP, NWT, CHAIN>;
    // the ring, or the output staging of 16 rows per wave if that is larger (8 waves, fp32 output)
    const size_t lds = std::max((size_t)(NWT == 8 ? NS8 : NS) * HT_H * sizeof(_Float16), (size_t)NWT * 16 * ORS<OutT> * sizeof(OutT));
    hipLaunchKernelGGL(kern, dim3(nb), dim3(NWT * 64), lds, s, p);
    return hipGetLastError();
}
template <typename InT, typename OutT, bool QN, bool RP>
static hipError_t launch_sel(AttnParams p, int Tq, int units, hipStream_t s) {
    // 8-wave workgroups where 256-row query tiles give every CU whole rounds of work (config 4: 512 tiles on 256
    // CUs), or at least one round of long units (keys >= 2048: config 5's self-attention, 448 tiles, whose 4-wave
    // form also needs two full rounds); elsewhere the 128-row tiles fill the chip more evenly and short units pay
    // less prologue per flop (and key-split launches need them)
    const long t8 = (long)((Tq + 255) / 256) * units;
    const int cus = resident_slots() / 2;
    bool longk = true;
    for (int i = 0; i < p.njobs; i++) longk &= p.job[i].Tk >= 2048;
    // context chains run 4-wave units: at config 5's cross-attention (432 units of three 512-key contexts) 8-wave
    // units (224 on 256 CUs) measured 62.1 against 58.1 us
    if (p.chain) return launch_nw<InT, OutT, QN, RP, 4, true>(p, Tq, units, s);
    if (p.ksplit <= 1 && cus > 0 && (t8 % cus == 0 || (longk && t8 >= cus)))
        return launch_nw<InT, OutT, QN, RP, 8>(p, Tq, units, s);
    hipError_t e = launch_nw<InT, OutT, QN, RP, 4>(p, Tq, units, s);
    if (e != hipSuccess) return e;
    if (p.ksplit > 1) hipLaunchKernelGGL(k_attn_merge<OutT>, dim3(4 * p.qtiles * units), dim3(256), 0, s, p);
    return hipGetLastError();
}

template <typename InT, typename OutT>
static hipError_t dispatch_attn(const AttnParams& p, int units, bool qnorm, bool rope, hipStream_t s) {
    if (qnorm && rope) return launch_sel<InT, OutT, true, true>(p, p.Tq, units, s);
    if (qnorm) return launch_sel<InT, OutT, true, false>(p, p.Tq, units, s);
    if (rope) return launch_sel<InT, OutT, false, true>(p, p.Tq, units, s);
    return launch_sel<InT, OutT, false, false>(p, p.Tq, units, s);
}

hipError_t launch_attn_fwd(const AttnLaunch& a, hipStream_t s) {
    AttnParams p{};
    for (int i = 0; i < a.njobs; i++) p.job[i] = a.job[i];
    p.njobs = a.njobs;
    p.Tq = a.Tq;
    p.H = a.H;
    p.ldq = a.ldq;
    p.ldo = a.ldo;
    const size_t osz = a.out == DT::F16 ? 2 : 4;
    bool pairs = (a.ldo * osz) % (4 * osz) != 0;
    for (int i = 0; i < a.njobs; i++) pairs |= ((uintptr_t)a.job[i].o % (4 * osz)) != 0;
    p.store_pairs = pairs;
    bool rows = (a.ldo * osz) % 16 == 0;
    for (int i = 0; i < a.njobs; i++) rows &= ((uintptr_t)a.job[i].o % 16) == 0;
    p.store_rows = rows;
    p.qw = a.qw;
    p.eps = a.eps;
    p.qscale = a.q_prescaled ? 1.0f : LOG2E / sqrtf((float)HD);
    p.rcos = a.rcos;
    p.rsin = a.rsin;
    p.ksplit = a.part && a.ksplit > 1 && !a.chain ? a.ksplit : 1;
    p.part = a.part;
    // context chains only where the per-context units take more than one round of the resident 4-wave slots
    // (config 5's cross-attention: 1296 units, 2.53 rounds); below that a chain only empties slots (config 3:
    // 384 per-context units, 192 chained: 27.7 -> 31.8 us)
    p.chain = a.chain && a.njobs > 1 && (long)((a.Tq + BM - 1) / BM) * a.H * a.njobs > resident_slots();
    const bool qn = a.qw != nullptr, rp = a.rcos != nullptr;
    const int units = a.H * (p.chain ? 1 : a.njobs);
    if (a.Tq <= 0 || units <= 0) return hipSuccess;
    if (a.in == DT::F16) {
        if (a.out == DT::F16) return dispatch_attn<_Float16, _Float16>(p, units, qn, rp, s);
        return dispatch_attn<_Float16, float>(p, units, qn, rp, s);
    }
    if (a.out == DT::F16) return dispatch_attn<float, _Float16>(p, units, qn, rp, s);
    return dispatch_attn<float, float>(p, units, qn, rp, s);
}

template <typename InT>
static hipError_t dispatch_prep(const PrepParams& p, int njobs, int H, hipStream_t s) {
    dim3 grid((2 * kv_tiles(p.Tk) + p.tpb - 1) / p.tpb, H, njobs), block(256);
    if (p.kw && p.rcos) hipLaunchKernelGGL((k_kv_prep<InT, true, true>), grid, block, 0, s, p);
    else if (p.kw) hipLaunchKernelGGL((k_kv_prep<InT, true, false>), grid, block, 0, s, p);
    else if (p.rcos) hipLaunchKernelGGL((k_kv_prep<InT, false, true>), grid, block, 0, s, p);
    else hipLaunchKernelGGL((k_kv_prep<InT, false, false>), grid, block, 0, s, p);
    return hipGetLastError();
}

hipError_t launch_kv_prep(const KVPrepJob* jobs, int njobs, DT in, int Tk, int H, const uint16_t* kw, float eps,
                          const float* rcos, const float* rsin, hipStream_t s) {
    if (Tk <= 0 || H <= 0 || njobs <= 0) return hipSuccess;
    if (njobs > MAX_JOBS) return hipErrorInvalidValue;
    PrepParams p{};
    for (int i = 0; i < njobs; i++) p.job[i] = jobs[i];
    p.Tk = Tk;
    // each block walks two consecutive 32-key half tiles of one head, the second one's loads in flight while
    // the first is converted and stored (measured best at T = 1536 and 4096; one per block for small inputs)
    const int halves = 2 * kv_tiles(Tk) * H * njobs;
    p.tpb = halves >= 1024 ? 2 : 1;
    p.kw = kw;
    p.eps = eps;
    p.rcos = rcos;
    p.rsin = rsin;
    if (in == DT::F16) return dispatch_prep<_Float16>(p, njobs, H, s);
    return dispatch_prep<float>(p, njobs, H, s);
}

}  // namespace kiln

