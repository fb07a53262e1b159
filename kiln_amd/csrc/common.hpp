// Shared device helpers and the kernel-side layout constants of the gfx950 attention path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kiln {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int HD = 128;            // head dim of the flash path
constexpr int KT = 64;             // keys per K/V tile
constexpr int TILE_H = KT * HD;    // halves in one K (or V) tile = 16 KB
constexpr int KV_TILE_H = 2 * TILE_H;  // K tile followed by V tile, 32 KB
constexpr float LOG2E = 1.4426950408889634f;

// Prepared K/V buffer of one context: [H][ntiles][64-key tile], fp16, zero beyond Tk. A 64-key tile is
// two 32-key half tiles c = 0, 1, each [K_c 8 KB | V_c 8 KB], in the operand order of v_mfma_f32_16x16x32_f16
// (lane l of an operand holds row l%16 and the 8 consecutive contraction elements 8*(l/16) .. +7):
//  K_c order [s 8][lane 64][e 8]:  key = 32c + 16*(s%2) + lane%16,  d = 32*(s/2) + 8*(lane/16) + e
//    (the A operand of S^T = K Q^T for key block s%2 and d chunk s/2)
//  V_c order [db 8][lane 64][j 8]:  d = 16*db + lane%16,  key = 32c + 16*(j/4) + 4*(lane/16) + j%4
//    (the A operand of O^T = V^T P^T whose B operand P^T is taken straight from the two S^T accumulators of
//    the half tile: lane l of the key-block-kb accumulator holds keys 16*kb + 4*(l/16) + i, i = 0..3)
constexpr int HT_H = 32 * HD * 2;  // halves in one half tile (K_c and V_c), 16 KB
// element offsets, within a 64-key tile, of key k32 of half tile c and dimension d
__host__ __device__ inline int kv_k_el(int c, int k32, int d) {
    const int s = 2 * (d >> 5) + (k32 >> 4), lane = (k32 & 15) + 16 * ((d >> 3) & 3);
    return c * HT_H + (s * 64 + lane) * 8 + (d & 7);
}
__host__ __device__ inline int kv_v_el(int c, int k32, int d) {
    const int db = d >> 4, lane = (d & 15) + 16 * ((k32 >> 2) & 3), j = 4 * (k32 >> 4) + (k32 & 3);
    return c * HT_H + 32 * HD + (db * 64 + lane) * 8 + j;
}
// the 16-byte V_c operand unit (db, lane)
__host__ __device__ inline int kv_v_off(int c, int db, int lane) { return c * HT_H + 32 * HD + (db * 64 + lane) * 8; }
__host__ __device__ inline int kv_tiles(int Tk) { return (Tk + KT - 1) / KT; }
__host__ __device__ inline size_t kv_head_stride(int Tk) { return (size_t)kv_tiles(Tk) * KV_TILE_H; }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// 8 consecutive elements of a row as fp32 (fp16 or fp32 storage); p is 16-byte aligned.
__device__ __forceinline__ void load8(const _Float16* p, float (&x)[8]) {
    half8 h = *reinterpret_cast<const half8*>(p);
#pragma unroll
    for (int e = 0; e < 8; e++) x[e] = (float)h[e];
}
__device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
    floatx4 a = *reinterpret_cast<const floatx4*>(p);
    floatx4 b = *reinterpret_cast<const floatx4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) { x[e] = a[e]; x[e + 4] = b[e]; }
}

__device__ __forceinline__ half8 to_half8(const float (&x)[8]) {
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = (_Float16)x[e];  // RN-even
    return h;
}

// lanes l and l^32 exchange: returns (own + partner) for every lane (v_permlane32_swap).
__device__ __forceinline__ float pair_sum(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair_max(float v) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// sum / max over the four lanes n, n+16, n+32, n+48 (rows of 16 lanes swapped pairwise, then halves)
__device__ __forceinline__ float quad_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return pair_sum(__uint_as_float(r[0]) + __uint_as_float(r[1]));
}
__device__ __forceinline__ float quad_max(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return pair_max(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}

}  // namespace kiln
