// Shared device helpers for the gfx950 tree-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tree_attn.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define TT_LOG2E 1.4426950408889634f
#define TT_LN2 0.6931471805599453f

// Tile geometry shared by the plan builder and the bf16 kernels.
//   forward / dQ pass: a workgroup owns TT_BQ queries of one q head, its four
//   waves own 32 queries each; key tiles hold TT_BK keys.
//   dK/dV pass: a workgroup owns TT_BKB keys of one kv head (32 per wave) and
//   walks its visible query range in blocks of TT_BQB.
#define TT_BQ 128
#define TT_BK 64
#define TT_BKB 128
#define TT_BQB 32

// Plan buffer layout (bytes):
//   [0,8)   uint64 visible pairs per head
//   [8,12)  int32 n_qb, [12,16) int32 n_kt
//   [64, 64 + 4*n_qb)            row_cnt
//   [.., + 4*n_qb*n_kt)          row_list: (kt << 1) | full, ascending kt
#define TT_PLAN_HDR 64

__host__ __device__ inline int tt_cdiv(int a, int b) { return (a + b - 1) / b; }

// v_mfma_f32_32x32x16_bf16: D[32x32] += A[32x16] * B[16x32].
// Lane l supplies row (l & 31) of A and column (l & 31) of B, 8 k-values
// each from lane half (l >> 5). Accumulator element r of lane l holds
// D[row = 8*(r/4) + 4*(l>>5) + (r%4)][col = l & 31].
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int acc_row(int r, int half) { return 8 * (r >> 2) + 4 * half + (r & 3); }

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    return x;
}
__device__ __forceinline__ int wave_min_i(int x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = min(x, __shfl_xor(x, o));
    return x;
}
__device__ __forceinline__ int wave_max_i(int x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = max(x, __shfl_xor(x, o));
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Pack 8 floats (round-to-nearest-even) into a bf16x8 MFMA operand.
__device__ __forceinline__ bf16x8 pack8(float a0, float a1, float a2, float a3, float a4, float a5,
                                        float a6, float a7) {
    bf16x8 r;
    r[0] = (__bf16)a0; r[1] = (__bf16)a1; r[2] = (__bf16)a2; r[3] = (__bf16)a3;
    r[4] = (__bf16)a4; r[5] = (__bf16)a5; r[6] = (__bf16)a6; r[7] = (__bf16)a7;
    return r;
}

// Concatenate two 4-element bf16 groups (8 bytes each) into one operand.
__device__ __forceinline__ bf16x8 cat44(const bf16x4& lo, const bf16x4& hi) {
    bf16x8 r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return r;
}
