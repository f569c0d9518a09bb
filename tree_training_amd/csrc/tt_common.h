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
//   walks at most tt_qch(n_q) queries of their visible range (one work item),
//   in blocks of TT_BQB; longer ranges are split into several items.
#define TT_BQ 128
#define TT_BK 64
#define TT_BKB 128
#define TT_BQB 32
#define TT_GDN_CHUNK 32

__host__ __device__ inline int tt_cdiv(int a, int b) { return (a + b - 1) / b; }

// Query window of one dK/dV work item: half the largest power of two <= n_q,
// clamped to [256, 4096] (a multiple of TT_BQB). Long windows mean fewer split
// key tiles (fewer V reloads and fp32 partial sums); short ones mean more,
// shorter items to balance over the chip, which small problems need: a
// partition of a few hundred queries under a gateway of thousands of keys has
// few key tiles, each a long serial walk if it is not split.
__host__ __device__ inline int tt_qch(int n_q) {
    const int half = n_q >= 2 ? (1 << (31 - __builtin_clz((unsigned)n_q))) / 2 : 0;   // half the largest power of 2 <= n_q
    return half > 4096 ? 4096 : (half < 256 ? 256 : half);
}
// Key-range split of the bf16 forward and dQ passes. Their grids hold one
// workgroup per (query block, q head) pair; with at most 256 pairs (one per
// CU) half the chip's resident slots idle while each workgroup walks its whole
// key list, as for a partition of a few hundred queries under a gateway of
// thousands of keys. Such problems cut every pair's key tiles into 4
// contiguous ranges, one workgroup each; a combine pass merges the fp32
// partials in range order. (Splitting 257-511 pairs in two or three did not
// pay for the partials' traffic and the combine launch.)
__host__ __device__ inline int tt_key_splits(int n_q, int hq) {
    return tt_cdiv(n_q, TT_BQ) * hq <= 256 ? 4 : 1;
}
// dK/dV work items of a key tile whose visible queries are [qlo, qhi). A range
// of at most qch queries is one item; a longer one is cut at multiples of qch
// in absolute query index, so workgroups busy with different key tiles at the
// same time walk the same query windows (and share them in L2).
__host__ __device__ inline int tt_kb_items(int qlo, int qhi, int qch) {
    if (qhi - qlo <= qch) return 1;
    return (qhi - 1) / qch - qlo / qch + 1;
}
// Upper bound on the dK/dV work items beyond the first of each key tile
// (n_kb tiles): a tile's items never exceed (n_q - 1) / qch + 1, whatever its
// visible range. The deterministic backward keeps one partial-sum slot for each.
__host__ __device__ inline int64_t tt_det_slots(int n_q, int n_keys) {
    return (int64_t)tt_cdiv(n_keys, TT_BKB) * ((n_q - 1) / tt_qch(n_q));
}
// Query range [q_start, q_stop) of item `item`; q_start is a multiple of TT_BQB.
__host__ __device__ inline void tt_kb_item_range(int qlo, int qhi, int qch, int item, int& q_start, int& q_stop) {
    q_start = q_stop = 0;
    if (qhi <= qlo) return;
    const int a = (qlo / TT_BQB) * TT_BQB;
    if (qhi - qlo <= qch) {
        q_start = a;
        q_stop = qhi;
        return;
    }
    const int w = qlo / qch + item;
    q_start = a > w * qch ? a : w * qch;
    q_stop = qhi < (w + 1) * qch ? qhi : (w + 1) * qch;
}

// Plan buffer layout. Header (bytes): [0,8) uint64 visible pairs per head;
// int32 at 8: n_qb, 12: n_kt, 16: n_kb, 20: n_items (dK/dV work items), 24:
// n_split (key tiles of more than one work item), 28: kb_item's order (1:
// longest item first, ties by query window; 2: window-major).
// Then int32 arrays:
//   row_cnt[n_qb]           non-empty key tiles per query block
//   row_order[n_qb]         query blocks by decreasing tile count
//   row_list[n_qb * n_kt]   (kt << 1) | full, ascending kt
//   kb_qlo[n_kb], kb_qhi[n_kb]  visible query range of each 128-key tile
//   kb_order[n_kb]          key tiles by decreasing range
//   kb_base[n_kb + 1]       first work item of each key tile, in kb_order order
//   kb_srank[n_kb]          rank of each key tile among the split ones, in key
//                           order (-1: not split): its rows in the split sums
// then int2 kb_item[n_items] (8-byte aligned; room for n_kb * query windows):
// (tile rank in kb_order, chunk) of each dK/dV work item in the order the
// persistent grid takes them, and a byte array cls[n_qb * n_kt] (tile
// classes, build scratch).
#define TT_PLAN_HDR 64
struct PlanLayout {
    int n_qb, n_kt, n_kb;
    int n_pb;   // 256-key blocks of the pair count
    size_t row_cnt, row_order, row_list, kb_qlo, kb_qhi, kb_order, kb_base, kb_srank, kb_item, pair_part, cls,
        total;
    __host__ __device__ PlanLayout(int n_q, int n_keys) {
        n_qb = tt_cdiv(n_q, TT_BQ);
        n_kt = tt_cdiv(n_keys, TT_BK);
        n_kb = tt_cdiv(n_keys, TT_BKB);
        n_pb = tt_cdiv(n_keys, 256);
        size_t o = TT_PLAN_HDR;
        row_cnt = o;   o += 4 * (size_t)n_qb;
        row_order = o; o += 4 * (size_t)n_qb;
        row_list = o;  o += 4 * (size_t)n_qb * n_kt;
        kb_qlo = o;    o += 4 * (size_t)n_kb;
        kb_qhi = o;    o += 4 * (size_t)n_kb;
        kb_order = o;  o += 4 * (size_t)n_kb;
        kb_base = o;   o += 4 * ((size_t)n_kb + 1);
        kb_srank = o;  o += 4 * (size_t)n_kb;
        o = (o + 7) & ~(size_t)7;
        kb_item = o;   o += 8 * (size_t)n_kb * ((n_q - 1) / tt_qch(n_q) + 1);
        pair_part = o; o += 8 * (size_t)n_pb;
        cls = o;       o += (size_t)n_qb * n_kt;
        total = (o + 255) & ~(size_t)255;
    }
};

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

// Max / sum of x over lanes l and l ^ 32 (the two halves of a wave), with
// gfx950's v_permlane32_swap: of the returned pair, one element is the lane's
// own x and the other its partner's, in either order.
__device__ __forceinline__ float halves_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

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
