// Device helpers shared by the tree gated-delta-rule kernels (tt_gdn.hip:
// the exact rule's prep, scans and backward; tt_gdn_trunc.hip: the
// reference's truncated within-node correction).
#pragma once

#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr int GD = 128;           // head dim (Dk = Dv)
constexpr int GC = TT_GDN_CHUNK;  // chunk length (32)
constexpr int GT = 256;           // threads per workgroup
constexpr int RS = GD + 4;        // row stride of [GC x GD] tiles (floats): rows 4 banks apart
constexpr int MS = GC + 4;        // row stride of [GC x GC] matrices
constexpr int RR = GC + 1;        // row stride of per-wave 32 x 32 partial products

// Workspace per (chunk, v head), floats: W [GC][GD], U [GC][GD], A [GC][GC],
// T [GC][GC] (the inverse, for the backward), G [GC] and its low part Glo [GC].
constexpr size_t kWsW = 0, kWsU = GC * GD, kWsA = 2 * GC * GD, kWsT = kWsA + GC * GC, kWsG = kWsT + GC * GC;
constexpr size_t kWsGlo = kWsG + GC;
constexpr size_t kWsChunk = kWsGlo + GC;

// The cumulative decay G of a chunk is kept as an unevaluated sum hi + lo,
// lo holding the rounding errors of the prefix sum. A strongly decaying head
// reaches |G| of several hundred within 32 tokens, where one float rounds
// G by up to |G| 2^-24 (3e-5 at 500): every factor e^{G_i - G_j} of two
// late tokens that is not negligible would carry that as a relative error.
// With both parts the difference is exact up to its own final rounding
// (hi_i - hi_j is exact whenever it is not large, Sterbenz).
__device__ __forceinline__ float gdiff(float hi_i, float lo_i, float hi_j, float lo_j) {
    return (hi_i - hi_j) + (lo_i - lo_j);
}

template <int I>
struct IntC4 {
    static constexpr int value = I;
};

template <typename T>
__device__ __forceinline__ void load16(const T* p, float (&x)[16]) {
    if constexpr (sizeof(T) == 2) {
        const bf16x8 a = *(const bf16x8*)p, b = *(const bf16x8*)(p + 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            x[e] = (float)a[e];
            x[8 + e] = (float)b[e];
        }
    } else {
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
            const f32x4 a = *(const f32x4*)(p + e);
            x[e] = a[0]; x[e + 1] = a[1]; x[e + 2] = a[2]; x[e + 3] = a[3];
        }
    }
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const f32x4& x) {
    if constexpr (sizeof(T) == 2) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (__bf16)x[e];
        *(bf16x4*)p = w;
    } else {
        *(f32x4*)p = x;
    }
}

// Sum over the 8 consecutive lanes that hold one row.
__device__ __forceinline__ float row8_sum(float x) {
    x += __shfl_xor(x, 1);
    x += __shfl_xor(x, 2);
    x += __shfl_xor(x, 4);
    return x;
}

// Chunk `c` -> (first token, length); false for a malformed chunk list.
__device__ __forceinline__ bool chunk_span(const GdnDev& p, int c, int& start, int& len) {
    const int node = p.chunk_node[c];
    if (node < 0 || node >= p.n_nodes) return false;
    const int ci = c - p.node_chunk0[node];
    const int ns = p.node_start[node], nl = p.node_len[node];
    if (ns < 0 || nl < 0 || ns > p.n_tokens - nl || ci < 0 || GC * ci >= nl) return false;
    start = ns + GC * ci;
    len = min(GC, nl - GC * ci);
    return true;
}

// Rows of one chunk (zeros past its length): l2-normalised q (times scale),
// k, and, when V is given, v; thread t handles row t/8, 16 dims.
template <typename TIn>
__device__ __forceinline__ void load_chunk_rows(const GdnDev& p, int start, int len, int h, float* Q, float* K,
                                                float* V) {
    const int t = threadIdx.x, i = t >> 3, d0 = 16 * (t & 7), hk = h / p.rep;
    const bool valid = i < len;
    const int64_t tok = start + i;
    float qv[16], kv[16], vv[16];
    if (valid) {
        load16((const TIn*)p.q + tok * p.q_st + hk * p.q_sh + d0, qv);
        load16((const TIn*)p.k + tok * p.k_st + hk * p.k_sh + d0, kv);
        if (V) load16((const TIn*)p.v + tok * p.v_st + h * p.v_sh + d0, vv);
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) qv[e] = kv[e] = vv[e] = 0.0f;
    }
    float sq = 0.0f, sk = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        sq = fmaf(qv[e], qv[e], sq);
        sk = fmaf(kv[e], kv[e], sk);
    }
    sq = row8_sum(sq);
    sk = row8_sum(sk);
    const float fq = (p.l2 ? 1.0f / sqrtf(sq + 1e-6f) : 1.0f) * p.scale;
    const float fk = p.l2 ? 1.0f / sqrtf(sk + 1e-6f) : 1.0f;
#pragma unroll
    for (int e = 0; e < 16; e += 4) {
        *(f32x4*)&Q[i * RS + d0 + e] = (f32x4){qv[e] * fq, qv[e + 1] * fq, qv[e + 2] * fq, qv[e + 3] * fq};
        *(f32x4*)&K[i * RS + d0 + e] = (f32x4){kv[e] * fk, kv[e + 1] * fk, kv[e + 2] * fk, kv[e + 3] * fk};
        if (V) *(f32x4*)&V[i * RS + d0 + e] = (f32x4){vv[e], vv[e + 1], vv[e + 2], vv[e + 3]};
    }
}

// v_mfma_f32_32x32x2_f32: D[32x32] += A[32x2] B[2x32]; lane l supplies
// A[l & 31][l >> 5] and B[l >> 5][l & 31], and accumulator element r of lane l
// is D[acc_row(r, l >> 5)][l & 31]. The contraction order is free, so step r
// of a 32-deep contraction pairs k = acc_row(r, 0) (lanes 0-31) with
// k = acc_row(r, 1) (lanes 32-63): a matrix held as accumulators (rows k,
// columns j) is then directly the B operand, element r of each lane.
__device__ __forceinline__ f32x16 mfma_f32(float a, float b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x4_f32: D[16x16] += A[16x4] B[4x16]; lane l supplies
// A[l & 15][l >> 4] and B[l >> 4][l & 15], and accumulator element v of lane
// l is D[4 (l >> 4) + v][l & 15]. Step v of a 16-deep contraction pairs
// k = 4 (l >> 4) + v across the four lane groups, so a 16-row block held as
// accumulators is directly the B operand, element v of each lane.
__device__ __forceinline__ f32x4 mfma16_f32(float a, float b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// A 16 x 16 tile of a row-major fp32 matrix of GD-float rows in the layout
// of mfma16_f32's accumulators: element v of lane l is row 4 (l >> 4) + v,
// column l & 15, of the tile at `base`.
__device__ __forceinline__ f32x4 load_t16(const float* base, int lane) {
    const float* p = base + 4 * (lane >> 4) * GD + (lane & 15);
    return (f32x4){p[0], p[GD], p[2 * GD], p[3 * GD]};
}
__device__ __forceinline__ void store_t16(float* base, int lane, const f32x4& x) {
    float* p = base + 4 * (lane >> 4) * GD + (lane & 15);
    p[0] = x[0];
    p[GD] = x[1];
    p[2 * GD] = x[2];
    p[3 * GD] = x[3];
}

// Accumulator-layout access to a row-major fp32 matrix of GD-float rows:
// element r of lane l is row ROW0 + acc_row(r, l >> 5), column `col`. One
// buffer resource (scalar registers), four lane offsets (rows r % 4); the
// uniform part of the row, ROW0 + 8 (r / 4), goes in the scalar offset.
struct AccMat {
    __amdgpu_buffer_rsrc_t rs;
    int vo[4];
};
__device__ __forceinline__ AccMat acc_mat(const float* base, int rows, int half, int col) {
    AccMat m;
    m.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, rows * GD * 4, 0x00020000);
#pragma unroll
    for (int k = 0; k < 4; ++k) m.vo[k] = ((4 * half + k) * GD + col) * 4;
    return m;
}
template <int ROW0>
__device__ __forceinline__ f32x16 load_acc(const AccMat& m) {
    f32x16 v;
#pragma unroll
    for (int r = 0; r < 16; ++r)
        v[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(m.rs, m.vo[r & 3], (ROW0 + 8 * (r >> 2)) * GD * 4, 0));
    return v;
}
template <int ROW0>
__device__ __forceinline__ void store_acc(const AccMat& m, const f32x16& v) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[r]), m.rs, m.vo[r & 3], (ROW0 + 8 * (r >> 2)) * GD * 4, 0);
}
template <typename F>
__device__ __forceinline__ void for_tiles(F&& f) {
    f(IntC4<0>{});
    f(IntC4<1>{});
    f(IntC4<2>{});
    f(IntC4<3>{});
}

template <typename T>
__device__ __forceinline__ f32x4 load4(const T* p) {
    if constexpr (sizeof(T) == 2) {
        const bf16x4 a = *(const bf16x4*)p;
        return (f32x4){(float)a[0], (float)a[1], (float)a[2], (float)a[3]};
    } else {
        return *(const f32x4*)p;
    }
}

__device__ __forceinline__ float dot4(const f32x4& a, const f32x4& b) {
    return fmaf(a[0], b[0], fmaf(a[1], b[1], fmaf(a[2], b[2], a[3] * b[3])));
}

// Rows of a [GC x GD] tile into LDS (stride RS): thread t copies row t/8,
// dims 16*(t%8)..+15; rows at or past `len` are zero.
template <typename T>
__device__ __forceinline__ void tile_in(const T* base, int64_t row_stride, int len, float* dst) {
    const int i = threadIdx.x >> 3, d0 = 16 * (threadIdx.x & 7);
    float x[16];
    if (i < len) {
        load16(base + i * row_stride + d0, x);
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) x[e] = 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 16; e += 4) *(f32x4*)&dst[i * RS + d0 + e] = (f32x4){x[e], x[e + 1], x[e + 2], x[e + 3]};
}

// fp32 MFMA operands from LDS, in the k order of mfma_f32 (step r pairs
// k = acc_row(r, 0) on lanes 0-31 with k = acc_row(r, 1) on lanes 32-63).
// Row operand X[col][kb + k]: four steps per 16-byte read.
__device__ __forceinline__ f32x4 op_row4(const float* X, int stride, int col, int half, int kb, int m) {
    return *(const f32x4*)&X[col * stride + kb + 8 * m + 4 * half];
}
// Column operand X[kb + k][c0 + col], one step.
__device__ __forceinline__ float op_col(const float* X, int stride, int half, int kb, int r, int c0, int col) {
    return X[(kb + acc_row(r, half)) * stride + c0 + col];
}
// 32 x 32 partial product over this wave's quarter of a 128-deep contraction:
// D[i][j] = sum_k A[i][k] B[j][k] (both read as rows), B scaled by bs (a
// per-column factor), added to acc.
__device__ __forceinline__ f32x16 quarter_nt(const float* A, const float* B, float bs, int col, int half, int wave,
                                             f32x16 acc) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const f32x4 a = op_row4(A, RS, col, half, 32 * wave, m), b = op_row4(B, RS, col, half, 32 * wave, m);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = mfma_f32(a[e], b[e] * bs, acc);
    }
    return acc;
}
__device__ __forceinline__ void put_partial(float* R, const f32x16& acc, int col, int half) {
#pragma unroll
    for (int r = 0; r < 16; ++r) R[acc_row(r, half) * RR + col] = acc[r];
}

}  // namespace
