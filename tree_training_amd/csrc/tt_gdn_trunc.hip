// The reference's own within-node correction for the tree gated delta rule
// (tt_gdn_problem.reference_truncated = 1; tree_dfs_ssm.py:100-150): each whole
// node is one chunk and its correction is built from the uncorrected rows,
//   R = -strictly_lower(beta k^ k^T * D),  D[i][m] = exp(G_i - G_m),
//   [U | W] = (I + R + R^2) Y0,  Y0 = [beta v | beta e^G k^],
// with G the node's cumulative log decay (node-level, not chunk-level). The
// level scans then take V' = U - W S_parent for every chunk of the node.
//
// R is never stored: a node is cut into the same 32-row blocks the scans walk
// (one block = one chunk), and R applied to a block-row is a sum over the
// node's other blocks (earlier ones for R, later ones for R^T), each R block
// formed on the fly from k^ k^T (fp32 MFMA) and the decays. The work is
// quadratic in the node length, like the reference's L x L matrices.
//
// Backward, given dF = [dV' | dW] of every chunk (level scans):
//   dF1 = R^T dF,  dY0 = dF + dF1 + R^T dF1,
//   E = strictly_lower(dF (Y0 + R Y0)^T + dF1 Y0^T)     (the gradient of R),
// and through R[i][m] = -beta_i (k^_i . k^_m) D[i][m], with M = E * D:
//   dbeta_i -= sum_m M[i][m] (k^_i . k^_m),  dG_i -= beta_i sum_m M[i][m] (k^_i . k^_m),
//   dk^_i  -= beta_i sum_m M[i][m] k^_m,     dk^_m -= sum_i M[i][m] beta_i k^_i,
//   dG_m  += sum_i beta_i M[i][m] (k^_i . k^_m),
// plus the Y0 terms (dv = beta dY0_v, dbeta, dk^ and dG from beta e^G k^). The
// node-level dG becomes dg by a suffix sum over the node; the chunk backward
// (tt_gdn.hip) adds dk^ and that suffix sum to its own terms.
#include "tt_gdn_common.h"

namespace {

constexpr int GW = 2 * GD;        // width of [v | k] rows
constexpr int RX = GW + 8;        // LDS row stride of [GC x GW] tiles: rows 4 apart land 32 banks apart

// Node of chunk c and the chunk's block index within it; false for a malformed list.
__device__ __forceinline__ bool chunk_block(const GdnDev& p, int c, int& node, int& b, int& nb) {
    node = p.chunk_node[c];
    if (node < 0 || node >= p.n_nodes) return false;
    const int len = p.node_len[node], c0 = p.node_chunk0[node];
    nb = tt_cdiv(len, GC);
    b = c - c0;
    return len >= 1 && b >= 0 && b < nb && c0 >= 0 && c0 <= p.n_chunks - nb;
}

// l2-normalised k rows of one chunk into K (stride RS), zeros past len; with
// X, also that chunk's Y0 rows [beta v | beta e^G k^] (stride RX). gn: the
// chunk's 32 node-level decays. Thread t handles row t/8, dims 16*(t%8)..+15.
template <typename TIn>
__device__ __forceinline__ void load_k_rows(const GdnDev& p, int start, int len, int h, float* K, float* X,
                                            const float* gn) {
    const int t = threadIdx.x, i = t >> 3, d0 = 16 * (t & 7), hk = h / p.rep;
    const bool valid = i < len;
    const int64_t tok = start + i;
    float kv[16], vv[16];
    if (valid) {
        load16((const TIn*)p.k + tok * p.k_st + hk * p.k_sh + d0, kv);
        if (X) load16((const TIn*)p.v + tok * p.v_st + h * p.v_sh + d0, vv);
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) kv[e] = vv[e] = 0.0f;
    }
    float sk = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) sk = fmaf(kv[e], kv[e], sk);
    sk = row8_sum(sk);
    const float fk = p.l2 ? 1.0f / sqrtf(sk + 1e-6f) : 1.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) kv[e] *= fk;
#pragma unroll
    for (int e = 0; e < 16; e += 4)
        *(f32x4*)&K[i * RS + d0 + e] = (f32x4){kv[e], kv[e + 1], kv[e + 2], kv[e + 3]};
    if (X) {
        const float bt = valid ? p.beta[tok * p.b_st + h] : 0.0f;
        const float bg = bt * expf(gn[i]);
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
            *(f32x4*)&X[i * RX + d0 + e] = (f32x4){bt * vv[e], bt * vv[e + 1], bt * vv[e + 2], bt * vv[e + 3]};
            *(f32x4*)&X[i * RX + GD + d0 + e] =
                (f32x4){bg * kv[e], bg * kv[e + 1], bg * kv[e + 2], bg * kv[e + 3]};
        }
    }
}

// Decays and betas of one chunk's 32 rows (beta zero past len), threads < 32.
__device__ __forceinline__ void load_gb(const GdnDev& p, int start, int len, int h, const float* gn, float* G,
                                        float* B) {
    const int t = threadIdx.x;
    if (t < GC) {
        G[t] = gn[t];
        B[t] = t < len ? p.beta[(int64_t)(start + t) * p.b_st + h] : 0.0f;
    }
}

// k^_t k^_p^T partial over head dims 32w .. 32w+31 (wave w), into KP[w] as
// rows of the target block, columns of the partner block.
__device__ __forceinline__ void kk_partial(const float* Kt, const float* Kp, float* KP) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, col = lane & 31, half = lane >> 5;
    f32x16 kk = {};
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
        const int k0 = 32 * wave + 8 * q4 + 4 * half;
        const f32x4 a = *(const f32x4*)&Kt[col * RS + k0];
        const f32x4 b = *(const f32x4*)&Kp[col * RS + k0];
#pragma unroll
        for (int e = 0; e < 4; ++e) kk = mfma_f32(a[e], b[e], kk);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) KP[wave * GC * MS + acc_row(r, half) * MS + col] = kk[r];
}

__device__ __forceinline__ float sum4(const float* P, int idx) {
    return P[idx] + P[GC * MS + idx] + P[2 * GC * MS + idx] + P[3 * GC * MS + idx];
}

// ----------------------------------------------------------------------------
// node-level decay: gn = the chunk cumulative sums (prep) plus the sum over the
// node's earlier chunks
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(64) void gdn_gnode_kernel(GdnDev p, const float* __restrict__ prep,
                                                       float* __restrict__ gn) {
    const int node = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int len = p.node_len[node], c0 = p.node_chunk0[node], nch = tt_cdiv(len, GC);
    if (len < 1 || c0 < 0 || c0 > p.n_chunks - nch) return;
    float carry = 0.0f;
    for (int b = 0; b < nch; ++b) {
        const size_t chn = (size_t)(c0 + b) * p.hv + h;
        const float gv = lane < GC ? prep[chn * kWsChunk + kWsG + lane] : 0.0f;
        const float last = __shfl(gv, GC - 1);
        if (lane < GC) gn[chn * GC + lane] = gv + carry;
        carry += last;
    }
}

// ----------------------------------------------------------------------------
// out = R X over a node's blocks (lower: target block b, partners b' <= b) or
// out = R^T X (upper: partners b' >= b), [32 x 256] per (chunk, v head).
// ----------------------------------------------------------------------------
enum { TRI_Y1 = 0, TRI_UW = 1, TRI_DF1 = 2, TRI_DY0 = 3 };
struct TriArgs {
    const float* gn;      // [chunk, hv, 32] node-level decay
    const float* xa;      // TRI_UW: y1; TRI_DF1: dV'; TRI_DY0: dF1
    const float* xb;      // TRI_DF1: dW
    const float* fa;      // TRI_DY0: dV' and dW (the target's dF)
    const float* fb;
    float* out;           // TRI_Y1: y1; TRI_DF1: dF1; TRI_DY0: dY0 ([chunk, hv, 32, 256])
    float* prep;          // TRI_UW: U and W slots of the chunk terms
};

struct TriLds {
    float Kt[GC * RS];
    float Kp[GC * RS];
    float X[GC * RX];
    float KP[4 * GC * MS];
    float R[GC * MS];
    float Gt[GC], Gp[GC], Bt[GC], Bp[GC];
};

// MODE: TRI_Y1   y1 = R Y0 (Y0 from the inputs)
//       TRI_UW   [U | W] = Y0 + y1 + R y1, into the chunk terms
//       TRI_DF1  dF1 = R^T [dV' | dW]
//       TRI_DY0  dY0 = dF + dF1 + R^T dF1
// Wave w owns output columns 64w .. 64w+63 (two accumulator tiles).
template <int MODE, typename TIn>
__global__ __launch_bounds__(GT) void gdn_tri_kernel(GdnDev p, TriArgs a) {
    constexpr bool UPPER = MODE >= TRI_DF1;
    __shared__ __attribute__((aligned(16))) TriLds L;
    const int c = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63, col = lane & 31, half = lane >> 5;
    int node, b, nb, start, len;
    if (!chunk_block(p, c, node, b, nb) || !chunk_span(p, c, start, len)) return;
    const int nstart = p.node_start[node], nlen = p.node_len[node], chunk0 = p.node_chunk0[node];
    const size_t chn = (size_t)c * p.hv + h;

    load_k_rows<TIn>(p, start, len, h, L.Kt, nullptr, nullptr);
    load_gb(p, start, len, h, a.gn + chn * GC, L.Gt, L.Bt);
    f32x16 acc0 = {}, acc1 = {};
    const int bp0 = UPPER ? b : 0, bp1 = UPPER ? nb : b + 1;
    for (int bp = bp0; bp < bp1; ++bp) {
        const int cp = chunk0 + bp, startp = nstart + GC * bp, lenp = min(GC, nlen - GC * bp);
        const size_t chp = (size_t)cp * p.hv + h;
        __syncthreads();   // the previous partner's readers are done
        if constexpr (MODE == TRI_Y1) {
            load_k_rows<TIn>(p, startp, lenp, h, L.Kp, L.X, a.gn + chp * GC);
        } else {
            load_k_rows<TIn>(p, startp, lenp, h, L.Kp, nullptr, nullptr);
            const int i = t >> 3, c0 = 32 * (t & 7);
            const float* src;
            if constexpr (MODE == TRI_DF1)
                src = c0 < GD ? a.xa + (chp * GC + i) * GD + c0 : a.xb + (chp * GC + i) * GD + (c0 - GD);
            else
                src = a.xa + (chp * GC + i) * GW + c0;
#pragma unroll
            for (int e = 0; e < 32; e += 4) *(f32x4*)&L.X[i * RX + c0 + e] = *(const f32x4*)(src + e);
        }
        load_gb(p, startp, lenp, h, a.gn + chp * GC, L.Gp, L.Bp);
        __syncthreads();
        kk_partial(L.Kt, L.Kp, L.KP);
        __syncthreads();
        {   // R[target row][partner row] (R^T of the partner's rows for UPPER)
            const int i = t >> 3;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = (t & 7) + 8 * e;
                const float kk = sum4(L.KP, i * MS + m);
                const bool vis = i < len && m < lenp && (UPPER ? (bp > b || m > i) : (bp < b || m < i));
                float r = 0.0f;
                if (vis) r = UPPER ? -L.Bp[m] * kk * expf(L.Gp[m] - L.Gt[i]) : -L.Bt[i] * kk * expf(L.Gt[i] - L.Gp[m]);
                L.R[i * MS + m] = r;
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 rv = *(const f32x4*)&L.R[col * MS + 8 * q + 4 * half];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int k = 8 * q + 4 * half + e;
                acc0 = mfma_f32(rv[e], L.X[k * RX + 64 * wave + col], acc0);
                acc1 = mfma_f32(rv[e], L.X[k * RX + 64 * wave + 32 + col], acc1);
            }
        }
    }

    // Accumulator element r: row acc_row(r, half), column 64 wave + 32 tile + col.
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
        const f32x16& acc = tile ? acc1 : acc0;
        const int j = 64 * wave + 32 * tile + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = acc_row(r, half);
            float val = acc[r];
            if constexpr (MODE == TRI_UW) {
                float y0;
                if (j < GD) {
                    const float vj = i < len ? (float)((const TIn*)p.v)[(int64_t)(start + i) * p.v_st +
                                                                         (int64_t)h * p.v_sh + j]
                                             : 0.0f;
                    y0 = L.Bt[i] * vj;
                } else {
                    y0 = L.Bt[i] * expf(L.Gt[i]) * L.Kt[i * RS + (j - GD)];
                }
                val += y0 + a.xa[(chn * GC + i) * GW + j];
                float* dst = a.prep + chn * kWsChunk + (j < GD ? kWsU + i * GD + j : kWsW + i * GD + (j - GD));
                *dst = val;
            } else {
                if constexpr (MODE == TRI_DY0)
                    val += (j < GD ? a.fa[(chn * GC + i) * GD + j] : a.fb[(chn * GC + i) * GD + (j - GD)]) +
                           a.xa[(chn * GC + i) * GW + j];
                a.out[(chn * GC + i) * GW + j] = val;
            }
        }
    }
}

// ----------------------------------------------------------------------------
// gradient of R, row side: per target block b over partners b' <= b
// ----------------------------------------------------------------------------
struct EArgs {
    const float* gn;
    const float* y1;      // R Y0
    const float* dvp;     // dV' ([chunk, hv, 32, 128])
    const float* dw;      // dW
    const float* df1;     // R^T dF ([chunk, hv, 32, 256])
    const float* dy0;     // dF + dF1 + R^T dF1
    float* dkr;           // dk^ from the correction, [chunk, hv, 32, 128]
    float* dgn;           // node-level dG, [chunk, hv, 32]
    void* dv;             // [T, Hv, 128] problem dtype (row side only)
    float* dbeta;         // [T, Hv] (row side only)
};

struct ELds {
    float Kt[GC * RS];
    float Kp[GC * RS];
    float EP[4 * GC * MS];
    float KP[4 * GC * MS];
    float M[GC * MS];
    float Gt[GC], Gp[GC], Bt[GC], Bp[GC];
};

// Wave w's columns of the 512-wide contraction E = [dF | dF1] [Y0 + y1 | Y0]^T:
//   w = 0: dV' . (beta v + y1_v)      w = 1: dW . (beta e^G k^ + y1_k)
//   w = 2: dF1_v . beta v             w = 3: dF1_k . beta e^G k^
// A row of [dF | dF1] (source `side` 0) or of [Y0 + y1 | Y0] (side 1) for the
// lane's MFMA operand: 16 groups of 4 at columns 8 g + 4 half.
template <typename TIn>
__device__ __forceinline__ f32x4 e_operand_y(const GdnDev& p, const EArgs& a, int wave, int g, int half,
                                             size_t ch, int row, int tok, bool in, int h, float bm, float bgm,
                                             const float* K) {
    const int d = 8 * g + 4 * half;
    f32x4 y = {};
    if (wave == 0 || wave == 2) {
        if (in) y = load4((const TIn*)p.v + (int64_t)tok * p.v_st + (int64_t)h * p.v_sh + d) * bm;
        if (wave == 0) y += *(const f32x4*)(a.y1 + (ch * GC + row) * GW + d);
    } else {
        y = *(const f32x4*)&K[row * RS + d] * bgm;
        if (wave == 1) y += *(const f32x4*)(a.y1 + (ch * GC + row) * GW + GD + d);
    }
    return y;
}
__device__ __forceinline__ f32x4 e_operand_f(const EArgs& a, int wave, int g, int half, size_t ch, int row) {
    const int d = 8 * g + 4 * half;
    switch (wave) {
        case 0: return *(const f32x4*)(a.dvp + (ch * GC + row) * GD + d);
        case 1: return *(const f32x4*)(a.dw + (ch * GC + row) * GD + d);
        case 2: return *(const f32x4*)(a.df1 + (ch * GC + row) * GW + d);
        default: return *(const f32x4*)(a.df1 + (ch * GC + row) * GW + GD + d);
    }
}

template <typename TIn>
__global__ __launch_bounds__(GT) void gdn_erow_kernel(GdnDev p, EArgs a) {
    __shared__ __attribute__((aligned(16))) ELds L;
    const int c = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63, col = lane & 31, half = lane >> 5;
    int node, b, nb, start, len;
    if (!chunk_block(p, c, node, b, nb) || !chunk_span(p, c, start, len)) return;
    const int nstart = p.node_start[node], nlen = p.node_len[node], chunk0 = p.node_chunk0[node];
    const size_t chn = (size_t)c * p.hv + h;

    load_k_rows<TIn>(p, start, len, h, L.Kt, nullptr, nullptr);
    load_gb(p, start, len, h, a.gn + chn * GC, L.Gt, L.Bt);
    f32x4 ar[16];   // this lane's row of the target's [dF | dF1] slice
#pragma unroll
    for (int g = 0; g < 16; ++g) ar[g] = e_operand_f(a, wave, g, half, chn, col);
    f32x16 dk = {};
    float s_acc = 0.0f;   // row t/8: sum_m M (k^ . k^)
    for (int bp = 0; bp <= b; ++bp) {
        const int cp = chunk0 + bp, startp = nstart + GC * bp, lenp = min(GC, nlen - GC * bp);
        const size_t chp = (size_t)cp * p.hv + h;
        __syncthreads();
        load_k_rows<TIn>(p, startp, lenp, h, L.Kp, nullptr, nullptr);
        load_gb(p, startp, lenp, h, a.gn + chp * GC, L.Gp, L.Bp);
        __syncthreads();
        {
            const bool in = col < lenp;
            const float bm = L.Bp[col], bgm = bm * expf(L.Gp[col]);
            f32x16 ep = {};
#pragma unroll
            for (int g = 0; g < 16; ++g) {
                const f32x4 y = e_operand_y<TIn>(p, a, wave, g, half, chp, col, startp + col, in, h, bm, bgm, L.Kp);
#pragma unroll
                for (int e = 0; e < 4; ++e) ep = mfma_f32(ar[g][e], y[e], ep);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) L.EP[wave * GC * MS + acc_row(r, half) * MS + col] = ep[r];
        }
        kk_partial(L.Kt, L.Kp, L.KP);
        __syncthreads();
        {
            const int i = t >> 3;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = (t & 7) + 8 * e;
                const bool vis = i < len && m < lenp && (bp < b || m < i);
                float mv = 0.0f;
                if (vis) mv = sum4(L.EP, i * MS + m) * expf(L.Gt[i] - L.Gp[m]);
                s_acc = fmaf(mv, sum4(L.KP, i * MS + m), s_acc);
                L.M[i * MS + m] = mv;
            }
        }
        __syncthreads();
        // dk^ (rows of the target) += M k^_p over head dims 32 wave + col
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 mv = *(const f32x4*)&L.M[col * MS + 8 * q + 4 * half];
#pragma unroll
            for (int e = 0; e < 4; ++e) dk = mfma_f32(mv[e], L.Kp[(8 * q + 4 * half + e) * RS + 32 * wave + col], dk);
        }
    }
    const float s_row = row8_sum(s_acc);
    __syncthreads();   // Kp readers done: it takes -beta (M k^_p) in row order
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int i = acc_row(r, half);
        L.Kp[i * RS + 32 * wave + col] = -L.Bt[i] * dk[r];
    }
    __syncthreads();
    // The Y0 terms, per row: thread t owns row t/8, dims 16 (t % 8) .. +15 of v and of k.
    {
        const int i = t >> 3, d0 = 16 * (t & 7);
        const bool in = i < len;
        const int64_t tok = start + i;
        const float bt = L.Bt[i], eg = expf(L.Gt[i]);
        const float* dyr = a.dy0 + (chn * GC + i) * GW;
        float vv[16];
        if (in) load16((const TIn*)p.v + tok * p.v_st + (int64_t)h * p.v_sh + d0, vv);
        else
#pragma unroll
            for (int e = 0; e < 16; ++e) vv[e] = 0.0f;
        float vdot = 0.0f, kdot = 0.0f;
        f32x4 dvo[4];
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            const f32x4 dyv = *(const f32x4*)(dyr + d0 + 4 * e4);
            const f32x4 dyk = *(const f32x4*)(dyr + GD + d0 + 4 * e4);
            const f32x4 kh = *(const f32x4*)&L.Kt[i * RS + d0 + 4 * e4];
            f32x4 kr = *(const f32x4*)&L.Kp[i * RS + d0 + 4 * e4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                vdot = fmaf(dyv[e], vv[4 * e4 + e], vdot);
                kdot = fmaf(dyk[e], kh[e], kdot);
                kr[e] = fmaf(bt * eg, dyk[e], kr[e]);
                dvo[e4][e] = bt * dyv[e];
            }
            *(f32x4*)(a.dkr + (chn * GC + i) * GD + d0 + 4 * e4) = kr;
        }
        if (in)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) store4((TIn*)a.dv + tok * p.dv_st + h * GD + d0 + 4 * e4, dvo[e4]);
        vdot = row8_sum(vdot);
        kdot = row8_sum(kdot);
        if ((t & 7) == 0) {
            if (in) a.dbeta[tok * p.hv + h] = -s_row + vdot + eg * kdot;
            a.dgn[chn * GC + i] = in ? bt * (eg * kdot - s_row) : 0.0f;
        }
    }
}

// ----------------------------------------------------------------------------
// gradient of R, column side: per target block b over partners b' >= b (rows
// of R in the partner, columns in the target)
// ----------------------------------------------------------------------------
template <typename TIn>
__global__ __launch_bounds__(GT) void gdn_ecol_kernel(GdnDev p, EArgs a) {
    __shared__ __attribute__((aligned(16))) ELds L;
    const int c = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63, col = lane & 31, half = lane >> 5;
    int node, b, nb, start, len;
    if (!chunk_block(p, c, node, b, nb) || !chunk_span(p, c, start, len)) return;
    const int nstart = p.node_start[node], nlen = p.node_len[node], chunk0 = p.node_chunk0[node];
    const size_t chn = (size_t)c * p.hv + h;

    load_k_rows<TIn>(p, start, len, h, L.Kt, nullptr, nullptr);
    load_gb(p, start, len, h, a.gn + chn * GC, L.Gt, L.Bt);
    __syncthreads();
    f32x4 br[16];   // this lane's row of the target's [Y0 + y1 | Y0] slice
    {
        const bool in = col < len;
        const float bm = L.Bt[col], bgm = bm * expf(L.Gt[col]);
#pragma unroll
        for (int g = 0; g < 16; ++g) br[g] = e_operand_y<TIn>(p, a, wave, g, half, chn, col, start + col, in, h, bm, bgm, L.Kt);
    }
    f32x16 dk = {};
    float cs_acc = 0.0f;   // column t/8: sum_i beta_i M (k^ . k^)
    for (int bq = b; bq < nb; ++bq) {
        const int cp = chunk0 + bq, startp = nstart + GC * bq, lenp = min(GC, nlen - GC * bq);
        const size_t chp = (size_t)cp * p.hv + h;
        __syncthreads();
        load_k_rows<TIn>(p, startp, lenp, h, L.Kp, nullptr, nullptr);
        load_gb(p, startp, lenp, h, a.gn + chp * GC, L.Gp, L.Bp);
        __syncthreads();
        {   // E[partner row][target row]
            f32x16 ep = {};
#pragma unroll
            for (int g = 0; g < 16; ++g) {
                const f32x4 f = e_operand_f(a, wave, g, half, chp, col);
#pragma unroll
                for (int e = 0; e < 4; ++e) ep = mfma_f32(f[e], br[g][e], ep);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) L.EP[wave * GC * MS + acc_row(r, half) * MS + col] = ep[r];
        }
        kk_partial(L.Kp, L.Kt, L.KP);   // [partner row][target row]
        __syncthreads();
        {
            const int m = t >> 3;   // target row
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = (t & 7) + 8 * e;   // partner row
                const bool vis = i < lenp && m < len && (bq > b || i > m);
                float mv = 0.0f;
                if (vis) mv = sum4(L.EP, i * MS + m) * expf(L.Gp[i] - L.Gt[m]);
                cs_acc = fmaf(L.Bp[i] * mv, sum4(L.KP, i * MS + m), cs_acc);
                L.M[m * MS + i] = mv;   // transposed: rows = target
            }
        }
        __syncthreads();
        // dk^ (rows of the target) += M^T (beta k^)_p over head dims 32 wave + col
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 mv = *(const f32x4*)&L.M[col * MS + 8 * q + 4 * half];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int k = 8 * q + 4 * half + e;
                dk = mfma_f32(mv[e], L.Bp[k] * L.Kp[k * RS + 32 * wave + col], dk);
            }
        }
    }
    const float cs_row = row8_sum(cs_acc);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) L.Kp[acc_row(r, half) * RS + 32 * wave + col] = -dk[r];
    __syncthreads();
    {
        const int i = t >> 3, d0 = 16 * (t & 7);
        float* dst = a.dkr + (chn * GC + i) * GD + d0;
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4)
            *(f32x4*)(dst + 4 * e4) = *(const f32x4*)(dst + 4 * e4) + *(const f32x4*)&L.Kp[i * RS + d0 + 4 * e4];
        if ((t & 7) == 0 && i < len) a.dgn[chn * GC + i] += cs_row;
    }
}

// ----------------------------------------------------------------------------
// node-level dG -> its suffix sums over the node (in place): dg_i gets
// sum_{j >= i in the node} dG_j, G being the node's cumulative sum
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(64) void gdn_gsuffix_kernel(GdnDev p, float* __restrict__ dgn) {
    const int node = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int len = p.node_len[node], c0 = p.node_chunk0[node], nch = tt_cdiv(len, GC);
    if (len < 1 || c0 < 0 || c0 > p.n_chunks - nch) return;
    float carry = 0.0f;
    for (int b = nch - 1; b >= 0; --b) {
        const size_t chn = (size_t)(c0 + b) * p.hv + h;
        const int lenc = min(GC, len - GC * b);
        float v = lane < lenc ? dgn[chn * GC + lane] : 0.0f;
#pragma unroll
        for (int o = 1; o < GC; o <<= 1) {
            const float up = __shfl_down(v, o, GC);
            if ((lane & (GC - 1)) + o < GC) v += up;
        }
        const float total = __shfl(v, 0);
        if (lane < GC) dgn[chn * GC + lane] = lane < lenc ? v + carry : 0.0f;
        carry += total;
    }
}

template <typename TIn>
int trunc_fwd(const GdnDev& d, float* prep, float* gn, float* y1, hipStream_t s) {
    hipLaunchKernelGGL(gdn_gnode_kernel, dim3(d.n_nodes, d.hv), dim3(64), 0, s, d, prep, gn);
    TriArgs a{gn, nullptr, nullptr, nullptr, nullptr, y1, prep};
    hipLaunchKernelGGL((gdn_tri_kernel<TRI_Y1, TIn>), dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, a);
    a.xa = y1;
    a.out = nullptr;
    hipLaunchKernelGGL((gdn_tri_kernel<TRI_UW, TIn>), dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, a);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

template <typename TIn>
int trunc_bwd(const GdnDev& d, const GdnTruncBwd& w, void* dv, float* dbeta, hipStream_t s) {
    TriArgs t1{w.gn, w.dvp, w.dw, nullptr, nullptr, w.df1, nullptr};
    hipLaunchKernelGGL((gdn_tri_kernel<TRI_DF1, TIn>), dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, t1);
    TriArgs t2{w.gn, w.df1, nullptr, w.dvp, w.dw, w.dy0, nullptr};
    hipLaunchKernelGGL((gdn_tri_kernel<TRI_DY0, TIn>), dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, t2);
    EArgs e{w.gn, w.y1, w.dvp, w.dw, w.df1, w.dy0, w.dkr, w.dgn, dv, dbeta};
    hipLaunchKernelGGL(gdn_erow_kernel<TIn>, dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, e);
    hipLaunchKernelGGL(gdn_ecol_kernel<TIn>, dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, e);
    hipLaunchKernelGGL(gdn_gsuffix_kernel, dim3(d.n_nodes, d.hv), dim3(64), 0, s, d, w.dgn);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

}  // namespace

int tt_gdn_trunc_fwd_launch(const GdnDev& d, float* prep, float* gn, float* y1, hipStream_t s) {
    return d.dtype == TT_DTYPE_BF16 ? trunc_fwd<__bf16>(d, prep, gn, y1, s) : trunc_fwd<float>(d, prep, gn, y1, s);
}

int tt_gdn_trunc_bwd_launch(const GdnDev& d, const GdnTruncBwd& w, void* dv, float* dbeta, hipStream_t s) {
    return d.dtype == TT_DTYPE_BF16 ? trunc_bwd<__bf16>(d, w, dv, dbeta, s) : trunc_bwd<float>(d, w, dv, dbeta, s);
}
