// Tree gated delta rule (the linear-attention layers of Qwen3.5-style models)
// over a DFS-packed tree: forward for gfx950.
//
// Semantics: the gated delta rule token by token along every root-to-leaf
// path — each node continues from its parent's final state (a root from the
// caller's initial state, or zero) — evaluated exactly in TT_GDN_CHUNK =
// 32-token chunks (a node is cut into consecutive chunks; its last chunk may
// be short):
//   G = cumsum(g), D[i][j] = exp(G_i - G_j) (j <= i),
//   N = -strictly_lower(beta k k^T * D),  T = (I - N)^-1,
//   U = T (beta v),  W = T (beta e^G k),  A = lower_incl(q k^T * D),
//   V' = U - W S,  O = e^G (q S) + A V',  S <- e^{G_last} S + (k e^{G_last - G})^T V'.
// q and k are l2-normalised in the kernels and q is scaled; v head h reads q/k
// head h / (Hv / Hk).
//
// Two kernels:
//  * gdn_prep_kernel — one workgroup per (chunk, v head), all chunks at once:
//    everything that does not depend on the state (A, T by a product of
//    (I + N^(2^r)) factors, U, W, G) into the workspace.
//  * gdn_scan_cols_kernel — per (node, v head) two workgroups of four waves,
//    one launch per tree level so a node's parent state (in the caller's
//    node_states buffer) is complete when it starts; each wave holds a
//    128 x 16 value slice of the state in MFMA accumulators (the delta rule is
//    independent per value column) and walks the node's chunks. Levels of
//    one or two nodes use gdn_scan_rows_kernel instead (eight workgroups per
//    pair, each wave a 32 x 16 slice), which gives the same bits.
// fp32 end to end: the prep on fp32 MFMA (v_mfma_f32_32x32x2_f32) and the
// vector ALUs, the scans on v_mfma_f32_16x16x4_f32.
#include "tt_gdn_common.h"

namespace {


// ----------------------------------------------------------------------------
// prep: per (chunk, v head) A, T, U, W, G
// ----------------------------------------------------------------------------
struct PrepLds {
    float Q[GC * RS];     // q^ * scale; v once A is done
    float K[GC * RS];
    float R[8 * 16 * 17]; // q^ k^T at 0 and k^ k^T at GC * RR (rows of RR); then T's 16 x 16 blocks
    float N[GC * MS];     // N = -strictly_lower(beta k^ k^T * D)
    float Tm[GC * MS];    // I + N, then T = (I - N)^-1
    float G[GC];
    float Glo[GC];
    float beta[GC];
    float bg[GC];         // beta e^G
};
static_assert(2 * GC * RR <= 8 * 16 * 17, "the two 32 x 32 partial products fit the inverse's scratch");

// q^ k^T and k^ k^T on fp32 MFMA (waves 0-1 and 2-3, each half of the
// 128-deep contraction), the inverse T on the vector ALUs, then U and W on
// fp32 MFMA, split by columns over the waves.
// TRUNC (the reference's per-node correction): only A and G here; U and W
// come from the node-level kernels of tt_gdn_trunc.hip.
template <typename TIn, bool TRUNC>
__global__ __launch_bounds__(GT) void gdn_prep_kernel(GdnDev p, float* __restrict__ ws) {
    __shared__ __attribute__((aligned(16))) PrepLds L;
    const int c = blockIdx.x, h = blockIdx.y;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, col = lane & 31, half = lane >> 5;
    int start, len;
    if (!chunk_span(p, c, start, len)) return;
    float* out = ws + ((size_t)c * p.hv + h) * kWsChunk;

    load_chunk_rows<TIn>(p, start, len, h, L.Q, L.K, nullptr);
    if (wave == 0) {
        // cumulative decay over the chunk (lanes 0..31; padded rows add 0),
        // each step's rounding error (two-sum) carried in lo
        const bool valid = lane < len;
        const int64_t tok = start + lane;
        float gv = valid ? p.g[tok * p.g_st + h] : 0.0f, lo = 0.0f;
        const float bv = valid ? p.beta[tok * p.b_st + h] : 0.0f;
#pragma unroll
        for (int o = 1; o < GC; o <<= 1) {
            const float up = __shfl_up(gv, o, GC), up_lo = __shfl_up(lo, o, GC);
            if ((lane & (GC - 1)) >= o) {
                const float sum = gv + up, bp = sum - gv;
                lo += up_lo + ((gv - (sum - bp)) + (up - bp));
                gv = sum;
            }
        }
        if (lane < GC) {
            L.G[lane] = gv;
            L.Glo[lane] = lo;
            L.beta[lane] = bv;
            L.bg[lane] = bv * expf(gv + lo);
            out[kWsG + lane] = gv;
            out[kWsGlo + lane] = lo;
        }
    }
    __syncthreads();
    {   // the odd wave of each pair stores its half of the contraction, the
        // even one adds its own in place (two 32 x 32 buffers, not four)
        const float* X = wave < 2 ? L.Q : L.K;
        const int q0 = 2 * (wave & 1);
        f32x16 acc = quarter_nt(X, L.K, 1.0f, col, half, q0, (f32x16){});
        acc = quarter_nt(X, L.K, 1.0f, col, half, q0 + 1, acc);
        float* Rw = L.R + (wave >> 1) * GC * RR;
        if (wave & 1) put_partial(Rw, acc, col, half);
        __syncthreads();
        if constexpr (!TRUNC)   // Q's readers are done
            tile_in((const TIn*)p.v + (int64_t)start * p.v_st + (int64_t)h * p.v_sh, p.v_st, len, L.Q);
        if (!(wave & 1)) {
#pragma unroll
            for (int r = 0; r < 16; ++r) Rw[acc_row(r, half) * RR + col] += acc[r];
        }
    }
    __syncthreads();

    // A = lower_incl(q^ k^T * D), N = -strictly_lower(beta k^ k^T * D).
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int pi = t + GT * u, i = pi >> 5, j = pi & 31;
        const float dqk = L.R[i * RR + j];
        const float dkk = L.R[GC * RR + i * RR + j];
        const float dec = j <= i ? expf(gdiff(L.G[i], L.Glo[i], L.G[j], L.Glo[j])) : 0.0f;
        const float nij = j < i ? -L.beta[i] * dkk * dec : 0.0f;
        out[kWsA + i * GC + j] = dqk * dec;
        L.N[i * MS + j] = nij;
        L.Tm[i * MS + j] = nij + (i == j ? 1.0f : 0.0f);
    }
    if constexpr (TRUNC) return;
    __syncthreads();

    // T = (I - N)^-1 by 16 x 16 blocks. With N = [[N11, 0], [N21, N22]],
    // T = [[T11, 0], [T22 N21 T11, T22]] and, each Nbb strictly lower
    // triangular (Nbb^16 = 0), Tbb = (I + Nbb)(I + Nbb^2)(I + Nbb^4)(I + Nbb^8):
    // from T = I + Nbb, P = Nbb, three rounds of P <- P P, then T <- T + T P.
    // Waves 0-1 take block 1, waves 2-3 block 2 (thread u: row u/8, columns
    // 2 (u%8), +1), with double-buffered P and T in the partial-product
    // buffer R (free again); then X = N21 T11 and T21 = T22 X, a thread an
    // entry. A quarter of the work of squaring the whole 32 x 32 matrix.
    {
        constexpr int BS = 17;                                   // row stride of the 16 x 16 blocks
        constexpr int B16 = 16 * BS;
        float* sc = L.R;
        const int blk = t >> 7, u = t & 127, bi = u >> 3, bj = 2 * (u & 7), o = 16 * blk;
        // block blk: P buffers at pb, pb + B16; T buffers at pb + 2 B16, pb + 3 B16
        const int pb = blk * 4 * B16, tb = pb + 2 * B16;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int j = bj + e;
            const float n = L.N[(o + bi) * MS + o + j];
            sc[pb + bi * BS + j] = n;
            sc[tb + bi * BS + j] = n + (bi == j ? 1.0f : 0.0f);
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            const int pc = pb + (r & 1) * B16, pn = pb + ((r + 1) & 1) * B16;
            float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                const float pim = sc[pc + bi * BS + m];
                a0 = fmaf(pim, sc[pc + m * BS + bj], a0);
                a1 = fmaf(pim, sc[pc + m * BS + bj + 1], a1);
            }
            sc[pn + bi * BS + bj] = a0;
            sc[pn + bi * BS + bj + 1] = a1;
            __syncthreads();
            const int tc0 = tb + (r & 1) * B16, tn = tb + ((r + 1) & 1) * B16;
            float t0 = sc[tc0 + bi * BS + bj], t1 = sc[tc0 + bi * BS + bj + 1];
#pragma unroll
            for (int m = 0; m < 16; ++m) {
                const float tim = sc[tc0 + bi * BS + m];
                t0 = fmaf(tim, sc[pn + m * BS + bj], t0);
                t1 = fmaf(tim, sc[pn + m * BS + bj + 1], t1);
            }
            sc[tn + bi * BS + bj] = t0;
            sc[tn + bi * BS + bj + 1] = t1;
            __syncthreads();
        }
        // Tbb is in the second T buffer of its block; X = N21 T11 goes to
        // block 1's first P buffer.
        constexpr int T11 = 3 * B16, T22 = 4 * B16 + 3 * B16, X = 0;
        const int xi = t >> 4, xj = t & 15;
        {
            float x = 0.0f;
#pragma unroll
            for (int m = 0; m < 16; ++m) x = fmaf(L.N[(16 + xi) * MS + m], sc[T11 + m * BS + xj], x);
            sc[X + xi * BS + xj] = x;
        }
        __syncthreads();
        float t21 = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; ++m) t21 = fmaf(sc[T22 + xi * BS + m], sc[X + m * BS + xj], t21);
        L.Tm[(16 + xi) * MS + xj] = t21;
        L.Tm[xi * MS + 16 + xj] = 0.0f;
#pragma unroll
        for (int e = 0; e < 2; ++e) L.Tm[(o + bi) * MS + o + bj + e] = sc[tb + B16 + bi * BS + bj + e];
        __syncthreads();
        const int ti = t >> 3, tc = 4 * (t & 7);
        *(f32x4*)(out + kWsT + ti * GC + tc) = *(const f32x4*)&L.Tm[ti * MS + tc];
    }

    // U = T (beta v), W = T (beta e^G k^): wave w produces columns 32w .. 32w+31.
    {
        const int cw0 = 32 * wave;
        f32x16 u = {}, w = {};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const f32x4 a = op_row4(L.Tm, MS, col, half, 0, m);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * m + e, k = acc_row(r, half);
                u = mfma_f32(a[e], L.beta[k] * L.Q[k * RS + cw0 + col], u);
                w = mfma_f32(a[e], L.bg[k] * L.K[k * RS + cw0 + col], w);
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            out[kWsU + acc_row(r, half) * GD + cw0 + col] = u[r];
            out[kWsW + acc_row(r, half) * GD + cw0 + col] = w[r];
        }
    }
}

// ----------------------------------------------------------------------------
// scan: per (node, v head), the node's chunks in order, on fp32 MFMA
// ----------------------------------------------------------------------------

struct ScanLds {
    float W[GC * RS];     // W [token][state row]
    float Q[GC * RS];     // q^ * scale
    float K[GC * RS];     // k^ e^{G_L - G}
    float A[GC * MS];
    float G[GC];
};

// A chunk's scan inputs, held in registers one chunk ahead of their use (the
// loads of the next chunk are in flight while a chunk computes): this
// thread's share of the q and k rows (row t/8, dims 16 (t%8) .. +15, in the
// problem dtype), of W's rows, four entries of A and the decays, and this
// lane's 16 x 16 operand tiles of U (forward) or dO (reverse).
template <typename TIn>
struct ScanAhead {
    using Vec = typename std::conditional<sizeof(TIn) == 2, bf16x8, f32x4>::type;
    static constexpr int NV = 16 * (int)sizeof(TIn) / 16;   // vectors per 16 elements
    Vec q[NV], k[NV];
    f32x4 w[4];
    float a[4];
    float gi, gl, gt, gil, gll;   // G_i, G_L, G_t; low parts of G_i, G_L
    f32x4 x[2];
};

// Loads the parts of chunk (start, len) that do not depend on the state: q/k
// rows, W rows (with LOAD_W), A and the decays from its workspace slot cw.
template <typename TIn, bool LOAD_W>
__device__ __forceinline__ void scan_fetch_rows(const GdnDev& p, const float* cw, int start, int len, int h,
                                                ScanAhead<TIn>& x) {
    using Vec = typename ScanAhead<TIn>::Vec;
    constexpr int NV = ScanAhead<TIn>::NV, EV = 16 / NV;
    const int t = threadIdx.x, i = t >> 3, d0 = 16 * (t & 7), hk = h / p.rep;
    if (i < len) {
        const int64_t tok = start + i;
        const TIn* qp = (const TIn*)p.q + tok * p.q_st + (int64_t)hk * p.q_sh + d0;
        const TIn* kp = (const TIn*)p.k + tok * p.k_st + (int64_t)hk * p.k_sh + d0;
#pragma unroll
        for (int n = 0; n < NV; ++n) {
            x.q[n] = *(const Vec*)(qp + EV * n);
            x.k[n] = *(const Vec*)(kp + EV * n);
        }
    } else {
#pragma unroll
        for (int n = 0; n < NV; ++n) {
#pragma unroll
            for (int e = 0; e < EV; ++e) x.q[n][e] = x.k[n][e] = (TIn)0.0f;
        }
    }
    if constexpr (LOAD_W) {
#pragma unroll
        for (int e = 0; e < 4; ++e) x.w[e] = *(const f32x4*)(cw + kWsW + i * GD + d0 + 4 * e);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) x.a[e] = cw[kWsA + t + GT * e];
    x.gi = cw[kWsG + i];
    x.gl = cw[kWsG + GC - 1];
    x.gt = cw[kWsG + (t & (GC - 1))];
    x.gil = cw[kWsGlo + i];
    x.gll = cw[kWsGlo + GC - 1];
}

// Writes a fetched chunk to LDS: Q = q^ * scale * qmul_i, K = k^ * kmul_i
// (each rounded after the normalisation, then after the multiplier), W with
// STORE_W, A and G. qmul / kmul: e^{G_i} / e^{G_L - G_i} where the scan needs
// them (1 for none: the forward's Q).
template <typename TIn, bool STORE_W, bool QMUL>
__device__ __forceinline__ void scan_stage_rows(const GdnDev& p, const ScanAhead<TIn>& x, float* Q, float* K,
                                                float* W, float* A, float* G) {
    constexpr int NV = ScanAhead<TIn>::NV, EV = 16 / NV;
    const int t = threadIdx.x, i = t >> 3, d0 = 16 * (t & 7);
    float qv[16], kv[16];
#pragma unroll
    for (int n = 0; n < NV; ++n)
#pragma unroll
        for (int e = 0; e < EV; ++e) {
            qv[EV * n + e] = (float)x.q[n][e];
            kv[EV * n + e] = (float)x.k[n][e];
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
    const float eq = QMUL ? expf(x.gi) : 1.0f, ek = expf(gdiff(x.gl, x.gll, x.gi, x.gil));
#pragma unroll
    for (int e = 0; e < 16; e += 4) {
        f32x4 qo, ko;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            qo[v] = qv[e + v] * fq;
            ko[v] = kv[e + v] * fk;
            if constexpr (QMUL) qo[v] *= eq;
            ko[v] *= ek;
        }
        *(f32x4*)&Q[i * RS + d0 + e] = qo;
        *(f32x4*)&K[i * RS + d0 + e] = ko;
        if constexpr (STORE_W) *(f32x4*)&W[i * RS + d0 + e] = x.w[e / 4];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int pi = t + GT * e;
        A[(pi >> 5) * MS + (pi & 31)] = x.a[e];
    }
    if (t < GC) G[t] = x.gt;
}

// Column layout of the level scans. The value columns of the delta rule are
// independent (column j of V', O and S depends only on column j of U, S and
// V'); each wave owns 16 of them (16 x 16 fp32 MFMA tiles), and a (node,
// v head) takes two workgroups of four waves (64 columns each) on different
// CUs. A level with few nodes is a serial chain of chunks per node while most
// CUs idle, and each chunk then runs on twice the MFMA pipes of one
// workgroup. Workgroup x of a level launch takes a head and a column block;
// with Hv a multiple of 8 the two blocks of a head are 8 apart (same XCD and
// L2, dispatched together).
constexpr int SCAN_COLS = 64;
constexpr int kScanSplit = GD / SCAN_COLS;
__device__ __forceinline__ void scan_block(const GdnDev& p, int& h, int& c0) {
    const int bx = blockIdx.x;
    int cs;
    if ((p.hv & 7) == 0) {
        h = ((bx >> 4) << 3) | (bx & 7);
        cs = (bx >> 3) & 1;
    } else {
        h = bx >> 1;
        cs = bx & 1;
    }
    c0 = SCAN_COLS * cs;
}

// Wave w owns value columns c0 + 16w .. +15 of one (node, v head): its
// 128 x 16 state slice lives in eight 16 x 16 accumulator tiles (rows
// 16 rb + 4 (l >> 4) + v) for the whole node. Per chunk (two 16-token tiles):
//   V' = U - W S,  qS  (A = W / q^ rows from LDS, B = S from registers)
//   O = e^G qS + A V'  (B = V' from registers)
//   S <- e^{G_L} S + (k^ e^{G_L - G})^T V'  (A = k~ from LDS, B = V')
// out may be null (the backward's recompute); chunk_sin / chunk_vp, when
// given, receive each chunk's initial state and V' ([n_chunks, Hv, 128, 128]
// and [n_chunks, Hv, 32, 128] floats).
// TRUNC (the reference's per-node correction): V' = U - W S0 with S0 the
// node's initial state for every chunk of the node. A first pass over the
// node's chunks, while the state registers still hold S0, replaces each
// chunk's U by its V' in the workspace; the scan proper then reads V' there.
template <typename TIn, bool TRUNC>
__global__ __launch_bounds__(GT) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_scan_cols_kernel(GdnDev p, int lvl_begin, float* __restrict__ ws,
                                                      TIn* __restrict__ out, float* __restrict__ states,
                                                      float* __restrict__ chunk_sin, float* __restrict__ chunk_vp) {
    __shared__ __attribute__((aligned(16))) ScanLds L;
    const int node = p.level_nodes[lvl_begin + blockIdx.y];
    if (node < 0 || node >= p.n_nodes) return;
    int h, cb;
    scan_block(p, h, cb);
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, c16 = lane & 15, g4 = 4 * (lane >> 4);
    const int j = cb + 16 * wave + c16;                                   // this lane's value column
    const int jt = cb + 16 * wave;                                        // the wave's first column
    const int start = p.node_start[node], len = p.node_len[node], chunk0 = p.node_chunk0[node];
    int par = p.parent[node];
    if (start < 0 || len < 0 || start > p.n_tokens - len) return;        // malformed node: skipped
    if (chunk0 < 0 || chunk0 > p.n_chunks - tt_cdiv(len, GC)) return;
    if (par >= node || par < -1) par = -1;                               // parents precede children

    // S0: the parent's final state; a root's is the initial state (or zero).
    const float* s0 = par >= 0 ? states + ((size_t)par * p.hv + h) * GD * GD
                               : (p.init ? p.init + (size_t)h * GD * GD : nullptr);
    f32x4 S[8];
    if (s0) {
#pragma unroll
        for (int rb = 0; rb < 8; ++rb) S[rb] = load_t16(s0 + jt + 16 * rb * GD, lane);
    } else {
#pragma unroll
        for (int rb = 0; rb < 8; ++rb) S[rb] = (f32x4){};
    }

    if constexpr (TRUNC) {
        // V' = U - W S0 for every chunk (with S0 zero: V' = U as it is).
        for (int c0 = 0; s0 && c0 < len; c0 += GC) {
            float* cw = ws + ((size_t)(chunk0 + c0 / GC) * p.hv + h) * kWsChunk;
            __syncthreads();   // readers of the previous chunk's W are done
            {
                const int i = t >> 3, d0 = 16 * (t & 7);
#pragma unroll
                for (int e = 0; e < 16; e += 4)
                    *(f32x4*)&L.W[i * RS + d0 + e] = *(const f32x4*)(cw + kWsW + i * GD + d0 + e);
            }
            f32x4 vp[2];
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) vp[tb] = load_t16(cw + kWsU + 16 * tb * GD + jt, lane);
            __syncthreads();
#pragma unroll
            for (int rb = 0; rb < 8; ++rb)
#pragma unroll
                for (int tb = 0; tb < 2; ++tb) {
                    const f32x4 wv = *(const f32x4*)&L.W[(16 * tb + c16) * RS + 16 * rb + g4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) vp[tb] = mfma16_f32(-wv[v], S[rb][v], vp[tb]);
                }
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) store_t16(cw + kWsU + 16 * tb * GD + jt, lane, vp[tb]);   // read back by this lane
        }
    }

    // U (TRUNC: V', written by the first pass) and the state-independent
    // chunk terms, one chunk ahead.
    const int n_ch = tt_cdiv(len, GC);
    ScanAhead<TIn> nx;
    {
        const float* cw = ws + ((size_t)chunk0 * p.hv + h) * kWsChunk;
        scan_fetch_rows<TIn, !TRUNC>(p, cw, start, min(GC, len), h, nx);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) nx.x[tb] = load_t16(cw + kWsU + 16 * tb * GD + jt, lane);
    }
    for (int ci = 0; ci < n_ch; ++ci) {
        const int c0 = GC * ci, Lc = min(GC, len - c0);
        const size_t ch = (size_t)(chunk0 + ci) * p.hv + h;
        if (chunk_sin) {
            float* sp = chunk_sin + ch * GD * GD + jt;
#pragma unroll
            for (int rb = 0; rb < 8; ++rb) store_t16(sp + 16 * rb * GD, lane, S[rb]);
        }
        __syncthreads();   // readers of the previous chunk's tiles are done
        scan_stage_rows<TIn, !TRUNC, false>(p, nx, L.Q, L.K, L.W, L.A, L.G);
        f32x4 vp[2], qs[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            vp[tb] = nx.x[tb];
            qs[tb] = (f32x4){};
        }
        if (ci + 1 < n_ch) {
            const float* cw = ws + (ch + p.hv) * kWsChunk;
            scan_fetch_rows<TIn, !TRUNC>(p, cw, start + c0 + GC, min(GC, len - c0 - GC), h, nx);
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) nx.x[tb] = load_t16(cw + kWsU + 16 * tb * GD + jt, lane);
        }
        __syncthreads();

        // V' = U - W S and q^ S over the 128 state rows as four partial sums of
        // two row tiles each, added in order: the partition of the row layout's
        // waves (gdn_scan_rows_kernel), so both layouts give the same bits.
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4) {
            f32x4 pv[2] = {}, pq[2] = {};
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int rb = 2 * w4 + r;
#pragma unroll
                for (int tb = 0; tb < 2; ++tb) {
                    const int ro = (16 * tb + c16) * RS + 16 * rb + g4;
                    const f32x4 qv = *(const f32x4*)&L.Q[ro];
                    if constexpr (!TRUNC) {
                        const f32x4 wv = *(const f32x4*)&L.W[ro];
#pragma unroll
                        for (int v = 0; v < 4; ++v) pv[tb] = mfma16_f32(-wv[v], S[rb][v], pv[tb]);
                    }
#pragma unroll
                    for (int v = 0; v < 4; ++v) pq[tb] = mfma16_f32(qv[v], S[rb][v], pq[tb]);
                    __builtin_amdgcn_sched_barrier(0);   // operand reads one step ahead at most (registers)
                }
            }
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                if constexpr (!TRUNC) vp[tb] += pv[tb];
                qs[tb] += pq[tb];
            }
        }
        if (chunk_vp) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) store_t16(chunk_vp + ch * GC * GD + 16 * tb * GD + jt, lane, vp[tb]);
        }
        // O = e^G (q^ S) + A V', token tile by token tile.
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            f32x4 o;
#pragma unroll
            for (int v = 0; v < 4; ++v) o[v] = qs[tb][v] * expf(L.G[16 * tb + g4 + v]);
#pragma unroll
            for (int tb2 = 0; tb2 < 2; ++tb2) {
                const f32x4 av = *(const f32x4*)&L.A[(16 * tb + c16) * MS + 16 * tb2 + g4];
#pragma unroll
                for (int v = 0; v < 4; ++v) o = mfma16_f32(av[v], vp[tb2][v], o);
            }
            if (out) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int i = 16 * tb + g4 + v;
                    if (i < Lc) out[((int64_t)(start + c0 + i) * p.hv + h) * GD + j] = (TIn)o[v];
                }
            }
        }
        // S <- e^{G_L} S + k~^T V': A[state row][token] = k~[token][state row].
        {
            const float el = expf(L.G[GC - 1]);
#pragma unroll
            for (int rb = 0; rb < 8; ++rb) {
                S[rb] *= el;
#pragma unroll
                for (int tb = 0; tb < 2; ++tb) {
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        S[rb] = mfma16_f32(L.K[(16 * tb + g4 + v) * RS + 16 * rb + c16], vp[tb][v], S[rb]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    }

    // Final state of the node (the initial state of its children).
    float* sp = states + ((size_t)node * p.hv + h) * GD * GD + jt;
#pragma unroll
    for (int rb = 0; rb < 8; ++rb) store_t16(sp + 16 * rb * GD, lane, S[rb]);
}

// Row layout of the level scans, for levels of few nodes (the exact rule
// only): a workgroup takes 16 value columns of one (node, v head), eight
// workgroups per pair, and its wave w the state rows 32w .. 32w+31 of them.
// The products over the state rows (W S and q^ S) are summed over the four
// waves through LDS, in wave order; every wave then updates its own rows. A
// chunk costs each wave about a quarter of the column layout's MFMAs, for
// four times the workgroups: a level with few nodes runs a serial chain of
// chunks on a mostly idle chip, and that chain gets shorter.
constexpr int ROWS_COLS = 16;
constexpr int kRowsSplit = GD / ROWS_COLS;
__device__ __forceinline__ void rows_block(const GdnDev& p, int& h, int& c0) {
    const int bx = blockIdx.x;
    int cs;
    if ((p.hv & 7) == 0) {   // the eight column blocks of a head on one XCD (same L2)
        h = ((bx >> 6) << 3) | (bx & 7);
        cs = (bx >> 3) & 7;
    } else {
        h = bx >> 3;
        cs = bx & 7;
    }
    c0 = ROWS_COLS * cs;
}

struct ScanRowsLds {
    ScanLds T;
    f32x4 P[4][2][2][64];   // per wave: its partial W S and q^ S, both token tiles, lane-major
};

// As gdn_scan_cols_kernel (exact rule), in the row layout: wave w holds the
// 32 x 16 slice S[32w .., c0 ..] in two 16 x 16 accumulator tiles.
template <typename TIn>
__global__ __launch_bounds__(GT) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_scan_rows_kernel(GdnDev p, int lvl_begin, float* __restrict__ ws,
                                                      TIn* __restrict__ out, float* __restrict__ states,
                                                      float* __restrict__ chunk_sin, float* __restrict__ chunk_vp) {
    __shared__ __attribute__((aligned(16))) ScanRowsLds L;
    const int node = p.level_nodes[lvl_begin + blockIdx.y];
    if (node < 0 || node >= p.n_nodes) return;
    int h, cb;
    rows_block(p, h, cb);
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, c16 = lane & 15, g4 = 4 * (lane >> 4);
    const int j = cb + c16;                                               // this lane's value column
    const int rb0 = 2 * wave;                                             // the wave's first row tile
    const int start = p.node_start[node], len = p.node_len[node], chunk0 = p.node_chunk0[node];
    int par = p.parent[node];
    if (start < 0 || len < 0 || start > p.n_tokens - len) return;        // malformed node: skipped
    if (chunk0 < 0 || chunk0 > p.n_chunks - tt_cdiv(len, GC)) return;
    if (par >= node || par < -1) par = -1;                               // parents precede children

    const float* s0 = par >= 0 ? states + ((size_t)par * p.hv + h) * GD * GD
                               : (p.init ? p.init + (size_t)h * GD * GD : nullptr);
    f32x4 S[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) S[r] = s0 ? load_t16(s0 + cb + 16 * (rb0 + r) * GD, lane) : (f32x4){};

    const int n_ch = tt_cdiv(len, GC);
    ScanAhead<TIn> nx;
    {
        const float* cw = ws + ((size_t)chunk0 * p.hv + h) * kWsChunk;
        scan_fetch_rows<TIn, true>(p, cw, start, min(GC, len), h, nx);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) nx.x[tb] = load_t16(cw + kWsU + 16 * tb * GD + cb, lane);
    }
    for (int ci = 0; ci < n_ch; ++ci) {
        const int c0 = GC * ci, Lc = min(GC, len - c0);
        const size_t ch = (size_t)(chunk0 + ci) * p.hv + h;
        if (chunk_sin) {
            float* sp = chunk_sin + ch * GD * GD + cb;
#pragma unroll
            for (int r = 0; r < 2; ++r) store_t16(sp + 16 * (rb0 + r) * GD, lane, S[r]);
        }
        __syncthreads();   // readers of the previous chunk's tiles and partials are done
        scan_stage_rows<TIn, true, false>(p, nx, L.T.Q, L.T.K, L.T.W, L.T.A, L.T.G);
        f32x4 vp[2], qs[2], pv[2], pq[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            vp[tb] = nx.x[tb];
            pv[tb] = pq[tb] = (f32x4){};
        }
        if (ci + 1 < n_ch) {
            const float* cw = ws + (ch + p.hv) * kWsChunk;
            scan_fetch_rows<TIn, true>(p, cw, start + c0 + GC, min(GC, len - c0 - GC), h, nx);
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) nx.x[tb] = load_t16(cw + kWsU + 16 * tb * GD + cb, lane);
        }
        __syncthreads();

        // this wave's rows of -W S and q^ S
#pragma unroll
        for (int r = 0; r < 2; ++r) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
                const int ro = (16 * tb + c16) * RS + 16 * (rb0 + r) + g4;
                const f32x4 wv = *(const f32x4*)&L.T.W[ro];
                const f32x4 qv = *(const f32x4*)&L.T.Q[ro];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    pv[tb] = mfma16_f32(-wv[v], S[r][v], pv[tb]);
                    pq[tb] = mfma16_f32(qv[v], S[r][v], pq[tb]);
                }
            }
        }
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            L.P[wave][0][tb][lane] = pv[tb];
            L.P[wave][1][tb][lane] = pq[tb];
        }
        __syncthreads();
        // V' = U - W S and q^ S, the partials summed in wave order
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            qs[tb] = (f32x4){};
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                vp[tb] += L.P[w][0][tb][lane];
                qs[tb] += L.P[w][1][tb][lane];
            }
        }
        if (chunk_vp && wave == 0) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) store_t16(chunk_vp + ch * GC * GD + 16 * tb * GD + cb, lane, vp[tb]);
        }
        // O = e^G (q^ S) + A V': waves 0 and 1 take one token tile each
        if (wave < 2) {
            const int tb = wave;
            f32x4 o;
#pragma unroll
            for (int v = 0; v < 4; ++v) o[v] = qs[tb][v] * expf(L.T.G[16 * tb + g4 + v]);
#pragma unroll
            for (int tb2 = 0; tb2 < 2; ++tb2) {
                const f32x4 av = *(const f32x4*)&L.T.A[(16 * tb + c16) * MS + 16 * tb2 + g4];
#pragma unroll
                for (int v = 0; v < 4; ++v) o = mfma16_f32(av[v], vp[tb2][v], o);
            }
            if (out) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int i = 16 * tb + g4 + v;
                    if (i < Lc) out[((int64_t)(start + c0 + i) * p.hv + h) * GD + j] = (TIn)o[v];
                }
            }
        }
        // S <- e^{G_L} S + k~^T V' on this wave's rows
        const float el = expf(L.T.G[GC - 1]);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            S[r] *= el;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    S[r] = mfma16_f32(L.T.K[(16 * tb + g4 + v) * RS + 16 * (rb0 + r) + c16], vp[tb][v], S[r]);
        }
    }

    float* sp = states + ((size_t)node * p.hv + h) * GD * GD + cb;
#pragma unroll
    for (int r = 0; r < 2; ++r) store_t16(sp + 16 * (rb0 + r) * GD, lane, S[r]);
}

// ----------------------------------------------------------------------------
// backward
// ----------------------------------------------------------------------------
// The backward recomputes the forward (prep + level scans, keeping each
// chunk's initial state S and V'), then:
//  * gdn_rscan_cols_kernel — reverse level scan (deepest level first) of dS, the
//    gradient of the state after a chunk, per (node, v head), on fp32 MFMA:
//      dV' = A^T dO + (e^{G_L - G} k^) dS,
//      dS <- e^{G_L} dS + (e^G q^)^T dO - W^T dV'.
//    A node's last chunk starts from the incoming gradient of its final
//    state (if the caller gives one) plus the sum of its children's dS at
//    entry.
//  * gdn_init_grad_kernel — when the initial state's gradient is wanted: the
//    sum of the roots' dS at entry.
//  * gdn_bwd_state_kernel — per (chunk, v head), the products with the
//    128 x 128 states: X = dO S^T, dW = -dV' S^T, dK~ = V' dS^T, <S, dS>.
//  * gdn_bwd_chunk_kernel — per (chunk, q/k head, looping over its v heads),
//    everything else: the chunk's 32 x 32 algebra (A, T = (I - N)^-1, N),
//    dv, dbeta, dg (reverse cumulative sum of dG within the chunk), and
//    dq, dk summed over the v heads of the group, then through the l2 norm.


struct RscanLds {
    float Q[GC * RS];     // e^G q^ * scale
    float K[GC * RS];     // e^{G_L - G} k^
    float W[GC * RS];
    float A[GC * MS];
    float G[GC];
};

// Column layout as gdn_scan_cols_kernel (scan_block). Wave w owns value
// columns c0 + 16w .. +15: its 128 x 16 slice of dS lives in eight 16 x 16
// accumulator tiles, dO of the chunk is loaded in accumulator layout (rows =
// tokens, two 16-token tiles), and dV' is produced in it, so all three are
// used straight from registers as MFMA B operands.
// TRUNC (V' = U - W S0 with the node's initial state S0): the walk leaves out
// the W term, and a second pass over the node's chunks subtracts
// sum_c W_c^T dV'_c from the state gradient at the node's entry.
template <typename TIn, bool TRUNC>
__global__ __launch_bounds__(GT) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_rscan_cols_kernel(
        GdnDev p, int lvl_begin, const float* __restrict__ ws, const TIn* __restrict__ d_o, int64_t do_st,
        int64_t do_sh, float* __restrict__ chunk_dso, float* __restrict__ chunk_dvp, float* __restrict__ node_dsin) {
    __shared__ __attribute__((aligned(16))) RscanLds L;
    const int node = p.level_nodes[lvl_begin + blockIdx.y];
    if (node < 0 || node >= p.n_nodes) return;
    int h, cb;
    scan_block(p, h, cb);
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, c16 = lane & 15, g4 = 4 * (lane >> 4);
    const int j = cb + 16 * wave + c16;
    const int jt = cb + 16 * wave;
    const int start = p.node_start[node], len = p.node_len[node], chunk0 = p.node_chunk0[node];
    if (start < 0 || len < 1 || start > p.n_tokens - len) return;        // malformed node: skipped
    if (chunk0 < 0 || chunk0 > p.n_chunks - tt_cdiv(len, GC)) return;

    // dS after the node: its state's incoming gradient, if any, plus the sum
    // over its children of their dS at entry.
    f32x4 dS[8];
    if (p.d_states && (!p.d_states_last || node == p.n_nodes - 1)) {
        const float* sp = p.d_states + ((size_t)(p.d_states_last ? 0 : node) * p.hv + h) * GD * GD + jt;
#pragma unroll
        for (int rb = 0; rb < 8; ++rb) dS[rb] = load_t16(sp + 16 * rb * GD, lane);
    } else {
#pragma unroll
        for (int rb = 0; rb < 8; ++rb) dS[rb] = (f32x4){};
    }
    {
        const int c_lo = max(p.child_off[node], 0), c_hi = min(p.child_off[node + 1], p.n_nodes);
        for (int ci = c_lo; ci < c_hi; ++ci) {
            const int child = p.child[ci];
            if (child <= node || child >= p.n_nodes) continue;          // children follow their parent
            const float* sp = node_dsin + ((size_t)child * p.hv + h) * GD * GD + jt;
#pragma unroll
            for (int rb = 0; rb < 8; ++rb) dS[rb] += load_t16(sp + 16 * rb * GD, lane);
        }
    }

    // The chunk terms and dO rows of a chunk, one chunk ahead (the walk runs
    // backwards).
    const int n_ch = tt_cdiv(len, GC);
    auto fetch = [&](int ci, ScanAhead<TIn>& x) {
        const int c0 = GC * ci, Lc = min(GC, len - c0);
        const float* cw = ws + ((size_t)(chunk0 + ci) * p.hv + h) * kWsChunk;
        scan_fetch_rows<TIn, !TRUNC>(p, cw, start + c0, Lc, h, x);
        const TIn* base = d_o + (int64_t)(start + c0) * do_st + (int64_t)h * do_sh + j;
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {   // dO[token 16 tb + 4 (l >> 4) + v][j], zero past the chunk
                const int i = 16 * tb + g4 + v;
                x.x[tb][v] = i < Lc ? (float)base[(int64_t)i * do_st] : 0.0f;
            }
    };
    ScanAhead<TIn> nx;
    fetch(n_ch - 1, nx);
    for (int ci = n_ch - 1; ci >= 0; --ci) {
        const int c0 = GC * ci, Lc = min(GC, len - c0);
        const size_t chn = (size_t)(chunk0 + ci) * p.hv + h;
        {   // the gradient of this chunk's output state
            float* sp = chunk_dso + chn * GD * GD + jt;
#pragma unroll
            for (int rb = 0; rb < 8; ++rb) store_t16(sp + 16 * rb * GD, lane, dS[rb]);
        }
        __syncthreads();   // readers of the previous chunk's tiles are done
        scan_stage_rows<TIn, !TRUNC, true>(p, nx, L.Q, L.K, L.W, L.A, L.G);
        const f32x4 dov[2] = {nx.x[0], nx.x[1]};
        if (ci > 0) fetch(ci - 1, nx);
        __syncthreads();

        // dV' = A^T dO + k~ dS as four partial sums added in order, partial w4
        // holding the A^T dO term of token tiles (w4 / 2, w4 % 2) and the
        // state rows 32 w4 .. +31: the partition of the row layout's waves
        // (gdn_rscan_rows_kernel), so both layouts give the same bits.
        f32x4 dv[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            dv[tb] = (f32x4){};
#pragma unroll
            for (int w4 = 0; w4 < 4; ++w4) {
                f32x4 pd = {};
                if (tb == (w4 >> 1)) {
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        pd = mfma16_f32(L.A[(16 * (w4 & 1) + g4 + v) * MS + 16 * tb + c16], dov[w4 & 1][v], pd);
                }
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const int rb = 2 * w4 + r;
                    const f32x4 kv = *(const f32x4*)&L.K[(16 * tb + c16) * RS + 16 * rb + g4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) pd = mfma16_f32(kv[v], dS[rb][v], pd);
                    __builtin_amdgcn_sched_barrier(0);
                }
                dv[tb] += pd;
            }
        }
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) store_t16(chunk_dvp + chn * GC * GD + 16 * tb * GD + jt, lane, dv[tb]);

        // dS <- e^{G_L} dS + (e^G q^)^T dO - W^T dV'
        const float el = expf(L.G[GC - 1]);
#pragma unroll
        for (int rb = 0; rb < 8; ++rb) {
            dS[rb] *= el;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int ro = (16 * tb + g4 + v) * RS + 16 * rb + c16;
                    dS[rb] = mfma16_f32(L.Q[ro], dov[tb][v], dS[rb]);
                    if constexpr (!TRUNC) dS[rb] = mfma16_f32(-L.W[ro], dv[tb][v], dS[rb]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    if constexpr (TRUNC) {
        for (int ci = 0; ci < tt_cdiv(len, GC); ++ci) {
            const size_t chn = (size_t)(chunk0 + ci) * p.hv + h;
            const float* cw = ws + chn * kWsChunk;
            __syncthreads();   // readers of the previous chunk's W are done
            {
                const int i = t >> 3, d0 = 16 * (t & 7);
#pragma unroll
                for (int e = 0; e < 16; e += 4)
                    *(f32x4*)&L.W[i * RS + d0 + e] = *(const f32x4*)(cw + kWsW + i * GD + d0 + e);
            }
            f32x4 dv[2];   // this lane's own writes
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) dv[tb] = load_t16(chunk_dvp + chn * GC * GD + 16 * tb * GD + jt, lane);
            __syncthreads();
#pragma unroll
            for (int rb = 0; rb < 8; ++rb)
#pragma unroll
                for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        dS[rb] = mfma16_f32(-L.W[(16 * tb + g4 + v) * RS + 16 * rb + c16], dv[tb][v], dS[rb]);
        }
    }
    // dS at the node's entry, summed into its parent by the next (shallower) level.
    float* sp = node_dsin + ((size_t)node * p.hv + h) * GD * GD + jt;
#pragma unroll
    for (int rb = 0; rb < 8; ++rb) store_t16(sp + 16 * rb * GD, lane, dS[rb]);
}

struct RscanRowsLds {
    RscanLds T;
    f32x4 P[4][2][64];   // per wave: its partial dV', both token tiles, lane-major
};

// As gdn_rscan_cols_kernel (exact rule), in the row layout of
// gdn_scan_rows_kernel: wave w holds dS[32w .., c0 ..]. dV' = A^T dO + k~ dS
// is summed over the waves' rows through LDS, in wave order (wave w also adds
// the A^T dO term of token tiles (w / 2, w % 2)); every wave then updates its
// rows of dS.
template <typename TIn>
__global__ __launch_bounds__(GT) __attribute__((amdgpu_waves_per_eu(2, 2))) void gdn_rscan_rows_kernel(
        GdnDev p, int lvl_begin, const float* __restrict__ ws, const TIn* __restrict__ d_o, int64_t do_st,
        int64_t do_sh, float* __restrict__ chunk_dso, float* __restrict__ chunk_dvp, float* __restrict__ node_dsin) {
    __shared__ __attribute__((aligned(16))) RscanRowsLds L;
    const int node = p.level_nodes[lvl_begin + blockIdx.y];
    if (node < 0 || node >= p.n_nodes) return;
    int h, cb;
    rows_block(p, h, cb);
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, c16 = lane & 15, g4 = 4 * (lane >> 4);
    const int j = cb + c16;
    const int rb0 = 2 * wave;
    const int start = p.node_start[node], len = p.node_len[node], chunk0 = p.node_chunk0[node];
    if (start < 0 || len < 1 || start > p.n_tokens - len) return;        // malformed node: skipped
    if (chunk0 < 0 || chunk0 > p.n_chunks - tt_cdiv(len, GC)) return;

    f32x4 dS[2];
    if (p.d_states && (!p.d_states_last || node == p.n_nodes - 1)) {
        const float* sp = p.d_states + ((size_t)(p.d_states_last ? 0 : node) * p.hv + h) * GD * GD + cb;
#pragma unroll
        for (int r = 0; r < 2; ++r) dS[r] = load_t16(sp + 16 * (rb0 + r) * GD, lane);
    } else {
#pragma unroll
        for (int r = 0; r < 2; ++r) dS[r] = (f32x4){};
    }
    {
        const int c_lo = max(p.child_off[node], 0), c_hi = min(p.child_off[node + 1], p.n_nodes);
        for (int ci = c_lo; ci < c_hi; ++ci) {
            const int child = p.child[ci];
            if (child <= node || child >= p.n_nodes) continue;          // children follow their parent
            const float* sp = node_dsin + ((size_t)child * p.hv + h) * GD * GD + cb;
#pragma unroll
            for (int r = 0; r < 2; ++r) dS[r] += load_t16(sp + 16 * (rb0 + r) * GD, lane);
        }
    }

    const int n_ch = tt_cdiv(len, GC);
    auto fetch = [&](int ci, ScanAhead<TIn>& x) {
        const int c0 = GC * ci, Lc = min(GC, len - c0);
        const float* cw = ws + ((size_t)(chunk0 + ci) * p.hv + h) * kWsChunk;
        scan_fetch_rows<TIn, true>(p, cw, start + c0, Lc, h, x);
        const TIn* base = d_o + (int64_t)(start + c0) * do_st + (int64_t)h * do_sh + j;
#pragma unroll
        for (int tb = 0; tb < 2; ++tb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {   // dO[token 16 tb + 4 (l >> 4) + v][j], zero past the chunk
                const int i = 16 * tb + g4 + v;
                x.x[tb][v] = i < Lc ? (float)base[(int64_t)i * do_st] : 0.0f;
            }
    };
    ScanAhead<TIn> nx;
    fetch(n_ch - 1, nx);
    const int atb = wave >> 1, atb2 = wave & 1;   // this wave's A^T dO term
    for (int ci = n_ch - 1; ci >= 0; --ci) {
        const size_t chn = (size_t)(chunk0 + ci) * p.hv + h;
        {
            float* sp = chunk_dso + chn * GD * GD + cb;
#pragma unroll
            for (int r = 0; r < 2; ++r) store_t16(sp + 16 * (rb0 + r) * GD, lane, dS[r]);
        }
        __syncthreads();   // readers of the previous chunk's tiles and partials are done
        scan_stage_rows<TIn, true, true>(p, nx, L.T.Q, L.T.K, L.T.W, L.T.A, L.T.G);
        const f32x4 dov[2] = {nx.x[0], nx.x[1]};
        if (ci > 0) fetch(ci - 1, nx);
        __syncthreads();

        f32x4 pd[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            pd[tb] = (f32x4){};
            if (tb == atb) {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    pd[tb] = mfma16_f32(L.T.A[(16 * atb2 + g4 + v) * MS + 16 * tb + c16], dov[atb2][v], pd[tb]);
            }
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const f32x4 kv = *(const f32x4*)&L.T.K[(16 * tb + c16) * RS + 16 * (rb0 + r) + g4];
#pragma unroll
                for (int v = 0; v < 4; ++v) pd[tb] = mfma16_f32(kv[v], dS[r][v], pd[tb]);
            }
            L.P[wave][tb][lane] = pd[tb];
        }
        __syncthreads();
        f32x4 dv[2];
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
            dv[tb] = (f32x4){};
#pragma unroll
            for (int w = 0; w < 4; ++w) dv[tb] += L.P[w][tb][lane];
        }
        if (wave == 0) {
#pragma unroll
            for (int tb = 0; tb < 2; ++tb) store_t16(chunk_dvp + chn * GC * GD + 16 * tb * GD + cb, lane, dv[tb]);
        }

        // dS <- e^{G_L} dS + (e^G q^)^T dO - W^T dV' on this wave's rows
        const float el = expf(L.T.G[GC - 1]);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            dS[r] *= el;
#pragma unroll
            for (int tb = 0; tb < 2; ++tb)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int ro = (16 * tb + g4 + v) * RS + 16 * (rb0 + r) + c16;
                    dS[r] = mfma16_f32(L.T.Q[ro], dov[tb][v], dS[r]);
                    dS[r] = mfma16_f32(-L.T.W[ro], dv[tb][v], dS[r]);
                }
        }
    }
    float* sp = node_dsin + ((size_t)node * p.hv + h) * GD * GD + cb;
#pragma unroll
    for (int r = 0; r < 2; ++r) store_t16(sp + 16 * (rb0 + r) * GD, lane, dS[r]);
}

// Gradient of the initial state: the sum over the roots, in node order (the
// order in which a node's children's terms are summed), of their state
// gradient at entry. Thread: four consecutive floats of one v head's
// 128 x 128 block.
__global__ __launch_bounds__(GT) void gdn_init_grad_kernel(GdnDev p, const float* __restrict__ node_dsin) {
    const int h = blockIdx.y;
    const int e = 4 * (blockIdx.x * GT + threadIdx.x);
    f32x4 acc = {};
    for (int node = 0; node < p.n_nodes; ++node) {
        const int par = p.parent[node];
        if (par >= 0 && par < node) continue;   // roots only, by the forward scan's rule
        acc += *(const f32x4*)(node_dsin + ((size_t)node * p.hv + h) * GD * GD + e);
    }
    *(f32x4*)(p.d_init + (size_t)h * GD * GD + e) = acc;
}

// State products on fp32 MFMA. The contraction (value dimension, 128) runs in
// four 32-column chunks; per chunk the block stages, with coalesced loads,
// columns v0..v0+31 of all 128 rows of S and dS and of the 32 rows of dO, dV'
// and V' into LDS rows of SCS = 34 floats: the MFMA operand reads (lane =
// row, one float per lane, two adjacent columns per step) then reach all 64
// banks once. Wave w produces columns 32w .. 32w+31 of X, dW and dK~ (rows of
// S / dS 32w .. 32w+31) as accumulators.
constexpr int SCS = 34;
struct StateGradLds {     // gdn_dw_s0_kernel: one chunk of S0 and of dV'
    float S[GD * SCS];
    float A1[GC * SCS];
    float A2[GC * SCS];
    float red[GT / 64];
};

// One 32-column slice of the value dimension of both S and dS (all 128 rows)
// and the matching columns of dO, dV' and V', staged together: every input
// is read once.
struct StatePairLds {
    float S[GD * SCS];
    float dS[GD * SCS];
    float A1[GC * SCS];   // dO
    float A2[GC * SCS];   // dV'
    float A3[GC * SCS];   // V'
    float red[GT / 64];
};

// Registers of one slice: S and dS at the same positions (thread t: row
// t >> 1, columns 16 (t & 1) .. +15) and the 32-row tiles (row t >> 3,
// columns 4 (t & 7) .. +3).
template <typename TIn>
struct StateChunk {
    float s[16];
    float ds[16];
    f32x4 vp, dvp;
    u32x4 d;        // dO as loaded (bf16: two per word; converted when committed)
};

// X = dO S^T, dW = -dV' S^T, dK~ = V' dS^T ([GC x GD] each) and <S, dS>.
template <typename TIn>
__global__ __launch_bounds__(GT) void gdn_bwd_state_kernel(GdnDev p, const TIn* __restrict__ d_o, int64_t do_st,
                                                           int64_t do_sh, const float* __restrict__ chunk_sin,
                                                           const float* __restrict__ chunk_dso,
                                                           const float* __restrict__ chunk_vp,
                                                           const float* __restrict__ chunk_dvp,
                                                           float* __restrict__ xo, float* __restrict__ dwo,
                                                           float* __restrict__ dkto, float* __restrict__ sdot) {
    __shared__ __attribute__((aligned(16))) StatePairLds L;
    const int c = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    int start, len;
    if (!chunk_span(p, c, start, len)) return;
    const size_t chn = (size_t)c * p.hv + h;
    const int wave = t >> 6, lane = t & 63, col = lane & 31, half = lane >> 5;
    const float* Sin = chunk_sin + chn * GD * GD;
    const float* dSo = chunk_dso + chn * GD * GD;
    const float* dVp = chunk_dvp + chn * GC * GD;
    const float* Vp = chunk_vp + chn * GC * GD;
    const int sr = t >> 1, sc = 16 * (t & 1);      // S / dS staging: row, first column
    const int ar = t >> 3, ac = 4 * (t & 7);       // 32-row tiles: row, first column
    // rows past the chunk's length read its last row and are zeroed at commit
    const TIn* dor = d_o + (int64_t)(start + min(ar, len - 1)) * do_st + (int64_t)h * do_sh;
    const bool arow_in = ar < len;

    auto fetch = [&](int k, StateChunk<TIn>& r) {
        const int v0 = GC * k;
        const int so = sr * GD + v0 + sc;
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
            const f32x4 x4 = *(const f32x4*)(Sin + so + e);
            const f32x4 y4 = *(const f32x4*)(dSo + so + e);
            r.s[e] = x4[0]; r.s[e + 1] = x4[1]; r.s[e + 2] = x4[2]; r.s[e + 3] = x4[3];
            r.ds[e] = y4[0]; r.ds[e + 1] = y4[1]; r.ds[e + 2] = y4[2]; r.ds[e + 3] = y4[3];
        }
        if constexpr (sizeof(TIn) == 2) {
            const u32x2 raw = *(const u32x2*)(dor + v0 + ac);
            r.d = (u32x4){raw[0], raw[1], 0u, 0u};
        } else {
            r.d = *(const u32x4*)(dor + v0 + ac);
        }
        r.dvp = *(const f32x4*)(dVp + ar * GD + v0 + ac);
        r.vp = *(const f32x4*)(Vp + ar * GD + v0 + ac);
    };
    auto commit = [&](const StateChunk<TIn>& r) {
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
            *(float2*)&L.S[sr * SCS + sc + e] = (float2){r.s[e], r.s[e + 1]};
            *(float2*)&L.dS[sr * SCS + sc + e] = (float2){r.ds[e], r.ds[e + 1]};
        }
        const float z = arow_in ? 1.0f : 0.0f;   // dO rows past the chunk are zero
        float dv4[4];
        if constexpr (sizeof(TIn) == 2) {   // bf16 -> fp32: the high half of a float
            dv4[0] = __uint_as_float(r.d[0] << 16);
            dv4[1] = __uint_as_float(r.d[0] & 0xffff0000u);
            dv4[2] = __uint_as_float(r.d[1] << 16);
            dv4[3] = __uint_as_float(r.d[1] & 0xffff0000u);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) dv4[e] = __uint_as_float(r.d[e]);
        }
        *(float2*)&L.A1[ar * SCS + ac] = (float2){z * dv4[0], z * dv4[1]};
        *(float2*)&L.A1[ar * SCS + ac + 2] = (float2){z * dv4[2], z * dv4[3]};
        *(float2*)&L.A2[ar * SCS + ac] = (float2){r.dvp[0], r.dvp[1]};
        *(float2*)&L.A2[ar * SCS + ac + 2] = (float2){r.dvp[2], r.dvp[3]};
        *(float2*)&L.A3[ar * SCS + ac] = (float2){r.vp[0], r.vp[1]};
        *(float2*)&L.A3[ar * SCS + ac + 2] = (float2){r.vp[2], r.vp[3]};
    };

    f32x16 x = (f32x16){}, w = (f32x16){}, kt = (f32x16){};
    float sd = 0.0f;
    const float* brow = &L.S[(32 * wave + col) * SCS + half];    // B: S row 32w + col, columns 2 step + half
    const float* dbrow = &L.dS[(32 * wave + col) * SCS + half];  // B: the same row of dS
    const float* arow1 = &L.A1[col * SCS + half];                // A: row col, columns 2 step + half
    const float* arow2 = &L.A2[col * SCS + half];
    const float* arow3 = &L.A3[col * SCS + half];
    StateChunk<TIn> cur, nxt;
    fetch(0, cur);
#pragma unroll 1
    for (int k = 0; k < 4; ++k) {
        __syncthreads();   // the previous slice's readers are done
        commit(cur);
#pragma unroll
        for (int e = 0; e < 16; ++e) sd = fmaf(cur.s[e], cur.ds[e], sd);   // <S, dS>, this thread's share
        __syncthreads();
        if (k + 1 < 4) fetch(k + 1, nxt);
#pragma unroll
        for (int st = 0; st < GC / 2; ++st) {
            const float b = brow[2 * st];
            x = mfma_f32(arow1[2 * st], b, x);
            w = mfma_f32(arow2[2 * st], b, w);
            kt = mfma_f32(arow3[2 * st], dbrow[2 * st], kt);
        }
        cur = nxt;
    }
    // Accumulator element r: row acc_row(r, half) (token), column 32w + col.
    store_acc<0>(acc_mat(xo + chn * GC * GD, GC, half, 32 * wave + col), x);
    store_acc<0>(acc_mat(dwo + chn * GC * GD, GC, half, 32 * wave + col), -w);
    store_acc<0>(acc_mat(dkto + chn * GC * GD, GC, half, 32 * wave + col), kt);
    sd = wave_sum(sd);
    if (lane == 0) L.red[wave] = sd;
    __syncthreads();
    if (t == 0) {
        float tot = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < GT / 64; ++w2) tot += L.red[w2];
        sdot[chn] = tot;
    }
}

// The reference's per-node correction (V' = U - W S0 for every chunk of a
// node): dW = -dV' S0^T with S0 the node's initial state (its first chunk's
// S), per (chunk, v head); it replaces the dW of gdn_bwd_state_kernel, whose
// S is the chunk's own. Same staging as there: per 32-column chunk of the
// value dimension, all 128 rows of S0 and the 32 rows of dV' in LDS rows of
// SCS floats; wave w produces columns 32w .. 32w+31.
__global__ __launch_bounds__(GT) void gdn_dw_s0_kernel(GdnDev p, const float* __restrict__ chunk_sin,
                                                       const float* __restrict__ chunk_dvp,
                                                       float* __restrict__ dwo) {
    __shared__ __attribute__((aligned(16))) StateGradLds L;
    const int c = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    int start, len;
    if (!chunk_span(p, c, start, len)) return;
    const size_t chn = (size_t)c * p.hv + h;
    const int wave = t >> 6, lane = t & 63, col = lane & 31, half = lane >> 5;
    const float* S0 = chunk_sin + ((size_t)p.node_chunk0[p.chunk_node[c]] * p.hv + h) * GD * GD;
    const float* dVp = chunk_dvp + chn * GC * GD;
    const int sr = t >> 1, sc = 16 * (t & 1);      // S0 staging: row, first column
    const int ar = t >> 3, ac = 4 * (t & 7);       // dV' staging: row, first column
    f32x16 w = {};
#pragma unroll 1
    for (int k = 0; k < 4; ++k) {
        const int v0 = GC * k;
        __syncthreads();   // the previous chunk's readers are done
#pragma unroll
        for (int e = 0; e < 16; e += 4) {   // rows of SCS floats: 8-byte aligned stores
            const f32x4 x4 = *(const f32x4*)(S0 + sr * GD + v0 + sc + e);
            *(float2*)&L.S[sr * SCS + sc + e] = (float2){x4[0], x4[1]};
            *(float2*)&L.S[sr * SCS + sc + e + 2] = (float2){x4[2], x4[3]};
        }
        const f32x4 a2 = *(const f32x4*)(dVp + ar * GD + v0 + ac);
        *(float2*)&L.A2[ar * SCS + ac] = (float2){a2[0], a2[1]};
        *(float2*)&L.A2[ar * SCS + ac + 2] = (float2){a2[2], a2[3]};
        __syncthreads();
#pragma unroll
        for (int st = 0; st < GC / 2; ++st)
            w = mfma_f32(L.A2[col * SCS + half + 2 * st], L.S[(32 * wave + col) * SCS + half + 2 * st], w);
    }
    store_acc<0>(acc_mat(dwo + chn * GC * GD, GC, half, 32 * wave + col), -w);
}

struct ChunkGradLds {
    float Qs[GC * RS];    // q^ * scale
    float Ks[GC * RS];    // k^
    float P1[GC * RS];
    float P2[GC * RS];
    float P3[GC * RS];    // v; later Y = T^T dT (stride MS)
    float KK[GC * MS];    // k^ k^T
    float M1[GC * MS];    // A -> dP -> dT -> E
    float M2[GC * MS];    // T
    float M3[GC * MS];    // dA * A + dN * N (the pair terms of dG)
    float R[4][GC * RR];  // per-wave partial 32 x 32 products (contraction split over the waves)
    float G[GC];
    float Glo[GC];
    float B[GC];
    float Grow[GC];
    float Crow[GC];
};

// Thread t owns row i = t/8 of the element-wise work: in [GC x GD] results
// the columns 32m + 4s + e (s = t%8, m, e < 4), in [GC x GC] results s + 8e.
// The products run on fp32 MFMA: a [GC x GD] result is split by columns
// (wave w: columns 32w .. 32w+31, in accumulator layout), a [GC x GC] one by
// contraction (wave w: k in [32w, 32w+32), partials summed through LDS).
// TRUNC (the reference's per-node correction): U and W do not come from the
// chunk's T, so the T part is left out; dv and dbeta are complete already
// (tt_gdn_trunc.hip), and trk (dk^ of the correction, [chunk, Hv, 32, 128])
// and trg (the node-level suffix sums of its dG, [chunk, Hv, 32]) are added.
template <typename TIn, bool TRUNC>
__global__ __launch_bounds__(GT) void gdn_bwd_chunk_kernel(GdnDev p, const TIn* __restrict__ d_o, int64_t do_st,
                                                           int64_t do_sh, const float* __restrict__ ws,
                                                           const float* __restrict__ chunk_vp,
                                                           const float* __restrict__ chunk_dvp,
                                                           const float* __restrict__ xo, const float* __restrict__ dwo,
                                                           const float* __restrict__ dkto,
                                                           const float* __restrict__ sdot, TIn* __restrict__ dq,
                                                           TIn* __restrict__ dk, TIn* __restrict__ dv,
                                                           float* __restrict__ dg, float* __restrict__ dbeta,
                                                           const float* __restrict__ trk, const float* __restrict__ trg) {
    __shared__ __attribute__((aligned(16))) ChunkGradLds L;
    const int c = blockIdx.x, hk = blockIdx.y, t = threadIdx.x;
    int start, len;
    if (!chunk_span(p, c, start, len)) return;
    const int i = t >> 3, s = t & 7;
    const int wave = t >> 6, lane = t & 63, col = lane & 31, half = lane >> 5, cw0 = 32 * wave;
    const bool valid = i < len;
    const int64_t tok = start + i;

    load_chunk_rows<TIn>(p, start, len, hk * p.rep, L.Qs, L.Ks, nullptr);
    __syncthreads();
    put_partial(L.R[wave], quarter_nt(L.Ks, L.Ks, 1.0f, col, half, wave, (f32x16){}), col, half);   // k^ k^T
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = s + 8 * e;
        L.KK[i * MS + j] = L.R[0][i * RR + j] + L.R[1][i * RR + j] + L.R[2][i * RR + j] + L.R[3][i * RR + j];
    }
    float dqa[16], dka[16];   // element-wise terms (row layout)
#pragma unroll
    for (int e = 0; e < 16; ++e) dqa[e] = dka[e] = 0.0f;
    f32x16 dqm = {}, dkm = {};   // product terms (accumulator layout, columns cw0 + col)

#pragma unroll 1
    for (int hh = 0; hh < p.rep; ++hh) {
        const int h = hk * p.rep + hh;
        const size_t chn = (size_t)c * p.hv + h;
        const float* cw = ws + chn * kWsChunk;
        // e^{G_L} <S, dS> for dg, loaded here so its latency hides behind the head's work
        const float gsd = t < GC ? sdot[chn] : 0.0f;
        __syncthreads();   // the previous head's readers are done
        if (t < GC) {
            L.G[t] = cw[kWsG + t];
            L.Glo[t] = cw[kWsGlo + t];
            L.B[t] = t < len ? p.beta[(int64_t)(start + t) * p.b_st + h] : 0.0f;
        }
        tile_in(d_o + (int64_t)start * do_st + (int64_t)h * do_sh, do_st, len, L.P1);
        tile_in(chunk_vp + chn * GC * GD, GD, GC, L.P2);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = s + 8 * e;
            L.M1[i * MS + j] = cw[kWsA + i * GC + j];
            if constexpr (!TRUNC) L.M2[i * MS + j] = cw[kWsT + i * GC + j];
        }
        __syncthreads();
        // dA = dO V'^T (partials per wave)
        put_partial(L.R[wave], quarter_nt(L.P1, L.P2, 1.0f, col, half, wave, (f32x16){}), col, half);
        __syncthreads();
        const float gi = L.G[i], gl = L.G[GC - 1], egi = expf(gi), bi = L.B[i];
        const float gil = L.Glo[i], gll = L.Glo[GC - 1];
        // this thread's share of row i's own dG terms (those of e^{G_i} alone), dbeta, c
        float dgp = 0.0f, dbp = 0.0f, cp = 0.0f;

        // dG from A = (q^ k^T) * D, then dP = dA * D (j <= i).
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = s + 8 * e;
            const float da = L.R[0][i * RR + j] + L.R[1][i * RR + j] + L.R[2][i * RR + j] + L.R[3][i * RR + j];
            const float dae = j <= i ? da : 0.0f;
            const float pa = dae * L.M1[i * MS + j];
            L.M3[i * MS + j] = pa;
            L.M1[i * MS + j] = j <= i ? dae * expf(gdiff(gi, gil, L.G[j], L.Glo[j])) : 0.0f;
        }
        // O's state term e^G q^ S: dq^ += e^G X, dG += e^G q^ . X.
        {
            const float* xr = xo + chn * GC * GD + i * GD;
            float xq = 0.0f;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const f32x4 x = *(const f32x4*)(xr + 32 * m + 4 * s);
                const f32x4 q = *(const f32x4*)&L.Qs[i * RS + 32 * m + 4 * s];
#pragma unroll
                for (int e = 0; e < 4; ++e) dqa[4 * m + e] = fmaf(egi, x[e], dqa[4 * m + e]);
                xq += dot4(q, x);
            }
            dgp = fmaf(egi, xq, dgp);
        }
        __syncthreads();   // dP complete
        // dq^ += dP k^, dk^ += dP^T q^ (contraction over the chunk's 32 tokens).
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const f32x4 a = op_row4(L.M1, MS, col, half, 0, m);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * m + e;
                dqm = mfma_f32(a[e], op_col(L.Ks, RS, half, 0, r, cw0, col), dqm);
                dkm = mfma_f32(op_col(L.M1, MS, half, 0, r, 0, col), op_col(L.Qs, RS, half, 0, r, cw0, col), dkm);
            }
        }
        if constexpr (!TRUNC) {
            __syncthreads();   // P1, P2 and R readers are done
            tile_in(chunk_dvp + chn * GC * GD, GD, GC, L.P1);
            tile_in(dwo + chn * GC * GD, GD, GC, L.P2);
            tile_in((const TIn*)p.v + (int64_t)start * p.v_st + (int64_t)h * p.v_sh, p.v_st, len, L.P3);
            __syncthreads();

            // dT = dV' (beta v)^T + dW (beta e^G k^)^T (partials per wave); dBv =
            // T^T dV', dBk = T^T dW (columns of this wave).
            {
                const float bj = L.B[col], bgj = bj * expf(L.G[col] + L.Glo[col]);
                f32x16 tp = quarter_nt(L.P1, L.P3, bj, col, half, wave, (f32x16){});
                tp = quarter_nt(L.P2, L.Ks, bgj, col, half, wave, tp);
                put_partial(L.R[wave], tp, col, half);
            }
            f32x16 dbvm = {}, dbkm = {};
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float a = op_col(L.M2, MS, half, 0, r, 0, col);
                dbvm = mfma_f32(a, op_col(L.P1, RS, half, 0, r, cw0, col), dbvm);
                dbkm = mfma_f32(a, op_col(L.P2, RS, half, 0, r, cw0, col), dbkm);
            }
            __syncthreads();   // R complete; P1, P2 readers are done
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                L.P1[acc_row(r, half) * RS + cw0 + col] = dbvm[r];
                L.P2[acc_row(r, half) * RS + cw0 + col] = dbkm[r];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = s + 8 * e;
                L.M1[i * MS + j] = L.R[0][i * RR + j] + L.R[1][i * RR + j] + L.R[2][i * RR + j] + L.R[3][i * RR + j];
            }
            __syncthreads();   // dBv, dBk and dT complete
            // dv = beta dBv; dbeta, dk^, dG from U = T (beta v) and W = T (beta e^G k^).
            {
                float vb = 0.0f, kb = 0.0f;
                const float bge = bi * egi;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const f32x4 vv = *(const f32x4*)&L.P3[i * RS + 32 * m + 4 * s];
                    const f32x4 kv = *(const f32x4*)&L.Ks[i * RS + 32 * m + 4 * s];
                    const f32x4 dbv = *(const f32x4*)&L.P1[i * RS + 32 * m + 4 * s];
                    const f32x4 dbk = *(const f32x4*)&L.P2[i * RS + 32 * m + 4 * s];
                    f32x4 o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        vb = fmaf(vv[e], dbv[e], vb);
                        kb = fmaf(kv[e], dbk[e], kb);
                        dka[4 * m + e] = fmaf(bge, dbk[e], dka[4 * m + e]);
                        o[e] = bi * dbv[e];
                    }
                    if (valid) store4(dv + tok * p.dv_st + h * GD + 32 * m + 4 * s, o);
                }
                dbp += vb + egi * kb;
                dgp = fmaf(bge, kb, dgp);
            }
            __syncthreads();   // P3 (v) readers are done
            // Y = T^T dT into P3 (stride MS)
            {
                float y[4] = {};
#pragma unroll 4
                for (int m = 0; m < GC; ++m) {
                    const float tmi = L.M2[m * MS + i];
#pragma unroll
                    for (int e = 0; e < 4; ++e) y[e] = fmaf(tmi, L.M1[m * MS + s + 8 * e], y[e]);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) L.P3[i * MS + s + 8 * e] = y[e];
            }
            __syncthreads();
            // dN = Y T^T (strictly lower): dbeta, dG and E = dL/d(k^ k^T) from
            // N = -beta (k^ k^T) * D.
            {
                float ev[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int j = s + 8 * e;
                    float dn = 0.0f;
#pragma unroll 4
                    for (int m = 0; m < GC; ++m) dn = fmaf(L.P3[i * MS + m], L.M2[j * MS + m], dn);
                    ev[e] = 0.0f;
                    if (j < i) {
                        const float dd = expf(gdiff(gi, gil, L.G[j], L.Glo[j])), kk = L.KK[i * MS + j];
                        const float pa = dn * (-bi * kk * dd);
                        dbp = fmaf(dn, -kk * dd, dbp);
                        ev[e] = -dn * bi * dd;
                        L.M3[i * MS + j] += pa;
                    }
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) L.M1[i * MS + s + 8 * e] = ev[e];   // dT's readers passed the last barrier
            }
            __syncthreads();
            // dk^ += (E + E^T) k^
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const f32x4 a = op_row4(L.M1, MS, col, half, 0, m);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * m + e;
                    const float ae = a[e] + op_col(L.M1, MS, half, 0, r, 0, col);
                    dkm = mfma_f32(ae, op_col(L.Ks, RS, half, 0, r, cw0, col), dkm);
                }
            }
        } else {   // the correction's dk^ (its dv, dbeta are complete)
            const float* kr = trk + (chn * GC + i) * GD;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const f32x4 x = *(const f32x4*)(kr + 32 * m + 4 * s);
#pragma unroll
                for (int e = 0; e < 4; ++e) dka[4 * m + e] += x[e];
            }
        }
        // M3 holds every pair term of dG (its last writers passed a barrier):
        // its rows become exclusive prefix sums, M3[i][c] = sum_{j < c} p_ij
        // (thread (i, s): four columns, a scan over the row's eight threads),
        // for the dg sums below.
        {
            f32x4 v = *(const f32x4*)&L.M3[i * MS + 4 * s];
            const float tot = v[0] + v[1] + v[2] + v[3];
            float pre = __shfl_up(tot, 1, 8);
            if (s == 0) pre = 0.0f;
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) {
                const float up = __shfl_up(pre, o, 8);
                if (s >= o) pre += up;
            }
            f32x4 x;
            x[0] = pre;
            x[1] = pre + v[0];
            x[2] = x[1] + v[1];
            x[3] = x[2] + v[2];
            *(f32x4*)&L.M3[i * MS + 4 * s] = x;
        }
        // The output state S_out = e^{G_L} S + (e^{G_L - G} k^)^T V': dk^ and dG.
        {
            const float* kr = dkto + chn * GC * GD + i * GD;
            const float ed = expf(gdiff(gl, gll, gi, gil));
            float kt = 0.0f;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const f32x4 x = *(const f32x4*)(kr + 32 * m + 4 * s);
                const f32x4 kv = *(const f32x4*)&L.Ks[i * RS + 32 * m + 4 * s];
                kt += dot4(kv, x);
#pragma unroll
                for (int e = 0; e < 4; ++e) dka[4 * m + e] = fmaf(ed, x[e], dka[4 * m + e]);
            }
            cp = ed * kt;
        }
        dgp = row8_sum(dgp);
        dbp = row8_sum(dbp);
        cp = row8_sum(cp);
        if (s == 0) {
            L.Grow[i] = dgp;
            L.Crow[i] = cp;
            if (!TRUNC && valid) dbeta[tok * p.hv + h] = dbp;
        }
        // dg_t = sum of dG_u over u >= t within the chunk (G is its cumulative
        // sum). A pair term p_ij (M3, i > j: the factors e^{G_i - G_j} of A and
        // N) adds to dG_i and subtracts from dG_j, so it reaches dg_t exactly
        // when i >= t > j; a term c_i of the output state's e^{G_L - G_i}
        // (Crow) reaches it when i < t; e^{G_L} S's reaches every t. Summing
        // just those sets, rather than suffix sums of row minus column sums
        // in which the pairs inside [t, L] cancel only up to rounding, keeps
        // dg accurate relative to its own size: dg_t = sum_{i >= t} M3[i][t]
        // + sum_{i < t} c_i + the e^{G_L} term + the suffix sum of the terms
        // of e^{G_i} alone.
        __syncthreads();
        if (t < GC) {
            float cross = 0.0f, cpre = 0.0f;
#pragma unroll 4
            for (int r = 0; r < GC; ++r) {
                cross += r >= t ? L.M3[r * MS + t] : 0.0f;
                cpre += r < t ? L.Crow[r] : 0.0f;
            }
            float dG = L.Grow[t];
#pragma unroll
            for (int o = 1; o < GC; o <<= 1) {
                const float up = __shfl_down(dG, o, GC);
                if (t + o < GC) dG += up;
            }
            dG += cross + cpre + expf(gl) * gsd;
            if constexpr (TRUNC) dG += trg[chn * GC + t];
            if (t < len) dg[(int64_t)(start + t) * p.hv + h] = dG;
        }
    }

    // The product terms join the element-wise ones (through P1, P2).
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        L.P1[acc_row(r, half) * RS + cw0 + col] = dqm[r];
        L.P2[acc_row(r, half) * RS + cw0 + col] = dkm[r];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const f32x4 a = *(const f32x4*)&L.P1[i * RS + 32 * m + 4 * s];
        const f32x4 b = *(const f32x4*)&L.P2[i * RS + 32 * m + 4 * s];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dqa[4 * m + e] += a[e];
            dka[4 * m + e] += b[e];
        }
    }

    // Through q^ = scale q / sqrt(|q|^2 + eps) and k^ = k / sqrt(|k|^2 + eps).
    if (valid) {
        const TIn* qr = (const TIn*)p.q + tok * p.q_st + (int64_t)hk * p.q_sh;
        const TIn* kr = (const TIn*)p.k + tok * p.k_st + (int64_t)hk * p.k_sh;
        f32x4 qv[4], kv[4];
        float sq = 0.0f, sk = 0.0f, dq_dot = 0.0f, dk_dot = 0.0f;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            qv[m] = load4(qr + 32 * m + 4 * s);
            kv[m] = load4(kr + 32 * m + 4 * s);
            sq += dot4(qv[m], qv[m]);
            sk += dot4(kv[m], kv[m]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dq_dot = fmaf(qv[m][e], dqa[4 * m + e], dq_dot);
                dk_dot = fmaf(kv[m][e], dka[4 * m + e], dk_dot);
            }
        }
        sq = row8_sum(sq);
        sk = row8_sum(sk);
        dq_dot = row8_sum(dq_dot);
        dk_dot = row8_sum(dk_dot);
        float aq = p.scale, bq = 0.0f, ak = 1.0f, bk = 0.0f;
        if (p.l2) {
            const float rq = 1.0f / sqrtf(sq + 1e-6f), rk = 1.0f / sqrtf(sk + 1e-6f);
            aq = p.scale * rq;
            bq = -p.scale * rq * rq * rq * dq_dot;
            ak = rk;
            bk = -rk * rk * rk * dk_dot;
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            f32x4 oq, ok;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                oq[e] = fmaf(aq, dqa[4 * m + e], bq * qv[m][e]);
                ok[e] = fmaf(ak, dka[4 * m + e], bk * kv[m][e]);
            }
            store4(dq + tok * p.dq_st + hk * GD + 32 * m + 4 * s, oq);
            store4(dk + tok * p.dk_st + hk * GD + 32 * m + 4 * s, ok);
        }
    }
}

}  // namespace

// Float counts per (chunk, v head) of the truncated mode's node-level terms:
// the node-level decay [32] and R (beta [v | e^G k]) rows [32 x 256].
constexpr size_t kTrGn = GC, kTrY1 = (size_t)GC * 2 * GD;

size_t tt_gdn_ws_bytes_impl(int n_chunks, int n_heads_v, bool trunc) {
    return (size_t)n_chunks * (size_t)n_heads_v * (kWsChunk + (trunc ? kTrGn + kTrY1 : 0)) * sizeof(float);
}

namespace {
constexpr int kMaxGridY = 65535;   // grid y limit: a level's nodes beyond it go to further launches


template <typename TIn, bool TRUNC>
void launch_prep(const GdnDev& d, float* prep, hipStream_t s) {
    hipLaunchKernelGGL((gdn_prep_kernel<TIn, TRUNC>), dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, prep);
}
// A level of n nodes runs in the row layout (exact rule) when the column
// layout would leave most of the chip idle: at most TT_GDN_ROWS_MAX_PAIRS
// (node, v head) pairs, two column workgroups each. On the 16K agent tree (32
// v heads) 64 pairs (levels of one or two nodes) timed best: 5.60 -> 5.40 ms
// per step, against 5.43 ms for 128 and for 256.
#ifndef TT_GDN_ROWS_MAX_PAIRS
#define TT_GDN_ROWS_MAX_PAIRS 64
#endif
template <bool TRUNC>
bool use_rows(const GdnDev& d, int n) {
    return !TRUNC && (int64_t)n * d.hv <= TT_GDN_ROWS_MAX_PAIRS;
}

template <typename TIn, bool TRUNC>
void launch_scan(const GdnDev& d, int b, int n, float* prep, TIn* out, float* states, float* sin, float* vp,
                 hipStream_t s) {
    // grid (v head x column block, node): all heads of a level's first
    // (longest) nodes are dispatched first
    for (int b0 = 0; b0 < n; b0 += kMaxGridY) {
        if (use_rows<TRUNC>(d, n))
            hipLaunchKernelGGL((gdn_scan_rows_kernel<TIn>), dim3(d.hv * kRowsSplit, min(kMaxGridY, n - b0)),
                               dim3(GT), 0, s, d, b + b0, prep, out, states, sin, vp);
        else
            hipLaunchKernelGGL((gdn_scan_cols_kernel<TIn, TRUNC>), dim3(d.hv * kScanSplit, min(kMaxGridY, n - b0)),
                               dim3(GT), 0, s, d, b + b0, prep, out, states, sin, vp);
    }
}

// The forward: chunk terms (prep; TRUNC: plus the node-level U, W), then one
// scan launch per tree level. gn, y1: TRUNC scratch.
template <typename TIn, bool TRUNC>
int gdn_forward(const GdnDev& d, const int32_t* level_offsets, int n_levels, TIn* out, float* states, float* prep,
                float* sin, float* vp, float* gn, float* y1, hipStream_t s) {
    launch_prep<TIn, TRUNC>(d, prep, s);
    if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    if constexpr (TRUNC) {
        const int rc = tt_gdn_trunc_fwd_launch(d, prep, gn, y1, s);
        if (rc != TT_OK) return rc;
    }
    for (int l = 0; l < n_levels; ++l) {
        const int b = level_offsets[l], n = level_offsets[l + 1] - b;
        if (n <= 0) continue;
        launch_scan<TIn, TRUNC>(d, b, n, prep, out, states, sin, vp, s);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    return TT_OK;
}

template <typename TIn>
int gdn_forward_any(const GdnDev& d, const int32_t* level_offsets, int n_levels, TIn* out, float* states,
                    float* prep, float* sin, float* vp, float* gn, float* y1, hipStream_t s) {
    return d.trunc ? gdn_forward<TIn, true>(d, level_offsets, n_levels, out, states, prep, sin, vp, gn, y1, s)
                   : gdn_forward<TIn, false>(d, level_offsets, n_levels, out, states, prep, sin, vp, gn, y1, s);
}
}  // namespace

int tt_gdn_fwd_launch(const GdnDev& d, const int32_t* level_offsets, int n_levels, void* out, float* states,
                      float* ws, hipStream_t s) {
    const size_t ch = (size_t)d.n_chunks * d.hv;
    float* gn = ws + ch * kWsChunk;
    float* y1 = gn + ch * kTrGn;
    if (d.dtype == TT_DTYPE_BF16)
        return gdn_forward_any<__bf16>(d, level_offsets, n_levels, (__bf16*)out, states, ws, nullptr, nullptr, gn,
                                       y1, s);
    return gdn_forward_any<float>(d, level_offsets, n_levels, (float*)out, states, ws, nullptr, nullptr, gn, y1, s);
}

// The backward's float buffers. "Saved" (what the forward can keep for it):
// per (chunk, v head) the prep terms [kWsChunk], the chunk's initial state S
// [128 x 128] and V' [32 x 128]; TRUNC: also the node-level decay [32] and
// R-rows y1 [32 x 256]. Scratch: per (chunk, v head) dS [128 x 128], dV', X,
// dW, dK~ [32 x 128]; TRUNC: dF1, dY0 [32 x 256], the correction's dk^
// [32 x 128] and dG [32]; per (node, v head) dS at entry [128 x 128]; when the
// backward recomputes the forward, the node states [128 x 128]; <S, dS> per
// (chunk, v head) last (it breaks 16-byte alignment).
namespace {
struct GdnBwdWs {
    float *prep, *sin, *vp, *gn, *y1, *dso, *dvp, *x, *dw, *dkt, *df1, *dy0, *dkr, *dgn, *dsn, *nstate, *sdot;
};
size_t gdn_saved_floats(size_t ch, bool trunc) {
    return ch * (kWsChunk + GD * GD + GC * GD + (trunc ? kTrGn + kTrY1 : 0));
}
size_t gdn_scratch_floats(size_t ch, size_t nd, bool recompute, bool trunc) {
    return ch * (GD * GD + 4 * GC * GD + 1 + (trunc ? 2 * kTrY1 + GC * GD + GC : 0)) +
           nd * GD * GD * (recompute ? 2 : 1);
}
GdnBwdWs gdn_bwd_carve(float* saved, float* scratch, size_t n_chunks, size_t n_nodes, size_t hv, bool recompute,
                       bool trunc) {
    const size_t ch = n_chunks * hv, nd = n_nodes * hv;
    GdnBwdWs w = {};
    float* q = saved;
    w.prep = q; q += ch * kWsChunk;
    w.sin = q; q += ch * GD * GD;
    w.vp = q; q += ch * GC * GD;
    if (trunc) {
        w.gn = q; q += ch * kTrGn;
        w.y1 = q; q += ch * kTrY1;
    }
    q = scratch;
    if (!q) return w;
    w.dso = q; q += ch * GD * GD;
    w.dvp = q; q += ch * GC * GD;
    w.x = q; q += ch * GC * GD;
    w.dw = q; q += ch * GC * GD;
    w.dkt = q; q += ch * GC * GD;
    if (trunc) {
        w.df1 = q; q += ch * kTrY1;
        w.dy0 = q; q += ch * kTrY1;
        w.dkr = q; q += ch * GC * GD;
        w.dgn = q; q += ch * GC;
    }
    w.dsn = q; q += nd * GD * GD;
    w.nstate = nullptr;
    if (recompute) { w.nstate = q; q += nd * GD * GD; }
    w.sdot = q;
    return w;
}
}  // namespace

size_t tt_gdn_saved_bytes_impl(int n_chunks, int n_heads_v, bool trunc) {
    return gdn_saved_floats((size_t)n_chunks * n_heads_v, trunc) * sizeof(float);
}
size_t tt_gdn_bwd_ws_bytes_impl(int n_chunks, int n_nodes, int n_heads_v, bool recompute, bool trunc) {
    const size_t ch = (size_t)n_chunks * n_heads_v, nd = (size_t)n_nodes * n_heads_v;
    return ((recompute ? gdn_saved_floats(ch, trunc) : 0) + gdn_scratch_floats(ch, nd, recompute, trunc)) *
           sizeof(float);
}

int tt_gdn_fwd_save_launch(const GdnDev& d, const int32_t* level_offsets, int n_levels, void* out, float* states,
                           float* saved, hipStream_t s) {
    const GdnBwdWs w = gdn_bwd_carve(saved, nullptr, d.n_chunks, d.n_nodes, d.hv, false, d.trunc);
    if (d.dtype == TT_DTYPE_BF16)
        return gdn_forward_any<__bf16>(d, level_offsets, n_levels, (__bf16*)out, states, w.prep, w.sin, w.vp, w.gn,
                                       w.y1, s);
    return gdn_forward_any<float>(d, level_offsets, n_levels, (float*)out, states, w.prep, w.sin, w.vp, w.gn, w.y1,
                                  s);
}

// saved == nullptr: recompute the forward into the front of ws; otherwise
// saved holds what tt_gdn_fwd_save_launch wrote for the same problem.
template <typename TIn, bool TRUNC>
static int gdn_bwd_run(const GdnDev& d, const int32_t* level_offsets, int n_levels, const TIn* d_o, int64_t do_st,
                       int64_t do_sh, TIn* dq, TIn* dk, TIn* dv, float* dg, float* dbeta, const float* saved,
                       float* ws, hipStream_t s) {
    const bool recompute = saved == nullptr;
    float* sv = recompute ? ws : const_cast<float*>(saved);
    float* scratch = recompute ? ws + gdn_saved_floats((size_t)d.n_chunks * d.hv, TRUNC) : ws;
    const GdnBwdWs w = gdn_bwd_carve(sv, scratch, d.n_chunks, d.n_nodes, d.hv, recompute, TRUNC);
    if (recompute) {
        const int rc = gdn_forward<TIn, TRUNC>(d, level_offsets, n_levels, (TIn*)nullptr, w.nstate, w.prep, w.sin,
                                               w.vp, w.gn, w.y1, s);
        if (rc != TT_OK) return rc;
    }
    for (int l = n_levels - 1; l >= 0; --l) {
        const int b = level_offsets[l], n = level_offsets[l + 1] - b;
        if (n <= 0) continue;
        for (int b0 = 0; b0 < n; b0 += kMaxGridY) {
            if (use_rows<TRUNC>(d, n))
                hipLaunchKernelGGL((gdn_rscan_rows_kernel<TIn>), dim3(d.hv * kRowsSplit, min(kMaxGridY, n - b0)),
                                   dim3(GT), 0, s, d, b + b0, w.prep, d_o, do_st, do_sh, w.dso, w.dvp, w.dsn);
            else
                hipLaunchKernelGGL((gdn_rscan_cols_kernel<TIn, TRUNC>),
                                   dim3(d.hv * kScanSplit, min(kMaxGridY, n - b0)), dim3(GT), 0, s, d, b + b0,
                                   w.prep, d_o, do_st, do_sh, w.dso, w.dvp, w.dsn);
        }
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    if (d.d_init) {
        static_assert(GD * GD % (4 * GT) == 0, "one f32x4 per thread");
        hipLaunchKernelGGL(gdn_init_grad_kernel, dim3(GD * GD / (4 * GT), d.hv), dim3(GT), 0, s, d, w.dsn);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    hipLaunchKernelGGL(gdn_bwd_state_kernel<TIn>, dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, d_o, do_st, do_sh,
                       w.sin, w.dso, w.vp, w.dvp, w.x, w.dw, w.dkt, w.sdot);
    if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    if constexpr (TRUNC) {
        hipLaunchKernelGGL(gdn_dw_s0_kernel, dim3(d.n_chunks, d.hv), dim3(GT), 0, s, d, w.sin, w.dvp, w.dw);
        const GdnTruncBwd tb{w.gn, w.y1, w.dvp, w.dw, w.df1, w.dy0, w.dkr, w.dgn};
        const int rc = tt_gdn_trunc_bwd_launch(d, tb, dv, dbeta, s);
        if (rc != TT_OK) return rc;
    }
    hipLaunchKernelGGL((gdn_bwd_chunk_kernel<TIn, TRUNC>), dim3(d.n_chunks, d.hk), dim3(GT), 0, s, d, d_o, do_st,
                       do_sh, w.prep, w.vp, w.dvp, w.x, w.dw, w.dkt, w.sdot, dq, dk, dv, dg, dbeta, w.dkr, w.dgn);
    if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    return TT_OK;
}

template <typename TIn>
static int gdn_bwd_any(const GdnDev& d, const int32_t* level_offsets, int n_levels, const TIn* d_o, int64_t do_st,
                       int64_t do_sh, TIn* dq, TIn* dk, TIn* dv, float* dg, float* dbeta, const float* saved,
                       float* ws, hipStream_t s) {
    return d.trunc ? gdn_bwd_run<TIn, true>(d, level_offsets, n_levels, d_o, do_st, do_sh, dq, dk, dv, dg, dbeta,
                                            saved, ws, s)
                   : gdn_bwd_run<TIn, false>(d, level_offsets, n_levels, d_o, do_st, do_sh, dq, dk, dv, dg, dbeta,
                                             saved, ws, s);
}

int tt_gdn_bwd_launch(const GdnDev& d, const int32_t* level_offsets, int n_levels, const void* d_o, int64_t do_st,
                      int64_t do_sh, void* dq, void* dk, void* dv, float* dg, float* dbeta, const float* saved,
                      float* ws, hipStream_t s) {
    if (d.dtype == TT_DTYPE_BF16)
        return gdn_bwd_any<__bf16>(d, level_offsets, n_levels, (const __bf16*)d_o, do_st, do_sh, (__bf16*)dq,
                                   (__bf16*)dk, (__bf16*)dv, dg, dbeta, saved, ws, s);
    return gdn_bwd_any<float>(d, level_offsets, n_levels, (const float*)d_o, do_st, do_sh, (float*)dq, (float*)dk,
                              (float*)dv, dg, dbeta, saved, ws, s);
}
