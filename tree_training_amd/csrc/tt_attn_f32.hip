// Tree-masked GQA attention in fp32 on gfx950's fp32 matrix cores
// (v_mfma_f32_32x32x2_f32), for fp32 models: the tiling, plan walk, masks and
// dK/dV work items of the bf16 path (tt_bf16_tiles.h), with fp32 operands.
//
// The MFMA takes one k per lane half per instruction: step r of a 32-deep
// contraction pairs k = acc_row(r, 0) (lanes 0-31) with k = acc_row(r, 1)
// (lanes 32-63), the accumulator row order, so a score accumulator (rows =
// keys or queries, one column per lane) is directly the operand of the next
// product, and a row operand X[lane row][k..k+3] is one 16-byte LDS read for
// four steps. Column operands X[k][lane column] are 4-byte reads; tiles read
// that way have rows of ROWC = 136 floats, so the two lane halves (rows 4
// apart) hit disjoint banks; tiles read only row-wise have ROWR = 132.
//
// Forward and dQ: S^T = K Q^T (Q of the lane's query in 64 registers), P^T
// feeds O^T = V^T P^T; dP^T = V dO^T, dQ^T = K^T dS^T. dK/dV: S = Q K^T and
// dP = dO V^T with rows = queries and a lane per key (K of the lane's key in
// registers, V of the workgroup's 128 keys in LDS), dV = P^T dO, dK = dS^T Q.
// K/V tiles (forward, dQ) and Q/dO blocks (dK/dV) are staged through
// registers: the next one's global loads are in flight while the current one
// computes; one LDS stage, two barriers per step.
#include "tt_bf16_tiles.h"

namespace {

constexpr int ROWR = D + 4;   // fp32 rows read as row operands
constexpr int ROWC = D + 8;   // fp32 rows read as column operands

__device__ __forceinline__ f32x16 mfma_x2(float a, float b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ const float* key_row_f(const AttnDev& a, int kk, int g, bool isv) {
    if (kk < a.n_past) {
        return isv ? (const float*)a.vp + kk * a.vp_st + g * a.vp_sh
                   : (const float*)a.kp + kk * a.kp_st + g * a.kp_sh;
    }
    const int64_t t = kk - a.n_past;
    return isv ? (const float*)a.v + t * a.v_st + g * a.v_sh : (const float*)a.k + t * a.k_st + g * a.k_sh;
}

// Register staging of NROWS fp32 rows of 128: thread t holds rows t/32 + 8i,
// floats 4(t%32) .. +3; 32 lanes cover a 512-byte row.
template <int NROWS>
struct RowRegsF {
    f32x4 x[NROWS / 8];
};

// NROWS rows that all exist: row 0 at `base`, rows `stb` bytes apart; one
// buffer resource (scalar), one lane offset, the row steps as scalar offsets.
template <int NROWS>
__device__ __forceinline__ void fetch_rows_fbuf(RowRegsF<NROWS>& r, const float* base, uint32_t stb) {
    const uint32_t bytes = (NROWS - 1) * stb + 4 * D;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes, 0x00020000);
    const uint32_t vo = (threadIdx.x >> 5) * stb + 16 * (threadIdx.x & 31);
#pragma unroll
    for (int i = 0; i < NROWS / 8; ++i)
        r.x[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)vo, (int)(8 * i * stb), 0));
}

template <int NROWS, int STRIDE>
__device__ __forceinline__ void store_rows_f(const RowRegsF<NROWS>& r, float* X) {
    const int dc = 4 * (threadIdx.x & 31), r0 = threadIdx.x >> 5;
#pragma unroll
    for (int i = 0; i < NROWS / 8; ++i) *(f32x4*)(X + (r0 + 8 * i) * STRIDE + dc) = r.x[i];
}

// ----------------------------------------------------------------------------
// forward and dQ: K/V tiles of 64 keys
// ----------------------------------------------------------------------------
struct KvStageF {
    float K[TT_BK * ROWR];
    float V[TT_BK * ROWC];
    int lo[TT_BK];
    int hi[TT_BK];
};

// Rows past the last key alias it (their empty bounds mask
// them); a tile straddling gateway and own keys is copied at commit.
struct KvTileStagerF {
    RowRegsF<TT_BK> k, v;
    int k0;
    bool direct;
    __device__ __forceinline__ void begin(const AttnDev& a, int kt, int g) {
        k0 = kt * TT_BK;
        direct = false;
        if (k0 + TT_BK <= a.n_past) {
            fetch_rows_fbuf(k, (const float*)a.kp + k0 * a.kp_st + g * a.kp_sh, 4 * a.kp_st);
            fetch_rows_fbuf(v, (const float*)a.vp + k0 * a.vp_st + g * a.vp_sh, 4 * a.vp_st);
        } else if (k0 >= a.n_past && k0 + TT_BK <= a.n_keys) {
            const int64_t t0 = k0 - a.n_past;
            fetch_rows_fbuf(k, (const float*)a.k + t0 * a.k_st + g * a.k_sh, 4 * a.k_st);
            fetch_rows_fbuf(v, (const float*)a.v + t0 * a.v_st + g * a.v_sh, 4 * a.v_st);
        } else {
            direct = true;
#pragma unroll
            for (int i = 0; i < TT_BK / 8; ++i) k.x[i] = v.x[i] = (f32x4){};
        }
    }
    __device__ __forceinline__ void commit(const AttnDev& a, int g, KvStageF& S) {
        if (!direct) {
            store_rows_f<TT_BK, ROWR>(k, S.K);
            store_rows_f<TT_BK, ROWC>(v, S.V);
            return;
        }
        const int dc = 4 * (threadIdx.x & 31), r0 = threadIdx.x >> 5;
        for (int i = 0; i < TT_BK / 8; ++i) {
            const int r = r0 + 8 * i, kk = min(k0 + r, a.n_keys - 1);
            *(f32x4*)(S.K + r * ROWR + dc) = *(const f32x4*)(key_row_f(a, kk, g, false) + dc);
            *(f32x4*)(S.V + r * ROWC + dc) = *(const f32x4*)(key_row_f(a, kk, g, true) + dc);
        }
    }
};

// Row `qi` of a [*, 128] fp32 tensor in operand order: x[4 db + m] holds
// columns 32 db + 8 m + 4 half .. +3 (zeros past n_q).
__device__ __forceinline__ void load_row_ops(const float* row, bool valid, int half, f32x4 (&x)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
        x[i] = valid ? *(const f32x4*)(row + 32 * (i >> 2) + 8 * (i & 3) + 4 * half) : (f32x4){};
}

// S^T of the 32 keys kb0 .. kb0+31 of the tile against the lane's query.
__device__ __forceinline__ f32x16 scores_t(const float* K, int kb0, const f32x4 (&q)[16], int col, int half) {
    f32x16 s = {};
    const float* kr = K + (kb0 + col) * ROWR + 4 * half;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const f32x4 kv = *(const f32x4*)(kr + 32 * (i >> 2) + 8 * (i & 3));
#pragma unroll
        for (int e = 0; e < 4; ++e) s = mfma_x2(kv[e], q[i][e], s);
    }
    return s;
}

// acc[db] += X^T P^T over the 32 keys kb0.. of a tile X (ROWC rows): column
// operand X[key][32 db + col].
__device__ __forceinline__ void accum_t(const float* X, int kb0, const f32x16& p, int col, int half,
                                        f32x16 (&acc)[4]) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float* xr = X + (kb0 + acc_row(r, half)) * ROWC + col;
#pragma unroll
        for (int db = 0; db < 4; ++db) acc[db] = mfma_x2(xr[32 * db], p[r], acc[db]);
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void fwd_f32_kernel(
    AttnDev a, float* __restrict__ out, float* __restrict__ lse) {
    __shared__ __attribute__((aligned(16))) KvStageF S;

    int qb, h;
    decode_qblock(a, qb, h);
    const int g = __builtin_amdgcn_readfirstlane(h / a.rep);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = lane & 31, half = lane >> 5;
    const int qi = qb * TT_BQ + wave * 32 + col;
    const float c = a.scale * TT_LOG2E;

    f32x4 q[16];
    load_row_ops((const float*)a.q + (int64_t)min(qi, a.n_q - 1) * a.q_st + h * a.q_sh, qi < a.n_q, half, q);
    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (f32x16){};
    float m_run = -INFINITY, l_run = 0.0f;

    const int cnt = __builtin_amdgcn_readfirstlane(a.row_cnt[qb]);
    const int* list = a.row_list + (size_t)qb * a.n_kt;
    KvTileStagerF stg;
    Bounds nb;
    if (cnt > 0) {
        const int kt0 = __builtin_amdgcn_readfirstlane(list[0] >> 1);
        stg.begin(a, kt0, g);
        fetch_bounds(a, kt0, nb);
    }
    for (int it = 0; it < cnt; ++it) {
        const bool full = __builtin_amdgcn_readfirstlane(list[it]) & 1;
        __syncthreads();   // the previous tile's readers are done
        stg.commit(a, g, S);
        store_bounds(nb, S.lo, S.hi);
        __syncthreads();
        {
            const int kt1 = __builtin_amdgcn_readfirstlane(list[it + 1 < cnt ? it + 1 : it] >> 1);
            stg.begin(a, kt1, g);
            fetch_bounds(a, kt1, nb);
        }
        f32x16 s[2];
        s[0] = scores_t(S.K, 0, q, col, half);
        s[1] = scores_t(S.K, 32, q, col, half);
        if (!full) mask_scores(s, S.lo, S.hi, qi, half);

        float mx0 = -INFINITY, mx1 = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            mx0 = fmaxf(mx0, s[0][r]);
            mx1 = fmaxf(mx1, s[1][r]);
        }
        const float mxc = halves_max(fmaxf(mx0, mx1)) * c;
        const bool grow = mxc > m_run + TT_RESCALE_LOG2;
        if (__ballot(grow)) {
            const float alpha = grow ? fast_exp2(m_run - mxc) : 1.0f;
            m_run = grow ? mxc : m_run;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] *= alpha;
        }
        const float m_use = (m_run == -INFINITY) ? 0.0f : m_run;
        float ps = 0.0f;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[b][r] = fast_exp2(fmaf(s[b][r], c, -m_use));
                ps += s[b][r];
            }
            accum_t(S.V, 32 * b, s[b], col, half, o);
        }
        l_run += ps;
    }

    const float l_tot = halves_sum(l_run);
    if (qi < a.n_q) {
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        float* op = out + ((size_t)qi * a.hq + h) * D;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                f32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = o[db][4 * grp + e] * inv;
                *(f32x4*)(op + 32 * db + 8 * grp + 4 * half) = w;
            }
        if (half == 0) {
            const float m_fin = (m_run == -INFINITY) ? 0.0f : m_run;
            lse[(size_t)h * a.n_q + qi] = l_tot > 0.0f ? (m_fin + __log2f(l_tot)) * TT_LN2 : -INFINITY;
        }
    }
}

// delta = rowsum(dO * O), one row per 16 threads (when TT_BWD_DELTA runs
// without TT_BWD_DQ; otherwise the dQ pass computes it).
__global__ __launch_bounds__(256) void bwd_delta_f32_kernel(AttnDev a, BwdDev b) {
    const int row = blockIdx.x * 16 + (threadIdx.x >> 4), sub = threadIdx.x & 15;
    const int total = a.n_q * a.hq;
    float acc = 0.0f;
    int i = 0, h = 0;
    if (row < total) {
        i = row / a.hq;
        h = row - i * a.hq;
        const float* op = (const float*)b.o + ((size_t)i * a.hq + h) * D + 8 * sub;
        const float* dp = (const float*)b.dout + i * b.do_st + h * b.do_sh + 8 * sub;
#pragma unroll
        for (int e = 0; e < 8; e += 4) {
            const f32x4 ov = *(const f32x4*)(op + e), dv = *(const f32x4*)(dp + e);
            acc += ov[0] * dv[0] + ov[1] * dv[1] + ov[2] * dv[2] + ov[3] * dv[3];
        }
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    if (row < total && sub == 0) b.delta[(size_t)h * a.n_q + i] = acc;
}

// dQ: per tile and 32-key half, S^T and dP^T, dS^T = P^T (dP^T - delta), then
// dQ^T += K^T dS^T. FUSE_DELTA: delta of the rows is computed here (and
// stored for the dK/dV pass) instead of read.
template <bool FUSE_DELTA>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void bwd_dq_f32_kernel(AttnDev a,
                                                                                                   BwdDev bw) {
    __shared__ __attribute__((aligned(16))) KvStageF S;
    __shared__ __attribute__((aligned(16))) float Kc[TT_BK * ROWC];   // K again, for the column reads of dQ

    int qb, h;
    decode_qblock(a, qb, h);
    const int g = __builtin_amdgcn_readfirstlane(h / a.rep);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = lane & 31, half = lane >> 5;
    const int qi = qb * TT_BQ + wave * 32 + col;
    const bool valid = qi < a.n_q;
    const int qr = min(qi, a.n_q - 1);
    const float c = a.scale * TT_LOG2E;

    f32x4 q[16], dov[16];
    load_row_ops((const float*)a.q + (int64_t)qr * a.q_st + h * a.q_sh, valid, half, q);
    load_row_ops((const float*)bw.dout + (int64_t)qr * bw.do_st + h * bw.do_sh, valid, half, dov);
    float lse2 = INFINITY, dlt = 0.0f;
    if (valid) {
        lse2 = bw.lse[(size_t)h * a.n_q + qi] * TT_LOG2E;
        if constexpr (FUSE_DELTA) {
            const float* orow = (const float*)bw.o + ((size_t)qi * a.hq + h) * D;
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const f32x4 ov = *(const f32x4*)(orow + 32 * (i >> 2) + 8 * (i & 3) + 4 * half);
                acc += ov[0] * dov[i][0] + ov[1] * dov[i][1] + ov[2] * dov[i][2] + ov[3] * dov[i][3];
            }
            dlt = acc;
        } else {
            dlt = bw.delta[(size_t)h * a.n_q + qi];
        }
    }
    if constexpr (FUSE_DELTA) {
        dlt = halves_sum(dlt);
        if (valid && half == 0) bw.delta[(size_t)h * a.n_q + qi] = dlt;
    }

    f32x16 dq[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) dq[i] = (f32x16){};

    const int cnt = __builtin_amdgcn_readfirstlane(a.row_cnt[qb]);
    const int* list = a.row_list + (size_t)qb * a.n_kt;
    KvTileStagerF stg;
    Bounds nb;
    if (cnt > 0) {
        const int kt0 = __builtin_amdgcn_readfirstlane(list[0] >> 1);
        stg.begin(a, kt0, g);
        fetch_bounds(a, kt0, nb);
    }
    for (int it = 0; it < cnt; ++it) {
        const bool full = __builtin_amdgcn_readfirstlane(list[it]) & 1;
        __syncthreads();
        stg.commit(a, g, S);
        store_rows_f<TT_BK, ROWC>(stg.k, Kc);
        if (stg.direct) {   // copied at commit: K rows again with the column stride
            const int dc = 4 * (threadIdx.x & 31), r0 = threadIdx.x >> 5;
            for (int i = 0; i < TT_BK / 8; ++i) {
                const int r = r0 + 8 * i;
                *(f32x4*)(Kc + r * ROWC + dc) = *(const f32x4*)(S.K + r * ROWR + dc);
            }
        }
        store_bounds(nb, S.lo, S.hi);
        __syncthreads();
        {
            const int kt1 = __builtin_amdgcn_readfirstlane(list[it + 1 < cnt ? it + 1 : it] >> 1);
            stg.begin(a, kt1, g);
            fetch_bounds(a, kt1, nb);
        }
        // a partial tile's 32-key half that none of the wave's queries sees is skipped
        const int run = full ? 3 : visible_halves(S.lo, S.hi, qb * TT_BQ + wave * 32, lane);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (!((run >> b) & 1)) continue;
            f32x16 sh = scores_t(S.K, 32 * b, q, col, half);
            f32x16 dph = {};
            {
                const float* vr = S.V + (32 * b + col) * ROWC + 4 * half;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const f32x4 vv = *(const f32x4*)(vr + 32 * (i >> 2) + 8 * (i & 3));
#pragma unroll
                    for (int e = 0; e < 4; ++e) dph = mfma_x2(vv[e], dov[i][e], dph);
                }
            }
            if (!full) mask_half(sh, S.lo + 32 * b, S.hi + 32 * b, qi, half);
#pragma unroll
            for (int r = 0; r < 16; ++r) sh[r] = fast_exp2(fmaf(sh[r], c, -lse2)) * (dph[r] - dlt);   // dS^T
            accum_t(Kc, 32 * b, sh, col, half, dq);
        }
    }

    if (valid) {
        float* op = (float*)bw.dq + ((size_t)qi * a.hq + h) * D;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                f32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = dq[db][4 * grp + e] * a.scale;
                *(f32x4*)(op + 32 * db + 8 * grp + 4 * half) = w;
            }
    }
}

// ----------------------------------------------------------------------------
// dK, dV (key-major, persistent over the plan's work items)
// ----------------------------------------------------------------------------
struct QStageF {
    float Q[TT_BQB * ROWC];
    float Dn[TT_BQB * ROWC];
    float lse[TT_BQB];    // log2 units
    float ndlt[TT_BQB];   // -delta
};

// Q and dO rows of a 32-query block of head h (rows past n_q alias the last
// query; their lse is +inf), plus its lse (wave 0) and delta (wave 1).
struct QBlockStagerF {
    RowRegsF<TT_BQB> q, d;
    float sv;
    int q0, h;
    __device__ __forceinline__ void begin(const AttnDev& a, const BwdDev& bw, int q0_, int h_) {
        q0 = q0_;
        h = h_;
        if (q0 + TT_BQB <= a.n_q) {
            fetch_rows_fbuf(q, (const float*)a.q + (int64_t)q0 * a.q_st + h * a.q_sh, 4 * a.q_st);
            fetch_rows_fbuf(d, (const float*)bw.dout + (int64_t)q0 * bw.do_st + h * bw.do_sh, 4 * bw.do_st);
        }
        const int wave = threadIdx.x >> 6;
        if (wave < 2) {
            const float* src = (wave == 0 ? bw.lse : bw.delta) + (size_t)h * a.n_q;
            sv = src[min(q0 + (int)(threadIdx.x & 31), a.n_q - 1)];
        }
    }
    __device__ __forceinline__ void commit(const AttnDev& a, const BwdDev& bw, QStageF& S) {
        if (q0 + TT_BQB <= a.n_q) {
            store_rows_f<TT_BQB, ROWC>(q, S.Q);
            store_rows_f<TT_BQB, ROWC>(d, S.Dn);
        } else {
            const int dc = 4 * (threadIdx.x & 31), r0 = threadIdx.x >> 5;
            for (int i = 0; i < TT_BQB / 8; ++i) {
                const int r = r0 + 8 * i;
                const int64_t qq = min(q0 + r, a.n_q - 1);
                *(f32x4*)(S.Q + r * ROWC + dc) = *(const f32x4*)((const float*)a.q + qq * a.q_st + h * a.q_sh + dc);
                *(f32x4*)(S.Dn + r * ROWC + dc) =
                    *(const f32x4*)((const float*)bw.dout + qq * bw.do_st + h * bw.do_sh + dc);
            }
        }
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        if (wave < 2 && lane < TT_BQB) {
            const bool in = q0 + lane < a.n_q;
            if (wave == 0) S.lse[lane] = in ? sv * TT_LOG2E : INFINITY;
            else S.ndlt[lane] = in ? -sv : 0.0f;
        }
    }
};

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void bwd_dkdv_f32_kernel(AttnDev a,
                                                                                                     BwdDev bw) {
    __shared__ __attribute__((aligned(16))) QStageF St[2];
    __shared__ __attribute__((aligned(16))) float Vs[TT_BKB * ROWR];   // V rows of the item's keys

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = lane & 31, half = lane >> 5;
    const float c = a.scale * TT_LOG2E;
    const int n_work = (*a.n_items) * a.hkv;

    for (int w_id = blockIdx.x; w_id < n_work; w_id += gridDim.x) {
        const int g = __builtin_amdgcn_readfirstlane(w_id % a.hkv);
        const int item = __builtin_amdgcn_readfirstlane(w_id / a.hkv);
        const int2 rc = a.kb_item[item];           // (tile rank, chunk): the plan's item order
        const int lo_r = __builtin_amdgcn_readfirstlane(rc.x);
        const int chunk = __builtin_amdgcn_readfirstlane(rc.y);
        const int kb = __builtin_amdgcn_readfirstlane(a.kb_order[lo_r]);
        // a later item's slot: the tile's items before it that are not its
        // first, after those of the tiles ranked before it
        const int64_t slot = (int64_t)a.kb_base[lo_r] - lo_r + chunk - 1;
        const int qlo = __builtin_amdgcn_readfirstlane(a.kb_qlo[kb]);
        const int qhi = __builtin_amdgcn_readfirstlane(a.kb_qhi[kb]);
        const int qch = tt_qch(a.n_q);
        const bool split = tt_kb_items(qlo, qhi, qch) > 1;
        int q_start, q_stop;
        tt_kb_item_range(qlo, qhi, qch, chunk, q_start, q_stop);
        // a tile of gateway keys that no query sees adds nothing anywhere
        if (q_stop <= q_start && kb * TT_BKB + TT_BKB <= a.n_past) continue;

        {   // V rows of the tile's 128 keys (keys past the end alias the last key)
            const int dc = 4 * (threadIdx.x & 31), r0 = threadIdx.x >> 5;
            for (int i = 0; i < TT_BKB / 8; ++i) {
                const int r = r0 + 8 * i, kk = min(kb * TT_BKB + r, a.n_keys - 1);
                *(f32x4*)(Vs + r * ROWR + dc) = *(const f32x4*)(key_row_f(a, kk, g, true) + dc);
            }
        }
        const int kk = kb * TT_BKB + wave * 32 + col;   // this lane's key
        int lo = 0, hi = 0;
        f32x4 kr[16];
        load_row_ops(key_row_f(a, min(kk, a.n_keys - 1), g, false), kk < a.n_keys, half, kr);
        if (kk < a.n_keys) {
            lo = max(a.key_lo[kk], 0);
            hi = min(a.key_hi[kk], a.n_q);
        }
        if (lo >= hi) { lo = a.n_q; hi = 0; }
        const unsigned vis_w = (unsigned)(hi - lo);
        const int w_lo = wave_min_i(lo), w_hi = wave_max_i(hi);
        const int w_maxlo = wave_max_i(lo < hi ? lo : -1), w_minhi = wave_min_i(lo < hi ? hi : -1);
        const bool w_all_vis = wave_min_i((kk < a.n_keys && lo < hi) ? 1 : 0) == 1;

        f32x16 dk[4], dv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) { dk[i] = (f32x16){}; dv[i] = (f32x16){}; }

        const int q_top = (q_stop > q_start) ? ((q_stop - 1) / TT_BQB) * TT_BQB : 0;
        const int n_steps = (q_stop > q_start) ? ((q_top - q_start) / TT_BQB + 1) * a.rep : 0;
        QBlockStagerF stg;
        int q0 = q_top, hh = 0;
        if (n_steps > 0) stg.begin(a, bw, q0, g * a.rep);
        const float* vrow = Vs + (wave * 32 + col) * ROWR + 4 * half;
        for (int s = 0; s < n_steps; ++s) {
            // Two stages: the one written here was last read in step s - 2, and
            // every wave passed the barrier of step s - 1 after finishing it.
            QStageF& S = St[s & 1];
            stg.commit(a, bw, S);
            __syncthreads();   // the stage (and, at step 0, Vs) written
            const int q0_cur = q0;
            if (++hh == a.rep) {
                hh = 0;
                q0 -= TT_BQB;
            }
            if (s + 1 < n_steps) stg.begin(a, bw, q0, g * a.rep + hh);
            const int q1 = min(q0_cur + TT_BQB, a.n_q);
            if (!((q0_cur < w_hi) && (q1 > w_lo))) continue;   // no key of this wave is seen here
            const bool full = w_all_vis && (w_maxlo <= q0_cur) && (w_minhi >= q1);

            // S = Q K^T and dP = dO V^T: rows = queries, lane = key column.
            f32x16 sc = {}, dp = {};
            {
                const float* qrow = S.Q + col * ROWC + 4 * half;
                const float* drow = S.Dn + col * ROWC + 4 * half;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int o = 32 * (i >> 2) + 8 * (i & 3);
                    const f32x4 qv = *(const f32x4*)(qrow + o), dv4 = *(const f32x4*)(drow + o);
                    const f32x4 vv = *(const f32x4*)(vrow + o);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        sc = mfma_x2(qv[e], kr[i][e], sc);
                        dp = mfma_x2(dv4[e], vv[e], dp);
                    }
                }
            }
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                const int r0 = 8 * grp + 4 * half;
                const f32x4 l2 = *(const f32x4*)(S.lse + r0);
                const f32x4 nd = *(const f32x4*)(S.ndlt + r0);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float p = fast_exp2(fmaf(sc[4 * grp + e], c, -l2[e]));
                    sc[4 * grp + e] = p;
                    dp[4 * grp + e] = p * (dp[4 * grp + e] + nd[e]);
                }
            }
            if (!full) {
#pragma unroll
                for (int grp = 0; grp < 4; ++grp)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const bool vis = (unsigned)(q0_cur + 8 * grp + 4 * half + e - lo) < vis_w;
                        sc[4 * grp + e] = vis ? sc[4 * grp + e] : 0.0f;
                        dp[4 * grp + e] = vis ? dp[4 * grp + e] : 0.0f;
                    }
            }
            // dV += P^T dO, dK += dS^T Q: contraction over the 32 queries.
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float* dr = S.Dn + acc_row(r, half) * ROWC + col;
                const float* qc = S.Q + acc_row(r, half) * ROWC + col;
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    dv[db] = mfma_x2(sc[r], dr[32 * db], dv[db]);
                    dk[db] = mfma_x2(dp[r], qc[32 * db], dk[db]);
                }
            }
        }

        // Epilogue: rows of dk/dv = this wave's keys, columns = d (as the bf16 pass).
        const bool det_split = split && bw.det;
        // a split tile's rows in the split sums (first items) and a later item's
        // slot: one that lies beyond the workspace writes nothing (the tile's
        // gradients become NaN in the finalize)
        const SplitRows sr = split ? split_rows(a, bw, kb) : SplitRows{0, false};
        const bool det_skip = det_split && (chunk > 0 ? slot >= bw.det_cap : !sr.ok);
        float* const sk = chunk == 0 ? bw.dk_ws : bw.dk_slot;
        float* const sv = chunk == 0 ? bw.dv_ws : bw.dv_slot;
        const int64_t srow = chunk == 0 ? sr.row0 : slot * TT_BKB - kb * TT_BKB;
        const int kbase = kb * TT_BKB + wave * 32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kbase + acc_row(r, half);
            if (key >= a.n_keys || det_skip) continue;
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const int d = 32 * db + col;
                const float gk = dk[db][r] * a.scale, gv = dv[db][r];
                const size_t widx = ((size_t)key * a.hkv + g) * D + d;
                if (det_split) {
                    const size_t sidx = ((size_t)(srow + key) * a.hkv + g) * D + d;
                    sk[sidx] = gk;
                    sv[sidx] = gv;
                } else if (key < a.n_past) {
                    if (bw.dk_acc) {
                        if (split) {
                            atomicAdd(bw.dk_acc + widx, gk);
                            atomicAdd(bw.dv_acc + widx, gv);
                        } else {
                            bw.dk_acc[widx] += gk;
                            bw.dv_acc[widx] += gv;
                        }
                    }
                } else if (split) {
                    if (sr.ok) {
                        const size_t cidx = ((size_t)(sr.row0 + key) * a.hkv + g) * D + d;
                        atomicAdd(bw.dk_ws + cidx, gk);
                        atomicAdd(bw.dv_ws + cidx, gv);
                    }
                } else {
                    const size_t idx = ((size_t)(key - a.n_past) * a.hkv + g) * D + d;
                    ((float*)bw.dk)[idx] = gk;
                    ((float*)bw.dv)[idx] = gv;
                }
            }
        }
        __syncthreads();   // Vs and the stage are reused by the next item
    }
}

}  // namespace

int tt_fwd_f32_launch(const AttnDev& a, void* o, float* lse, hipStream_t s) {
    hipLaunchKernelGGL(fwd_f32_kernel, dim3(a.n_qb * a.hq), dim3(256), 0, s, a, (float*)o, lse);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

int tt_bwd_f32_launch(const AttnDev& a, const BwdDev& b, hipStream_t s) {
    const bool fuse = (b.parts & TT_BWD_DELTA) && (b.parts & TT_BWD_DQ);
    if ((b.parts & TT_BWD_DELTA) && !fuse) {
        hipLaunchKernelGGL(bwd_delta_f32_kernel, dim3(tt_cdiv(a.n_q * a.hq, 16)), dim3(256), 0, s, a, b);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    if (b.parts & TT_BWD_DQ) {
        if (fuse)
            hipLaunchKernelGGL(bwd_dq_f32_kernel<true>, dim3(a.n_qb * a.hq), dim3(256), 0, s, a, b);
        else
            hipLaunchKernelGGL(bwd_dq_f32_kernel<false>, dim3(a.n_qb * a.hq), dim3(256), 0, s, a, b);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    if (b.parts & TT_BWD_DKDV) {
        // one workgroup per CU (the kernel holds 256 VGPRs per lane and 103 KB of LDS)
        const int grid = (1024 / a.hkv) * a.hkv > 0 ? (1024 / a.hkv) * a.hkv : a.hkv;
        if (b.det) {
            hipLaunchKernelGGL(bwd_dkdv_f32_kernel, dim3(grid), dim3(256), 0, s, a, b);
            hipLaunchKernelGGL(bwd_split_finalize_det_kernel<float>, dim3(a.n_kb, a.hkv), dim3(256), 0, s, a, b);
        } else {
            hipLaunchKernelGGL(bwd_split_zero_kernel, dim3(a.n_kb, a.hkv), dim3(256), 0, s, a, b);
            hipLaunchKernelGGL(bwd_dkdv_f32_kernel, dim3(grid), dim3(256), 0, s, a, b);
            hipLaunchKernelGGL(bwd_split_finalize_kernel<float>, dim3(a.n_kb, a.hkv, 4), dim3(256), 0, s, a, b);
        }
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    return TT_OK;
}
