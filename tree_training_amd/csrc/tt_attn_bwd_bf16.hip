// Tree-masked GQA flash attention backward for gfx950 (bf16 in, fp32
// accumulate): delta, dQ (query-major) and dK/dV (key-major); the tiling is
// described in tt_bf16_tiles.h.
#include "tt_bf16_tiles.h"

namespace {

// ----------------------------------------------------------------------------
// backward: delta = rowsum(dO * O)
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void bwd_delta_bf16_kernel(AttnDev a, BwdDev b) {
    const int row = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15;
    const int total = a.n_q * a.hq;
    float acc = 0.0f;
    int i = 0, h = 0;
    if (row < total) {
        i = row / a.hq;
        h = row - i * a.hq;
        const bf16x8 ov = *(const bf16x8*)((const bf16*)b.o + ((size_t)i * a.hq + h) * D + 8 * sub);
        const bf16x8 dv = *(const bf16x8*)((const bf16*)b.dout + i * b.do_st + h * b.do_sh + 8 * sub);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc += (float)ov[e] * (float)dv[e];
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    if (row < total && sub == 0) b.delta[(size_t)h * a.n_q + i] = acc;
}

// ----------------------------------------------------------------------------
// backward: dQ (query-major, same tiling as the forward; key tiles staged by
// direct global -> LDS loads)
// ----------------------------------------------------------------------------
struct DqStage {
    bf16 K[TT_BK / 4 * GPITCH];   // read as rows (S^T) and transposed (dQ^T)
    bf16 V[TT_BK / 4 * GPITCH];   // read as rows (dP^T)
    int lo[TT_BK];
    int hi[TT_BK];
};

// FUSE_DELTA: the kernel also computes delta = rowsum(dO * O) of its rows (and
// stores it for the dK/dV pass) instead of reading it. SPLIT: workgroup
// (pair, blockIdx.y) walks the blockIdx.y-th of bw.n_split contiguous ranges
// of the pair's key tiles and writes its unscaled fp32 dQ partial for
// bwd_dq_combine_kernel (split 0 stores delta).
template <bool FUSE_DELTA, bool SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void bwd_dq_bf16_kernel(AttnDev a, BwdDev bw) {
    __shared__ __attribute__((aligned(16))) DqStage st[2];

    int qb, h;
    decode_qblock(a, qb, h);
    const int g = __builtin_amdgcn_readfirstlane(h / a.rep);   // the division runs on the VALU
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = lane & 31, half = lane >> 5;
    const int qi = qb * TT_BQ + wave * 32 + col;
    const float c = a.scale * TT_LOG2E;

    bf16x8 qa[8], da[8];
    float lse2 = INFINITY, dlt = 0.0f;
    if (qi < a.n_q) {
        const bf16* qp = (const bf16*)a.q + qi * a.q_st + h * a.q_sh + 8 * half;
        const bf16* dp = (const bf16*)bw.dout + qi * bw.do_st + h * bw.do_sh + 8 * half;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            qa[t] = *(const bf16x8*)(qp + 16 * t);
            da[t] = *(const bf16x8*)(dp + 16 * t);
        }
        lse2 = bw.lse[(size_t)h * a.n_q + qi] * TT_LOG2E;
        if constexpr (FUSE_DELTA) {
            // lanes l and l ^ 32 hold the two halves of the row (same query)
            const bf16* op = (const bf16*)bw.o + ((size_t)qi * a.hq + h) * D + 8 * half;
            float acc = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const bf16x8 ov = *(const bf16x8*)(op + 16 * t);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc += (float)ov[e] * (float)da[t][e];
            }
            dlt = halves_sum(acc);
            if (half == 0 && (!SPLIT || blockIdx.y == 0)) bw.delta[(size_t)h * a.n_q + qi] = dlt;
        } else {
            dlt = bw.delta[(size_t)h * a.n_q + qi];
        }
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) { qa[t] = zero8(); da[t] = zero8(); }
    }

    f32x16 dq[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) dq[i] = (f32x16){};

    const int cnt = a.row_cnt[qb];
    const int* list = a.row_list + (size_t)qb * a.n_kt;
    int it0 = 0, it1 = cnt;
    if constexpr (SPLIT) {
        it0 = cnt * (int)blockIdx.y / bw.n_split;
        it1 = cnt * ((int)blockIdx.y + 1) / bw.n_split;
    }
    KvTileDma stg;
    Bounds nb;
    const RowOffsG kro = row_offsg(col, half);   // this lane's key row in either 32-key half of a tile
    const TrOffsG tro = tr_offsg(lane);
    if (it1 > it0) {
        stg.begin(a, list[it0] >> 1, g, st[it0 & 1].K, st[it0 & 1].V);
        fetch_bounds(a, list[it0] >> 1, nb);
    }
    for (int it = it0; it < it1; ++it) {
        DqStage& S = st[it & 1];
        const bool full = list[it] & 1;
        stg.commit(a, g, S.K, S.V);
        store_bounds(nb, S.lo, S.hi);
        __syncthreads();
        if (it + 1 < it1) {   // the other stage was last read in step it - 1, which every wave has left
            const int kt1 = list[it + 1] >> 1;
            stg.begin(a, kt1, g, st[(it + 1) & 1].K, st[(it + 1) & 1].V);
            fetch_bounds(a, kt1, nb);
        }

        // The tile as two 32-key halves: scores, dS and the dQ update of one
        // half before the next. Half the score registers are live at a time
        // (the whole tile at once spills), which leaves room for operand
        // reads ahead of their MFMAs. A partial tile's half that no query of
        // the wave sees is skipped.
        const int run = full ? 3 : visible_halves(S.lo, S.hi, qb * TT_BQ + wave * 32, lane);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (!((run >> b) & 1)) continue;
            f32x16 sh = (f32x16){}, dph = (f32x16){};
            {   // the K / V operands of MFMA pair t + 1 are read before pair t issues
                const bf16* kh = S.K + 8 * b * GPITCH;
                const bf16* vh = S.V + 8 * b * GPITCH;
                bf16x8 ko[2], vo[2];
                ko[0] = read_rowg<0>(kh, kro);
                vo[0] = read_rowg<0>(vh, kro);
                static_for<8>([&](auto tt) {
                    constexpr int t = decltype(tt)::value;
                    if constexpr (t + 1 < 8) {
                        ko[(t + 1) & 1] = read_rowg<t + 1>(kh, kro);
                        vo[(t + 1) & 1] = read_rowg<t + 1>(vh, kro);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    sh = mfma32(ko[t & 1], qa[t], sh);
                    dph = mfma32(vo[t & 1], da[t], dph);
                    __builtin_amdgcn_sched_barrier(0);
                });
            }
            if (!full) mask_half(sh, S.lo + 32 * b, S.hi + 32 * b, qi, half);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = fast_exp2(fmaf(sh[r], c, -lse2));
                sh[r] = p * (dph[r] - dlt);   // dS^T
            }
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const int r0 = 8 * s2;
                const bf16x8 pk = pack8(sh[r0 + 0], sh[r0 + 1], sh[r0 + 2], sh[r0 + 3], sh[r0 + 4], sh[r0 + 5],
                                        sh[r0 + 6], sh[r0 + 7]);
#pragma unroll
                for (int db = 0; db < 4; ++db)
                    dq[db] = mfma32(read_trg(S.K, tro, 16 * (2 * b + s2), db), pk, dq[db]);
            }
        }
    }

    if constexpr (SPLIT) {
        if (qi < a.n_q) {
            float* op = bw.dq_part + (((size_t)blockIdx.y * a.n_q + qi) * a.hq + h) * D;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int grp = 0; grp < 4; ++grp) {
                    f32x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = dq[db][4 * grp + e];
                    *(f32x4*)(op + 32 * db + 8 * grp + 4 * half) = w;
                }
        }
    } else if (qi < a.n_q) {
        bf16* op = (bf16*)bw.dq + ((size_t)qi * a.hq + h) * D;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                bf16x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = (bf16)(dq[db][4 * grp + e] * a.scale);
                *(bf16x4*)(op + 32 * db + 8 * grp + 4 * half) = w;
            }
    }
    // The dK/dV pass of the same call needs its split sums cleared: each
    // workgroup takes every n-th (key tile, kv head), which saves that pass a
    // launch of its own.
    if (bw.zero_in_dq) {
        const int n_wg = gridDim.x * gridDim.y;
        for (int t = blockIdx.x + blockIdx.y * gridDim.x; t < a.n_kb * a.hkv; t += n_wg)
            split_zero_tile(a, bw, t / a.hkv, t % a.hkv);
    }
}

// dQ = scale * (sum of the key-range partials, in range order), four
// elements per thread.
__global__ __launch_bounds__(256) void bwd_dq_combine_kernel(AttnDev a, BwdDev bw) {
    const size_t n4 = (size_t)a.n_q * a.hq * (D / 4);
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    const size_t stride = (size_t)a.n_q * a.hq * D;
    f32x4 acc = *(const f32x4*)(bw.dq_part + 4 * i);
    for (int s = 1; s < bw.n_split; ++s) {
        const f32x4 v = *(const f32x4*)(bw.dq_part + s * stride + 4 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += v[e];
    }
    bf16x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = (bf16)(acc[e] * a.scale);
    *(bf16x4*)((bf16*)bw.dq + 4 * i) = w;
}

// ----------------------------------------------------------------------------
// backward: dK, dV (key-major, persistent over work items)
// ----------------------------------------------------------------------------
struct KvStage {
    bf16 Q[TT_BQB * ROWX];     // swizzled: read row-wise and transposed
    bf16 Dn[TT_BQB * ROWX];
    float nlse[TT_BQB];    // -lse / scale: the score accumulators start here
    float ndlt[TT_BQB];    // -delta: the dP accumulators start here
};

// Staging of a 32-query block of q head h: the Q and dO rows move straight
// from global memory into the swizzled tiles (direct loads: waves 0-1 move Q,
// waves 2-3 dO, five 1 KB pieces of the 10 KB tile each; the pieces' buffer
// offsets per lane are fixed for the kernel, the padding bytes of each row
// take row data that nothing reads); rows past the last query read as zeros.
// The block's lse (wave 0) and delta (wave 1) come through registers.
struct QBlockStager {
    uint32_t vo[5];   // this lane's buffer offset in each of its wave's pieces
    float sv;
    int q0;
    __device__ __forceinline__ void init(const AttnDev& a, const BwdDev& bw) {
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        const uint32_t stb = 2u * (uint32_t)(wave < 2 ? a.q_st : bw.do_st);
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int byte = 1024 * (5 * (wave & 1) + i) + 16 * lane;   // in the tile
            const int r = byte / (2 * ROWX), b = byte - r * (2 * ROWX);
            const int c = b < 2 * D ? ((b >> 4) ^ ((r >> 2) & 3)) : 0;   // 16-byte chunk of row r (tile_offx)
            vo[i] = (uint32_t)r * stb + 16u * (uint32_t)c;
        }
    }
    // Issues the direct loads of query block q0_, q head h into stage S.
    __device__ __forceinline__ void begin(const AttnDev& a, const BwdDev& bw, int q0_, int h, KvStage& S) {
        q0 = q0_;
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        const int rows = min(TT_BQB, a.n_q - q0);
        const bool isq = wave < 2;
        const uint32_t stb = 2u * (uint32_t)(isq ? a.q_st : bw.do_st);
        const bf16* base = isq ? (const bf16*)a.q + (int64_t)q0 * a.q_st + h * a.q_sh
                               : (const bf16*)bw.dout + (int64_t)q0 * bw.do_st + h * bw.do_sh;
        const i32x4 rs = dma_rsrc(base, (uint32_t)(rows - 1) * stb + 2u * D);
        const uint32_t l0 = lds_addr(isq ? S.Q : S.Dn) + 5120u * (uint32_t)(wave & 1);
#pragma unroll
        for (int i = 0; i < 5; ++i) lds_dma16(rs, l0 + 1024u * i, vo[i]);
        if (wave < 2) {
            const float* src = (wave == 0 ? bw.lse : bw.delta) + (size_t)h * a.n_q;
            sv = src[min(q0 + (int)(threadIdx.x & 31), a.n_q - 1)];
        }
    }
    // Completes the stage (before the barrier that publishes it). Rows past
    // the last query get -inf for -lse / scale, so they contribute nothing.
    __device__ __forceinline__ void commit(const AttnDev& a, KvStage& S) {
        const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
        if (wave < 2 && lane < TT_BQB) {
            const bool in = q0 + lane < a.n_q;
            if (wave == 0) S.nlse[lane] = in ? -sv / a.scale : -INFINITY;
            else S.ndlt[lane] = in ? -sv : 0.0f;
        }
        wait_vmem();
    }
};

#ifndef TT_DKDV_WAVES_PER_EU
#define TT_DKDV_WAVES_PER_EU 2
#endif
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TT_DKDV_WAVES_PER_EU, TT_DKDV_WAVES_PER_EU))) void bwd_dkdv_bf16_kernel(AttnDev a, BwdDev bw) {
    __shared__ __attribute__((aligned(16))) KvStage st[2];
    __shared__ __attribute__((aligned(16))) bf16 Vs[TT_BKB * ROW_R];   // V rows of the item's keys (row reads only)

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = lane & 31, half = lane >> 5;
    const float c = a.scale * TT_LOG2E;
    const int n_work = (*a.n_items) * a.hkv;
    const RowOffsX qro = row_offsx(col, half);   // this lane's query row in the Q / dO blocks
    const TrOffsX tro = tr_offsx(lane);
    QBlockStager stg;
    stg.init(a, bw);

    for (int w_id = blockIdx.x; w_id < n_work; w_id += gridDim.x) {
        // Workgroup-uniform values (the integer divisions run on the VALU):
        // readfirstlane keeps them, and everything derived from them, scalar.
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
        // the first query block's direct loads go out before the item's V and
        // K loads (stage 0 was last read before the previous item's final
        // barrier)
        const int q_top = (q_stop > q_start) ? ((q_stop - 1) / TT_BQB) * TT_BQB : 0;
        const int n_steps = (q_stop > q_start) ? ((q_top - q_start) / TT_BQB + 1) * a.rep : 0;
        if (n_steps > 0) stg.begin(a, bw, q_top, g * a.rep, st[0]);

        // V rows of the tile's 128 keys go to LDS (read as MFMA operands every
        // step); K of the lane's key stays in registers. Keys past the end alias
        // the last key and are never visible.
        {
            const int k0 = kb * TT_BKB;
            RowRegs<TT_BKB> vr;
            if (k0 + TT_BKB <= a.n_past) {
                fetch_rows_buf(vr, threadIdx.x, (const bf16*)a.vp + k0 * a.vp_st + g * a.vp_sh, 2 * a.vp_st);
            } else if (k0 >= a.n_past && k0 + TT_BKB <= a.n_keys) {
                fetch_rows_buf(vr, threadIdx.x, (const bf16*)a.v + (int64_t)(k0 - a.n_past) * a.v_st + g * a.v_sh,
                               2 * a.v_st);
            } else {
                auto vrow = [&](int r) { return key_row(a, min(k0 + r, a.n_keys - 1), g, true); };
                fetch_rows(vr, threadIdx.x, vrow);
            }
            store_rows<TT_BKB, ROW_R>(vr, threadIdx.x, Vs);
        }
        const int kk = kb * TT_BKB + wave * 32 + col;   // this lane's key (MFMA column)
        int lo = 0, hi = 0;
        bf16x8 kbv[8];
        if (kk < a.n_keys) {
            lo = max(a.key_lo[kk], 0);
            hi = min(a.key_hi[kk], a.n_q);
            const bf16* kp = key_row(a, kk, g, false) + 8 * half;
#pragma unroll
            for (int t = 0; t < 8; ++t) kbv[t] = *(const bf16x8*)(kp + 16 * t);
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) kbv[t] = zero8();
        }
        if (lo >= hi) { lo = a.n_q; hi = 0; }          // invisible key: neutral for min/max
        const unsigned vis_w = (unsigned)(hi - lo);     // query q sees the key iff q - lo < vis_w (unsigned)
        const int w_lo = wave_min_i(lo), w_hi = wave_max_i(hi);
        const int w_maxlo = wave_max_i(lo < hi ? lo : -1), w_minhi = wave_min_i(lo < hi ? hi : -1);
        const bool w_all_vis = wave_min_i((kk < a.n_keys && lo < hi) ? 1 : 0) == 1;

        f32x16 dk[4], dv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) { dk[i] = (f32x16){}; dv[i] = (f32x16){}; }

        // Query blocks are walked from the top of the range down, so items whose
        // ranges end at the same subtree end read the same rows at the same time.
        // step s covers query block q0 of q head g*rep + hh; (q0, hh) of the next
        // step are kept incrementally
        int q0 = q_top, hh = 0;
        for (int s = 0; s < n_steps; ++s) {
            KvStage& S = st[s & 1];
            stg.commit(a, S);
            __syncthreads();
            const int q0_cur = q0;
            if (++hh == a.rep) {
                hh = 0;
                q0 -= TT_BQB;
            }
            // the other stage was last read in step s - 1, which every wave has left
            if (s + 1 < n_steps) stg.begin(a, bw, q0, g * a.rep + hh, st[(s + 1) & 1]);
            const int q1 = min(q0_cur + TT_BQB, a.n_q);
            if (!((q0_cur < w_hi) && (q1 > w_lo))) continue;   // no key of this wave is seen here
            const bool full = w_all_vis && (w_maxlo <= q0_cur) && (w_minhi >= q1);

            // S = Q K^T and dP = dO V^T (rows = queries, lane = key column),
            // the accumulators started at -lse / scale and -delta of their rows:
            // P = exp2(c S') and dS = P dP' need no row terms afterwards. The
            // operands of MFMA pair t + 1 are read before pair t issues.
            f32x16 sc, dp;
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                const int r0 = 8 * grp + 4 * half;
                const f32x4 nl = *(const f32x4*)(S.nlse + r0);
                const f32x4 nd = *(const f32x4*)(S.ndlt + r0);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sc[4 * grp + e] = nl[e];
                    dp[4 * grp + e] = nd[e];
                }
            }
            {
                bf16x8 qo[2], doo[2], vo[2];
                qo[0] = read_rowx<0>(S.Q, qro);
                doo[0] = read_rowx<0>(S.Dn, qro);
                vo[0] = read_row_operand<ROW_R>(Vs, wave * 32 + col, 8 * half);
                static_for<8>([&](auto tt) {
                    constexpr int t = decltype(tt)::value;
                    if constexpr (t + 1 < 8) {
                        qo[(t + 1) & 1] = read_rowx<t + 1>(S.Q, qro);
                        doo[(t + 1) & 1] = read_rowx<t + 1>(S.Dn, qro);
                        vo[(t + 1) & 1] = read_row_operand<ROW_R>(Vs, wave * 32 + col, 16 * (t + 1) + 8 * half);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    sc = mfma32(qo[t & 1], kbv[t], sc);
                    dp = mfma32(doo[t & 1], vo[t & 1], dp);
                    __builtin_amdgcn_sched_barrier(0);
                });
            }
            // P = exp(S*scale - lse), dS = P (dP - delta); on the few steps where
            // some key of the wave is invisible to some query, those entries are
            // then zeroed (selects, so an overflowing exp of an invisible score
            // never propagates).
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float p = fast_exp2(sc[i] * c);
                sc[i] = p;
                dp[i] = p * dp[i];
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
            {   // P and dS packed at once (the score registers die here); the
                // transposed dO / Q operands of MFMA pair i + 1 are read before
                // pair i issues, so the LDS latency hides behind the MFMAs.
                bf16x8 pa[2], sa[2];
#pragma unroll
                for (int stp = 0; stp < 2; ++stp) {
                    const int r0 = 8 * stp;
                    pa[stp] = pack8(sc[r0 + 0], sc[r0 + 1], sc[r0 + 2], sc[r0 + 3], sc[r0 + 4], sc[r0 + 5],
                                    sc[r0 + 6], sc[r0 + 7]);
                    sa[stp] = pack8(dp[r0 + 0], dp[r0 + 1], dp[r0 + 2], dp[r0 + 3], dp[r0 + 4], dp[r0 + 5],
                                    dp[r0 + 6], dp[r0 + 7]);
                }
                bf16x8 od[2], oq[2];
                od[0] = read_trx(S.Dn, tro, 0, 0);
                oq[0] = read_trx(S.Q, tro, 0, 0);
                static_for<8>([&](auto ii) {   // pair i: query half i / 4, d block i % 4
                    constexpr int i = decltype(ii)::value, n = i + 1;
                    if constexpr (n < 8) {
                        od[n % 2] = read_trx(S.Dn, tro, 16 * (n / 4), 32 * (n % 4));
                        oq[n % 2] = read_trx(S.Q, tro, 16 * (n / 4), 32 * (n % 4));
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    dv[i % 4] = mfma32(pa[i / 4], od[i % 2], dv[i % 4]);
                    dk[i % 4] = mfma32(sa[i / 4], oq[i % 2], dk[i % 4]);
                });
            }
        }

        // Epilogue: rows of dk/dv = this wave's keys, columns = d. In the
        // deterministic mode a split tile's first item stores its partial sums
        // in the fp32 rows and each later item in its own slot (`slot` above);
        // the finalize pass adds them in chunk order.
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
                } else if (key < a.n_past) {   // gateway key: fp32, added to the caller's accumulators
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
                    ((bf16*)bw.dk)[idx] = (bf16)gk;
                    ((bf16*)bw.dv)[idx] = (bf16)gv;
                }
            }
        }
        __syncthreads();   // LDS stages are reused by the next item
    }
}

// Device self-test of the MFMA lane layout every bf16 kernel above relies on:
// D = A[32x16] * B[16x32] (row-major bf16), written back through acc_row().
__global__ __launch_bounds__(64) void selftest_mfma_kernel(const bf16* __restrict__ A, const bf16* __restrict__ B,
                                                           float* __restrict__ Dm) {
    const int lane = threadIdx.x, col = lane & 31, half = lane >> 5;
    bf16x8 av, bv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        av[e] = A[col * 16 + 8 * half + e];
        bv[e] = B[(8 * half + e) * 32 + col];
    }
    const f32x16 acc = mfma32(av, bv, (f32x16){});
#pragma unroll
    for (int r = 0; r < 16; ++r) Dm[acc_row(r, half) * 32 + col] = acc[r];
}

}  // namespace

int tt_selftest_mfma_launch(const void* a, const void* b, float* d, hipStream_t s) {
    hipLaunchKernelGGL(selftest_mfma_kernel, dim3(1), dim3(64), 0, s, (const bf16*)a, (const bf16*)b, d);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

// Persistent grid for the dK/dV pass: a multiple of Hkv so every workgroup
// keeps one kv head (and, with Hkv = 8, one XCD). 2048 workgroups (four per
// resident slot) leave at most one work item per workgroup on the 16K tree,
// so the hardware's dispatch balances the uneven items (6 % faster than 1024,
// which pairs items statically).
static int dkdv_grid(const AttnDev& a) {
    const int target = 2048;
    const int gsz = (target / a.hkv) * a.hkv;
    return gsz > 0 ? gsz : a.hkv;
}

int tt_bwd_bf16_launch(const AttnDev& a, const BwdDev& b, hipStream_t s) {
    const int rows = a.n_q * a.hq;
    // delta and dQ requested together: the dQ kernel computes delta itself
    const bool fuse = (b.parts & TT_BWD_DELTA) && (b.parts & TT_BWD_DQ);
    if ((b.parts & TT_BWD_DELTA) && !fuse) {
        hipLaunchKernelGGL(bwd_delta_bf16_kernel, dim3(tt_cdiv(rows, 16)), dim3(256), 0, s, a, b);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    if (b.parts & TT_BWD_DQ) {
        if (b.n_split > 1) {
            const dim3 grid(a.n_qb * a.hq, b.n_split);
            if (fuse)
                hipLaunchKernelGGL((bwd_dq_bf16_kernel<true, true>), grid, dim3(256), 0, s, a, b);
            else
                hipLaunchKernelGGL((bwd_dq_bf16_kernel<false, true>), grid, dim3(256), 0, s, a, b);
            const size_t n4 = (size_t)a.n_q * a.hq * (D / 4);
            hipLaunchKernelGGL(bwd_dq_combine_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, a, b);
        } else if (fuse) {
            hipLaunchKernelGGL((bwd_dq_bf16_kernel<true, false>), dim3(a.n_qb * a.hq), dim3(256), 0, s, a, b);
        } else {
            hipLaunchKernelGGL((bwd_dq_bf16_kernel<false, false>), dim3(a.n_qb * a.hq), dim3(256), 0, s, a, b);
        }
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    if (b.parts & TT_BWD_DKDV) {
        if (b.det) {
            hipLaunchKernelGGL(bwd_dkdv_bf16_kernel, dim3(dkdv_grid(a)), dim3(256), 0, s, a, b);
            hipLaunchKernelGGL(bwd_split_finalize_det_kernel<bf16>, dim3(a.n_kb, a.hkv), dim3(256), 0, s, a, b);
        } else {
            // split sums start at zero: cleared by the dQ pass of this call,
            // else by a launch of their own
            if (!b.zero_in_dq)
                hipLaunchKernelGGL(bwd_split_zero_kernel, dim3(a.n_kb, a.hkv), dim3(256), 0, s, a, b);
            hipLaunchKernelGGL(bwd_dkdv_bf16_kernel, dim3(dkdv_grid(a)), dim3(256), 0, s, a, b);
            hipLaunchKernelGGL(bwd_split_finalize_kernel<bf16>, dim3(a.n_kb, a.hkv, 4), dim3(256), 0, s, a, b);
        }
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    return TT_OK;
}

