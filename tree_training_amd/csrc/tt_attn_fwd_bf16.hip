// Tree-masked GQA flash attention forward for gfx950 (bf16 in, fp32
// accumulate); the tiling is described in tt_bf16_tiles.h.
//
// Built without NaN semantics and with IEEE mode off (see build.py): masked
// scores are -inf, never NaN, and every exp2/max/sum on them is guarded, so the
// row max runs as v_max3_f32 straight on MFMA results.
#include "tt_bf16_tiles.h"

namespace {

// ----------------------------------------------------------------------------
// forward
// ----------------------------------------------------------------------------
struct FwdStage {
    bf16 K[TT_BK / 4 * GPITCH];   // row-group tiles: K read as rows, V transposed
    bf16 V[TT_BK / 4 * GPITCH];
    int lo[TT_BK];
    int hi[TT_BK];
};

// SPLIT: workgroup (pair, blockIdx.y) walks the blockIdx.y-th of sp.n
// contiguous ranges of the pair's key tiles and writes the unnormalised
// output, row max and row sum of that range for fwd_combine_kernel.
template <bool SPLIT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void fwd_bf16_kernel(AttnDev a, bf16* __restrict__ out, float* __restrict__ lse, FwdSplit sp) {
    __shared__ __attribute__((aligned(16))) FwdStage st[2];

    int qb, h;
    decode_qblock(a, qb, h);
    const int g = __builtin_amdgcn_readfirstlane(h / a.rep);   // the division runs on the VALU
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = lane & 31, half = lane >> 5;
    const int qi = qb * TT_BQ + wave * 32 + col;
    const float c = a.scale * TT_LOG2E;

    bf16x8 qa[8];
    if (qi < a.n_q) {
        const bf16* qp = (const bf16*)a.q + qi * a.q_st + h * a.q_sh + 8 * half;
#pragma unroll
        for (int t = 0; t < 8; ++t) qa[t] = *(const bf16x8*)(qp + 16 * t);
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) qa[t] = zero8();
    }

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (f32x16){};
    float m_run = -INFINITY, l_run = 0.0f;

    // The plan entries are wave-uniform; readfirstlane keeps everything derived
    // from them (tile bases, buffer descriptors) in scalar registers.
    const int cnt = __builtin_amdgcn_readfirstlane(a.row_cnt[qb]);
    const int* list = a.row_list + (size_t)qb * a.n_kt;
    int it0 = 0, it1 = cnt;
    if constexpr (SPLIT) {
        it0 = cnt * (int)blockIdx.y / sp.n;
        it1 = cnt * ((int)blockIdx.y + 1) / sp.n;
    }
    KvTileDma stg;
    Bounds nb;
    const RowOffsG kro = row_offsg(col, half);   // this lane's key row in either 32-key half of a tile
    const TrOffsG tro = tr_offsg(lane);
    if (it1 > it0) {
        const int kt0 = __builtin_amdgcn_readfirstlane(list[it0] >> 1);
        stg.begin(a, kt0, g, st[it0 & 1].K, st[it0 & 1].V);
        fetch_bounds(a, kt0, nb);
    }
    for (int it = it0; it < it1; ++it) {
        FwdStage& S = st[it & 1];
        const bool full = __builtin_amdgcn_readfirstlane(list[it]) & 1;
        stg.commit(a, g, S.K, S.V);
        store_bounds(nb, S.lo, S.hi);
        __syncthreads();
        if (it + 1 < it1) {   // the other stage was last read in step it - 1, which every wave has left
            const int kt1 = __builtin_amdgcn_readfirstlane(list[it + 1] >> 1);
            stg.begin(a, kt1, g, st[(it + 1) & 1].K, st[(it + 1) & 1].V);
            fetch_bounds(a, kt1, nb);
        }

        f32x16 s[2];
        {
            // K operand reads run AH MFMAs ahead of their use (the scheduler
            // would otherwise issue them two at a time, just before use).
            constexpr int AH = 4;
            bf16x8 kop[16];
            static_for<AH>([&](auto i) {
                constexpr int n = decltype(i)::value;
                kop[n] = read_rowg<n & 7>(S.K + 8 * (n >> 3) * GPITCH, kro);
            });
            s[0] = (f32x16){};
            s[1] = (f32x16){};
            static_for<16>([&](auto i) {
                constexpr int n = decltype(i)::value;
                if constexpr (n + AH < 16)
                    kop[n + AH] = read_rowg<(n + AH) & 7>(S.K + 8 * ((n + AH) >> 3) * GPITCH, kro);
                __builtin_amdgcn_sched_barrier(0);
                s[n >> 3] = mfma32(kop[n], qa[n & 7], s[n >> 3]);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
        if (!full) mask_scores(s, S.lo, S.hi, qi, half);

        // Tile row max (both lane halves hold the same query after the exchange).
        float mx0 = -INFINITY, mx1 = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            mx0 = fmaxf(mx0, fmaxf(s[0][r], s[0][r + 1]));
            mx1 = fmaxf(mx1, fmaxf(s[1][r], s[1][r + 1]));
        }
        const float mx = halves_max(fmaxf(mx0, mx1));
        // Lazy rescaling: the running max moves only when the tile's max exceeds
        // it by more than TT_RESCALE_LOG2; otherwise probabilities are taken
        // against the stale max, so they stay below 2^TT_RESCALE_LOG2.
        const float mxc = mx * c;
        const bool grow = mxc > m_run + TT_RESCALE_LOG2;
        if (__ballot(grow)) {
            const float alpha = grow ? fast_exp2(m_run - mxc) : 1.0f;
            m_run = grow ? mxc : m_run;
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] *= alpha;
        }
        const float m_use = (m_run == -INFINITY) ? 0.0f : m_run;

        // P^T (bf16) feeds O^T += V^T P^T; the row sum is taken from the same
        // rounded values.
        float ps0 = 0.0f, ps1 = 0.0f;
#pragma unroll
        for (int stp = 0; stp < 4; ++stp) {
            const f32x16& sb = s[stp >> 1];
            const int r0 = 8 * (stp & 1);
            float p[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) p[e] = fast_exp2(fmaf(sb[r0 + e], c, -m_use));
            const bf16x8 pk = pack8(p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]);
            ps0 = sum4_bf16(pk, 0, ps0);
            ps1 = sum4_bf16(pk, 4, ps1);
#pragma unroll
            for (int db = 0; db < 4; ++db)
                o[db] = mfma32(read_trg(S.V, tro, 16 * stp, db), pk, o[db]);
        }
        l_run += ps0 + ps1;
    }

    const float l_tot = halves_sum(l_run);
    if constexpr (SPLIT) {
        if (qi < a.n_q) {
            const int s = blockIdx.y;
            float* op = sp.o + (((size_t)s * a.n_q + qi) * a.hq + h) * D;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int grp = 0; grp < 4; ++grp) {
                    f32x4 w;
#pragma unroll
                    for (int e = 0; e < 4; ++e) w[e] = o[db][4 * grp + e];
                    *(f32x4*)(op + 32 * db + 8 * grp + 4 * half) = w;
                }
            if (half == 0) {
                const size_t mi = ((size_t)s * a.hq + h) * a.n_q + qi;
                sp.m[mi] = (m_run == -INFINITY) ? 0.0f : m_run;
                sp.l[mi] = l_tot;
            }
        }
        return;
    }
    if (qi < a.n_q) {
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        bf16* op = out + ((size_t)qi * a.hq + h) * D;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                bf16x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = (bf16)(o[db][4 * grp + e] * inv);
                *(bf16x4*)(op + 32 * db + 8 * grp + 4 * half) = w;
            }
        if (half == 0) {
            const float m_fin = (m_run == -INFINITY) ? 0.0f : m_run;
            lse[(size_t)h * a.n_q + qi] = l_tot > 0.0f ? (m_fin + __log2f(l_tot)) * TT_LN2 : -INFINITY;
        }
    }
}

// Merges the key-range partials of each (query, q head) row: with M the
// largest row max of the ranges that saw a key, O = sum_s 2^(m_s - M) O_s /
// sum_s 2^(m_s - M) l_s, lse = (M + log2 of that sum) ln 2, ranges added in
// order. 32 threads per row, four columns each.
__global__ __launch_bounds__(256) void fwd_combine_kernel(AttnDev a, bf16* __restrict__ out, float* __restrict__ lse,
                                                          FwdSplit sp) {
    const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
    if (row >= a.n_q * a.hq) return;
    const int qi = row / a.hq, h = row - qi * a.hq;
    const int c4 = (threadIdx.x & 31) * 4;
    float mx = -INFINITY;
    for (int s = 0; s < sp.n; ++s) {
        const size_t mi = ((size_t)s * a.hq + h) * a.n_q + qi;
        if (sp.l[mi] > 0.0f) mx = fmaxf(mx, sp.m[mi]);
    }
    float l_sum = 0.0f;
    f32x4 acc = {};
    for (int s = 0; s < sp.n; ++s) {
        const size_t mi = ((size_t)s * a.hq + h) * a.n_q + qi;
        const float l = sp.l[mi];
        if (!(l > 0.0f)) continue;
        const float w = exp2f(sp.m[mi] - mx);
        l_sum = fmaf(w, l, l_sum);
        const f32x4 v = *(const f32x4*)(sp.o + ((size_t)s * a.n_q + qi) * a.hq * D + (size_t)h * D + c4);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = fmaf(w, v[e], acc[e]);
    }
    const float inv = l_sum > 0.0f ? 1.0f / l_sum : 0.0f;
    bf16x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (bf16)(acc[e] * inv);
    *(bf16x4*)(out + ((size_t)qi * a.hq + h) * D + c4) = r;
    if (c4 == 0) lse[(size_t)h * a.n_q + qi] = l_sum > 0.0f ? (mx + __log2f(l_sum)) * TT_LN2 : -INFINITY;
}

}  // namespace

int tt_fwd_bf16_launch(const AttnDev& a, void* o, float* lse, const FwdSplit& sp, hipStream_t s) {
    if (sp.n > 1) {
        hipLaunchKernelGGL(fwd_bf16_kernel<true>, dim3(a.n_qb * a.hq, sp.n), dim3(256), 0, s, a, (bf16*)o, lse, sp);
        hipLaunchKernelGGL(fwd_combine_kernel, dim3(tt_cdiv(a.n_q * a.hq, 8)), dim3(256), 0, s, a, (bf16*)o, lse,
                           sp);
    } else {
        hipLaunchKernelGGL(fwd_bf16_kernel<false>, dim3(a.n_qb * a.hq), dim3(256), 0, s, a, (bf16*)o, lse, sp);
    }
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}
