// Tree-masked GQA attention in fp32 (VALU), for fp32 models and as an
// independent second implementation of the bf16 path.
//
// One wavefront per output row: lane l holds head-dim elements l and l + 64.
// Dot products reduce across the wave; the softmax state is wave-uniform.
// Forward and dQ walk the plan's non-empty key tiles of the row's query
// block; dK/dV walk the key's contiguous visible query interval for the
// Hq/Hkv q heads of its group. Deterministic, no atomics.
#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr int D = 128;

__device__ __forceinline__ const float* key_row_f(const AttnDev& a, int kk, int g, bool isv) {
    if (kk < a.n_past) {
        return isv ? (const float*)a.vp + kk * a.vp_st + g * a.vp_sh
                   : (const float*)a.kp + kk * a.kp_st + g * a.kp_sh;
    }
    const int64_t t = kk - a.n_past;
    return isv ? (const float*)a.v + t * a.v_st + g * a.v_sh : (const float*)a.k + t * a.k_st + g * a.k_sh;
}

__global__ __launch_bounds__(64) void fwd_f32_kernel(AttnDev a, float* __restrict__ out, float* __restrict__ lse) {
    const int i = blockIdx.x, h = blockIdx.y, g = h / a.rep;
    const int l = threadIdx.x;
    const float* qp = (const float*)a.q + i * a.q_st + h * a.q_sh;
    const float q0 = qp[l], q1 = qp[l + 64];
    float o0 = 0.0f, o1 = 0.0f, m = -INFINITY, den = 0.0f;
    const int qb = i / TT_BQ;
    const int cnt = a.row_cnt[qb];
    const int* list = a.row_list + (size_t)qb * a.n_kt;
    for (int it = 0; it < cnt; ++it) {
        const int kt = list[it] >> 1;
        const int jend = min(kt * TT_BK + TT_BK, a.n_keys);
        for (int j = kt * TT_BK; j < jend; ++j) {
            if (!(a.key_lo[j] <= i && i < a.key_hi[j])) continue;
            const float* kr = key_row_f(a, j, g, false);
            const float* vr = key_row_f(a, j, g, true);
            const float s = wave_sum(fmaf(q0, kr[l], q1 * kr[l + 64])) * a.scale;
            const float m_new = fmaxf(m, s);
            const float alpha = expf(m - m_new);
            const float p = expf(s - m_new);
            den = den * alpha + p;
            o0 = o0 * alpha + p * vr[l];
            o1 = o1 * alpha + p * vr[l + 64];
            m = m_new;
        }
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    float* op = out + ((size_t)i * a.hq + h) * D;
    op[l] = o0 * inv;
    op[l + 64] = o1 * inv;
    if (l == 0) lse[(size_t)h * a.n_q + i] = den > 0.0f ? m + logf(den) : -INFINITY;
}

__global__ __launch_bounds__(64) void bwd_delta_f32_kernel(AttnDev a, BwdDev b) {
    const int i = blockIdx.x, h = blockIdx.y, l = threadIdx.x;
    const float* op = (const float*)b.o + ((size_t)i * a.hq + h) * D;
    const float* dp = (const float*)b.dout + i * b.do_st + h * b.do_sh;
    const float s = wave_sum(fmaf(op[l], dp[l], op[l + 64] * dp[l + 64]));
    if (l == 0) b.delta[(size_t)h * a.n_q + i] = s;
}

__global__ __launch_bounds__(64) void bwd_dq_f32_kernel(AttnDev a, BwdDev b) {
    const int i = blockIdx.x, h = blockIdx.y, g = h / a.rep;
    const int l = threadIdx.x;
    const float* qp = (const float*)a.q + i * a.q_st + h * a.q_sh;
    const float* dop = (const float*)b.dout + i * b.do_st + h * b.do_sh;
    const float q0 = qp[l], q1 = qp[l + 64], d0 = dop[l], d1 = dop[l + 64];
    const float L = b.lse[(size_t)h * a.n_q + i], dl = b.delta[(size_t)h * a.n_q + i];
    float g0 = 0.0f, g1 = 0.0f;
    const int qb = i / TT_BQ;
    const int cnt = a.row_cnt[qb];
    const int* list = a.row_list + (size_t)qb * a.n_kt;
    for (int it = 0; it < cnt; ++it) {
        const int kt = list[it] >> 1;
        const int jend = min(kt * TT_BK + TT_BK, a.n_keys);
        for (int j = kt * TT_BK; j < jend; ++j) {
            if (!(a.key_lo[j] <= i && i < a.key_hi[j])) continue;
            const float* kr = key_row_f(a, j, g, false);
            const float* vr = key_row_f(a, j, g, true);
            const float s = wave_sum(fmaf(q0, kr[l], q1 * kr[l + 64])) * a.scale;
            const float dpv = wave_sum(fmaf(d0, vr[l], d1 * vr[l + 64]));
            const float ds = expf(s - L) * (dpv - dl);
            g0 = fmaf(ds, kr[l], g0);
            g1 = fmaf(ds, kr[l + 64], g1);
        }
    }
    float* out = (float*)b.dq + ((size_t)i * a.hq + h) * D;
    out[l] = g0 * a.scale;
    out[l + 64] = g1 * a.scale;
}

__global__ __launch_bounds__(64) void bwd_dkdv_f32_kernel(AttnDev a, BwdDev b) {
    const int j = blockIdx.x, g = blockIdx.y, l = threadIdx.x;
    const float* kr = key_row_f(a, j, g, false);
    const float* vr = key_row_f(a, j, g, true);
    const float k0 = kr[l], k1 = kr[l + 64], v0 = vr[l], v1 = vr[l + 64];
    const int lo = max(a.key_lo[j], 0), hi = min(a.key_hi[j], a.n_q);
    float gk0 = 0.0f, gk1 = 0.0f, gv0 = 0.0f, gv1 = 0.0f;
    for (int hh = 0; hh < a.rep; ++hh) {
        const int h = g * a.rep + hh;
        for (int i = lo; i < hi; ++i) {
            const float* qp = (const float*)a.q + i * a.q_st + h * a.q_sh;
            const float* dop = (const float*)b.dout + i * b.do_st + h * b.do_sh;
            const float s = wave_sum(fmaf(qp[l], k0, qp[l + 64] * k1)) * a.scale;
            const float p = expf(s - b.lse[(size_t)h * a.n_q + i]);
            const float dpv = wave_sum(fmaf(dop[l], v0, dop[l + 64] * v1));
            const float ds = p * (dpv - b.delta[(size_t)h * a.n_q + i]);
            gv0 = fmaf(p, dop[l], gv0);
            gv1 = fmaf(p, dop[l + 64], gv1);
            gk0 = fmaf(ds, qp[l], gk0);
            gk1 = fmaf(ds, qp[l + 64], gk1);
        }
    }
    gk0 *= a.scale;
    gk1 *= a.scale;
    if (j < a.n_past) {
        if (b.dk_acc) {
            const size_t idx = ((size_t)j * a.hkv + g) * D;
            b.dk_acc[idx + l] += gk0;
            b.dk_acc[idx + l + 64] += gk1;
            b.dv_acc[idx + l] += gv0;
            b.dv_acc[idx + l + 64] += gv1;
        }
    } else {
        const size_t idx = ((size_t)(j - a.n_past) * a.hkv + g) * D;
        ((float*)b.dk)[idx + l] = gk0;
        ((float*)b.dk)[idx + l + 64] = gk1;
        ((float*)b.dv)[idx + l] = gv0;
        ((float*)b.dv)[idx + l + 64] = gv1;
    }
}

}  // namespace

int tt_fwd_f32_launch(const AttnDev& a, void* o, float* lse, hipStream_t s) {
    hipLaunchKernelGGL(fwd_f32_kernel, dim3(a.n_q, a.hq), dim3(64), 0, s, a, (float*)o, lse);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

int tt_bwd_f32_launch(const AttnDev& a, const BwdDev& b, hipStream_t s) {
    if (b.parts & TT_BWD_DELTA) {
        hipLaunchKernelGGL(bwd_delta_f32_kernel, dim3(a.n_q, a.hq), dim3(64), 0, s, a, b);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    if (b.parts & TT_BWD_DQ) {
        hipLaunchKernelGGL(bwd_dq_f32_kernel, dim3(a.n_q, a.hq), dim3(64), 0, s, a, b);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    if (b.parts & TT_BWD_DKDV) {
        hipLaunchKernelGGL(bwd_dkdv_f32_kernel, dim3(a.n_keys, a.hkv), dim3(64), 0, s, a, b);
        if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    }
    return TT_OK;
}
