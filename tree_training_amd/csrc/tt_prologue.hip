// Attention prologue for gfx950: per (token, head) row of the projected q and
// k, RMSNorm over the 128 head dims then the rotate-half rotary embedding,
// written in the [T, H, 128] layout the attention kernels read; and its
// backward (dx, and the two norm weights' gradients summed in a fixed order).
//
//   y = w * x / sqrt(mean(x^2) + eps),  out = y * cos + rot(y) * sin,
//   rot(y) = [-y[64:], y[:64]]   (cos/sin: the model's table at the token's
//   position, read from the caller, so any rotary scaling variant works).
//
// 16 lanes hold one row (8 dims each, one 16-byte load); the rotary partner
// of dims 8l..8l+7 sits in lane l ^ 8. Rows are enumerated token-major over
// the Hq query heads then the Hkv key heads. fp32 arithmetic, one rounding.
// Memory-bound: 2 x row bytes + the cos/sin row per token.
#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr int PD = 128;
constexpr int PT = 256;              // threads per workgroup = 16 rows
constexpr int PROWS = PT / 16;

template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&x)[8]) {
    if constexpr (sizeof(T) == 2) {
        const bf16x8 a = *(const bf16x8*)p;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (float)a[e];
    } else {
        const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[e] = a[e];
            x[4 + e] = b[e];
        }
    }
}

template <typename T>
__device__ __forceinline__ void st8(T* p, const float (&x)[8]) {
    if constexpr (sizeof(T) == 2) {
        bf16x8 a;
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = (__bf16)x[e];
        *(bf16x8*)p = a;
    } else {
        *(f32x4*)p = (f32x4){x[0], x[1], x[2], x[3]};
        *(f32x4*)(p + 4) = (f32x4){x[4], x[5], x[6], x[7]};
    }
}

__device__ __forceinline__ float sum16(float v) {
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 8);
    return v;
}

// Row `row` -> token, whether it is a k row, and its input / output pointers.
template <typename T>
struct RowRef {
    int tok, h;
    bool is_k;
    const T* x;
    const T* w;
    float eps;
    int64_t out_off;   // element offset into the q or k output / gradient ([T, H, 128] contiguous)
};

template <typename T>
__device__ __forceinline__ RowRef<T> row_ref(const PrologueDev& p, int row) {
    const int per_tok = p.hq + p.hkv;
    const int tok = row / per_tok, hh = row - tok * per_tok;
    RowRef<T> r;
    r.tok = tok;
    r.is_k = hh >= p.hq;
    const int h = r.is_k ? hh - p.hq : hh;
    r.h = h;
    r.x = r.is_k ? (const T*)p.k + (int64_t)tok * p.k_st + (int64_t)h * p.k_sh
                 : (const T*)p.q + (int64_t)tok * p.q_st + (int64_t)h * p.q_sh;
    r.w = (const T*)(r.is_k ? p.kw : p.qw);
    r.eps = r.is_k ? p.eps_k : p.eps_q;
    r.out_off = ((int64_t)tok * (r.is_k ? p.hkv : p.hq) + h) * PD;
    return r;
}

constexpr int FWD_RPG = 4;           // rows per 16-lane group in the forward

template <typename T>
__device__ __forceinline__ void fwd_row(const PrologueDev& p, int row, int lane16, T* q_out, T* k_out) {
    const RowRef<T> r = row_ref<T>(p, row);
    const int d0 = 8 * lane16;
    float x[8], w[8], cs[8], sn[8];
    ld8(r.x + d0, x);
    ld8(r.w + d0, w);
    ld8((const T*)p.cos + (int64_t)r.tok * p.cs_st + d0, cs);
    ld8((const T*)p.sin + (int64_t)r.tok * p.cs_st + d0, sn);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
    const float rr = rsqrtf(sum16(ss) * (1.0f / PD) + r.eps);
    float y[8], o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = w[e] * (x[e] * rr);
    const float sgn = lane16 < 8 ? -1.0f : 1.0f;   // rot(y)[d] = -y[d+64] (d < 64), y[d-64]
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float partner = __shfl_xor(y[e], 8);
        o[e] = fmaf(y[e], cs[e], sgn * partner * sn[e]);
    }
    st8((r.is_k ? k_out : q_out) + r.out_off + d0, o);
}

// A workgroup covers FWD_RPG * 16 consecutive rows; group g takes rows
// g, g + 16, ... (each row's 16 lanes read 256 contiguous bytes).
template <typename T>
__global__ __launch_bounds__(PT) void prologue_fwd_kernel(PrologueDev p, T* __restrict__ q_out,
                                                          T* __restrict__ k_out) {
    const int lane16 = threadIdx.x & 15;
    const int base = blockIdx.x * (PROWS * FWD_RPG) + (threadIdx.x >> 4);
#pragma unroll
    for (int i = 0; i < FWD_RPG; ++i) {
        const int row = base + PROWS * i;
        if (row < p.n_rows) fwd_row<T>(p, row, lane16, q_out, k_out);   // uniform over the 16 lanes
    }
}

// Backward: dy = dout * cos + rot^T(dout * sin), rot^T(z) = [z[64:], -z[:64]];
// dxn = w * dy; dx = r (dxn - xn mean(xn * dxn)); dw += dy * xn. Each
// workgroup walks rows with a grid stride and keeps its dw partial sums (q and
// k weights) in LDS; part[block][2][128] is reduced in a fixed order after.
template <typename T>
__global__ __launch_bounds__(PT) void prologue_bwd_kernel(PrologueDev p, const T* __restrict__ dq_out,
                                                          int64_t dq_st, int64_t dq_sh,
                                                          const T* __restrict__ dk_out, int64_t dk_st,
                                                          int64_t dk_sh, T* __restrict__ dq_raw,
                                                          T* __restrict__ dk_raw, float* __restrict__ part) {
    __shared__ float acc[PROWS][2][PD];
    const int lane16 = threadIdx.x & 15, grp = threadIdx.x >> 4;
    const int d0 = 8 * lane16;
    float awq[8], awk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) awq[e] = awk[e] = 0.0f;
    const float sgn = lane16 < 8 ? 1.0f : -1.0f;    // rot^T(z)[d] = z[d+64] (d < 64), -z[d-64]
    for (int row = blockIdx.x * PROWS + grp; row < p.n_rows; row += gridDim.x * PROWS) {
        const RowRef<T> r = row_ref<T>(p, row);
        const T* go = r.is_k ? dk_out + (int64_t)r.tok * dk_st + (int64_t)r.h * dk_sh
                             : dq_out + (int64_t)r.tok * dq_st + (int64_t)r.h * dq_sh;
        float x[8], w[8], cs[8], sn[8], g[8];
        ld8(r.x + d0, x);
        ld8(r.w + d0, w);
        ld8((const T*)p.cos + (int64_t)r.tok * p.cs_st + d0, cs);
        ld8((const T*)p.sin + (int64_t)r.tok * p.cs_st + d0, sn);
        ld8(go + d0, g);
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
        const float rr = rsqrtf(sum16(ss) * (1.0f / PD) + r.eps);
        float xn[8], dxn[8], dot = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float zs = g[e] * sn[e];
            const float partner = __shfl_xor(zs, 8);
            const float dy = fmaf(g[e], cs[e], sgn * partner);
            xn[e] = x[e] * rr;
            dxn[e] = w[e] * dy;
            dot = fmaf(xn[e], dxn[e], dot);
            const float c = dy * xn[e];
            awq[e] += r.is_k ? 0.0f : c;
            awk[e] += r.is_k ? c : 0.0f;
        }
        const float m = sum16(dot) * (1.0f / PD);
        float dx[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) dx[e] = rr * (dxn[e] - xn[e] * m);
        st8((r.is_k ? dk_raw : dq_raw) + r.out_off + d0, dx);
    }
    // This workgroup's dw partials: groups' sums in LDS, then one fixed-order pass.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        acc[grp][0][d0 + e] = awq[e];
        acc[grp][1][d0 + e] = awk[e];
    }
    __syncthreads();
    {
        const int s = threadIdx.x >> 7, d = threadIdx.x & 127;   // 256 threads = 2 x 128 outputs
        float t = 0.0f;
#pragma unroll
        for (int g2 = 0; g2 < PROWS; ++g2) t += acc[g2][s][d];
        part[((size_t)blockIdx.x * 2 + s) * PD + d] = t;
    }
}

// dw[s][d] = sum over workgroups b of part[b][s][d]: one workgroup per
// output, each thread a fixed strided subset, then a fixed-order tree.
__global__ __launch_bounds__(PT) void prologue_dw_reduce_kernel(const float* __restrict__ part, int n_parts,
                                                                float* __restrict__ dqw, float* __restrict__ dkw) {
    __shared__ float red[PT];
    const int o = blockIdx.x, s = o >> 7, d = o & 127;
    float t = 0.0f;
    for (int b = threadIdx.x; b < n_parts; b += PT) t += part[((size_t)b * 2 + s) * PD + d];
    red[threadIdx.x] = t;
    __syncthreads();
    for (int w = PT / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) (s ? dkw : dqw)[d] = red[0];
}

constexpr int kBwdBlocks = 1024;

}  // namespace

size_t tt_prologue_bwd_ws_bytes_impl() { return (size_t)kBwdBlocks * 2 * PD * sizeof(float); }

int tt_prologue_fwd_launch(const PrologueDev& p, void* q_out, void* k_out, hipStream_t s) {
    const dim3 grid(tt_cdiv(p.n_rows, PROWS * FWD_RPG));
    if (p.dtype == TT_DTYPE_BF16)
        hipLaunchKernelGGL(prologue_fwd_kernel<__bf16>, grid, dim3(PT), 0, s, p, (__bf16*)q_out, (__bf16*)k_out);
    else
        hipLaunchKernelGGL(prologue_fwd_kernel<float>, grid, dim3(PT), 0, s, p, (float*)q_out, (float*)k_out);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}

int tt_prologue_bwd_launch(const PrologueDev& p, const void* dq_out, int64_t dq_st, int64_t dq_sh, const void* dk_out,
                           int64_t dk_st, int64_t dk_sh, void* dq_raw, void* dk_raw, float* dqw, float* dkw,
                           float* ws, hipStream_t s) {
    const int blocks = min(kBwdBlocks, tt_cdiv(p.n_rows, PROWS));
    if (p.dtype == TT_DTYPE_BF16)
        hipLaunchKernelGGL(prologue_bwd_kernel<__bf16>, dim3(blocks), dim3(PT), 0, s, p, (const __bf16*)dq_out,
                           dq_st, dq_sh, (const __bf16*)dk_out, dk_st, dk_sh, (__bf16*)dq_raw, (__bf16*)dk_raw, ws);
    else
        hipLaunchKernelGGL(prologue_bwd_kernel<float>, dim3(blocks), dim3(PT), 0, s, p, (const float*)dq_out, dq_st,
                           dq_sh, (const float*)dk_out, dk_st, dk_sh, (float*)dq_raw, (float*)dk_raw, ws);
    if (hipGetLastError() != hipSuccess) return TT_E_HIP;
    hipLaunchKernelGGL(prologue_dw_reduce_kernel, dim3(2 * PD), dim3(PT), 0, s, (const float*)ws, blocks, dqw, dkw);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}
