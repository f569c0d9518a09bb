// Row-wise softmax cross-entropy with its logit gradient, for gfx950: the
// leaf-loss step after the tree forward, applied to one chunk of lm_head
// logits at a time so the [T, V] logits never exist at once.
//
// Row r (label y, weight c): lse = log sum_j exp(x_j),
//   loss[r] = c (lse - x_y),   grad[r][j] = c (exp(x_j - lse) - [j == y]);
// a row whose label is ignore_index gets loss 0 and a zero gradient. grad may
// alias the logits (each element is read before the same thread writes it).
// One workgroup per row; an online max/sum pass then the gradient pass
// (3 x row bytes of HBM traffic). fp32 arithmetic.
#include "tt_common.h"
#include "tt_internal.h"

namespace {

constexpr int CE_T = 256;

template <typename T>
__device__ __forceinline__ void ce_ld8(const T* p, float (&x)[8]) {
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
__device__ __forceinline__ void ce_st8(T* p, const float (&x)[8]) {
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

// (m, s) <- merge of two online-softmax partials (s relative to m).
__device__ __forceinline__ void merge_ms(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) return;
    s = s * exp2f((m - mn) * TT_LOG2E) + s2 * exp2f((m2 - mn) * TT_LOG2E);
    m = mn;
}

template <typename T>
__global__ __launch_bounds__(CE_T) void ce_rows_kernel(const T* logits, int64_t ld, int V,
                                                       const int32_t* __restrict__ labels,
                                                       const float* __restrict__ row_scale, int ignore_index,
                                                       float* __restrict__ loss, T* grad, int64_t ldg) {
    __shared__ float red_m[CE_T / 64], red_s[CE_T / 64];
    __shared__ float row_lse;
    const int row = blockIdx.x, tid = threadIdx.x;
    const T* x = logits + (int64_t)row * ld;
    T* g = grad + (int64_t)row * ldg;
    const int lab = labels[row];
    const bool ignore = lab == ignore_index;
    const bool valid = !ignore && lab >= 0 && lab < V;
    const float sc = row_scale[row];
    const int v8 = V & ~7;

    float m = -INFINITY, s = 0.0f;
    for (int j = 8 * tid; j < v8; j += 8 * CE_T) {
        float v[8];
        ce_ld8(x + j, v);
        float m8 = v[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) m8 = fmaxf(m8, v[e]);
        float s8 = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s8 += exp2f((v[e] - m8) * TT_LOG2E);
        merge_ms(m, s, m8, s8);
    }
    for (int j = v8 + tid; j < V; j += CE_T) merge_ms(m, s, (float)x[j], 1.0f);
    // wave, then workgroup
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
        merge_ms(m, s, m2, s2);
    }
    if ((tid & 63) == 0) {
        red_m[tid >> 6] = m;
        red_s[tid >> 6] = s;
    }
    __syncthreads();
    if (tid == 0) {
        float mm = red_m[0], ss = red_s[0];
#pragma unroll
        for (int w = 1; w < CE_T / 64; ++w) merge_ms(mm, ss, red_m[w], red_s[w]);
        const float lse = mm + logf(ss);
        row_lse = lse;
        loss[row] = ignore ? 0.0f : (valid ? sc * (lse - (float)x[lab]) : __builtin_nanf(""));
    }
    __syncthreads();   // the label's logit is read before any gradient overwrites it
    const float lse = row_lse;
    const float c = valid ? sc : 0.0f;
    for (int j = 8 * tid; j < v8; j += 8 * CE_T) {
        float v[8];
        ce_ld8(x + j, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = c * (exp2f((v[e] - lse) * TT_LOG2E) - (j + e == lab ? 1.0f : 0.0f));
        ce_st8(g + j, v);
    }
    for (int j = v8 + tid; j < V; j += CE_T) {
        const float v = (float)x[j];
        g[j] = (T)(c * (exp2f((v - lse) * TT_LOG2E) - (j == lab ? 1.0f : 0.0f)));
    }
}

}  // namespace

int tt_ce_rows_launch(int dtype, const void* logits, int64_t ld, int n_rows, int vocab, const int32_t* labels,
                      const float* row_scale, int ignore_index, float* loss, void* grad, int64_t ldg,
                      hipStream_t s) {
    if (dtype == TT_DTYPE_BF16)
        hipLaunchKernelGGL(ce_rows_kernel<__bf16>, dim3(n_rows), dim3(CE_T), 0, s, (const __bf16*)logits, ld, vocab,
                           labels, row_scale, ignore_index, loss, (__bf16*)grad, ldg);
    else
        hipLaunchKernelGGL(ce_rows_kernel<float>, dim3(n_rows), dim3(CE_T), 0, s, (const float*)logits, ld, vocab,
                           labels, row_scale, ignore_index, loss, (float*)grad, ldg);
    return hipGetLastError() == hipSuccess ? TT_OK : TT_E_HIP;
}
