// Graded sign / mask / permutation ops and norm_sq on gfx950, one HBM pass each.
//
// The reference applies these as eager torch expressions with a precomputed
// per-blade vector (src/cliffordcuda/algebra.py:195-334): reverse, grade
// involution and Clifford conjugation multiply by (-1)^{f(grade)}, grade
// projection by a 0/1 mask, dual is x.flip(-1) * signs, norm_sq is
// (x * x * w).sum(-1) (three passes). Here each is one streaming kernel whose
// per-blade factor is computed from the blade index in registers (popcount),
// so no table is read.
#include "clf_common.h"

namespace clf {

__device__ __forceinline__ float graded_factor(int kind, unsigned k, int grade) {
    const int g = __popc(k);
    switch (kind) {
        case CLF_GRADED_REVERSE: return ((g * (g - 1) / 2) & 1) ? -1.f : 1.f;
        case CLF_GRADED_INVOLUTION: return (g & 1) ? -1.f : 1.f;
        case CLF_GRADED_CONJUGATION: return ((g * (g + 1) / 2) & 1) ? -1.f : 1.f;
        default: return g == grade ? 1.f : 0.f;  // projection
    }
}

// dual sign s[m]: output position m reads input blade ~m, with
// s[m] = (1/I^2) * (-1)^{sum of positions in ~m} * prod_{i in ~m} metric[i]
// (reference algebra.py:240-265 and _shared/_einsum_refs.py:107-115).
__device__ __forceinline__ float dual_factor(unsigned m, unsigned full, unsigned neg, int isq_par) {
    const unsigned a = ~m & full;
    const int par = isq_par + bitsum_parity(a) + __popc(a & neg);
    return (par & 1) ? -1.f : 1.f;
}

// One thread per 4 consecutive blades of one row (n >= 2).
__global__ __launch_bounds__(256) void graded_vec4(int kind, int n, unsigned neg, int grade, int isq_par,
                                                    const float4* __restrict__ X, float4* __restrict__ Y,
                                                    long long nchunks) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nchunks) return;
    const int c_log = n - 2;
    const unsigned full = (1u << n) - 1u;
    const long long row = idx >> c_log;
    const unsigned f = (unsigned)(idx & ((1 << c_log) - 1));
    const unsigned k0 = f << 2;
    if (kind == CLF_GRADED_DUAL || kind == CLF_GRADED_DUAL_ADJ) {
        // y[m] = x[~m] * s(m)  (dual)   or   y[k] = x[~k] * s(~k)  (adjoint)
        const unsigned src = ((1u << c_log) - 1u) - f;
        const float4 v = X[(row << c_log) + src];
        float o[4] = {v.w, v.z, v.y, v.x};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const unsigned m = k0 + e;
            const unsigned at = (kind == CLF_GRADED_DUAL) ? m : (~m & full);
            o[e] *= dual_factor(at, full, neg, isq_par);
        }
        Y[idx] = make_float4(o[0], o[1], o[2], o[3]);
    } else {
        const float4 v = X[idx];
        Y[idx] = make_float4(v.x * graded_factor(kind, k0, grade), v.y * graded_factor(kind, k0 + 1, grade),
                             v.z * graded_factor(kind, k0 + 2, grade), v.w * graded_factor(kind, k0 + 3, grade));
    }
}

// Scalar fallback for n < 2.
__global__ __launch_bounds__(256) void graded_scalar(int kind, int n, unsigned neg, int grade, int isq_par,
                                                      const float* __restrict__ X, float* __restrict__ Y,
                                                      long long total) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const unsigned full = (1u << n) - 1u;
    const long long row = idx >> n;
    const unsigned k = (unsigned)(idx & full);
    if (kind == CLF_GRADED_DUAL || kind == CLF_GRADED_DUAL_ADJ) {
        const unsigned src = ~k & full;
        const unsigned at = (kind == CLF_GRADED_DUAL) ? k : src;
        Y[idx] = X[(row << n) + src] * dual_factor(at, full, neg, isq_par);
    } else {
        Y[idx] = X[idx] * graded_factor(kind, k, grade);
    }
}

__device__ __forceinline__ float norm_weight(unsigned b, unsigned neg, unsigned nul) {
    if (b & nul) return 0.f;
    return (__popc(b & neg) & 1) ? -1.f : 1.f;
}

// out[r] = sum_b x[r,b]^2 w[b]; `tpr` lanes per row (power of two <= 64),
// each lane strides over the row's float4 chunks, then a butterfly reduce.
__global__ __launch_bounds__(256) void norm_sq_fwd_kernel(int n, unsigned neg, unsigned nul, int tpr_log,
                                                           const float* __restrict__ X, float* __restrict__ OUT,
                                                           long long batch) {
    const int tpr = 1 << tpr_log;
    const long long row = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> tpr_log;
    const int t = threadIdx.x & (tpr - 1);
    float acc = 0.f;
    if (row < batch) {
        const unsigned D = 1u << n;
        const float* x = X + (row << n);
        if (n >= 2) {
            const float4* x4 = reinterpret_cast<const float4*>(x);
            for (unsigned f = t; f < (D >> 2); f += tpr) {
                const float4 v = x4[f];
                const unsigned k = f << 2;
                acc = __builtin_fmaf(v.x * v.x, norm_weight(k, neg, nul), acc);
                acc = __builtin_fmaf(v.y * v.y, norm_weight(k + 1, neg, nul), acc);
                acc = __builtin_fmaf(v.z * v.z, norm_weight(k + 2, neg, nul), acc);
                acc = __builtin_fmaf(v.w * v.w, norm_weight(k + 3, neg, nul), acc);
            }
        } else {
            for (unsigned k = t; k < D; k += tpr) acc = __builtin_fmaf(x[k] * x[k], norm_weight(k, neg, nul), acc);
        }
    }
    for (int off = tpr >> 1; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (row < batch && t == 0) OUT[row] = acc;
}

__global__ __launch_bounds__(256) void norm_sq_bwd_kernel(int n, unsigned neg, unsigned nul,
                                                           const float* __restrict__ X,
                                                           const float* __restrict__ GOUT,
                                                           float* __restrict__ GX, long long total) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const unsigned k = (unsigned)(idx & ((1u << n) - 1u));
    const long long row = idx >> n;
    GX[idx] = 2.f * norm_weight(k, neg, nul) * X[idx] * GOUT[row];
}

static int check_graded_common(int n, uint32_t neg, uint32_t nul, int64_t batch) {
    if (n < 1 || n > kMaxNGraded)
        return set_error(CLF_ERR_ARG, "n must be in [1, " + std::to_string(kMaxNGraded) + "], got " + std::to_string(n));
    const uint32_t full = (1u << n) - 1u;
    if ((neg & ~full) || (nul & ~full)) return set_error(CLF_ERR_ARG, "metric masks have bits above n");
    if (neg & nul) return set_error(CLF_ERR_ARG, "neg_mask and null_mask overlap");
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    return CLF_OK;
}

int graded(int kind, int n, uint32_t neg, uint32_t nul, int grade, const float* x, float* y, int64_t batch,
           void* stream) {
    int rc = check_graded_common(n, neg, nul, batch);
    if (rc) return rc;
    if (kind < CLF_GRADED_REVERSE || kind > CLF_GRADED_DUAL_ADJ)
        return set_error(CLF_ERR_ARG, "unknown graded kind " + std::to_string(kind));
    const bool is_dual = kind == CLF_GRADED_DUAL || kind == CLF_GRADED_DUAL_ADJ;
    if (kind == CLF_GRADED_PROJECTION && (grade < 0 || grade > n))
        return set_error(CLF_ERR_ARG,
                         "grade must be in [0, " + std::to_string(n) + "] for n=" + std::to_string(n) + "; got " +
                             std::to_string(grade));
    if (is_dual && nul)
        return set_error(CLF_ERR_UNSUPPORTED,
                         "dual is undefined for degenerate metrics (any 0 in the metric makes the pseudoscalar I "
                         "non-invertible).");
    if (batch == 0) return CLF_OK;
    if (!x || !y) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (is_dual && x == y) return set_error(CLF_ERR_ARG, "dual output must not alias its input");
    if ((((uintptr_t)x) | ((uintptr_t)y)) & 15u) return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    // I^2 = (-1)^{n(n-1)/2} prod(metric): its parity
    const int isq_par = ((n * (n - 1) / 2) + popc_rt(neg)) & 1;
    hipStream_t s = (hipStream_t)stream;
    if (n >= 2) {
        const long long nchunks = (long long)batch << (n - 2);
        hipLaunchKernelGGL(graded_vec4, dim3((unsigned)((nchunks + 255) / 256)), dim3(256), 0, s, kind, n, neg, grade,
                           isq_par, reinterpret_cast<const float4*>(x), reinterpret_cast<float4*>(y), nchunks);
    } else {
        const long long total = (long long)batch << n;
        hipLaunchKernelGGL(graded_scalar, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, kind, n, neg, grade,
                           isq_par, x, y, total);
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int norm_sq_fwd(int n, uint32_t neg, uint32_t nul, const float* x, float* out, int64_t batch, void* stream) {
    int rc = check_graded_common(n, neg, nul, batch);
    if (rc) return rc;
    if (batch == 0) return CLF_OK;
    if (!x || !out) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (((uintptr_t)x) & 15u) return set_error(CLF_ERR_ARG, "x must be 16-byte aligned");
    const int chunks = n >= 2 ? (1 << (n - 2)) : (1 << n);
    int tpr_log = 0;
    while ((1 << tpr_log) < chunks && tpr_log < 6) ++tpr_log;
    const long long threads = (long long)batch << tpr_log;
    hipLaunchKernelGGL(norm_sq_fwd_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       n, neg, nul, tpr_log, x, out, (long long)batch);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int norm_sq_bwd(int n, uint32_t neg, uint32_t nul, const float* x, const float* gout, float* gx, int64_t batch,
                void* stream) {
    int rc = check_graded_common(n, neg, nul, batch);
    if (rc) return rc;
    if (batch == 0) return CLF_OK;
    if (!x || !gout || !gx) return set_error(CLF_ERR_ARG, "null pointer argument");
    const long long total = (long long)batch << n;
    hipLaunchKernelGGL(norm_sq_bwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, n,
                       neg, nul, x, gout, gx, total);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
