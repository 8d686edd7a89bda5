// Broadcast-weight products on gfx950 MFMA: y = op(x, w) (or op(w, x)) with one
// weight multivector w shared by every row, as the product layers compute it
// (reference layers.py:43-47, which expands w to (batch, 2^n) and runs the
// per-row kernel).
//
// For a fixed w the product is linear in x: y = x M_w with the signed D x D
// matrix
//   side 0 (x op w): M_w[i, kout] = sigma_op(i, i^k)     w[i^k]
//   side 1 (w op x): M_w[j, kout] = sigma_op(j^k, j)     w[j^k]
// (kout = k, or ~k for the regressive product). Forward is one fp32 MFMA GEMM
// (batch x D) * (D x D); backward is gx = gy M_w^T (a second GEMM) and
// gw[m] = sum_{(i,kout) fed by w[m]} sigma * G[i, kout] with G = x^T gy, a
// split-K MFMA GEMM over the batch followed by a deterministic reduction.
//
// GEMM kernel: 256 threads, 128 x 128 output tile, K staged through LDS in
// chunks of 32, each wave a 64 x 64 sub-tile of 2 x 2 v_mfma_f32_32x32x2f32
// blocks (operand lanes: A[m = l%32][k = l/32], B[k = l/32][n = l%32];
// accumulator element e of lane l: row 8*(e/4) + 4*(l/32) + e%4, column l%32).
#include "clf_common.h"

namespace clf {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 128, GBK = 32, GPAD = 4;
constexpr int kBcastMinN = 7;  // D >= 128: whole 128-wide tiles

// C[M x N] (+ split stride) = op(A) * B over the K range of this split.
//   TA == false: A row-major [M x K], lda = K
//   TA == true : A row-major [K x M], lda = M (op(A) = A^T)
//   B row-major [K x N], ldb = N; C row-major, ldc = N
template <bool TA>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const float* __restrict__ A, const float* __restrict__ Bm,
                                                         float* __restrict__ C, long long M, int N, long long K,
                                                         long long k_per_split) {
    __shared__ float As[GBK][GBM + GPAD];
    __shared__ float Bs[GBK][GBN + GPAD];
    const long long m_base = (long long)blockIdx.x * GBM;
    const int n_base = blockIdx.y * GBN;
    const long long k_begin = (long long)blockIdx.z * k_per_split;
    const long long k_end = (k_begin + k_per_split < K) ? (k_begin + k_per_split) : K;
    C += (long long)blockIdx.z * M * N;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    for (long long k0 = k_begin; k0 < k_end; k0 += GBK) {
        __syncthreads();  // the previous chunk's fragments have been read
        // A tile -> As[k][m]
        if (!TA) {
            // 128 rows x 32 k: thread reads 4 consecutive k of one row, 4 passes
#pragma unroll
            for (int pass = 0; pass < 4; ++pass) {
                const int mr = pass * 32 + (tid >> 3);
                const int kc = (tid & 7) * 4;
                const long long gm = m_base + mr;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (gm < M) v = *reinterpret_cast<const float4*>(A + gm * K + k0 + kc);
                As[kc + 0][mr] = v.x;
                As[kc + 1][mr] = v.y;
                As[kc + 2][mr] = v.z;
                As[kc + 3][mr] = v.w;
            }
        } else {
            // 32 k-rows x 128 m: thread reads 4 consecutive m of one k-row, 4 passes
#pragma unroll
            for (int pass = 0; pass < 4; ++pass) {
                const int kr = pass * 8 + (tid >> 5);
                const int mc = (tid & 31) * 4;
                const long long gk = k0 + kr;
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (gk < k_end) v = *reinterpret_cast<const float4*>(A + gk * M + m_base + mc);
                *reinterpret_cast<float4*>(&As[kr][mc]) = v;
            }
        }
        // B tile -> Bs[k][n]
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) {
            const int kr = pass * 8 + (tid >> 5);
            const int nc = (tid & 31) * 4;
            const long long gk = k0 + kr;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (gk < k_end) v = *reinterpret_cast<const float4*>(Bm + gk * N + n_base + nc);
            *reinterpret_cast<float4*>(&Bs[kr][nc]) = v;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < GBK; kk += 2) {
            const float a0 = As[kk + lk][wm * 64 + lr];
            const float a1 = As[kk + lk][wm * 64 + 32 + lr];
            const float b0 = Bs[kk + lk][wn * 64 + lr];
            const float b1 = Bs[kk + lk][wn * 64 + 32 + lr];
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const long long row = m_base + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
                const int col = n_base + wn * 64 + j * 32 + lr;
                if (row < M) C[row * N + col] = acc[i][j][e];
            }
}

// M (and/or its transpose) from w
__global__ __launch_bounds__(256) void bcast_build_kernel(int op, int side, int n, unsigned neg, unsigned nul,
                                                           const float* __restrict__ w, float* __restrict__ Mw,
                                                           float* __restrict__ MwT) {
    const unsigned D = 1u << n;
    const unsigned idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= D * D) return;
    const unsigned r = idx >> n;        // input blade (row of M)
    const unsigned kout = idx & (D - 1);
    const unsigned k = (op == OP_REGR) ? (~kout & (D - 1)) : kout;
    const unsigned m = r ^ k;           // weight blade
    const int s = side == 0 ? full_sign(op, n, r, m, neg, nul) : full_sign(op, n, m, r, neg, nul);
    const float v = s ? (float)s * w[m] : 0.f;
    if (Mw) Mw[idx] = v;
    if (MwT) MwT[kout * D + r] = v;
}

// G = sum over splits of the partial products (D*D entries, one per thread)
__global__ __launch_bounds__(256) void bcast_reduce_kernel(const float* __restrict__ parts, int nsplit, int DD,
                                                            float* __restrict__ G) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= DD) return;
    float t = 0.f;
    for (int s = 0; s < nsplit; ++s) t += parts[(long long)s * DD + idx];
    G[idx] = t;
}

__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ p, long long count) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = 0.f;
}

// gw[m] = sum_r sigma * G[r, kout(r ^ m)]
__global__ __launch_bounds__(256) void bcast_gw_kernel(int op, int side, int n, unsigned neg, unsigned nul,
                                                        const float* __restrict__ G, float* __restrict__ gw) {
    const unsigned D = 1u << n;
    const unsigned m = blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= D) return;
    float t = 0.f;
    for (unsigned r = 0; r < D; ++r) {
        const int s = side == 0 ? full_sign(op, n, r, m, neg, nul) : full_sign(op, n, m, r, neg, nul);
        if (!s) continue;
        const unsigned k = r ^ m;
        const unsigned kout = (op == OP_REGR) ? (~k & (D - 1)) : k;
        t = __builtin_fmaf((float)s, G[r * D + kout], t);
    }
    gw[m] = t;
}

// ---- host side --------------------------------------------------------------

static int bcast_splits(int64_t batch) {
    long long s = (batch + 2047) / 2048;
    if (s > 128) s = 128;
    if (s < 1) s = 1;
    return (int)s;
}

size_t bcast_ws_bytes(int n, int64_t batch) {
    if (n < kBcastMinN || n > kMaxN || batch < 0) return 0;
    const size_t DD = (size_t)1 << (2 * n);
    return (2 + (size_t)bcast_splits(batch) + 1) * DD * sizeof(float);
}

static int check_bcast(int op, int side, int n, uint32_t neg, uint32_t nul, int64_t batch) {
    if (op < CLF_OP_GEOM || op > CLF_OP_REGRESSIVE) return set_error(CLF_ERR_ARG, "unknown product op");
    if (side != 0 && side != 1) return set_error(CLF_ERR_ARG, "side must be 0 (x op w) or 1 (w op x)");
    if (n < kBcastMinN || n > 10)
        return set_error(CLF_ERR_ARG, "broadcast products support n in [" + std::to_string(kBcastMinN) + ", 10], got " +
                                          std::to_string(n));
    const uint32_t full = (1u << n) - 1u;
    if ((neg & ~full) || (nul & ~full)) return set_error(CLF_ERR_ARG, "metric masks have bits above n");
    if (neg & nul) return set_error(CLF_ERR_ARG, "neg_mask and null_mask overlap");
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (op == CLF_OP_REGRESSIVE && nul)
        return set_error(CLF_ERR_UNSUPPORTED,
                         "regressive_prod is undefined for degenerate metrics (any 0 in the metric makes the "
                         "pseudoscalar non-invertible)");
    return CLF_OK;
}

static void launch_gemm(bool ta, const float* A, const float* B, float* C, long long M, int N, long long K,
                        long long kps, int splits, hipStream_t s) {
    const dim3 grid((unsigned)((M + GBM - 1) / GBM), (unsigned)(N / GBN), (unsigned)splits);
    if (ta) hipLaunchKernelGGL((gemm_mfma_kernel<true>), grid, dim3(256), 0, s, A, B, C, M, N, K, kps);
    else hipLaunchKernelGGL((gemm_mfma_kernel<false>), grid, dim3(256), 0, s, A, B, C, M, N, K, kps);
}

int bcast_fwd(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w, float* y,
              int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = check_bcast(op, side, n, neg, nul, batch)) return rc;
    if (!w || !ws) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (ws_bytes < bcast_ws_bytes(n, batch))
        return set_error(CLF_ERR_WORKSPACE, "workspace of at least " + std::to_string(bcast_ws_bytes(n, batch)) +
                                                " bytes required");
    if (batch == 0) return CLF_OK;
    if (!x || !y) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (x == y) return set_error(CLF_ERR_ARG, "output must not alias the input");
    if ((((uintptr_t)x) | ((uintptr_t)y) | ((uintptr_t)ws)) & 15u)
        return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    const int D = 1 << n;
    float* Mw = (float*)ws;
    hipLaunchKernelGGL(bcast_build_kernel, dim3((unsigned)((D * D + 255) / 256)), dim3(256), 0, s, op, side, n, neg,
                       nul, w, Mw, (float*)nullptr);
    launch_gemm(false, x, Mw, y, batch, D, D, D, 1, s);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int bcast_bwd(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w, const float* gy,
              float* gx, float* gw, int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = check_bcast(op, side, n, neg, nul, batch)) return rc;
    if (!gx && !gw) return CLF_OK;
    if (!w || !ws || (batch > 0 && (!gy || (gw && !x)))) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (ws_bytes < bcast_ws_bytes(n, batch))
        return set_error(CLF_ERR_WORKSPACE, "workspace of at least " + std::to_string(bcast_ws_bytes(n, batch)) +
                                                " bytes required");
    if ((((uintptr_t)x) | ((uintptr_t)gy) | ((uintptr_t)gx) | ((uintptr_t)ws)) & 15u)
        return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    const int D = 1 << n;
    const size_t DD = (size_t)D * D;
    float* MwT = (float*)ws + DD;
    float* parts = (float*)ws + 2 * DD;
    const int splits = bcast_splits(batch);
    float* G = parts + (size_t)splits * DD;
    if (gx && batch > 0) {
        hipLaunchKernelGGL(bcast_build_kernel, dim3((unsigned)((DD + 255) / 256)), dim3(256), 0, s, op, side, n, neg,
                           nul, w, (float*)nullptr, MwT);
        launch_gemm(false, gy, MwT, gx, batch, D, D, D, 1, s);
    }
    if (gw) {
        if (batch > 0) {
            const long long kps = ((batch + splits - 1) / splits + GBK - 1) / GBK * GBK;
            const int used = (int)((batch + kps - 1) / kps);
            launch_gemm(true, x, gy, parts, D, D, batch, kps, used, s);
            hipLaunchKernelGGL(bcast_reduce_kernel, dim3((unsigned)((DD + 255) / 256)), dim3(256), 0, s, parts, used,
                               (int)DD, G);
        } else {
            hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((DD + 255) / 256)), dim3(256), 0, s, G, (long long)DD);
        }
        hipLaunchKernelGGL(bcast_gw_kernel, dim3((unsigned)((D + 255) / 256)), dim3(256), 0, s, op, side, n, neg, nul,
                           G, gw);
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
