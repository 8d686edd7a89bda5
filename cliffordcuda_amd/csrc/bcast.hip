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
// GEMM kernels: 256 threads, 128 x 128 output tile, K staged through LDS in
// chunks of 32, each wave a 64 x 64 sub-tile of 2 x 2 v_mfma_f32_32x32x2f32
// blocks (operand lanes: A[m = l%32][k = l/32], B[k = l/32][n = l%32];
// accumulator element e of lane l: row 8*(e/4) + 4*(l/32) + e%4, column l%32).
#include <atomic>
#include <mutex>

#include "clf_common.h"

namespace clf {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 128, GBK = 32, GPAD = 4;
constexpr int kBcastMinN = 7;  // D >= 128: whole 128-wide tiles

// Split-K C_z[M x N] = A^T B over rows [z * k_per_split, ...) of A and B,
// A row-major [K x M], B row-major [K x N] (the weight-gradient product
// x^T gy). Both tiles are stored k-major in LDS exactly as they sit in HBM;
// rows past the split's end are loaded clamped and zeroed (no branches). The
// next chunk is prefetched into registers while the current one is consumed.
// ldb: floats between the k-rows of Bm (N, or 0 for one row broadcast over K)
__global__ __launch_bounds__(256) void gemm_tn_kernel(const float* __restrict__ A, const float* __restrict__ Bm,
                                                       float* __restrict__ C, int M, int N, long long K,
                                                       long long k_per_split, long long ldb) {
    __shared__ float As[GBK][GBM + GPAD];
    __shared__ float Bs[GBK][GBN + GPAD];
    const int m_base = blockIdx.x * GBM;
    const int n_base = blockIdx.y * GBN;
    const long long k_begin = (long long)blockIdx.z * k_per_split;
    const long long k_end = (k_begin + k_per_split < K) ? (k_begin + k_per_split) : K;
    C += (long long)blockIdx.z * M * N;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lg = lane >> 5;
    const int krow = tid >> 5, col4 = (tid & 31) * 4;  // loader: 8 k-rows x 32 float4 per pass

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    float4 ra0, ra1, ra2, ra3, rb0, rb1, rb2, rb3;
#define CLF_TN_FETCH1(P, K0)                                                               \
    {                                                                                      \
        const long long kr = (K0) + (P) * 8 + krow;                                        \
        const bool ok = kr < k_end;                                                        \
        const long long kc = ok ? kr : (k_end - 1);                                        \
        ra##P = *reinterpret_cast<const float4*>(A + kc * M + m_base + col4);              \
        rb##P = *reinterpret_cast<const float4*>(Bm + kc * ldb + n_base + col4);           \
        if (!ok) {                                                                         \
            ra##P = make_float4(0.f, 0.f, 0.f, 0.f);                                       \
            rb##P = make_float4(0.f, 0.f, 0.f, 0.f);                                       \
        }                                                                                  \
    }
#define CLF_TN_FETCH(K0) CLF_TN_FETCH1(0, K0) CLF_TN_FETCH1(1, K0) CLF_TN_FETCH1(2, K0) CLF_TN_FETCH1(3, K0)
    CLF_TN_FETCH(k_begin)
    for (long long k0 = k_begin; k0 < k_end; k0 += GBK) {
        __syncthreads();  // the previous chunk's fragments have been read
        *reinterpret_cast<float4*>(&As[krow][col4]) = ra0;
        *reinterpret_cast<float4*>(&As[8 + krow][col4]) = ra1;
        *reinterpret_cast<float4*>(&As[16 + krow][col4]) = ra2;
        *reinterpret_cast<float4*>(&As[24 + krow][col4]) = ra3;
        *reinterpret_cast<float4*>(&Bs[krow][col4]) = rb0;
        *reinterpret_cast<float4*>(&Bs[8 + krow][col4]) = rb1;
        *reinterpret_cast<float4*>(&Bs[16 + krow][col4]) = rb2;
        *reinterpret_cast<float4*>(&Bs[24 + krow][col4]) = rb3;
        __syncthreads();
        {
            const long long kn = (k0 + GBK < k_end) ? (k0 + GBK) : k0;
            CLF_TN_FETCH(kn)
        }
#pragma unroll
        for (int kk = 0; kk < GBK; kk += 2) {
            const float a0 = As[kk + lg][wm * 64 + lr];
            const float a1 = As[kk + lg][wm * 64 + 32 + lr];
            const float b0 = Bs[kk + lg][wn * 64 + lr];
            const float b1 = Bs[kk + lg][wn * 64 + 32 + lr];
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
        }
    }
#undef CLF_TN_FETCH
#undef CLF_TN_FETCH1
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m_base + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * lg + (e & 3);
                const int col = n_base + wn * 64 + j * 32 + lr;
                C[(long long)row * N + col] = acc[i][j][e];
            }
}

// C[M x N] = A * B with A row-major [M x K] and B given transposed, Bt
// row-major [N x K]: both operand tiles are k-contiguous in LDS, so a lane reads
// four k values of its row with one 16-byte LDS read. The reduction index is
// permuted inside each 8-wide k block (MFMA step s takes k = 8kb + s on lanes
// 0-31 and k = 8kb + 4 + s on lanes 32-63; A and B use the same permutation).
// The next K chunk is loaded into registers while the current one is consumed.
constexpr int NBK = 32, NPAD = 4;
// lda: floats between the rows of A (K, or 0 for one row broadcast over M)
__global__ __launch_bounds__(256) void gemm_nn_kernel(const float* __restrict__ A, const float* __restrict__ Bt,
                                                       float* __restrict__ C, long long M, int N, int K,
                                                       long long lda) {
    __shared__ float As[GBM][NBK + NPAD];
    __shared__ float Bs[GBN][NBK + NPAD];
    const long long m_base = (long long)blockIdx.x * GBM;
    const int n_base = blockIdx.y * GBN;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lg = lane >> 5;
    const int lrow = tid >> 3, lk = (tid & 7) * 4;  // loader: 32 rows x 8 float4 per pass

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    float4 ra0, ra1, ra2, ra3, rb0, rb1, rb2, rb3;
#define CLF_NN_FETCH1(P, K0)                                                                                  \
    {                                                                                                         \
        /* rows past M read row M-1 (always valid); their results are never stored */                  \
        const long long gm = (m_base + (P) * 32 + lrow) < M ? (m_base + (P) * 32 + lrow) : (M - 1);          \
        ra##P = *reinterpret_cast<const float4*>(A + gm * lda + (K0) + lk);                                  \
        rb##P = *reinterpret_cast<const float4*>(Bt + (long long)(n_base + (P) * 32 + lrow) * K + (K0) + lk);   \
    }
#define CLF_NN_FETCH(K0) CLF_NN_FETCH1(0, K0) CLF_NN_FETCH1(1, K0) CLF_NN_FETCH1(2, K0) CLF_NN_FETCH1(3, K0)
    CLF_NN_FETCH(0)
    for (int k0 = 0; k0 < K; k0 += NBK) {
        __syncthreads();  // the previous chunk's fragments have been read
        *reinterpret_cast<float4*>(&As[lrow][lk]) = ra0;
        *reinterpret_cast<float4*>(&As[32 + lrow][lk]) = ra1;
        *reinterpret_cast<float4*>(&As[64 + lrow][lk]) = ra2;
        *reinterpret_cast<float4*>(&As[96 + lrow][lk]) = ra3;
        *reinterpret_cast<float4*>(&Bs[lrow][lk]) = rb0;
        *reinterpret_cast<float4*>(&Bs[32 + lrow][lk]) = rb1;
        *reinterpret_cast<float4*>(&Bs[64 + lrow][lk]) = rb2;
        *reinterpret_cast<float4*>(&Bs[96 + lrow][lk]) = rb3;
        __syncthreads();
        {
            // prefetch the next chunk (the last iteration re-reads its own chunk: no branch)
            const int kn = (k0 + NBK < K) ? (k0 + NBK) : k0;
            CLF_NN_FETCH(kn)
        }
#pragma unroll
        for (int kb = 0; kb < NBK / 8; ++kb) {
            const int kc = kb * 8 + 4 * lg;
            const float4 a0 = *reinterpret_cast<const float4*>(&As[wm * 64 + lr][kc]);
            const float4 a1 = *reinterpret_cast<const float4*>(&As[wm * 64 + 32 + lr][kc]);
            const float4 b0 = *reinterpret_cast<const float4*>(&Bs[wn * 64 + lr][kc]);
            const float4 b1 = *reinterpret_cast<const float4*>(&Bs[wn * 64 + 32 + lr][kc]);
#define CLF_NN_STEP(F)                                                                       \
    acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.F, b0.F, acc[0][0], 0, 0, 0);        \
    acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.F, b1.F, acc[0][1], 0, 0, 0);        \
    acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.F, b0.F, acc[1][0], 0, 0, 0);        \
    acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.F, b1.F, acc[1][1], 0, 0, 0);
            CLF_NN_STEP(x)
            CLF_NN_STEP(y)
            CLF_NN_STEP(z)
            CLF_NN_STEP(w)
#undef CLF_NN_STEP
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const long long row = m_base + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * lg + (e & 3);
                const int col = n_base + wn * 64 + j * 32 + lr;
                if (row < M) C[row * N + col] = acc[i][j][e];
            }
#undef CLF_NN_FETCH
#undef CLF_NN_FETCH1
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

// G = sum over splits of the partial products (four entries per thread)
__global__ __launch_bounds__(256) void bcast_reduce_kernel(const float4* __restrict__ parts, int nsplit, int DD4,
                                                            float4* __restrict__ G) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= DD4) return;
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < nsplit; ++s) {
        const float4 v = parts[(long long)s * DD4 + idx];
        t.x += v.x;
        t.y += v.y;
        t.z += v.z;
        t.w += v.w;
    }
    G[idx] = t;
}

__global__ __launch_bounds__(256) void zero_kernel(float* __restrict__ p, long long count) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = 0.f;
}

// gw[m] = sum_r sigma * G[r, kout(r ^ m)]: one wave per output blade m, lanes
// stride over r, then a butterfly sum
__global__ __launch_bounds__(256) void bcast_gw_kernel(int op, int side, int n, unsigned neg, unsigned nul,
                                                        const float* __restrict__ G, float* __restrict__ gw) {
    const unsigned D = 1u << n;
    const unsigned m = blockIdx.x * 4 + (threadIdx.x >> 6);
    const unsigned lane = threadIdx.x & 63;
    float t = 0.f;
    if (m < D) {
        for (unsigned r = lane; r < D; r += 64) {
            const int s = side == 0 ? full_sign(op, n, r, m, neg, nul) : full_sign(op, n, m, r, neg, nul);
            if (!s) continue;
            const unsigned k = r ^ m;
            const unsigned kout = (op == OP_REGR) ? (~k & (D - 1)) : k;
            t = __builtin_fmaf((float)s, G[r * D + kout], t);
        }
    }
    for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, 64);
    if (m < D && lane == 0) gw[m] = t;
}

// ---- host side --------------------------------------------------------------

bool rep_bcast_applicable(int op, int n, uint32_t neg, uint32_t nul);
size_t rep_bcast_ws_floats(int64_t batch);
int rep_bcast_fwd(int side, int n, uint32_t neg, const float* x, const float* w, float* y, int64_t batch,
                  void* stream);
int rep_bcast_bwd(int side, int n, uint32_t neg, const float* x, const float* w, const float* gy, int64_t ldg,
                  float* gx, float* gw, int64_t batch, float* ws, void* stream);

static int bcast_splits(int64_t batch, int cap = 128) {
    long long s = (batch + 2047) / 2048;
    if (s > cap) s = cap;
    if (s < 1) s = 1;
    return (int)s;
}

// The GEMM path's workspace; it also covers the matrix-representation path's
// weight-gradient partials (256 floats per workgroup, at most 2048 workgroups
// and at most 16 * batch floats, below (3 + splits) * 2^(2n) for n >= 7).
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

static void launch_tn(const float* A, const float* B, float* C, int D, long long K, long long kps, int splits,
                      hipStream_t s, long long ldb) {
    const dim3 grid((unsigned)(D / GBM), (unsigned)(D / GBN), (unsigned)splits);
    hipLaunchKernelGGL(gemm_tn_kernel, grid, dim3(256), 0, s, A, B, C, D, D, K, kps, ldb);
}

// C = A * Bt^T, A (rows x D, rows lda apart), Bt (D x D) given transposed
static void launch_nn(const float* A, const float* Bt, float* C, long long rows, int D, hipStream_t s,
                      long long lda) {
    const dim3 grid((unsigned)((rows + GBM - 1) / GBM), (unsigned)(D / GBN));
    hipLaunchKernelGGL(gemm_nn_kernel, grid, dim3(256), 0, s, A, Bt, C, rows, D, D, lda);
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
    if (rep_bcast_applicable(op, n, neg, nul)) return rep_bcast_fwd(side, n, neg, x, w, y, batch, stream);
    hipStream_t s = (hipStream_t)stream;
    const int D = 1 << n;
    float* MwT = (float*)ws;
    hipLaunchKernelGGL(bcast_build_kernel, dim3((unsigned)((D * D + 255) / 256)), dim3(256), 0, s, op, side, n, neg,
                       nul, w, (float*)nullptr, MwT);
    launch_nn(x, MwT, y, batch, D, s, D);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

// Argument checks shared by both backward entry points (no HIP call).
// gy's rows are ldg floats apart: 2^n, or 0 for one row broadcast over the batch
static int check_bcast_bwd_args(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w,
                                const float* gy, int64_t ldg, float* gx, float* gw, int64_t batch) {
    if (int rc = check_bcast(op, side, n, neg, nul, batch)) return rc;
    if (ldg != 0 && ldg != (1LL << n)) return set_error(CLF_ERR_ARG, "gy row stride must be 0 or 2^n");
    if (!gx && !gw) return CLF_OK;
    if (!w || (batch > 0 && (!gy || (gw && !x)))) return set_error(CLF_ERR_ARG, "null pointer argument");
    if ((((uintptr_t)x) | ((uintptr_t)gy) | ((uintptr_t)gx)) & 15u)
        return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    return CLF_OK;
}

// The backward's launches on an already checked workspace. GEMM path layout:
// [0, DD) the weight matrix for gx, [DD, 2 DD) unused (the forward's transposed
// matrix), then `splits` partial products of x^T gy and their sum G; the split
// count is at most max_splits.
static int bcast_bwd_launch(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w,
                            const float* gy, int64_t ldg, float* gx, float* gw, int64_t batch, float* ws,
                            int max_splits, void* stream) {
    if (rep_bcast_applicable(op, n, neg, nul))
        return rep_bcast_bwd(side, n, neg, x, w, gy, ldg, gx, gw, batch, ws, stream);
    hipStream_t s = (hipStream_t)stream;
    const int D = 1 << n;
    const size_t DD = (size_t)D * D;
    float* parts = ws + 2 * DD;
    const int splits = bcast_splits(batch, max_splits);
    float* G = parts + (size_t)splits * DD;
    if (gx && batch > 0) {
        float* Mw = ws;
        hipLaunchKernelGGL(bcast_build_kernel, dim3((unsigned)((DD + 255) / 256)), dim3(256), 0, s, op, side, n, neg,
                           nul, w, Mw, (float*)nullptr);
        launch_nn(gy, Mw, gx, batch, D, s, ldg);
    }
    if (gw) {
        if (batch > 0) {
            const long long kps = ((batch + splits - 1) / splits + GBK - 1) / GBK * GBK;
            const int used = (int)((batch + kps - 1) / kps);
            launch_tn(x, gy, parts, D, batch, kps, used, s, ldg);
            hipLaunchKernelGGL(bcast_reduce_kernel, dim3((unsigned)((DD / 4 + 255) / 256)), dim3(256), 0, s,
                               reinterpret_cast<const float4*>(parts), used, (int)(DD / 4), reinterpret_cast<float4*>(G));
        } else {
            hipLaunchKernelGGL(zero_kernel, dim3((unsigned)((DD + 255) / 256)), dim3(256), 0, s, G, (long long)DD);
        }
        hipLaunchKernelGGL(bcast_gw_kernel, dim3((unsigned)((D + 3) / 4)), dim3(256), 0, s, op, side, n, neg, nul, G,
                           gw);
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int bcast_bwd(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w, const float* gy,
              int64_t ldg, float* gx, float* gw, int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = check_bcast_bwd_args(op, side, n, neg, nul, x, w, gy, ldg, gx, gw, batch)) return rc;
    if (!gx && !gw) return CLF_OK;
    if (!ws) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (((uintptr_t)ws) & 15u) return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    if (ws_bytes < bcast_ws_bytes(n, batch))
        return set_error(CLF_ERR_WORKSPACE, "workspace of at least " + std::to_string(bcast_ws_bytes(n, batch)) +
                                                " bytes required");
    if (rep_bcast_applicable(op, n, neg, nul) && rep_bcast_ws_floats(batch) * sizeof(float) > ws_bytes)
        return set_error(CLF_ERR_WORKSPACE, "workspace too small for the weight-gradient partials");
    return bcast_bwd_launch(op, side, n, neg, nul, x, w, gy, ldg, gx, gw, batch, (float*)ws, 128, stream);
}

// ---- allocation-free backward ------------------------------------------------
// The same backward with its workspace in a fixed device array instead of a
// caller buffer, for callers that cannot allocate (code under graph capture,
// serving loops). The array lives for the whole process on every device the
// entry point runs on. Its host-side name is only a stand-in for the symbol:
// the device address comes from hipGetSymbolAddress, looked up once per device
// with that device current, and only that address is ever passed to kernels.
// Every call on a device shares the array; calls that overlap on one device
// (different streams or threads) race on it. No kernel relies on its previous
// contents: every workspace entry a launch reads was written earlier in the
// same call.
constexpr size_t kBcastScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) float scratch[kBcastScratchBytes / sizeof(float)];

constexpr int kScratchMaxDevices = 64;
static std::atomic<float*> g_scratch_ptr[kScratchMaxDevices];
static std::mutex g_scratch_mu;

static int scratch_address(float** out) {
    int dev = 0;
    CLF_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= kScratchMaxDevices) return set_error(CLF_ERR_ARG, "device index beyond the scratch table");
    float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            void* addr = nullptr;
            CLF_HIP_CHECK(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)));
            if (!addr) return set_error(CLF_ERR_HIP, "hipGetSymbolAddress returned a null scratch address");
            p = (float*)addr;
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return CLF_OK;
}

size_t bcast_scratch_bytes() { return kBcastScratchBytes; }

// Split count that keeps the GEMM path's workspace inside the scratch array.
static int noalloc_max_splits(int n) {
    const size_t DD = (size_t)1 << (2 * n);
    const long long slots = (long long)(kBcastScratchBytes / (DD * sizeof(float)));
    return (int)(slots - 3);
}

int bcast_bwd_noalloc(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w,
                      const float* gy, int64_t ldg, float* gx, float* gw, int64_t batch, void* stream) {
    if (int rc = check_bcast_bwd_args(op, side, n, neg, nul, x, w, gy, ldg, gx, gw, batch)) return rc;
    if (!gx && !gw) return CLF_OK;
    size_t need;
    if (rep_bcast_applicable(op, n, neg, nul)) {
        need = rep_bcast_ws_floats(batch) * sizeof(float);
    } else {
        const int cap = noalloc_max_splits(n);
        if (cap < 1)
            return set_error(CLF_ERR_WORKSPACE, "n = " + std::to_string(n) + " needs more than the " +
                                                    std::to_string(kBcastScratchBytes) + "-byte scratch array");
        need = (3 + (size_t)bcast_splits(batch, cap)) * ((size_t)1 << (2 * n)) * sizeof(float);
    }
    if (need > kBcastScratchBytes)
        return set_error(CLF_ERR_WORKSPACE, "this call needs " + std::to_string(need) + " bytes of scratch; the " +
                                                "allocation-free backward has " + std::to_string(kBcastScratchBytes));
    float* ws = nullptr;
    if (int rc = scratch_address(&ws)) return rc;
    return bcast_bwd_launch(op, side, n, neg, nul, x, w, gy, ldg, gx, gw, batch, ws, noalloc_max_splits(n),
                            stream);
}

}  // namespace clf
