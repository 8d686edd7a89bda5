// Rotor path on gfx950: bivector -> rotation -> plane-rotation chain, the
// sandwich ~R x R applied to a batch of multivectors, and gradients to the
// bivector and to x.
//
// What is computed (the composite of reference algebra.py:343-373, Euclidean):
//   B = 2 (M - M^T), M[i_m, j_m] = b_m (lex pairs, kernels/rotor/eigh_exp.cu:283-288)
//   Q = expm(-B)                 the grade-1 action of ~R x R, R = exp(sum b_m e_{i_m} e_{j_m})
//   Q = G_1 G_2 ... G_C          Givens factorisation, planes (p, q) in lex order,
//                                G_k e_p = c e_p + s e_q, G_k e_q = -s e_p + c e_q
//   y = Lambda(Q) x              outermorphism: Lambda(G_1)(...(Lambda(G_C) x))
// A plane rotation acts on the blade pairs (I with p not q, J = I ^ {p,q}):
//   y_I = c x_I - s sig x_J,  y_J = c x_J + s sig x_I,  sig = (-1)^{|I & (p, q)|}
// (bits of I strictly between p and q).
//
// Gradients. With gx = Lambda(Q)^T gy (the chain run backwards with s -> -s),
//   dL/dQ = Q Gamma,  Gamma_ab = sum_rows sum_{I: b in I, a not in I} sig x_I gx_{I^{a,b}}
// (the derivation extension of Q^{-1} dQ; only its antisymmetric part matters,
// since Q stays orthogonal), and the bivector gradient follows
// from the adjoint Frechet derivative of expm:
//   dL/dA = [expm([[A^T, dL/dQ], [0, A^T]])]_{12},  A = -B,
//   dL/db_m = 2 (dL/dB[i_m][j_m] - dL/dB[j_m][i_m]),  dL/dB = -dL/dA.
// The reference instead runs torch eigh + a closed form + Givens kernels with
// host syncs and returns no gradient to x (extensions/rotor/*.py).
//
// Apply layout: one row is spread over 2^(n-RB) lanes, each holding 2^RB
// consecutive blades in registers. Planes inside the register bits are pure
// FMAs; planes touching lane bits exchange partner values with lane shuffles.
// The plane list is unrolled at compile time per n.
#include <utility>

#include "rep_common.h"

namespace clf {

constexpr int kRotorMinN = 2;
constexpr int kRotorMaxN = 10;

__host__ __device__ constexpr int n_planes(int n) { return n * (n - 1) / 2; }
__host__ __device__ constexpr int plane_p(int n, int k) {
    int p = 0;
    while (k >= n - 1 - p) {
        k -= n - 1 - p;
        ++p;
    }
    return p;
}
__host__ __device__ constexpr int plane_q(int n, int k) {
    int p = 0;
    while (k >= n - 1 - p) {
        k -= n - 1 - p;
        ++p;
    }
    return p + 1 + k;
}
// register bits per lane: rows of n <= 8 use 4 lanes (partner exchanges are
// quad-local DPP permutes), n = 9, 10 use 8 / 16 lanes of 64 blades each
__host__ __device__ constexpr int rotor_rb(int n) { return n < 4 ? n : (n <= 8 ? n - 2 : 6); }
// parity of the bits of r strictly between positions p and q (p < q)
__host__ __device__ constexpr int between_par(unsigned r, int p, int q) {
    int c = 0;
    for (int b = p + 1; b < q; ++b) c += (r >> b) & 1u;
    return c & 1;
}
// state: Q (n x n), the (c, s) pairs of the chain, and for n = 8 also the
// 16 x 16 matrix U = phi(R) of the Cl(8,0) representation (row-major)
__host__ __device__ constexpr int spin_offset(int n) { return n * n + 2 * n_planes(n); }
__host__ __device__ constexpr int state_floats(int n) { return spin_offset(n) + (n == kSpinN ? 256 : 0); }

// ---- the plane-rotation chain on register-resident rows ---------------------

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// value of v in lane (lane ^ MASK) for MASK < 32: quad-local bits by DPP quad
// permutes (full-rate VALU), bits 2..4 by one ds_swizzle in bit-mask mode
template <unsigned MASK>
__device__ __forceinline__ float lane_xor(float v) {
    static_assert(MASK < 32, "lane exchange limited to 32 lanes");
    float r = v;
    if constexpr ((MASK & 3u) == 1u) r = dpp_mov<0xB1>(r);       // quad_perm [1,0,3,2]
    else if constexpr ((MASK & 3u) == 2u) r = dpp_mov<0x4E>(r);  // quad_perm [2,3,0,1]
    else if constexpr ((MASK & 3u) == 3u) r = dpp_mov<0x1B>(r);  // quad_perm [3,2,1,0]
    if constexpr ((MASK & 0x1Cu) != 0u) {
        constexpr int pattern = (int)(((MASK & 0x1Cu) << 10) | 0x1Fu);  // and 0x1F, or 0, xor MASK
        r = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(r), pattern));
    }
    return r;
}

template <int N, int RB, int K, bool FWD>
__device__ __forceinline__ void rot_plane(float (&v)[1 << RB], const float* __restrict__ cs, unsigned L) {
    constexpr int P = plane_p(N, K), Qb = plane_q(N, K);
    constexpr int V = 1 << RB;
    const float c = cs[2 * K];
    const float s = FWD ? cs[2 * K + 1] : -cs[2 * K + 1];
    if constexpr (Qb < RB) {  // both generators in the register bits
        constexpr unsigned mp = 1u << P, mq = 1u << Qb;
#pragma unroll
        for (int r = 0; r < V; ++r) {
            if ((r & mp) && !(r & mq)) {
                const int rj = r ^ (int)(mp | mq);
                const float sg = between_par((unsigned)r, P, Qb) ? -s : s;
                const float xi = v[r], xj = v[rj];
                v[r] = __builtin_fmaf(c, xi, -sg * xj);
                v[rj] = __builtin_fmaf(c, xj, sg * xi);
            }
        }
    } else if constexpr (P < RB) {  // p in registers, q in lanes
        // Pair (I, J): the q-clear lane holds I in r1 = r0 | 2^p, the q-set
        // partner holds J in r0. Both lanes exchange both registers and apply
        //   x1' = a1 x1 + b1 (partner x0),  x0' = a0 x0 + b0 (partner x1)
        // with lane constants (q clear: a1 = c, b1 = -s sig, a0 = 1, b0 = 0;
        // q set: a1 = 1, b1 = 0, a0 = c, b0 = s sig): no selects per pair.
        constexpr unsigned mp = 1u << P;
        constexpr int ql = Qb - RB;
        const bool qset = (L >> ql) & 1u;
        const int lpar = __popc(L & ((1u << ql) - 1u)) & 1;
        const float s_l = lpar ? -s : s;
        const float a1 = qset ? 1.f : c, b1 = qset ? 0.f : -s_l;
        const float a0 = qset ? c : 1.f, b0 = qset ? s_l : 0.f;
#pragma unroll
        for (int r0 = 0; r0 < V; ++r0) {
            if (r0 & mp) continue;
            const int r1 = r0 | (int)mp;
            const bool neg = between_par((unsigned)r1, P, RB);
            const float x0 = v[r0], x1 = v[r1];
            const float p0 = lane_xor<(1u << ql)>(x0);
            const float p1 = lane_xor<(1u << ql)>(x1);
            v[r1] = __builtin_fmaf(a1, x1, (neg ? -b1 : b1) * p0);
            v[r0] = __builtin_fmaf(a0, x0, (neg ? -b0 : b0) * p1);
        }
    } else {  // both in lanes
        constexpr int pl = P - RB, ql = Qb - RB;
        const bool pset = (L >> pl) & 1u, qset = (L >> ql) & 1u;
        const bool part = pset != qset;
        const unsigned between = ((1u << ql) - 1u) & ~((2u << pl) - 1u);
        const int lpar = __popc(L & between) & 1;
        const float sg = lpar ? -s : s;
        const float ce = part ? c : 1.f;
        const float se = part ? (qset ? sg : -sg) : 0.f;
#pragma unroll
        for (int r = 0; r < V; ++r) {
            const float recv = lane_xor<(1u << pl) | (1u << ql)>(v[r]);
            v[r] = __builtin_fmaf(ce, v[r], se * recv);
        }
    }
}

template <int N, int RB, bool FWD, int... Ks>
__device__ __forceinline__ void rot_chain_seq(float (&v)[1 << RB], const float* __restrict__ cs, unsigned L,
                                              std::integer_sequence<int, Ks...>) {
    // forward: Lambda(G_1)(...(Lambda(G_C) x)) -> planes C-1 .. 0; transpose: 0 .. C-1
    constexpr int C = n_planes(N);
    (rot_plane<N, RB, FWD ? (C - 1 - Ks) : Ks, FWD>(v, cs, L), ...);
}

template <int N, int RB, bool FWD>
__device__ __forceinline__ void rot_chain(float (&v)[1 << RB], const float* __restrict__ cs, unsigned L) {
    rot_chain_seq<N, RB, FWD>(v, cs, L, std::make_integer_sequence<int, n_planes(N)>{});
}

template <int RB>
__device__ __forceinline__ void load_row_part(float (&v)[1 << RB], const float* __restrict__ src) {
    if constexpr (RB >= 2) {
        const float4* s4 = reinterpret_cast<const float4*>(src);
#pragma unroll
        for (int q = 0; q < (1 << RB) / 4; ++q) {
            const float4 t = s4[q];
            v[4 * q] = t.x;
            v[4 * q + 1] = t.y;
            v[4 * q + 2] = t.z;
            v[4 * q + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int r = 0; r < (1 << RB); ++r) v[r] = src[r];
    }
}

template <int RB>
__device__ __forceinline__ void store_row_part(const float (&v)[1 << RB], float* __restrict__ dst) {
    if constexpr (RB >= 2) {
        float4* d4 = reinterpret_cast<float4*>(dst);
#pragma unroll
        for (int q = 0; q < (1 << RB) / 4; ++q) d4[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    } else {
#pragma unroll
        for (int r = 0; r < (1 << RB); ++r) dst[r] = v[r];
    }
}

// y = Lambda(Q) x (FWD) or Lambda(Q)^T x (!FWD), one row per 2^(N-RB) lanes.
// Persistent: the lanes of a row walk rows with a grid stride and load the
// next row part while the current one is rotated. Rows past the end are never
// stored; their prefetch re-reads the last row (a cache hit, no branch).
// The loop condition is the same for all lanes of a row, so a row's lanes
// stay active together and every shuffle partner is active.
template <int N, bool FWD>
__global__ __launch_bounds__(256) void rotor_apply_kernel(const float* __restrict__ state,
                                                           const float* __restrict__ X, float* __restrict__ Y,
                                                           long long batch) {
    constexpr int RB = rotor_rb(N);
    constexpr int LB = N - RB;
    const float* cs = state + N * N;
    const unsigned L = threadIdx.x & ((1u << LB) - 1u);
    const long long rows_per_block = 256 >> LB;
    const long long stride = (long long)gridDim.x * rows_per_block;
    long long row = (long long)blockIdx.x * rows_per_block + (threadIdx.x >> LB);
    const long long lane_off = (long long)L << RB;
    float v[1 << RB];
    load_row_part<RB>(v, X + ((row < batch ? row : batch - 1) << N) + lane_off);
    for (; row < batch; row += stride) {
        const long long nrow = row + stride;
        float nv[1 << RB];
        load_row_part<RB>(nv, X + ((nrow < batch ? nrow : batch - 1) << N) + lane_off);
        // an opaque copy of L per row keeps the per-plane lane factors inside
        // the loop instead of being hoisted into VGPRs for all planes
        unsigned Lr = L;
        asm volatile("" : "+v"(Lr));
        rot_chain<N, RB, FWD>(v, cs, Lr);
        store_row_part<RB>(v, Y + (row << N) + lane_off);
#pragma unroll
        for (int r = 0; r < (1 << RB); ++r) v[r] = nv[r];
    }
}

// ---- backward: gx = Lambda(Q)^T gy and the per-workgroup partial skew(Gamma) --
//
// Only the antisymmetric part of Gamma reaches the bivector: Q stays in SO(n),
// so Q^{-1} dQ is antisymmetric and <Gamma, Q^{-1} dQ> = <skew Gamma, Q^{-1} dQ>.
// Per plane (p < q) the kernels accumulate
//   K_pq = Gamma_pq - Gamma_qp = sum_rows sum_pairs sig (x_J gx_I - x_I gx_J)
// (I holds p not q, J = I ^ {p,q}). One accumulator per plane and lane; the
// lane-dependent sign of a term (which side of the pair the lane holds, and the
// lane bits between p and q) is applied when the per-lane sums are combined.

template <int N, int RB, int K>
__device__ __forceinline__ void skew_plane(float* __restrict__ acc, const float (&x)[1 << RB],
                                           const float (&g)[1 << RB], unsigned L) {
    constexpr int P = plane_p(N, K), Qb = plane_q(N, K);
    constexpr int V = 1 << RB;
    if constexpr (Qb < RB) {
        constexpr unsigned mp = 1u << P, mq = 1u << Qb;
#pragma unroll
        for (int r = 0; r < V; ++r) {
            if ((r & mp) && !(r & mq)) {
                const int rj = r ^ (int)(mp | mq);
                const bool neg = between_par((unsigned)r, P, Qb);
                // sig (x_J g_I - x_I g_J)
                acc[K] = __builtin_fmaf(neg ? -x[rj] : x[rj], g[r], acc[K]);
                acc[K] = __builtin_fmaf(neg ? x[r] : -x[r], g[rj], acc[K]);
            }
        }
    } else if constexpr (P < RB) {
        constexpr unsigned mp = 1u << P;
        constexpr int ql = Qb - RB;
        const bool qset = (L >> ql) & 1u;
#pragma unroll
        for (int r0 = 0; r0 < V; ++r0) {
            if (r0 & mp) continue;
            const int r1 = r0 | (int)mp;
            const bool neg = between_par((unsigned)r1, P, RB);
            // q-clear lane owns I = (L, r1), q-set lane owns J = (L, r0); each
            // multiplies its own x by the partner's g (sign applied later)
            const float x0 = x[r0], x1 = x[r1], g0 = g[r0], g1 = g[r1];
            const float xo = qset ? x0 : x1;
            const float go = qset ? g0 : g1;
            const float gp = lane_xor<(1u << ql)>(go);
            acc[K] = __builtin_fmaf(neg ? -xo : xo, gp, acc[K]);
        }
    } else {
        constexpr int pl = P - RB, ql = Qb - RB;
#pragma unroll
        for (int r = 0; r < V; ++r) {
            const float gp = lane_xor<(1u << pl) | (1u << ql)>(g[r]);
            acc[K] = __builtin_fmaf(x[r], gp, acc[K]);
        }
    }
}

template <int N, int RB, int... Ks>
__device__ __forceinline__ void skew_all_seq(float* __restrict__ acc, const float (&x)[1 << RB],
                                             const float (&g)[1 << RB], unsigned L,
                                             std::integer_sequence<int, Ks...>) {
    (skew_plane<N, RB, Ks>(acc, x, g, L), ...);
}

// sign of lane position Lp's accumulator for plane k (0 if the lane holds no pair)
template <int N, int RB>
__device__ __forceinline__ float skew_lane_sign(int k, unsigned Lp) {
    const int p = plane_p(N, k), q = plane_q(N, k);
    if (q < RB) return 1.f;
    if (p < RB) {
        const int ql = q - RB;
        const bool qset = (Lp >> ql) & 1u;
        const bool lneg = __popc(Lp & ((1u << ql) - 1u)) & 1;
        // q-set lane: +sig x_J g_I ; q-clear lane: -sig x_I g_J
        return (qset != lneg) ? 1.f : -1.f;
    }
    const int pl = p - RB, ql = q - RB;
    const bool pset = (Lp >> pl) & 1u, qset = (Lp >> ql) & 1u;
    if (pset == qset) return 0.f;
    const unsigned between = ((1u << ql) - 1u) & ~((2u << pl) - 1u);
    const bool lneg = __popc(Lp & between) & 1;
    return (qset != lneg) ? 1.f : -1.f;
}

// Persistent: each workgroup walks rows with a grid stride, writes gx (if
// requested) and, if gamma_ws != nullptr, its partial K (C(N,2) floats) to
// gamma_ws[blockIdx.x * C(N,2)].
template <int N>
__global__ __launch_bounds__(256) void rotor_apply_bwd_kernel(const float* __restrict__ state,
                                                               const float* __restrict__ X,
                                                               const float* __restrict__ GY,
                                                               float* __restrict__ GX,
                                                               float* __restrict__ gamma_ws, long long batch) {
    constexpr int RB = rotor_rb(N);
    constexpr int LB = N - RB;
    constexpr int LPR = 1 << LB;
    constexpr int C = n_planes(N);
    const float* cs = state + N * N;
    const unsigned L = threadIdx.x & (LPR - 1);
    const int rows_per_block = blockDim.x >> LB;
    const bool want_gamma = gamma_ws != nullptr;
    float acc[C];
#pragma unroll
    for (int i = 0; i < C; ++i) acc[i] = 0.f;
    for (long long row0 = (long long)blockIdx.x * rows_per_block; row0 < batch;
         row0 += (long long)gridDim.x * rows_per_block) {
        const long long row = row0 + (threadIdx.x >> LB);
        // rows past the end sit out as whole groups of lanes (never split a row)
        if (row < batch) {
            // an opaque copy of L per row keeps the per-plane lane factors
            // inside the loop instead of being hoisted into VGPRs for all planes
            unsigned Lr = L;
            asm volatile("" : "+v"(Lr));
            const long long off = (row << N) + ((long long)Lr << RB);
            float g[1 << RB];
            load_row_part<RB>(g, GY + off);
            rot_chain<N, RB, false>(g, cs, Lr);
            if (GX) store_row_part<RB>(g, GX + off);
            if (want_gamma) {
                float x[1 << RB];
                load_row_part<RB>(x, X + off);
                skew_all_seq<N, RB>(acc, x, g, Lr, std::make_integer_sequence<int, C>{});
            }
        }
    }
    if (!want_gamma) return;  // uniform: a kernel argument
    // 1) sum over the rows of each wave: lanes with equal L sit at stride LPR
#pragma unroll
    for (int i = 0; i < C; ++i)
        for (int off = LPR; off < 64; off <<= 1) acc[i] += __shfl_xor(acc[i], off, 64);
    __shared__ float red[4][C][LPR];  // blockDim.x == 256: four waves
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane < LPR) {
#pragma unroll
        for (int i = 0; i < C; ++i) red[wave][i][lane] = acc[i];
    }
    __syncthreads();
    // 2) sum over waves and lane positions with each position's sign
    for (int k = threadIdx.x; k < C; k += blockDim.x) {
        float t = 0.f;
        for (int Lp = 0; Lp < LPR; ++Lp) {
            const float sgn = skew_lane_sign<N, RB>(k, (unsigned)Lp);
            t += sgn * (red[0][k][Lp] + red[1][k][Lp] + red[2][k][Lp] + red[3][k][Lp]);
        }
        gamma_ws[(long long)blockIdx.x * C + k] = t;
    }
}

// ---- small dense fp64 matrix functions in one wave -----------------------
// Taylor degree after scaling to norm <= 1/4: the truncation (1/4)^9 / 9! ~ 1e-11
// is far below the fp32 precision of the rotor state and the bivector gradient.
constexpr int kTaylorDegree = 8;

// Lane j (< M) holds column j of an M x M matrix in registers (compile-time M,
// so the row indices are register names); the other lanes run along idle.

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const long long bits = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(bits & 0xffffffffll), lane);
    const int hi = __builtin_amdgcn_readlane((int)(bits >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

__device__ __forceinline__ double wave_max_f64(double v) {
    for (int off = 32; off > 0; off >>= 1) {
        const double o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

// col <- column j of expm(Z), Z row-major M x M in LDS, by scaling to 1-norm
// <= 1/4 and squaring, with the degree-8 Taylor series (Horner form; truncation
// (1/4)^9 / 9! = 1e-11 relative, far below the fp32 results).
template <int M>
__device__ __forceinline__ void expm_cols(double (&col)[M], const double* __restrict__ Z, int j) {
    // 1-norm, then the number of squarings that brings it to <= 1/2
    double cs = 0.0;
    if (j < M)
        for (int i = 0; i < M; ++i) cs += fabs(Z[i * M + j]);
    double nrm = wave_max_f64(cs);
    int sq = 0;
    while (nrm > 0.25 && sq < 60) {
        nrm *= 0.5;
        ++sq;
    }
    const double scale = ldexp(1.0, -sq);
#pragma unroll
    for (int i = 0; i < M; ++i) col[i] = (i == j) ? 1.0 : 0.0;
    for (int k = kTaylorDegree; k >= 1; --k) {
        const double f = scale / (double)k;
        double t[M];
#pragma unroll
        for (int i = 0; i < M; ++i) {
            double acc = 0.0;
#pragma unroll
            for (int l = 0; l < M; ++l) acc += Z[i * M + l] * col[l];
            t[i] = acc;
        }
#pragma unroll
        for (int i = 0; i < M; ++i) col[i] = ((i == j) ? 1.0 : 0.0) + f * t[i];
    }
    for (int r = 0; r < sq; ++r) {
        double t[M];
#pragma unroll
        for (int i = 0; i < M; ++i) t[i] = 0.0;
#pragma unroll
        for (int l = 0; l < M; ++l) {
            const double cjl = col[l];
#pragma unroll
            for (int i = 0; i < M; ++i) t[i] += readlane_f64(col[i], l) * cjl;
        }
#pragma unroll
        for (int i = 0; i < M; ++i) col[i] = t[i];
    }
}

// c, s of the plane rotation that zeroes b against a: 1 / sqrt(a^2 + b^2) by the
// hardware reciprocal square root refined with two Newton steps (full fp64
// precision), instead of a square root and a division
__device__ __forceinline__ void givens_cs(double a, double b, double& c, double& s) {
    const double r2 = a * a + b * b;
    c = 1.0;
    s = 0.0;
    if (r2 > 1e-300) {
        double y = __builtin_amdgcn_rsq(r2);
        y = y * (1.5 - 0.5 * r2 * y * y);
        y = y * (1.5 - 0.5 * r2 * y * y);
        c = a * y;
        s = b * y;
    }
}

__device__ __forceinline__ double shfl_f64(double v, int src) {
    const long long bits = __double_as_longlong(v);
    const int lo = __shfl((int)(bits & 0xffffffffll), src, 64);
    const int hi = __shfl((int)(bits >> 32), src, 64);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// E <- G_k^T E for the planes in lex order (E ends as I), lane j < N holding
// column j of E; lane 0 writes the (c, s) pairs
template <int N>
__device__ __forceinline__ void givens_cols(double (&col)[N], float* __restrict__ cs, int lane) {
#pragma unroll
    for (int p = 0; p < N - 1; ++p) {
#pragma unroll
        for (int q = p + 1; q < N; ++q) {
            const int k = p * N - p * (p + 1) / 2 + (q - p - 1);
            double c, s;
            givens_cs(readlane_f64(col[p], p), readlane_f64(col[q], p), c, s);
            const double ep = col[p], eq = col[q];
            col[p] = c * ep + s * eq;
            col[q] = -s * ep + c * eq;
            if (lane == 0) {
                cs[2 * k] = (float)c;
                cs[2 * k + 1] = (float)s;
            }
        }
    }
}

// ---- the spin matrix U = phi(R) of Cl(8,0) (n = 8) -------------------------
// R = exp(B) for the bivector B = sum_m b_m e_{i_m} e_{j_m}, so U = expm(phi(B)),
// phi(B)[r][r ^ x_m] += f_m(r) b_m (the plane table). U is a 16 x 16 matrix
// exponential, computed by a second wave of the compile kernel concurrently
// with the rotation and its plane chain, on the fp64 matrix cores
// (v_mfma_f64_16x16x4: A[i][k] from lane 16k + i, B[k][j] from lane 16k + j,
// D[i][j] in register i / 4 of lane 16 (i % 4) + j). A 16 x 16 x 16 product
// is four of them; chunk c takes k = 4c + g from lane group g, so the B
// operand of chunk c is register c of the previous product's D layout and a
// Horner step needs no data movement. Squaring also needs E as the A operand
// (row i in lane i), through one LDS round trip. Scaling to infinity norm
// <= 1/4, degree-8 Taylor, squaring.
typedef double doublex4 __attribute__((ext_vector_type(4)));
constexpr int kSpinLdsDoubles = 256;

__device__ __forceinline__ doublex4 mfma16_f64(const double (&a)[4], const doublex4& b) {
    doublex4 acc = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int c = 0; c < 4; ++c) acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a[c], b[c], acc, 0, 0, 0);
    return acc;
}

__device__ __forceinline__ void spin_expm(const float* __restrict__ biv, const SpinTable& spin, float* __restrict__ U,
                                          double* __restrict__ lds, int lane) {
    const int g = lane >> 4, i = lane & 15;
    // A operand of Z: za[c] = Z[i][4c + g]
    double za[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int m = 0; m < kSpinPlanes; ++m) {
        const unsigned pl = spin.plane[m];
        const unsigned col = (unsigned)i ^ (pl & 15u);
        const double b = (double)biv[m];
        const double fb = ((pl >> (16 + i)) & 1u) ? -b : b;
#pragma unroll
        for (int c = 0; c < 4; ++c) za[c] += (col == (unsigned)(4 * c + g)) ? fb : 0.0;
    }
    double rs = fabs(za[0]) + fabs(za[1]) + fabs(za[2]) + fabs(za[3]);
    rs += __shfl_xor(rs, 16, 64);
    rs += __shfl_xor(rs, 32, 64);
    double nrm = wave_max_f64(rs);
    int sq = 0;
    while (nrm > 0.25 && sq < 60) {
        nrm *= 0.5;
        ++sq;
    }
    const double scale = ldexp(1.0, -sq);
    // E in D layout: e[t] = E[4t + g][i]
    doublex4 e;
#pragma unroll
    for (int t = 0; t < 4; ++t) e[t] = (4 * t + g == i) ? 1.0 : 0.0;
    // E <- I + (scale / k) Z E
    for (int k = kTaylorDegree; k >= 1; --k) {
        const doublex4 p = mfma16_f64(za, e);
        const double f = scale / (double)k;
#pragma unroll
        for (int t = 0; t < 4; ++t) e[t] = ((4 * t + g == i) ? 1.0 : 0.0) + f * p[t];
    }
    // E <- E E: the A operand E[i][4c + g] through LDS (row-major E)
    for (int r = 0; r < sq; ++r) {
#pragma unroll
        for (int t = 0; t < 4; ++t) lds[(4 * t + g) * 16 + i] = e[t];
        wave_lds_sync();
        double ea[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) ea[c] = lds[i * 16 + 4 * c + g];
        wave_lds_sync();
        e = mfma16_f64(ea, e);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) U[(4 * t + g) * 16 + i] = (float)e[t];
}

// A = -B, B = 2 (M - M^T) from the lex-ordered bivector: A[i][j] = -2 b, A[j][i] = 2 b
__device__ __forceinline__ double generator_entry(const float* __restrict__ biv, int n, int i, int j) {
    if (i == j) return 0.0;
    const int a = i < j ? i : j, c = i < j ? j : i;
    const int m = a * n - a * (a + 1) / 2 + (c - a - 1);
    const double b = (double)biv[m];
    return i < j ? -2.0 * b : 2.0 * b;
}

template <int N>
__global__ __launch_bounds__(64) void rotor_compile_fwd_cols_kernel(const float* __restrict__ biv,
                                                                     float* __restrict__ state) {
    __shared__ double Z[N * N];
    const int j = threadIdx.x;
    for (int idx = j; idx < N * N; idx += 64) Z[idx] = generator_entry(biv, N, idx / N, idx % N);
    __syncthreads();
    double col[N];
    expm_cols<N>(col, Z, j);
    if (j < N)
#pragma unroll
        for (int i = 0; i < N; ++i) state[i * N + j] = (float)col[i];
    // Givens elimination E <- G_k^T E (planes in lex order); E ends as I (det = +1)
    givens_cols<N>(col, state + N * N, j);
}

// dL/dQ (tangent part) = Q skew(Gamma), skew(Gamma)[p][q] = K_pq / 2 = -skew(Gamma)[q][p],
// K = sum of the per-workgroup partials. Writes the Q slot of g_state and zeroes
// its chain slot. 1024 threads: entries padded to EP (a power of two >= C(n,2)),
// thread t sums partials p = t/EP, t/EP + 1024/EP, ... of entry t % EP, then the
// 1024/EP groups are added.
__global__ __launch_bounds__(1024) void rotor_gamma_finalize_kernel(int n, const float* __restrict__ state,
                                                                     const float* __restrict__ gamma_ws, int nparts,
                                                                     float* __restrict__ g_state) {
    __shared__ double part[1024];
    __shared__ double S[kRotorMaxN * kRotorMaxN];
    const int C = n_planes(n);
    int ep = 1;
    while (ep < C) ep <<= 1;
    const int ngrp = 1024 / ep;
    const int e = threadIdx.x & (ep - 1), grp = threadIdx.x / ep;
    // eight independent loads per iteration, so their latencies overlap
    double t[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    if (e < C) {
        int p = grp;
        for (; p + 7 * ngrp < nparts; p += 8 * ngrp)
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] += (double)gamma_ws[(long long)(p + u * ngrp) * C + e];
        for (; p < nparts; p += ngrp) t[0] += (double)gamma_ws[(long long)p * C + e];
    }
    part[threadIdx.x] = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
    for (int i = threadIdx.x; i < n * n; i += blockDim.x) S[i] = 0.0;
    __syncthreads();
    if ((int)threadIdx.x < C) {
        double u = 0.0;
        for (int g = 0; g < ngrp; ++g) u += part[g * ep + threadIdx.x];
        const int p = plane_p(n, threadIdx.x), q = plane_q(n, threadIdx.x);
        S[p * n + q] = 0.5 * u;
        S[q * n + p] = -0.5 * u;
    }
    __syncthreads();
    if ((int)threadIdx.x < n * n) {
        const int i = threadIdx.x / n, j = threadIdx.x % n;
        double v = 0.0;
        for (int k = 0; k < n; ++k) v += (double)state[i * n + k] * S[k * n + j];
        g_state[threadIdx.x] = (float)v;
    }
    for (int i = n * n + threadIdx.x; i < state_floats(n); i += blockDim.x) g_state[i] = 0.f;
}

// Frechet derivative of expm by the block identity
//   expm([[X, G], [0, X]]) = [[e^X, L], [0, e^X]]:
// Horner on the blocks (T_E <- I + X T_E / k, T_L <- (X T_L + G T_E) / k), then
// squaring (E <- E E, L <- E L + L E). Lane j (< N) ends with column j of L.
template <int N>
__device__ __forceinline__ void expm_frechet_cols(double (&Lc)[N], const double* __restrict__ X,
                                                  const double* __restrict__ G, int j) {
    // G is given pre-scaled to norm <= 1 by the caller (the result is linear in G)
    double cs = 0.0;
    if (j < N)
        for (int i = 0; i < N; ++i) cs += fabs(X[i * N + j]) + fabs(G[i * N + j]);
    double xs = 0.0;
    if (j < N)
        for (int i = 0; i < N; ++i) xs += fabs(X[i * N + j]);
    double nrm = wave_max_f64(cs > xs ? cs : xs);
    int sq = 0;
    while (nrm > 0.25 && sq < 60) {
        nrm *= 0.5;
        ++sq;
    }
    const double scale = ldexp(1.0, -sq);
    double Ec[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        Ec[i] = (i == j) ? 1.0 : 0.0;
        Lc[i] = 0.0;
    }
    for (int k = kTaylorDegree; k >= 1; --k) {
        const double f = scale / (double)k;
        double tE[N], tL[N];
#pragma unroll
        for (int i = 0; i < N; ++i) {
            double ae = 0.0, al = 0.0;
#pragma unroll
            for (int l = 0; l < N; ++l) {
                const double xil = X[i * N + l];
                ae += xil * Ec[l];
                al += xil * Lc[l] + G[i * N + l] * Ec[l];
            }
            tE[i] = ae;
            tL[i] = al;
        }
#pragma unroll
        for (int i = 0; i < N; ++i) {
            Ec[i] = ((i == j) ? 1.0 : 0.0) + f * tE[i];
            Lc[i] = f * tL[i];
        }
    }
    for (int r = 0; r < sq; ++r) {
        double tE[N], tL[N];
#pragma unroll
        for (int i = 0; i < N; ++i) {
            tE[i] = 0.0;
            tL[i] = 0.0;
        }
#pragma unroll
        for (int l = 0; l < N; ++l) {
            const double ej = Ec[l], lj = Lc[l];
#pragma unroll
            for (int i = 0; i < N; ++i) {
                const double eil = readlane_f64(Ec[i], l), lil = readlane_f64(Lc[i], l);
                tE[i] += eil * ej;
                tL[i] += eil * lj + lil * ej;
            }
        }
#pragma unroll
        for (int i = 0; i < N; ++i) {
            Ec[i] = tE[i];
            Lc[i] = tL[i];
        }
    }
}

// g_biv from dL/dQ (Q slot of g_state) through Q = expm(A), A = -B(biv):
// dL/dA = L(A^T, dL/dQ), the (1,2) block of expm([[A^T, dL/dQ], [0, A^T]]).
template <int N>
__global__ __launch_bounds__(64) void rotor_compile_bwd_cols_kernel(const float* __restrict__ biv,
                                                                     const float* __restrict__ g_state,
                                                                     float* __restrict__ g_biv) {
    __shared__ double X[N * N], G[N * N], F[N * N];
    const int j = threadIdx.x;
    double gmax = 0.0;
    for (int idx = j; idx < N * N; idx += 64) gmax = fmax(gmax, fabs((double)g_state[idx]));
    gmax = wave_max_f64(gmax) * N;  // bounds every column sum of |G|
    int gexp = 0;
    if (gmax > 1.0) frexp(gmax, &gexp);
    for (int idx = j; idx < N * N; idx += 64) {
        const int r = idx / N, c = idx % N;
        X[idx] = generator_entry(biv, N, c, r);  // A^T
        G[idx] = ldexp((double)g_state[idx], -gexp);
    }
    __syncthreads();
    double Lc[N];
    expm_frechet_cols<N>(Lc, X, G, j);
    if (j < N)
#pragma unroll
        for (int i = 0; i < N; ++i) F[i * N + j] = ldexp(Lc[i], gexp);
    __syncthreads();
    for (int k = j; k < n_planes(N); k += 64) {
        const int p = plane_p(N, k), q = plane_q(N, k);
        // dL/dB = -dL/dA; dL/db = 2 (dL/dB[p][q] - dL/dB[q][p])
        g_biv[k] = (float)(-2.0 * (F[p * N + q] - F[q * N + p]));
    }
}

// ---- entry per lane (N <= 8) ------------------------------------------------
// Lane e = i N + j holds entry (i, j) of each N x N matrix and row i of the
// fixed operands in registers; a product needs column j of the other factor,
// N doubles gathered with lane shuffles (ds_bpermute), so one step of the
// Taylor recursion or of squaring is N FMAs per lane instead of N^2 in N lanes.
// Lanes e >= N^2 compute on row/column 0 and never store.

// number of halvings that bring the infinity norm to <= 1/4 (rows in registers)
template <int N>
__device__ __forceinline__ int halvings(double rowsum) {
    double nrm = wave_max_f64(rowsum);
    int sq = 0;
    while (nrm > 0.25 && sq < 60) {
        nrm *= 0.5;
        ++sq;
    }
    return sq;
}

// entry (i, j) of expm(Z), row i of Z given in z (degree-8 Taylor, Horner form,
// after scaling; then squaring)
template <int N>
__device__ __forceinline__ double expm_entry(const double (&z)[N], int i, int j) {
    double rs = 0.0;
#pragma unroll
    for (int l = 0; l < N; ++l) rs += fabs(z[l]);
    const int sq = halvings<N>(rs);
    const double scale = ldexp(1.0, -sq);
    const double id = (i == j) ? 1.0 : 0.0;
    double e = id;
    for (int k = kTaylorDegree; k >= 1; --k) {
        const double f = scale / (double)k;
        double t = 0.0;
#pragma unroll
        for (int l = 0; l < N; ++l) t += z[l] * shfl_f64(e, l * N + j);
        e = id + f * t;
    }
    for (int r = 0; r < sq; ++r) {
        double t = 0.0;
#pragma unroll
        for (int l = 0; l < N; ++l) t += shfl_f64(e, i * N + l) * shfl_f64(e, l * N + j);
        e = t;
    }
    return e;
}

// Wave 0: Q = expm(A) one entry per lane, then the Givens chain. For n = 8 a
// second wave builds the spin matrix U concurrently (spin_expm).
template <int N>
__global__ __launch_bounds__(128) void rotor_compile_fwd_ent_kernel(const float* __restrict__ biv,
                                                                     float* __restrict__ state, SpinTable spin) {
    static_assert(N * N <= 64, "one entry per lane");
    if constexpr (N == kSpinN) {
        __shared__ double spin_lds[kSpinLdsDoubles];
        if (threadIdx.x >= 64) {  // uniform per wave
            spin_expm(biv, spin, state + spin_offset(N), spin_lds, (int)threadIdx.x - 64);
            return;
        }
    }
    const int lane = threadIdx.x;
    const bool active = lane < N * N;
    const int i = active ? lane / N : 0, j = active ? lane % N : 0;
    double z[N];
#pragma unroll
    for (int l = 0; l < N; ++l) z[l] = generator_entry(biv, N, i, l);
    const double e = expm_entry<N>(z, i, j);
    if (active) state[i * N + j] = (float)e;
    // Givens elimination on columns: lane j < N gathers column j, so the row
    // updates of a plane are register operations
    double col[N];
#pragma unroll
    for (int r = 0; r < N; ++r) col[r] = shfl_f64(e, r * N + (lane < N ? lane : 0));
    givens_cols<N>(col, state + N * N, lane);
}

// Adjoint Frechet derivative by the block identity (see the column version):
// lane (i, j) holds E[i][j] and L[i][j]; X = A^T and G rows in registers.
template <int N>
__global__ __launch_bounds__(64) void rotor_compile_bwd_ent_kernel(const float* __restrict__ biv,
                                                                    const float* __restrict__ g_state,
                                                                    float* __restrict__ g_biv) {
    static_assert(N * N <= 64, "one entry per lane");
    const int lane = threadIdx.x;
    const bool active = lane < N * N;
    const int i = active ? lane / N : 0, j = active ? lane % N : 0;
    double x[N], g[N];
    double xs = 0.0, gs = 0.0;
#pragma unroll
    for (int l = 0; l < N; ++l) {
        x[l] = generator_entry(biv, N, l, i);  // (A^T)[i][l]
        g[l] = (double)g_state[i * N + l];
        xs += fabs(x[l]);
        gs += fabs(g[l]);
    }
    // The derivative is linear in G: scale G to norm <= 1 by a power of two
    // (exact) so that the number of squarings depends on X only, and scale the
    // result back at the end. Summed over a batch, G is often 1e4 or larger.
    int gexp = 0;
    const double gmax = wave_max_f64(gs);
    if (gmax > 1.0) frexp(gmax, &gexp);
#pragma unroll
    for (int l = 0; l < N; ++l) g[l] = ldexp(g[l], -gexp);
    const int sq = halvings<N>(xs + ldexp(gs, -gexp));
    const double scale = ldexp(1.0, -sq);
    const double id = (i == j) ? 1.0 : 0.0;
    double e = id, L = 0.0;
    for (int k = kTaylorDegree; k >= 1; --k) {
        const double f = scale / (double)k;
        double te = 0.0, tl = 0.0;
#pragma unroll
        for (int l = 0; l < N; ++l) {
            const double el = shfl_f64(e, l * N + j), ll = shfl_f64(L, l * N + j);
            te += x[l] * el;
            tl += x[l] * ll + g[l] * el;
        }
        e = id + f * te;
        L = f * tl;
    }
    for (int r = 0; r < sq; ++r) {
        double te = 0.0, tl = 0.0;
#pragma unroll
        for (int l = 0; l < N; ++l) {
            const double eil = shfl_f64(e, i * N + l), lil = shfl_f64(L, i * N + l);
            const double elj = shfl_f64(e, l * N + j), llj = shfl_f64(L, l * N + j);
            te += eil * elj;
            tl += eil * llj + lil * elj;
        }
        e = te;
        L = tl;
    }
    // dL/dB = -dL/dA; dL/db = 2 (dL/dB[p][q] - dL/dB[q][p]), lane (p, q) with p < q
    L = ldexp(L, gexp);
    const double ft = shfl_f64(L, j * N + i);  // F[q][p]
    if (active && i < j) {
        const int k = i * N - i * (i + 1) / 2 + (j - i - 1);
        g_biv[k] = (float)(-2.0 * (L - ft));
    }
}

// ---- host side --------------------------------------------------------------

#define CLF_ROTOR_DISPATCH(n, CALL)       \
    switch (n) {                          \
        case 2: CALL(2); break;           \
        case 3: CALL(3); break;           \
        case 4: CALL(4); break;           \
        case 5: CALL(5); break;           \
        case 6: CALL(6); break;           \
        case 7: CALL(7); break;           \
        case 8: CALL(8); break;           \
        case 9: CALL(9); break;           \
        case 10: CALL(10); break;         \
        default: break;                   \
    }

// one entry per lane up to n = 8 (64 entries), one column per lane above
template <int N>
static int launch_compile_fwd(const float* biv, float* state, hipStream_t s) {
    if constexpr (N * N <= 64) {
        SpinTable spin{};
        if constexpr (N == kSpinN) {
            RepTable T;
            if (!spin_tables(T, spin)) return set_error(CLF_ERR_UNSUPPORTED, "Cl(8,0) representation tables unavailable");
        }
        hipLaunchKernelGGL((rotor_compile_fwd_ent_kernel<N>), dim3(1), dim3(N == kSpinN ? 128 : 64), 0, s, biv, state,
                           spin);
    } else {
        hipLaunchKernelGGL((rotor_compile_fwd_cols_kernel<N>), dim3(1), dim3(64), 0, s, biv, state);
    }
    return CLF_OK;
}

template <int N>
static void launch_compile_bwd(const float* biv, const float* g_state, float* g_biv, hipStream_t s) {
    if constexpr (N * N <= 64)
        hipLaunchKernelGGL((rotor_compile_bwd_ent_kernel<N>), dim3(1), dim3(64), 0, s, biv, g_state, g_biv);
    else hipLaunchKernelGGL((rotor_compile_bwd_cols_kernel<N>), dim3(1), dim3(64), 0, s, biv, g_state, g_biv);
}

static int check_rotor_n(int n) {
    if (n < kRotorMinN || n > kRotorMaxN)
        return set_error(CLF_ERR_ARG, "rotor kernels support n in [" + std::to_string(kRotorMinN) + ", " +
                                          std::to_string(kRotorMaxN) + "], got " + std::to_string(n));
    return CLF_OK;
}

int rotor_state_floats(int n) { return (n >= kRotorMinN && n <= kRotorMaxN) ? state_floats(n) : -1; }

static int rotor_bwd_grid(int n, int64_t batch) {
    const int lb = n - rotor_rb(n);
    const long long rows_per_block = 256 >> lb;
    long long g = (batch + rows_per_block - 1) / rows_per_block;
    if (g > 1024) g = 1024;
    if (g < 1) g = 1;
    return (int)g;
}

size_t rotor_apply_ws_bytes(int n, int64_t batch) {
    if (n < kRotorMinN || n > kRotorMaxN || batch < 0) return 0;
    return (size_t)rotor_bwd_grid(n, batch) * n_planes(n) * sizeof(float);
}

int rotor_compile_fwd(int n, const float* biv, float* state, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (!biv || !state) return set_error(CLF_ERR_ARG, "null pointer argument");
    hipStream_t s = (hipStream_t)stream;
    int rc = CLF_OK;
#define CLF_CALL(N) rc = launch_compile_fwd<N>(biv, state, s)
    CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
    if (rc) return rc;
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int rotor_compile_bwd(int n, const float* biv, const float* g_state, float* g_biv, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (!biv || !g_state || !g_biv) return set_error(CLF_ERR_ARG, "null pointer argument");
    hipStream_t s = (hipStream_t)stream;
#define CLF_CALL(N) launch_compile_bwd<N>(biv, g_state, g_biv, s)
    CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

template <int N>
static void launch_apply(bool fwd, const float* state, const float* x, float* y, int64_t batch, hipStream_t s) {
    constexpr int LB = N - rotor_rb(N);
    const long long threads = (long long)batch << LB;
    const long long wanted = (threads + 255) / 256;
    if (fwd) {
        const dim3 grid(resident_grid((const void*)rotor_apply_kernel<N, true>, 256, 0, wanted));
        hipLaunchKernelGGL((rotor_apply_kernel<N, true>), grid, dim3(256), 0, s, state, x, y, (long long)batch);
    } else {
        const dim3 grid(resident_grid((const void*)rotor_apply_kernel<N, false>, 256, 0, wanted));
        hipLaunchKernelGGL((rotor_apply_kernel<N, false>), grid, dim3(256), 0, s, state, x, y, (long long)batch);
    }
}

// Backward grid: at most rotor_bwd_grid (the workspace bound), at most the
// resident workgroups. The gamma finalize reads this many partials.
template <int N>
static unsigned bwd_launch_grid(int64_t batch) {
    return resident_grid((const void*)rotor_apply_bwd_kernel<N>, 256, 0, rotor_bwd_grid(N, batch));
}

template <int N>
static void launch_apply_bwd(const float* state, const float* x, const float* gy, float* gx, float* ws,
                             int64_t batch, hipStream_t s) {
    hipLaunchKernelGGL((rotor_apply_bwd_kernel<N>), dim3(bwd_launch_grid<N>(batch)), dim3(256), 0, s, state, x, gy,
                       gx, ws, (long long)batch);
}


bool rotor16_enabled(int n);
int rotor16_apply(bool fwd, const float* U, const float* x, float* y, int64_t batch, void* stream);
int rotor16_bwd(const float* U, const float* x, const float* gy, float* gx, float* gamma_ws, int64_t batch,
                unsigned grid, void* stream);
unsigned rotor16_bwd_grid(long long wanted);

int rotor_apply_fwd(int n, const float* state, const float* x, float* y, int64_t batch, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (batch == 0) return CLF_OK;
    if (!state || !x || !y) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (x == y) return set_error(CLF_ERR_ARG, "output must not alias the input");
    if ((((uintptr_t)x) | ((uintptr_t)y)) & 15u) return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    if (rotor16_enabled(n)) return rotor16_apply(true, state + spin_offset(n), x, y, batch, stream);
    hipStream_t s = (hipStream_t)stream;
#define CLF_CALL(N) launch_apply<N>(true, state, x, y, batch, s)
    CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int rotor_apply_bwd(int n, const float* state, const float* x, const float* gy, float* gx, float* g_state,
                    int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (!gx && !g_state) return CLF_OK;
    if (!state || !gy || (g_state && !x)) return set_error(CLF_ERR_ARG, "null pointer argument");
    if ((((uintptr_t)x) | ((uintptr_t)gy) | ((uintptr_t)gx)) & 15u)
        return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    if (gx && (gx == gy || gx == x)) return set_error(CLF_ERR_ARG, "gx must not alias x or gy");
    const size_t need = rotor_apply_ws_bytes(n, batch);
    if (g_state && (!ws || ws_bytes < need))
        return set_error(CLF_ERR_WORKSPACE, "workspace of at least " + std::to_string(need) + " bytes required");
    hipStream_t s = (hipStream_t)stream;
    float* gws = g_state ? (float*)ws : nullptr;
    const bool mat = rotor16_enabled(n);
    int nparts = 0;
    if (batch > 0) {
        if (!g_state) {
            if (mat) return rotor16_apply(false, state + spin_offset(n), gy, gx, batch, stream);
#define CLF_CALL(N) launch_apply<N>(false, state, gy, gx, batch, s)
            CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
        } else if (mat) {
            nparts = (int)rotor16_bwd_grid(rotor_bwd_grid(n, batch));
            if (int rc = rotor16_bwd(state + spin_offset(n), x, gy, gx, gws, batch, (unsigned)nparts, stream)) return rc;
        } else {
#define CLF_CALL(N) launch_apply_bwd<N>(state, x, gy, gx, gws, batch, s)
            CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
#define CLF_CALL(N) nparts = (int)bwd_launch_grid<N>(batch)
            CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
        }
        CLF_HIP_CHECK(hipGetLastError());
    }
    if (g_state) {
        hipLaunchKernelGGL(rotor_gamma_finalize_kernel, dim3(1), dim3(1024), 0, s, n, state, gws, nparts, g_state);
        CLF_HIP_CHECK(hipGetLastError());
    }
    return CLF_OK;
}

}  // namespace clf
