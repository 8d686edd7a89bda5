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
//                     Gamma_bb = sum_rows sum_{I: b in I} x_I gx_I
// (the derivation extension of Q^{-1} dQ), and the bivector gradient follows
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

#include "clf_common.h"

namespace clf {

constexpr int kRotorMinN = 2;
constexpr int kRotorMaxN = 10;
constexpr int kRotorMaxM = 2 * kRotorMaxN;  // block matrix of the Frechet derivative

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
__host__ __device__ constexpr int rotor_rb(int n) { return n < 4 ? n : (n - 4 <= 6 ? 4 : n - 6); }
// parity of the bits of r strictly between positions p and q (p < q)
__host__ __device__ constexpr int between_par(unsigned r, int p, int q) {
    int c = 0;
    for (int b = p + 1; b < q; ++b) c += (r >> b) & 1u;
    return c & 1;
}
__host__ __device__ constexpr int state_floats(int n) { return n * n + 2 * n_planes(n); }

// ---- the plane-rotation chain on register-resident rows ---------------------

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
        constexpr unsigned mp = 1u << P;
        constexpr int ql = Qb - RB;
        const bool qset = (L >> ql) & 1u;
        const int lpar = __popc(L & ((1u << ql) - 1u)) & 1;
        const float s_l = lpar ? -s : s;
#pragma unroll
        for (int r0 = 0; r0 < V; ++r0) {
            if (r0 & mp) continue;
            const int r1 = r0 | (int)mp;
            const float sg = between_par((unsigned)r1, P, RB) ? -s_l : s_l;
            // value selects only (a select of addresses would force the row into memory)
            const float x0 = v[r0], x1 = v[r1];
            const float own = qset ? x0 : x1;
            const float recv = __shfl_xor(own, 1 << ql, 64);
            const float nv = __builtin_fmaf(c, own, (qset ? sg : -sg) * recv);
            v[r0] = qset ? nv : x0;
            v[r1] = qset ? x1 : nv;
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
            const float recv = __shfl_xor(v[r], (1 << pl) | (1 << ql), 64);
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
template <int N, bool FWD>
__global__ __launch_bounds__(256) void rotor_apply_kernel(const float* __restrict__ state,
                                                           const float* __restrict__ X, float* __restrict__ Y,
                                                           long long batch) {
    constexpr int RB = rotor_rb(N);
    constexpr int LB = N - RB;
    const float* cs = state + N * N;
    const long long gtid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long row = gtid >> LB;
    const unsigned L = (unsigned)(gtid & ((1 << LB) - 1));
    // whole rows only: a row's lanes are in one wave, so every lane that
    // shuffles with a partner has that partner active
    if (row >= batch) return;
    float v[1 << RB];
    const long long off = (row << N) + ((long long)L << RB);
    load_row_part<RB>(v, X + off);
    rot_chain<N, RB, FWD>(v, cs, L);
    store_row_part<RB>(v, Y + off);
}

// ---- backward: gx = Lambda(Q)^T gy and the per-workgroup partial Gamma ----

// per-lane accumulator slots, per plane: 2 if both bits are register bits
// (Gamma_qp and Gamma_pq), else 1 (the lane's own type); then RB register-bit
// diagonals and one all-blades diagonal sum
template <int N, int RB>
struct AccLayout {
    static constexpr int slot(int k) {
        int s = 0;
        for (int j = 0; j < k; ++j) s += (plane_q(N, j) < RB) ? 2 : 1;
        return s;
    }
    static constexpr int planes_end = slot(n_planes(N));
    static constexpr int diag = planes_end;           // RB register-bit diagonals
    static constexpr int all = planes_end + RB;       // sum over all blades of the lane
    static constexpr int total = planes_end + RB + 1;
};

template <int N, int RB, int K>
__device__ __forceinline__ void gamma_plane(float* __restrict__ acc, const float (&x)[1 << RB],
                                            const float (&g)[1 << RB], unsigned L) {
    constexpr int P = plane_p(N, K), Qb = plane_q(N, K);
    constexpr int V = 1 << RB;
    constexpr int S = AccLayout<N, RB>::slot(K);
    if constexpr (Qb < RB) {
        constexpr unsigned mp = 1u << P, mq = 1u << Qb;
#pragma unroll
        for (int r = 0; r < V; ++r) {
            if ((r & mp) && !(r & mq)) {
                const int rj = r ^ (int)(mp | mq);
                const bool neg = between_par((unsigned)r, P, Qb);
                // Gamma_qp += sig x_I gx_J ; Gamma_pq += sig x_J gx_I
                acc[S] = __builtin_fmaf(neg ? -x[r] : x[r], g[rj], acc[S]);
                acc[S + 1] = __builtin_fmaf(neg ? -x[rj] : x[rj], g[r], acc[S + 1]);
            }
        }
    } else if constexpr (P < RB) {
        constexpr unsigned mp = 1u << P;
        constexpr int ql = Qb - RB;
        const bool qset = (L >> ql) & 1u;
        const bool lneg = __popc(L & ((1u << ql) - 1u)) & 1;
#pragma unroll
        for (int r0 = 0; r0 < V; ++r0) {
            if (r0 & mp) continue;
            const int r1 = r0 | (int)mp;
            const bool neg = between_par((unsigned)r1, P, RB) != lneg;
            // q-clear lane owns I = (L, r1): term x_I gx_J ; q-set lane owns J = (L, r0): term x_J gx_I
            const float x0 = x[r0], x1 = x[r1], g0 = g[r0], g1 = g[r1];
            const float xo = qset ? x0 : x1;
            const float go = qset ? g0 : g1;
            const float gp = __shfl_xor(go, 1 << ql, 64);
            acc[S] = __builtin_fmaf(neg ? -xo : xo, gp, acc[S]);
        }
    } else {
        constexpr int pl = P - RB, ql = Qb - RB;
        const bool pset = (L >> pl) & 1u, qset = (L >> ql) & 1u;
        const unsigned between = ((1u << ql) - 1u) & ~((2u << pl) - 1u);
        const bool neg = __popc(L & between) & 1;
        const float w = (pset != qset) ? (neg ? -1.f : 1.f) : 0.f;
#pragma unroll
        for (int r = 0; r < V; ++r) {
            const float gp = __shfl_xor(g[r], (1 << pl) | (1 << ql), 64);
            acc[S] = __builtin_fmaf(w * x[r], gp, acc[S]);
        }
    }
}

template <int N, int RB, int... Ks>
__device__ __forceinline__ void gamma_all_seq(float* __restrict__ acc, const float (&x)[1 << RB],
                                              const float (&g)[1 << RB], unsigned L,
                                              std::integer_sequence<int, Ks...>) {
    (gamma_plane<N, RB, Ks>(acc, x, g, L), ...);
}

template <int N, int RB>
__device__ __forceinline__ void gamma_accumulate(float* __restrict__ acc, const float (&x)[1 << RB],
                                                 const float (&g)[1 << RB], unsigned L) {
    gamma_all_seq<N, RB>(acc, x, g, L, std::make_integer_sequence<int, n_planes(N)>{});
    using AL = AccLayout<N, RB>;
#pragma unroll
    for (int r = 0; r < (1 << RB); ++r) {
        const float t = x[r] * g[r];
        acc[AL::all] += t;
#pragma unroll
        for (int b = 0; b < RB; ++b)
            if ((r >> b) & 1) acc[AL::diag + b] += t;
    }
}

// Persistent: each workgroup walks rows with a grid stride, writes gx (if
// requested) and, if gamma_ws != nullptr, its partial Gamma (N*N floats) to
// gamma_ws[blockIdx.x * N * N].
template <int N>
__global__ __launch_bounds__(256) void rotor_apply_bwd_kernel(const float* __restrict__ state,
                                                               const float* __restrict__ X,
                                                               const float* __restrict__ GY,
                                                               float* __restrict__ GX,
                                                               float* __restrict__ gamma_ws, long long batch) {
    constexpr int RB = rotor_rb(N);
    constexpr int LB = N - RB;
    constexpr int LPR = 1 << LB;
    using AL = AccLayout<N, RB>;
    const float* cs = state + N * N;
    const unsigned L = threadIdx.x & (LPR - 1);
    const int rows_per_block = blockDim.x >> LB;
    const bool want_gamma = gamma_ws != nullptr;
    float acc[AL::total];
#pragma unroll
    for (int i = 0; i < AL::total; ++i) acc[i] = 0.f;
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
                gamma_accumulate<N, RB>(acc, x, g, Lr);
            }
        }
    }
    if (!want_gamma) return;  // uniform: a kernel argument
    // 1) sum over the rows of each wave: lanes with equal L sit at stride LPR
#pragma unroll
    for (int i = 0; i < AL::total; ++i)
        for (int off = LPR; off < 64; off <<= 1) acc[i] += __shfl_xor(acc[i], off, 64);
    __shared__ float red[4][AL::total][LPR];  // blockDim.x == 256: four waves
    __shared__ float gam[N * N];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane < LPR) {
#pragma unroll
        for (int i = 0; i < AL::total; ++i) red[wave][i][lane] = acc[i];
    }
    __syncthreads();
    // 2) sum over waves and scatter the lane-position sums into Gamma
    if (threadIdx.x == 0) {
        for (int i = 0; i < N * N; ++i) gam[i] = 0.f;
        auto S = [&](int i, int Lp) { return red[0][i][Lp] + red[1][i][Lp] + red[2][i][Lp] + red[3][i][Lp]; };
        int slot = 0;
        for (int k = 0; k < n_planes(N); ++k) {
            const int p = plane_p(N, k), q = plane_q(N, k);
            for (int Lp = 0; Lp < LPR; ++Lp) {
                if (q < RB) {
                    gam[q * N + p] += S(slot, Lp);      // Gamma_qp
                    gam[p * N + q] += S(slot + 1, Lp);  // Gamma_pq
                } else if (p < RB) {
                    const bool qset = (Lp >> (q - RB)) & 1;
                    gam[qset ? (p * N + q) : (q * N + p)] += S(slot, Lp);
                } else {
                    const bool pset = (Lp >> (p - RB)) & 1, qset = (Lp >> (q - RB)) & 1;
                    if (pset != qset) gam[qset ? (p * N + q) : (q * N + p)] += S(slot, Lp);
                }
            }
            slot += (q < RB) ? 2 : 1;
        }
        for (int Lp = 0; Lp < LPR; ++Lp) {
            for (int b = 0; b < RB; ++b) gam[b * N + b] += S(AL::diag + b, Lp);
            for (int b = RB; b < N; ++b)
                if ((Lp >> (b - RB)) & 1) gam[b * N + b] += S(AL::all, Lp);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < N * N; i += blockDim.x) gamma_ws[(long long)blockIdx.x * N * N + i] = gam[i];
}

// ---- small dense fp64 helpers for one workgroup ------------------------------

// C = A * B for m x m row-major matrices in LDS (C must not alias A or B)
__device__ void mm(double* __restrict__ C, const double* __restrict__ A, const double* __restrict__ B, int m) {
    for (int idx = threadIdx.x; idx < m * m; idx += blockDim.x) {
        const int i = idx / m, j = idx % m;
        double t = 0.0;
        for (int k = 0; k < m; ++k) t += A[i * m + k] * B[k * m + j];
        C[idx] = t;
    }
    __syncthreads();
}

// E = expm(Z), m x m, by scaling and squaring of a degree-18 Taylor series.
// Z is left scaled; T1, T2 are scratch. All arrays m*m doubles in LDS.
__device__ void expm(double* __restrict__ E, double* __restrict__ Z, double* __restrict__ T1,
                     double* __restrict__ T2, int m) {
    __shared__ double s_norm;
    __shared__ int s_sq;
    if (threadIdx.x == 0) {
        double nrm = 0.0;
        for (int i = 0; i < m; ++i) {
            double r = 0.0;
            for (int j = 0; j < m; ++j) r += fabs(Z[i * m + j]);
            nrm = r > nrm ? r : nrm;
        }
        int sq = 0;
        while (nrm > 0.5 && sq < 60) {
            nrm *= 0.5;
            ++sq;
        }
        s_norm = nrm;
        s_sq = sq;
    }
    __syncthreads();
    const int sq = s_sq;
    const double scale = ldexp(1.0, -sq);
    for (int i = threadIdx.x; i < m * m; i += blockDim.x) Z[i] *= scale;
    // Horner: E = I + Z/1 (I + Z/2 (I + ... (I + Z/18)))
    for (int i = threadIdx.x; i < m * m; i += blockDim.x) E[i] = (i / m == i % m) ? 1.0 : 0.0;
    __syncthreads();
    for (int k = 18; k >= 1; --k) {
        mm(T1, Z, E, m);
        for (int i = threadIdx.x; i < m * m; i += blockDim.x) E[i] = ((i / m == i % m) ? 1.0 : 0.0) + T1[i] / k;
        __syncthreads();
    }
    for (int r = 0; r < sq; ++r) {
        mm(T2, E, E, m);
        for (int i = threadIdx.x; i < m * m; i += blockDim.x) E[i] = T2[i];
        __syncthreads();
    }
}

// A = -B, B = 2 (M - M^T) from the lex-ordered bivector
__device__ void build_generator(double* __restrict__ A, const float* __restrict__ biv, int n) {
    for (int i = threadIdx.x; i < n * n; i += blockDim.x) A[i] = 0.0;
    __syncthreads();
    if (threadIdx.x == 0) {
        int m = 0;
        for (int i = 0; i < n; ++i)
            for (int j = i + 1; j < n; ++j, ++m) {
                const double b = (double)biv[m];
                A[i * n + j] = -2.0 * b;
                A[j * n + i] = 2.0 * b;
            }
    }
    __syncthreads();
}

__global__ __launch_bounds__(256) void rotor_compile_fwd_kernel(int n, const float* __restrict__ biv,
                                                                 float* __restrict__ state) {
    __shared__ double A[kRotorMaxN * kRotorMaxN], E[kRotorMaxN * kRotorMaxN];
    __shared__ double T1[kRotorMaxN * kRotorMaxN], T2[kRotorMaxN * kRotorMaxN];
    build_generator(A, biv, n);
    expm(E, A, T1, T2, n);
    for (int i = threadIdx.x; i < n * n; i += blockDim.x) state[i] = (float)E[i];
    __syncthreads();
    if (threadIdx.x == 0) {
        // Givens elimination E <- G_k^T E column by column; E ends as I for det = +1
        float* cs = state + n * n;
        int k = 0;
        for (int p = 0; p < n - 1; ++p)
            for (int q = p + 1; q < n; ++q, ++k) {
                const double a = E[p * n + p], b = E[q * n + p];
                const double r = sqrt(a * a + b * b);
                double c = 1.0, s = 0.0;
                if (r > 1e-300) {
                    c = a / r;
                    s = b / r;
                }
                for (int j = 0; j < n; ++j) {
                    const double ep = E[p * n + j], eq = E[q * n + j];
                    E[p * n + j] = c * ep + s * eq;
                    E[q * n + j] = -s * ep + c * eq;
                }
                cs[2 * k] = (float)c;
                cs[2 * k + 1] = (float)s;
            }
    }
}

// dL/dQ = Q Gamma, Gamma = sum of the per-workgroup partials; writes the Q
// slot of g_state and zeroes its chain slot
__global__ __launch_bounds__(256) void rotor_gamma_finalize_kernel(int n, const float* __restrict__ state,
                                                                    const float* __restrict__ gamma_ws, int nparts,
                                                                    float* __restrict__ g_state) {
    __shared__ double G[kRotorMaxN * kRotorMaxN];
    for (int i = threadIdx.x; i < n * n; i += blockDim.x) {
        double t = 0.0;
        for (int p = 0; p < nparts; ++p) t += (double)gamma_ws[(long long)p * n * n + i];
        G[i] = t;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < n * n; idx += blockDim.x) {
        const int i = idx / n, j = idx % n;
        double t = 0.0;
        for (int k = 0; k < n; ++k) t += (double)state[i * n + k] * G[k * n + j];
        g_state[idx] = (float)t;
    }
    for (int i = n * n + threadIdx.x; i < state_floats(n); i += blockDim.x) g_state[i] = 0.f;
}

// g_biv from dL/dQ (Q slot of g_state) through Q = expm(-B(biv))
__global__ __launch_bounds__(256) void rotor_compile_bwd_kernel(int n, const float* __restrict__ biv,
                                                                 const float* __restrict__ g_state,
                                                                 float* __restrict__ g_biv) {
    constexpr int MM = kRotorMaxM * kRotorMaxM;
    __shared__ double A[kRotorMaxN * kRotorMaxN];
    __shared__ double Z[MM], E[MM], T1[MM], T2[MM];
    build_generator(A, biv, n);
    const int m = 2 * n;
    for (int idx = threadIdx.x; idx < m * m; idx += blockDim.x) {
        const int i = idx / m, j = idx % m;
        double v = 0.0;
        if (i < n && j < n) v = A[j * n + i];                              // A^T
        else if (i >= n && j >= n) v = A[(j - n) * n + (i - n)];           // A^T
        else if (i < n && j >= n) v = (double)g_state[i * n + (j - n)];    // dL/dQ
        Z[idx] = v;
    }
    __syncthreads();
    expm(E, Z, T1, T2, m);
    if (threadIdx.x == 0) {
        int k = 0;
        for (int i = 0; i < n; ++i)
            for (int j = i + 1; j < n; ++j, ++k) {
                const double dAij = E[i * m + (n + j)], dAji = E[j * m + (n + i)];
                // dL/dB = -dL/dA; dL/db = 2 (dL/dB[i][j] - dL/dB[j][i])
                g_biv[k] = (float)(-2.0 * (dAij - dAji));
            }
    }
}

// ---- host side --------------------------------------------------------------

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
    return (size_t)rotor_bwd_grid(n, batch) * n * n * sizeof(float);
}

int rotor_compile_fwd(int n, const float* biv, float* state, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (!biv || !state) return set_error(CLF_ERR_ARG, "null pointer argument");
    hipLaunchKernelGGL(rotor_compile_fwd_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, n, biv, state);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int rotor_compile_bwd(int n, const float* biv, const float* g_state, float* g_biv, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (!biv || !g_state || !g_biv) return set_error(CLF_ERR_ARG, "null pointer argument");
    hipLaunchKernelGGL(rotor_compile_bwd_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, n, biv, g_state, g_biv);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

template <int N>
static void launch_apply(bool fwd, const float* state, const float* x, float* y, int64_t batch, hipStream_t s) {
    constexpr int LB = N - rotor_rb(N);
    const long long threads = (long long)batch << LB;
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (fwd) hipLaunchKernelGGL((rotor_apply_kernel<N, true>), grid, dim3(256), 0, s, state, x, y, (long long)batch);
    else hipLaunchKernelGGL((rotor_apply_kernel<N, false>), grid, dim3(256), 0, s, state, x, y, (long long)batch);
}

template <int N>
static void launch_apply_bwd(const float* state, const float* x, const float* gy, float* gx, float* ws,
                             int64_t batch, hipStream_t s) {
    hipLaunchKernelGGL((rotor_apply_bwd_kernel<N>), dim3(rotor_bwd_grid(N, batch)), dim3(256), 0, s, state, x, gy, gx,
                       ws, (long long)batch);
}

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

int rotor_apply_fwd(int n, const float* state, const float* x, float* y, int64_t batch, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (batch == 0) return CLF_OK;
    if (!state || !x || !y) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (x == y) return set_error(CLF_ERR_ARG, "output must not alias the input");
    if ((((uintptr_t)x) | ((uintptr_t)y)) & 15u) return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
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
    if (batch > 0) {
        if (!g_state) {
#define CLF_CALL(N) launch_apply<N>(false, state, gy, gx, batch, s)
            CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
        } else {
#define CLF_CALL(N) launch_apply_bwd<N>(state, x, gy, gx, gws, batch, s)
            CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
        }
        CLF_HIP_CHECK(hipGetLastError());
    }
    if (g_state) {
        const int nparts = batch > 0 ? rotor_bwd_grid(n, batch) : 0;
        hipLaunchKernelGGL(rotor_gamma_finalize_kernel, dim3(1), dim3(256), 0, s, n, state, gws, nparts, g_state);
        CLF_HIP_CHECK(hipGetLastError());
    }
    return CLF_OK;
}

}  // namespace clf
