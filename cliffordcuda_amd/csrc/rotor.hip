// Rotor path on gfx950: bivector -> rotation -> plane-rotation chain, the
// sandwich ~R x R applied to a batch of multivectors, and gradients to the
// bivector and to x.
//
// What is computed (the composite of reference algebra.py:343-373, Euclidean):
//   B = 2 (M - M^T), M[i_m, j_m] = b_m (lex pairs, kernels/rotor/eigh_exp.cu:283-288)
//   R = expm(B)                  the matrix the reference factors (its closed form
//                                kernels/rotor/eigh_exp.cu:55-67 is exp(B))
//   Q = R^T = expm(-B)           the grade-1 action of ~R x R, R = exp(sum b_m e_{i_m} e_{j_m})
//   cs                           the reference's Givens factors of R (givens_factor.cu:23-38):
//                                planes (p, q) in lex order, c = a / r, s = b / r with
//                                a = A[p][p], b = A[q][p]; rows A[p] <- c A[p] + s A[q],
//                                A[q] <- -s A[p] + c A[q]; (c, s) of plane k stored at
//                                index C - 1 - k (C = C(n,2))
//   y = chain(cs) x              planes applied lex-first; plane (p, q) maps the blade
//                                pairs (I with p not q, J = I ^ {p,q}) as
//                                y_I = c x_I + s sig x_J,  y_J = c x_J - s sig x_I,
//                                sig = (-1)^{|I & (p, q)|} (bits strictly between p
//                                and q), the reference's givens_apply_mb_perm_packed.cu:33-64.
// For the factors of a rotation the chain is the outermorphism Lambda(Q).
//
// Gradients of the composite (bivector -> y). With gx = Lambda(Q)^T gy (the chain
// transposed),
//   dL/dQ = Q Gamma,  Gamma_ab = sum_rows sum_{I: b in I, a not in I} sig x_I gx_{I^{a,b}}
// (the derivation extension of Q^{-1} dQ; only its antisymmetric part matters,
// since Q stays orthogonal), and the bivector gradient follows
// from the adjoint Frechet derivative of expm:
//   dL/dA = [expm([[A^T, dL/dQ], [0, A^T]])]_{12},  A = -B,
//   dL/db_m = 2 (dL/dB[i_m][j_m] - dL/dB[j_m][i_m]),  dL/dB = -dL/dA.
// The reference instead runs torch eigh + a closed form + Givens kernels with
// host syncs and returns no gradient to x (extensions/rotor/*.py).
//
// Gradients of the chain on a caller's cs (apply_rotor(cs, x) with cs a free
// tensor): the reference's backward (givens_apply_mb_perm_packed.cu:111-160):
// walking the planes from the last applied, each plane's input is rebuilt from
// its output with the transposed pair map and
//   grad_c += g_I v_I + g_J v_J,  grad_s += sig (g_I v_J - g_J v_I)
// summed over the batch (exact for unit pairs, the reference's rule for any);
// and, through cs = Givens(expm(B)), the bivector gradient by reverse-mode
// through the factorisation (fp64) followed by the Frechet step above.
//
// Apply layout: one row is spread over 2^(n-RB) lanes, each holding 2^RB
// consecutive blades in registers. Planes inside the register bits are pure
// FMAs; planes touching lane bits exchange partner values with lane shuffles.
// The plane list is unrolled at compile time per n.
#include <utility>

#include "rep_common.h"

namespace clf {

constexpr int kRotorMinN = 2;
constexpr int kRotorMaxN = 12;

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
// quad-local DPP permutes), n = 9 .. 12 use 8 .. 64 lanes of 64 blades each
__host__ __device__ constexpr int rotor_rb(int n) { return n < 4 ? n : (n <= 8 ? n - 2 : 6); }
// parity of the bits of r strictly between positions p and q (p < q)
__host__ __device__ constexpr int between_par(unsigned r, int p, int q) {
    int c = 0;
    for (int b = p + 1; b < q; ++b) c += (r >> b) & 1u;
    return c & 1;
}
// state: Q (n x n), the cs pairs of the chain (the reference's layout), and for
// n = 8 also the 16 x 16 matrix U = phi(R) of the Cl(8,0) representation
// (row-major)
__host__ __device__ constexpr int spin_offset(int n) { return n * n + 2 * n_planes(n); }
__host__ __device__ constexpr int state_floats(int n) { return spin_offset(n) + (n == kSpinN ? 256 : 0); }

// ---- the plane-rotation chain on register-resident rows ---------------------

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// value of v in lane (lane ^ MASK) for MASK < 64: quad-local bits by DPP quad
// permutes (full-rate VALU), bits 2..4 by one ds_swizzle in bit-mask mode, bit 5
// (the other half of the wave) by ds_bpermute
template <unsigned MASK>
__device__ __forceinline__ float lane_xor(float v) {
    static_assert(MASK < 64, "lane exchange limited to one wave");
    float r = v;
    if constexpr ((MASK & 3u) == 1u) r = dpp_mov<0xB1>(r);       // quad_perm [1,0,3,2]
    else if constexpr ((MASK & 3u) == 2u) r = dpp_mov<0x4E>(r);  // quad_perm [2,3,0,1]
    else if constexpr ((MASK & 3u) == 3u) r = dpp_mov<0x1B>(r);  // quad_perm [3,2,1,0]
    if constexpr ((MASK & 0x1Cu) != 0u) {
        constexpr int pattern = (int)(((MASK & 0x1Cu) << 10) | 0x1Fu);  // and 0x1F, or 0, xor MASK
        r = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(r), pattern));
    }
    if constexpr ((MASK & 32u) != 0u) r = __shfl_xor(r, 32, 64);
    return r;
}

// One plane of the chain, in the form y_I = c x_I - s sig x_J,
// y_J = c x_J + s sig x_I: the reference's pair map has the opposite sign of s,
// so the forward uses s = -cs_s and the transposed map s = +cs_s. Plane K (lex)
// reads the pair stored at index C - 1 - K.
template <int N, int RB, int K, bool FWD>
__device__ __forceinline__ void rot_plane(float (&v)[1 << RB], const float* __restrict__ cs, unsigned L) {
    constexpr int P = plane_p(N, K), Qb = plane_q(N, K);
    constexpr int V = 1 << RB;
    constexpr int SLOT = n_planes(N) - 1 - K;
    const float c = cs[2 * SLOT];
    const float s = FWD ? -cs[2 * SLOT + 1] : cs[2 * SLOT + 1];
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
    // forward: lex plane 0 first; transpose: the reverse order
    constexpr int C = n_planes(N);
    (rot_plane<N, RB, FWD ? Ks : (C - 1 - Ks), FWD>(v, cs, L), ...);
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

// y = Lambda(Q) x (FWD) or Lambda(Q)^T x (!FWD), one row per 2^(N-RB) lanes
// (RB: 2^RB floats of a row per lane; rotor_rb(N), or N - 6 for one wave per
// row, where a row's planes run on 64 lanes with 2^(N-6) floats each instead
// of on 2^(N-6) lanes with 64 floats; use_wave_rows picks by n and batch).
// Persistent: the lanes of a row walk rows with a grid stride and load the
// next row part while the current one is rotated. Rows past the end are never
// stored; their prefetch re-reads the last row (a cache hit, no branch).
// The loop condition is the same for all lanes of a row, so a row's lanes
// stay active together and every shuffle partner is active.
// ldx: floats between the input's rows (2^N, or 0 for one row broadcast over
// the batch: the transposed action on the gradient of a sum)
template <int N, bool FWD, int RB = rotor_rb(N)>
__global__ __launch_bounds__(256) void rotor_apply_kernel(const float* __restrict__ cs,
                                                           const float* __restrict__ X, float* __restrict__ Y,
                                                           long long batch, long long ldx) {
    static_assert(RB >= 1 && N - RB <= 6, "a row spans at most one wave");
    constexpr int LB = N - RB;
    const unsigned L = threadIdx.x & ((1u << LB) - 1u);
    const long long rows_per_block = 256 >> LB;
    const long long stride = (long long)gridDim.x * rows_per_block;
    long long row = (long long)blockIdx.x * rows_per_block + (threadIdx.x >> LB);
    const long long lane_off = (long long)L << RB;
    float v[1 << RB];
    load_row_part<RB>(v, X + (row < batch ? row : batch - 1) * ldx + lane_off);
    for (; row < batch; row += stride) {
        const long long nrow = row + stride;
        float nv[1 << RB];
        load_row_part<RB>(nv, X + (nrow < batch ? nrow : batch - 1) * ldx + lane_off);
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

__device__ __forceinline__ float wave_sum_f32(float v) {
    for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Persistent: each workgroup walks rows with a grid stride, writes gx (if
// requested) and, if gamma_ws != nullptr, its partial K (C(N,2) floats) to
// gamma_ws[blockIdx.x * C(N,2)].
template <int N, int RB = rotor_rb(N)>
__global__ __launch_bounds__(256) void rotor_apply_bwd_kernel(const float* __restrict__ cs,
                                                               const float* __restrict__ X,
                                                               const float* __restrict__ GY,
                                                               float* __restrict__ GX,
                                                               float* __restrict__ gamma_ws, long long batch,
                                                               long long ldg) {
    static_assert(RB >= 1 && N - RB <= 6, "a row spans at most one wave");
    constexpr int LB = N - RB;
    constexpr int LPR = 1 << LB;
    constexpr int C = n_planes(N);
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
            load_row_part<RB>(g, GY + row * ldg + ((long long)Lr << RB));  // ldg: 2^N, or 0 (one row for all)
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
    // each lane position's sign, then one sum over the whole wave (rows and
    // lane positions), then over the four waves
    __shared__ float red[4][C];  // blockDim.x == 256: four waves
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < C; ++i) {
        const float t = wave_sum_f32(skew_lane_sign<N, RB>(i, L) * acc[i]);
        if (lane == 0) red[wave][i] = t;
    }
    __syncthreads();
    for (int k = threadIdx.x; k < C; k += blockDim.x)
        gamma_ws[(long long)blockIdx.x * C + k] = (red[0][k] + red[1][k]) + (red[2][k] + red[3][k]);
}

// ---- the chain with rows staged in LDS (any n up to 12, run-time planes) ----
// Used for the reference's backward on a caller's cs (every n) and for the
// n = 12 forward and transposed apply up to 768 rows; the other chain work at
// n = 11, 12 runs the register kernels with one wave per row (32 and 64
// floats per lane), which measured faster there. A workgroup stages
// kLdsBlades floats per array (whole rows; one row at n = 12) and walks the
// planes with a barrier between planes; each thread owns kLdsBlades / 1024
// blade pairs of every plane, found by inserting zero bits at p and q into
// the pair number:
//   base = deposit(t), I = base | 2^p (p set, q clear), J = base | 2^q.
// Modes:
//   LDS_FWD    y = chain(cs) x
//   LDS_TR     gx = chain(cs)^T gy
//   LDS_CS_BWD from (y, gy): gx and the cs gradient (the reference's rule:
//              inputs rebuilt with the transposed pair map,
//              grad_c += g_I v_I + g_J v_J, grad_s += sig (g_I v_J - g_J v_I))
//   LDS_GAMMA  from (x, gy): gx = chain^T gy and the statistics
//              K_pq = sum sig (x_J gx_I - x_I gx_J) of the composite backward
// Per-plane sums go through a wave reduction into a per-wave LDS slot (no
// atomics, fixed order), then one partial per workgroup.
constexpr int kLdsBlades = 4096;
enum LdsMode { LDS_FWD = 0, LDS_TR = 1, LDS_CS_BWD = 2, LDS_GAMMA = 3 };

__device__ __forceinline__ unsigned deposit2(unsigned t, int p, int q) {
    const unsigned lo = t & ((1u << p) - 1u);
    const unsigned mid = (t >> p) & ((1u << (q - p - 1)) - 1u);
    const unsigned hi = t >> (q - 1);
    return lo | (mid << (p + 1)) | (hi << (q + 1));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
    for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}

template <int MODE>
__global__ __launch_bounds__(256) void rotor_chain_lds_kernel(int n, const float* __restrict__ cs,
                                                               const float* __restrict__ A,
                                                               const float* __restrict__ B, float* __restrict__ OUT,
                                                               float* __restrict__ parts, long long batch,
                                                               long long lda, long long ldb) {
    constexpr bool TWO = (MODE == LDS_CS_BWD || MODE == LDS_GAMMA);
    constexpr int kMaxW = 2 * 66;  // 2 C(12, 2)
    __shared__ float va[kLdsBlades];
    __shared__ float vb[TWO ? kLdsBlades : 1];
    __shared__ float acc[TWO ? 4 : 1][TWO ? kMaxW : 1];
    const int D = 1 << n;
    const int C = n * (n - 1) / 2;
    const int rpb = kLdsBlades >> n > 0 ? kLdsBlades >> n : 1;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int pairs = (rpb * D) >> 2;  // per plane in the staged rows
    if (TWO)
        for (int e = tid; e < 4 * kMaxW; e += blockDim.x) (&acc[0][0])[e] = 0.f;
    for (long long row0 = (long long)blockIdx.x * rpb; row0 < batch; row0 += (long long)gridDim.x * rpb) {
        const long long rows = (batch - row0) < rpb ? (batch - row0) : rpb;
        const int nb = (int)(rows << n);
        __syncthreads();  // the previous group's last plane and stores are done
        for (int e = tid * 4; e < nb; e += blockDim.x * 4) {
            // rows of A and B are lda / ldb floats apart (2^n, or 0: one row for all)
            const long long r = row0 + (e >> n), c = e & (D - 1);
            *reinterpret_cast<float4*>(&va[e]) = *reinterpret_cast<const float4*>(A + r * lda + c);
            if (TWO) *reinterpret_cast<float4*>(&vb[e]) = *reinterpret_cast<const float4*>(B + r * ldb + c);
        }
        if (MODE == LDS_GAMMA) {
            // gx = chain^T gy on vb (planes last to first), then K from (va = x, vb = gx)
            for (int k = C - 1; k >= -C; --k) {
                __syncthreads();
                const bool stats = k < 0;
                const int kk = stats ? -1 - k : k;
                int p = 0, rem = kk;
                while (rem >= n - 1 - p) {
                    rem -= n - 1 - p;
                    ++p;
                }
                const int q = p + 1 + rem;
                const float c = cs[2 * (C - 1 - kk)], sv = cs[2 * (C - 1 - kk) + 1];
                const unsigned between = ((1u << q) - 1u) & ~((2u << p) - 1u);
                float part = 0.f;
                for (int t = tid; t < pairs; t += blockDim.x) {
                    const int r = t >> (n - 2), tt = t & ((D >> 2) - 1);
                    const unsigned base = deposit2((unsigned)tt, p, q);
                    const int I = (r << n) | (int)(base | (1u << p)), J = (r << n) | (int)(base | (1u << q));
                    const float sig = (__popc(base & between) & 1) ? -1.f : 1.f;
                    if (r >= rows) continue;
                    const float gI = vb[I], gJ = vb[J];
                    if (!stats) {
                        // transposed pair map: (gI, gJ) <- (c gI - s sig gJ, c gJ + s sig gI)
                        vb[I] = __builtin_fmaf(c, gI, -sv * sig * gJ);
                        vb[J] = __builtin_fmaf(c, gJ, sv * sig * gI);
                    } else {
                        part = __builtin_fmaf(sig, __builtin_fmaf(va[J], gI, -va[I] * gJ), part);
                    }
                }
                if (stats) {
                    part = wave_sum_dpp(part);
                    if (lane == 0) acc[wave][kk] += part;
                }
            }
            __syncthreads();
            for (int e = tid * 4; e < nb; e += blockDim.x * 4)
                if (OUT) *reinterpret_cast<float4*>(OUT + (row0 << n) + e) = *reinterpret_cast<const float4*>(&vb[e]);
            continue;
        }
        for (int step = 0; step < C; ++step) {
            __syncthreads();
            const int k = (MODE == LDS_FWD) ? step : C - 1 - step;
            int p = 0, rem = k;
            while (rem >= n - 1 - p) {
                rem -= n - 1 - p;
                ++p;
            }
            const int q = p + 1 + rem;
            const float c = cs[2 * (C - 1 - k)], sv = cs[2 * (C - 1 - k) + 1];
            const unsigned between = ((1u << q) - 1u) & ~((2u << p) - 1u);
            float dc = 0.f, dsum = 0.f;
            for (int t = tid; t < pairs; t += blockDim.x) {
                const int r = t >> (n - 2), tt = t & ((D >> 2) - 1);
                if (r >= rows) continue;
                const unsigned base = deposit2((unsigned)tt, p, q);
                const int I = (r << n) | (int)(base | (1u << p)), J = (r << n) | (int)(base | (1u << q));
                const float ss = (__popc(base & between) & 1) ? -sv : sv;
                const float xI = va[I], xJ = va[J];
                if (MODE == LDS_FWD) {
                    va[I] = __builtin_fmaf(c, xI, ss * xJ);
                    va[J] = __builtin_fmaf(c, xJ, -ss * xI);
                } else {
                    // rebuilt input (LDS_CS_BWD) or transposed gradient (LDS_TR)
                    const float pI = __builtin_fmaf(c, xI, -ss * xJ);
                    const float pJ = __builtin_fmaf(c, xJ, ss * xI);
                    va[I] = pI;
                    va[J] = pJ;
                    if (MODE == LDS_CS_BWD) {
                        const float gI = vb[I], gJ = vb[J];
                        const float sig = (__popc(base & between) & 1) ? -1.f : 1.f;
                        dc = __builtin_fmaf(gI, pI, __builtin_fmaf(gJ, pJ, dc));
                        dsum = __builtin_fmaf(sig, __builtin_fmaf(gI, pJ, -gJ * pI), dsum);
                        vb[I] = __builtin_fmaf(c, gI, -ss * gJ);
                        vb[J] = __builtin_fmaf(c, gJ, ss * gI);
                    }
                }
            }
            if (MODE == LDS_CS_BWD) {
                dc = wave_sum_dpp(dc);
                dsum = wave_sum_dpp(dsum);
                if (lane == 0) {
                    acc[wave][2 * (C - 1 - k)] += dc;
                    acc[wave][2 * (C - 1 - k) + 1] += dsum;
                }
            }
        }
        __syncthreads();
        const float* res = (MODE == LDS_CS_BWD) ? vb : va;
        if (OUT)
            for (int e = tid * 4; e < nb; e += blockDim.x * 4)
                *reinterpret_cast<float4*>(OUT + (row0 << n) + e) = *reinterpret_cast<const float4*>(&res[e]);
    }
    if (!TWO || !parts) return;
    __syncthreads();
    const int W = (MODE == LDS_CS_BWD) ? 2 * C : C;
    for (int e = tid; e < W; e += blockDim.x)
        parts[(long long)blockIdx.x * W + e] = (acc[0][e] + acc[1][e]) + (acc[2][e] + acc[3][e]);
}

// out[e] = sum_p parts[p * width + e] in fp64, one workgroup, deterministic
__global__ __launch_bounds__(256) void parts_sum_kernel(const float* __restrict__ parts, int nparts, int width,
                                                        float* __restrict__ out) {
    for (int e = threadIdx.x; e < width; e += blockDim.x) {
        double t0 = 0.0, t1 = 0.0, t2 = 0.0, t3 = 0.0;
        int p = 0;
        for (; p + 3 < nparts; p += 4) {
            t0 += (double)parts[(long long)p * width + e];
            t1 += (double)parts[(long long)(p + 1) * width + e];
            t2 += (double)parts[(long long)(p + 2) * width + e];
            t3 += (double)parts[(long long)(p + 3) * width + e];
        }
        for (; p < nparts; ++p) t0 += (double)parts[(long long)p * width + e];
        out[e] = (float)((t0 + t1) + (t2 + t3));
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

// The reference's Givens factorisation of R (lane j < N holding column j of
// E = R): for the planes in lex order E <- G_k E (E ends as I), and lane 0
// writes the (c, s) of plane k at index C - 1 - k of cs (and of cs2 if given).
template <int N>
__device__ __forceinline__ void givens_cols(double (&col)[N], float* __restrict__ cs, float* __restrict__ cs2,
                                            int lane) {
    constexpr int C = n_planes(N);
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
                cs[2 * (C - 1 - k)] = (float)c;
                cs[2 * (C - 1 - k) + 1] = (float)s;
                if (cs2) {
                    cs2[2 * (C - 1 - k)] = (float)c;
                    cs2[2 * (C - 1 - k) + 1] = (float)s;
                }
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

// Lane j < N computes column j of R = expm(B) = Q^T, i.e. row j of Q.
template <int N>
__global__ __launch_bounds__(64) void rotor_compile_fwd_cols_kernel(const float* __restrict__ biv,
                                                                     float* __restrict__ state,
                                                                     float* __restrict__ cs_out) {
    __shared__ double Z[N * N];
    const int j = threadIdx.x;
    for (int idx = j; idx < N * N; idx += 64) Z[idx] = generator_entry(biv, N, idx % N, idx / N);  // B = A^T
    __syncthreads();
    double col[N];
    expm_cols<N>(col, Z, j);
    if (j < N)
#pragma unroll
        for (int i = 0; i < N; ++i) state[j * N + i] = (float)col[i];
    // Givens elimination of R (planes in lex order); E ends as I (det = +1)
    givens_cols<N>(col, state + N * N, cs_out, j);
}

// dL/dQ (tangent part) = Q skew(Gamma), skew(Gamma)[p][q] = K_pq / 2 = -skew(Gamma)[q][p],
// K = sum of the per-workgroup partials. Called by all 1024 threads of the
// workgroup (it holds barriers); thread t < n^2 gets entry t (row-major) of
// Q skew(Gamma), the others 0. Entries are padded to EP (a power of two >=
// C(n,2)): thread t sums partials p = t/EP, t/EP + 1024/EP, ... of entry
// t % EP, then the 1024/EP groups are added.
__device__ double gamma_q_skew(int n, const float* __restrict__ state, const float* __restrict__ gamma_ws,
                               int nparts, double* __restrict__ part, double* __restrict__ S) {
    const int C = n_planes(n);
    int ep = 1;
    while (ep < C) ep <<= 1;
    const int ngrp = 1024 / ep;
    const int e = threadIdx.x & (ep - 1), grp = threadIdx.x / ep;
    // sixteen independent loads per iteration, so their latencies overlap (the
    // usual partial count, 512 at n = 8, takes one iteration)
    float t[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) t[u] = 0.f;
    double acc = 0.0;
    if (e < C) {
        int p = grp;
        for (; p + 15 * ngrp < nparts; p += 16 * ngrp) {
#pragma unroll
            for (int u = 0; u < 16; ++u) t[u] = gamma_ws[(long long)(p + u * ngrp) * C + e];
#pragma unroll
            for (int u = 0; u < 16; ++u) acc += (double)t[u];
        }
        for (; p < nparts; p += ngrp) acc += (double)gamma_ws[(long long)p * C + e];
    }
    part[threadIdx.x] = acc;
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
    double v = 0.0;
    if ((int)threadIdx.x < n * n) {
        const int i = threadIdx.x / n, j = threadIdx.x % n;
        for (int k = 0; k < n; ++k) v += (double)state[i * n + k] * S[k * n + j];
    }
    return v;
}

// Writes the Q slot of g_state (Q skew(Gamma)) and zeroes its other slots.
__global__ __launch_bounds__(1024) void rotor_gamma_finalize_kernel(int n, const float* __restrict__ state,
                                                                     const float* __restrict__ gamma_ws, int nparts,
                                                                     float* __restrict__ g_state) {
    __shared__ double part[1024];
    __shared__ double S[kRotorMaxN * kRotorMaxN];
    const double v = gamma_q_skew(n, state, gamma_ws, nparts, part, S);
    if ((int)threadIdx.x < n * n) g_state[threadIdx.x] = (float)v;
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

// g_biv from dL/dQ (row-major in G, LDS) through Q = expm(A), A = -B(biv):
// dL/dA = L(A^T, dL/dQ), the (1,2) block of expm([[A^T, dL/dQ], [0, A^T]]).
// One wave; X and F are N x N LDS scratch. G is scaled in place.
template <int N>
__device__ __forceinline__ void frechet_to_biv(const float* __restrict__ biv, double* __restrict__ G,
                                               double* __restrict__ X, double* __restrict__ F,
                                               float* __restrict__ g_biv, int j) {
    double gmax = 0.0;
    for (int idx = j; idx < N * N; idx += 64) gmax = fmax(gmax, fabs(G[idx]));
    gmax = wave_max_f64(gmax) * N;  // bounds every column sum of |G|
    int gexp = 0;
    if (gmax > 1.0) frexp(gmax, &gexp);
    wave_lds_sync();
    for (int idx = j; idx < N * N; idx += 64) {
        const int r = idx / N, c = idx % N;
        X[idx] = generator_entry(biv, N, c, r);  // A^T
        G[idx] = ldexp(G[idx], -gexp);
    }
    wave_lds_sync();
    double Lc[N];
    expm_frechet_cols<N>(Lc, X, G, j);
    if (j < N)
#pragma unroll
        for (int i = 0; i < N; ++i) F[i * N + j] = ldexp(Lc[i], gexp);
    wave_lds_sync();
    for (int k = j; k < n_planes(N); k += 64) {
        const int p = plane_p(N, k), q = plane_q(N, k);
        // dL/dB = -dL/dA; dL/db = 2 (dL/dB[p][q] - dL/dB[q][p])
        g_biv[k] = (float)(-2.0 * (F[p * N + q] - F[q * N + p]));
    }
}

template <int N>
__global__ __launch_bounds__(64) void rotor_compile_bwd_cols_kernel(const float* __restrict__ biv,
                                                                     const float* __restrict__ g_state,
                                                                     float* __restrict__ g_biv) {
    __shared__ double X[N * N], G[N * N], F[N * N];
    const int j = threadIdx.x;
    for (int idx = j; idx < N * N; idx += 64) G[idx] = (double)g_state[idx];
    wave_lds_sync();
    frechet_to_biv<N>(biv, G, X, F, g_biv, j);
}

// g_biv from the gradient of the reference-layout cs through
// cs = Givens(R), R = expm(B) = Q^T. One wave: R's columns in lanes (fp64),
// the factorisation replayed with each plane's input rows p and q recorded in
// LDS, then reverse mode through it:
//   rows P' = c P + s Qr, Q' = -s P + c Qr:  dc += <gP', P> + <gQ', Qr>,
//   ds += <gP', Qr> - <gQ', P>,  gP = c gP' - s gQ',  gQ = s gP' + c gQ';
//   (c, s) = (a, b) / r:  ga = (dc b^2 - ds a b) / r^3,  gb = (ds a^2 - dc a b) / r^3
// with a = E[p][p], b = E[q][p]. dL/dQ = (dL/dR)^T, then the Frechet step.
template <int N>
__global__ __launch_bounds__(64) void rotor_cs_compile_bwd_kernel(const float* __restrict__ biv,
                                                                   const float* __restrict__ g_cs,
                                                                   float* __restrict__ g_biv) {
    constexpr int C = n_planes(N);
    __shared__ double Z[N * N], F[N * N];
    __shared__ double rows[C][2][N];
    const int j = threadIdx.x;
    const bool act = j < N;
    for (int idx = j; idx < N * N; idx += 64) Z[idx] = generator_entry(biv, N, idx % N, idx / N);  // B = A^T
    wave_lds_sync();
    double col[N];
    expm_cols<N>(col, Z, j);
    // forward replay (column j of E in lane j), recording the rows p, q entering each plane
#pragma unroll
    for (int p = 0; p < N - 1; ++p) {
#pragma unroll
        for (int q = p + 1; q < N; ++q) {
            const int k = p * N - p * (p + 1) / 2 + (q - p - 1);
            if (act) {
                rows[k][0][j] = col[p];
                rows[k][1][j] = col[q];
            }
            double c, s;
            givens_cs(readlane_f64(col[p], p), readlane_f64(col[q], p), c, s);
            const double ep = col[p], eq = col[q];
            col[p] = c * ep + s * eq;
            col[q] = -s * ep + c * eq;
        }
    }
    wave_lds_sync();
    // reverse mode; gcol = column j of dL/dE (A_final is not an output: starts at 0)
    double gcol[N];
#pragma unroll
    for (int i = 0; i < N; ++i) gcol[i] = 0.0;
#pragma unroll
    for (int p = N - 2; p >= 0; --p) {
#pragma unroll
        for (int q = N - 1; q > p; --q) {
            const int k = p * N - p * (p + 1) / 2 + (q - p - 1);
            const double P = act ? rows[k][0][j] : 0.0, Qr = act ? rows[k][1][j] : 0.0;
            const double a = rows[k][0][p], b = rows[k][1][p];
            double c, s;
            givens_cs(a, b, c, s);
            const double gp = gcol[p], gq = gcol[q];
            double dc = gp * P + gq * Qr, ds = gp * Qr - gq * P;
            for (int off = 1; off < 64; off <<= 1) {
                dc += __shfl_xor(dc, off, 64);
                ds += __shfl_xor(ds, off, 64);
            }
            dc += (double)g_cs[2 * (C - 1 - k)];
            ds += (double)g_cs[2 * (C - 1 - k) + 1];
            gcol[p] = c * gp - s * gq;
            gcol[q] = s * gp + c * gq;
            const double r2 = a * a + b * b;
            if (r2 > 1e-300 && j == p) {
                const double r = sqrt(r2);
                const double ir3 = 1.0 / (r2 * r);
                gcol[p] += (dc * b * b - ds * a * b) * ir3;
                gcol[q] += (ds * a * a - dc * a * b) * ir3;
            }
        }
    }
    // dL/dQ[i][jj] = dL/dR[jj][i] = lane i's gcol[jj]
    if (act)
#pragma unroll
        for (int jj = 0; jj < N; ++jj) F[j * N + jj] = gcol[jj];
    wave_lds_sync();
    frechet_to_biv<N>(biv, F, Z, (double*)&rows[0][0][0], g_biv, j);
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
                                                                     float* __restrict__ state,
                                                                     float* __restrict__ cs_out, SpinTable spin) {
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
    // Givens elimination of R = Q^T on columns: lane j < N gathers column j of
    // R (row j of Q), so the row updates of a plane are register operations
    double col[N];
#pragma unroll
    for (int r = 0; r < N; ++r) col[r] = shfl_f64(e, (lane < N ? lane : 0) * N + r);
    givens_cols<N>(col, state + N * N, cs_out, lane);
}

// Adjoint Frechet derivative by the block identity (see the column version):
// lane (i, j) holds E[i][j] and L[i][j]; X = A^T and G rows in registers.
// Run by one whole wave (lanes 0..63); g holds row i of dL/dQ for lane
// (i, j) = (lane / N, lane % N) (row 0 for lanes past N^2).
template <int N>
__device__ __forceinline__ void compile_bwd_ent(const float* __restrict__ biv, double (&g)[N],
                                                float* __restrict__ g_biv) {
    static_assert(N * N <= 64, "one entry per lane");
    const int lane = threadIdx.x & 63;
    const bool active = lane < N * N;
    const int i = active ? lane / N : 0, j = active ? lane % N : 0;
    double x[N];
    double xs = 0.0, gs = 0.0;
#pragma unroll
    for (int l = 0; l < N; ++l) {
        x[l] = generator_entry(biv, N, l, i);  // (A^T)[i][l]
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

template <int N>
__global__ __launch_bounds__(64) void rotor_compile_bwd_ent_kernel(const float* __restrict__ biv,
                                                                    const float* __restrict__ g_state,
                                                                    float* __restrict__ g_biv) {
    const int lane = threadIdx.x;
    const int i = lane < N * N ? lane / N : 0;
    double g[N];
#pragma unroll
    for (int l = 0; l < N; ++l) g[l] = (double)g_state[i * N + l];
    compile_bwd_ent<N>(biv, g, g_biv);
}

// The bivector gradient straight from the apply backward's partials (n <= 8):
// the batch sum and Q skew(Gamma) of the finalize, kept in LDS in fp64, then
// wave 0 runs the compile backward on it. One launch instead of two, and no
// g_state round trip through memory.
template <int N>
__global__ __launch_bounds__(1024) void rotor_gamma_biv_kernel(const float* __restrict__ biv,
                                                                const float* __restrict__ state,
                                                                const float* __restrict__ gamma_ws, int nparts,
                                                                float* __restrict__ g_biv) {
    __shared__ double part[1024];
    __shared__ double S[N * N];
    __shared__ double G[N * N];
    const double v = gamma_q_skew(N, state, gamma_ws, nparts, part, S);
    if ((int)threadIdx.x < N * N) G[threadIdx.x] = v;
    __syncthreads();
    if (threadIdx.x >= 64) return;  // no barrier follows
    const int i = (int)threadIdx.x < N * N ? (int)threadIdx.x / N : 0;
    double g[N];
#pragma unroll
    for (int l = 0; l < N; ++l) g[l] = G[i * N + l];
    compile_bwd_ent<N>(biv, g, g_biv);
}

// ---- host side --------------------------------------------------------------

// register-layout kernels: n = 2 .. 10
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

// compile kernels: n = 2 .. 12
#define CLF_COMPILE_DISPATCH(n, CALL)     \
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
        case 11: CALL(11); break;         \
        case 12: CALL(12); break;         \
        default: break;                   \
    }

constexpr int kRegChainMaxN = 10;  // largest n of the default register layout (64 floats on 2^(n-6) lanes)

// one entry per lane up to n = 8 (64 entries), one column per lane above
template <int N>
static int launch_compile_fwd(const float* biv, float* state, float* cs, hipStream_t s) {
    if constexpr (N * N <= 64) {
        SpinTable spin{};
        if constexpr (N == kSpinN) {
            RepTable T;
            if (!spin_tables(T, spin)) return set_error(CLF_ERR_UNSUPPORTED, "Cl(8,0) representation tables unavailable");
        }
        hipLaunchKernelGGL((rotor_compile_fwd_ent_kernel<N>), dim3(1), dim3(N == kSpinN ? 128 : 64), 0, s, biv, state,
                           cs, spin);
    } else {
        hipLaunchKernelGGL((rotor_compile_fwd_cols_kernel<N>), dim3(1), dim3(64), 0, s, biv, state, cs);
    }
    return CLF_OK;
}

template <int N>
static void launch_compile_bwd(const float* biv, const float* g_state, float* g_biv, hipStream_t s) {
    if constexpr (N * N <= 64)
        hipLaunchKernelGGL((rotor_compile_bwd_ent_kernel<N>), dim3(1), dim3(64), 0, s, biv, g_state, g_biv);
    else hipLaunchKernelGGL((rotor_compile_bwd_cols_kernel<N>), dim3(1), dim3(64), 0, s, biv, g_state, g_biv);
}

// Partials -> g_biv: one fused launch while Q is n x n <= 64 entries (one per
// lane of the compile backward), else the finalize into g_state and the
// column compile backward.
template <int N>
static void launch_gamma_biv(const float* biv, const float* state, const float* gws, int nparts, float* g_state,
                             float* g_biv, hipStream_t s) {
    if constexpr (N * N <= 64) {
        hipLaunchKernelGGL((rotor_gamma_biv_kernel<N>), dim3(1), dim3(1024), 0, s, biv, state, gws, nparts, g_biv);
    } else {
        hipLaunchKernelGGL(rotor_gamma_finalize_kernel, dim3(1), dim3(1024), 0, s, N, state, gws, nparts, g_state);
        launch_compile_bwd<N>(biv, g_state, g_biv, s);
    }
}

static int check_rotor_n(int n) {
    if (n < kRotorMinN || n > kRotorMaxN)
        return set_error(CLF_ERR_ARG, "rotor kernels support n in [" + std::to_string(kRotorMinN) + ", " +
                                          std::to_string(kRotorMaxN) + "], got " + std::to_string(n));
    return CLF_OK;
}

int rotor_state_floats(int n) { return (n >= kRotorMinN && n <= kRotorMaxN) ? state_floats(n) : -1; }

// Workgroups of a backward launch (and so partials in the workspace): the
// register kernels take 256 >> (lanes per row) rows per workgroup, the
// LDS-staged kernel kLdsBlades / 2^n rows.
static bool use_wave_rows_bwd(int n, int64_t batch);

static int rotor_bwd_grid(int n, int64_t batch) {
    long long rows_per_block;
    if (use_wave_rows_bwd(n, batch)) rows_per_block = 4;
    else if (n <= kRegChainMaxN) rows_per_block = 256 >> (n - rotor_rb(n));
    else rows_per_block = kLdsBlades >> n > 0 ? kLdsBlades >> n : 1;
    long long g = (batch + rows_per_block - 1) / rows_per_block;
    if (g > 1024) g = 1024;
    if (g < 1) g = 1;
    return (int)g;
}

static long long lds_groups(int n, int64_t batch) {
    const long long rpb = kLdsBlades >> n > 0 ? kLdsBlades >> n : 1;
    return (batch + rpb - 1) / rpb;
}

static int cs_bwd_grid(int n, int64_t batch) {
    long long g = lds_groups(n, batch);
    if (g > 1024) g = 1024;
    if (g < 1) g = 1;
    return (int)g;
}

size_t rotor_apply_ws_bytes(int n, int64_t batch) {
    if (n < kRotorMinN || n > kRotorMaxN || batch < 0) return 0;
    return (size_t)rotor_bwd_grid(n, batch) * n_planes(n) * sizeof(float);
}

size_t rotor_cs_apply_ws_bytes(int n, int64_t batch) {
    if (n < kRotorMinN || n > kRotorMaxN || batch < 0) return 0;
    return (size_t)cs_bwd_grid(n, batch) * 2 * n_planes(n) * sizeof(float);
}

int rotor_compile_fwd(int n, const float* biv, float* state, float* cs, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (!biv || !state) return set_error(CLF_ERR_ARG, "null pointer argument");
    hipStream_t s = (hipStream_t)stream;
    int rc = CLF_OK;
#define CLF_CALL(N) rc = launch_compile_fwd<N>(biv, state, cs, s)
    CLF_COMPILE_DISPATCH(n, CLF_CALL)
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
    CLF_COMPILE_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

// LDS-staged chain launch: grid of at most `cap` workgroups and at most the
// resident workgroups, never more than the row groups.
template <int MODE>
static unsigned lds_grid(int n, int64_t batch, long long cap) {
    long long want = lds_groups(n, batch);
    if (want > cap) want = cap;
    return resident_grid((const void*)rotor_chain_lds_kernel<MODE>, 256, 0, want);
}

template <int MODE>
static void launch_lds(int n, const float* cs, const float* a, const float* b, float* out, float* parts, int64_t batch,
                       unsigned grid, hipStream_t s, long long lda, long long ldb) {
    hipLaunchKernelGGL((rotor_chain_lds_kernel<MODE>), dim3(grid), dim3(256), 0, s, n, cs, a, b, out, parts,
                       (long long)batch, lda, ldb);
}

template <int N>
static void launch_apply_reg(bool fwd, const float* cs, const float* x, float* y, int64_t batch, hipStream_t s,
                             long long ldx) {
    constexpr int LB = N - rotor_rb(N);
    const long long threads = (long long)batch << LB;
    const long long wanted = (threads + 255) / 256;
    if (fwd) {
        const dim3 grid(resident_grid((const void*)rotor_apply_kernel<N, true>, 256, 0, wanted));
        hipLaunchKernelGGL((rotor_apply_kernel<N, true>), grid, dim3(256), 0, s, cs, x, y, (long long)batch, ldx);
    } else {
        const dim3 grid(resident_grid((const void*)rotor_apply_kernel<N, false>, 256, 0, wanted));
        hipLaunchKernelGGL((rotor_apply_kernel<N, false>), grid, dim3(256), 0, s, cs, x, y, (long long)batch, ldx);
    }
}

// One wave per row (four rows per workgroup, 2^(n-6) floats per lane) where
// it measured faster than the default layouts (rotor_rb: 64 floats on
// 2^(n-6) lanes; the LDS-staged chain at n = 11, 12). Device time of one
// forward apply, old -> wave rows: n = 9 19.5 -> 9.2 us at 64 to 2048 rows,
// 24.2 -> 17.9 at 8192, even at 16384, 56 -> 66 at 32768 rows; n = 10
// 30 -> 14.5 at 64 rows, 532 -> 455 at 131072; n = 11 43 -> 26.4 at 64 rows,
// 1535 -> 532 at 65536; n = 12 51.4 -> 62.5 at 64 rows, 57.1 -> 63.8 at
// 512, 77.9 -> 66.6 at 1024, 1848 -> 1100 at 32768.
static bool use_wave_rows(int n, int64_t batch) {
    switch (n) {
        case 9: return batch <= 12288;
        case 10:
        case 11: return true;
        case 12: return batch > 768;
        default: return false;
    }
}

template <int N>
static void launch_apply_wave_rows(bool fwd, const float* cs, const float* x, float* y, int64_t batch, hipStream_t s,
                                   long long ldx) {
    const dim3 grid((unsigned)((batch + 3) / 4));
    if (fwd)
        hipLaunchKernelGGL((rotor_apply_kernel<N, true, N - 6>), grid, dim3(256), 0, s, cs, x, y, (long long)batch,
                           ldx);
    else
        hipLaunchKernelGGL((rotor_apply_kernel<N, false, N - 6>), grid, dim3(256), 0, s, cs, x, y, (long long)batch,
                           ldx);
}

// y = chain(cs) x (fwd) or chain(cs)^T x, any n in range, batch > 0; x's rows
// are ldx floats apart (2^n, or 0 for one row broadcast over the batch)
static void launch_chain(int n, bool fwd, const float* cs, const float* x, float* y, int64_t batch, hipStream_t s,
                         long long ldx) {
    if (use_wave_rows(n, batch)) {
        switch (n) {
            case 9: launch_apply_wave_rows<9>(fwd, cs, x, y, batch, s, ldx); break;
            case 10: launch_apply_wave_rows<10>(fwd, cs, x, y, batch, s, ldx); break;
            case 11: launch_apply_wave_rows<11>(fwd, cs, x, y, batch, s, ldx); break;
            default: launch_apply_wave_rows<12>(fwd, cs, x, y, batch, s, ldx); break;
        }
    } else if (n <= kRegChainMaxN) {
#define CLF_CALL(N) launch_apply_reg<N>(fwd, cs, x, y, batch, s, ldx)
        CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
    } else if (fwd) {
        launch_lds<LDS_FWD>(n, cs, x, nullptr, y, nullptr, batch, lds_grid<LDS_FWD>(n, batch, 1LL << 30), s, ldx, 0);
    } else {
        launch_lds<LDS_TR>(n, cs, x, nullptr, y, nullptr, batch, lds_grid<LDS_TR>(n, batch, 1LL << 30), s, ldx, 0);
    }
}

// Composite backward with the K statistics: the register kernel (n <= 10) or
// the LDS-staged kernel; returns the number of partials written.
template <int N>
static int launch_apply_bwd_reg(const float* cs, const float* x, const float* gy, long long ldg, float* gx, float* ws,
                                int64_t batch, hipStream_t s) {
    const unsigned grid = resident_grid((const void*)rotor_apply_bwd_kernel<N>, 256, 0, rotor_bwd_grid(N, batch));
    hipLaunchKernelGGL((rotor_apply_bwd_kernel<N>), dim3(grid), dim3(256), 0, s, cs, x, gy, gx, ws, (long long)batch,
                       ldg);
    return (int)grid;
}

// The backward with the statistics on one wave per row (2^(n-6) floats per
// lane) where it measured faster. Device time of one call (gx and the
// partials), old -> wave rows: n = 9 40.1 -> 23.0 us at 64 rows, 40.8 -> 24.4
// at 1024, 47.1 -> 50.5 at 8192; n = 10 55.8 -> 33.3 at 64, 58.5 -> 35.9 at
// 1024, 79.5 -> 81.5 at 8192; n = 11 108 -> 63.5 at 64, 602 -> 178 at 8192
// (the LDS-staged chain before); n = 12 132 -> 101 at 64, 725 -> 347 at 4096.
static bool use_wave_rows_bwd(int n, int64_t batch) {
    if (n == 9 || n == 10) return batch <= 4096;
    return n == 11 || n == 12;
}

template <int N>
static int launch_apply_bwd_wave_rows(const float* cs, const float* x, const float* gy, long long ldg, float* gx,
                                      float* ws, int64_t batch, hipStream_t s) {
    const unsigned grid =
        resident_grid((const void*)rotor_apply_bwd_kernel<N, N - 6>, 256, 0, rotor_bwd_grid(N, batch));
    hipLaunchKernelGGL((rotor_apply_bwd_kernel<N, N - 6>), dim3(grid), dim3(256), 0, s, cs, x, gy, gx, ws,
                       (long long)batch, ldg);
    return (int)grid;
}

static int launch_gamma(int n, const float* cs, const float* x, const float* gy, long long ldg, float* gx, float* ws,
                        int64_t batch, hipStream_t s) {
    int nparts = 0;
    if (use_wave_rows_bwd(n, batch)) {
        switch (n) {
            case 9: nparts = launch_apply_bwd_wave_rows<9>(cs, x, gy, ldg, gx, ws, batch, s); break;
            case 10: nparts = launch_apply_bwd_wave_rows<10>(cs, x, gy, ldg, gx, ws, batch, s); break;
            case 11: nparts = launch_apply_bwd_wave_rows<11>(cs, x, gy, ldg, gx, ws, batch, s); break;
            default: nparts = launch_apply_bwd_wave_rows<12>(cs, x, gy, ldg, gx, ws, batch, s); break;
        }
    } else if (n <= kRegChainMaxN) {
#define CLF_CALL(N) nparts = launch_apply_bwd_reg<N>(cs, x, gy, ldg, gx, ws, batch, s)
        CLF_ROTOR_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
    } else {
        const unsigned grid = lds_grid<LDS_GAMMA>(n, batch, rotor_bwd_grid(n, batch));
        launch_lds<LDS_GAMMA>(n, cs, x, gy, gx, ws, batch, grid, s, 1LL << n, ldg);
        nparts = (int)grid;
    }
    return nparts;
}

bool rotor16_enabled(int n);
int rotor16_apply(bool fwd, const float* U, const float* x, float* y, int64_t batch, void* stream,
                  long long ldx = 256);
int rotor16_bwd(const float* U, const float* x, const float* gy, long long ldg, float* gx, float* gamma_ws,
                int64_t batch, unsigned grid, void* stream);
unsigned rotor16_bwd_grid(long long wanted);

// gx (when given) and the per-workgroup partials of Gamma for the batch;
// nparts = the partial count (0 for an empty batch)
static int launch_gamma_parts(int n, const float* state, const float* x, const float* gy, int64_t ldg, float* gx,
                              float* gws, int64_t batch, hipStream_t s, int& nparts) {
    nparts = 0;
    if (batch == 0) return CLF_OK;
    if (rotor16_enabled(n)) {
        nparts = (int)rotor16_bwd_grid(rotor_bwd_grid(n, batch));
        if (int rc = rotor16_bwd(state + spin_offset(n), x, gy, ldg, gx, gws, batch, (unsigned)nparts, s)) return rc;
    } else {
        nparts = launch_gamma(n, state + n * n, x, gy, ldg, gx, gws, batch, s);
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int rotor_apply_fwd(int n, const float* state, const float* x, float* y, int64_t batch, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (batch == 0) return CLF_OK;
    if (!state || !x || !y) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (x == y) return set_error(CLF_ERR_ARG, "output must not alias the input");
    if ((((uintptr_t)x) | ((uintptr_t)y)) & 15u) return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    if (rotor16_enabled(n)) return rotor16_apply(true, state + spin_offset(n), x, y, batch, stream);
    launch_chain(n, true, state + n * n, x, y, batch, (hipStream_t)stream, 1LL << n);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

// gy's rows are ldg floats apart: 2^n, or 0 for one row broadcast over the batch
int rotor_apply_bwd(int n, const float* state, const float* x, const float* gy, int64_t ldg, float* gx,
                    float* g_state, int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (ldg != 0 && ldg != (1LL << n)) return set_error(CLF_ERR_ARG, "gy row stride must be 0 or 2^n");
    if (!gx && !g_state) return CLF_OK;
    if (!state || (batch > 0 && (!gy || (g_state && !x)))) return set_error(CLF_ERR_ARG, "null pointer argument");
    if ((((uintptr_t)x) | ((uintptr_t)gy) | ((uintptr_t)gx)) & 15u)
        return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    if (gx && (gx == gy || gx == x)) return set_error(CLF_ERR_ARG, "gx must not alias x or gy");
    const size_t need = rotor_apply_ws_bytes(n, batch);
    if (g_state && (!ws || ws_bytes < need))
        return set_error(CLF_ERR_WORKSPACE, "workspace of at least " + std::to_string(need) + " bytes required");
    hipStream_t s = (hipStream_t)stream;
    if (!g_state) {
        if (batch == 0) return CLF_OK;
        if (rotor16_enabled(n)) return rotor16_apply(false, state + spin_offset(n), gy, gx, batch, stream, ldg);
        launch_chain(n, false, state + n * n, gy, gx, batch, s, ldg);
        CLF_HIP_CHECK(hipGetLastError());
        return CLF_OK;
    }
    float* gws = (float*)ws;
    int nparts = 0;
    if (int rc = launch_gamma_parts(n, state, x, gy, ldg, gx, gws, batch, s, nparts)) return rc;
    hipLaunchKernelGGL(rotor_gamma_finalize_kernel, dim3(1), dim3(1024), 0, s, n, state, gws, nparts, g_state);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

size_t rotor_biv_apply_ws_bytes(int n, int64_t batch) {
    if (n < kRotorMinN || n > kRotorMaxN || batch < 0) return 0;
    return ((rotor_apply_ws_bytes(n, batch) + 255) & ~size_t(255)) + (size_t)state_floats(n) * sizeof(float);
}

// The backward of apply(compile(biv), x) to biv and x: the apply backward's
// partials, then their sum and the compile backward (one fused launch for
// n <= 8; the finalize into the workspace and the compile backward above).
int rotor_biv_apply_bwd(int n, const float* biv, const float* state, const float* x, const float* gy, int64_t ldg,
                        float* gx, float* g_biv, int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (ldg != 0 && ldg != (1LL << n)) return set_error(CLF_ERR_ARG, "gy row stride must be 0 or 2^n");
    if (!g_biv) return rotor_apply_bwd(n, state, x, gy, ldg, gx, nullptr, batch, nullptr, 0, stream);
    if (!biv || !state || (batch > 0 && (!gy || !x))) return set_error(CLF_ERR_ARG, "null pointer argument");
    if ((((uintptr_t)x) | ((uintptr_t)gy) | ((uintptr_t)gx)) & 15u)
        return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    if (gx && (gx == gy || gx == x)) return set_error(CLF_ERR_ARG, "gx must not alias x or gy");
    const size_t need = rotor_biv_apply_ws_bytes(n, batch);
    if (!ws || ws_bytes < need)
        return set_error(CLF_ERR_WORKSPACE, "workspace of at least " + std::to_string(need) + " bytes required");
    hipStream_t s = (hipStream_t)stream;
    float* gws = (float*)ws;
    int nparts = 0;
    if (int rc = launch_gamma_parts(n, state, x, gy, ldg, gx, gws, batch, s, nparts)) return rc;
    float* g_state = (float*)((char*)ws + ((rotor_apply_ws_bytes(n, batch) + 255) & ~size_t(255)));
#define CLF_CALL(N) launch_gamma_biv<N>(biv, state, gws, nparts, g_state, g_biv, s)
    CLF_COMPILE_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

// ---- the chain on a caller's cs (apply_rotor(cs, x)) ----------------------

int rotor_cs_apply_fwd(int n, const float* cs, const float* x, float* y, int64_t batch, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (batch == 0) return CLF_OK;
    if (!cs || !x || !y) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (x == y) return set_error(CLF_ERR_ARG, "output must not alias the input");
    if ((((uintptr_t)x) | ((uintptr_t)y)) & 15u) return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    launch_chain(n, true, cs, x, y, batch, (hipStream_t)stream, 1LL << n);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

// gy's rows are ldg floats apart: 2^n, or 0 for one row broadcast over the batch
int rotor_cs_apply_bwd(int n, const float* cs, const float* y, const float* gy, int64_t ldg, float* gx, float* g_cs,
                       int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (ldg != 0 && ldg != (1LL << n)) return set_error(CLF_ERR_ARG, "gy row stride must be 0 or 2^n");
    if (!gx && !g_cs) return CLF_OK;
    if (!cs || (batch > 0 && (!gy || (g_cs && !y)))) return set_error(CLF_ERR_ARG, "null pointer argument");
    if ((((uintptr_t)y) | ((uintptr_t)gy) | ((uintptr_t)gx)) & 15u)
        return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    if (gx && (gx == gy || gx == y)) return set_error(CLF_ERR_ARG, "gx must not alias y or gy");
    const size_t need = rotor_cs_apply_ws_bytes(n, batch);
    if (g_cs && (!ws || ws_bytes < need))
        return set_error(CLF_ERR_WORKSPACE, "workspace of at least " + std::to_string(need) + " bytes required");
    hipStream_t s = (hipStream_t)stream;
    float* parts = g_cs ? (float*)ws : nullptr;
    int nparts = 0;
    if (batch > 0) {
        if (!g_cs) {
            launch_chain(n, false, cs, gy, gx, batch, s, ldg);
        } else {
            const unsigned grid = lds_grid<LDS_CS_BWD>(n, batch, cs_bwd_grid(n, batch));
            launch_lds<LDS_CS_BWD>(n, cs, y, gy, gx, parts, batch, grid, s, 1LL << n, ldg);
            nparts = (int)grid;
        }
        CLF_HIP_CHECK(hipGetLastError());
    }
    if (g_cs) {
        hipLaunchKernelGGL(parts_sum_kernel, dim3(1), dim3(256), 0, s, parts, nparts, 2 * n_planes(n), g_cs);
        CLF_HIP_CHECK(hipGetLastError());
    }
    return CLF_OK;
}

int rotor_cs_compile_bwd(int n, const float* biv, const float* g_cs, float* g_biv, void* stream) {
    if (int rc = check_rotor_n(n)) return rc;
    if (!biv || !g_cs || !g_biv) return set_error(CLF_ERR_ARG, "null pointer argument");
    hipStream_t s = (hipStream_t)stream;
#define CLF_CALL(N) hipLaunchKernelGGL((rotor_cs_compile_bwd_kernel<N>), dim3(1), dim3(64), 0, s, biv, g_cs, g_biv)
    CLF_COMPILE_DISPATCH(n, CLF_CALL)
#undef CLF_CALL
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
