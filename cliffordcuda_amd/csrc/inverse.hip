// Multivector inverse on gfx950 (the reference's extensions/ga/inverse.py:139-194
// and inverse_rep.py): a fused versor inverse and an inverse through a complex
// matrix representation, one workgroup per row.
//
// Versor inverse: for each row, y = rev(x) / <x rev(x)>_0 together with the
// checks that x rev(x) (computed by the product kernel) is a scalar and that
// the scalar is not zero.
//
// Matrix representation. Let the algebra's non-null generators be g_0 < ... <
// g_{n'-1}, m = floor(n'/2), d = 2^m. On m qubits, with Pauli strings written
// i^e X^a Z^b (a, b m-bit masks, X^a Z^b = prod over qubits of X^{a_k} Z^{b_k}):
//   gamma_{2k}   = Z_0 .. Z_{k-1} X_k        (a = 2^k, b = 2^k - 1,         e = 0)
//   gamma_{2k+1} = Z_0 .. Z_{k-1} Y_k        (a = 2^k, b = 2^k - 1 | 2^k,   e = 1; Y = i X Z)
//   gamma_{2m}   = Z_0 .. Z_{m-1}            (odd n' only)
// times i for a generator squaring to -1. They anticommute and square to the
// metric. A blade's matrix is the ordered product of its generators' gammas:
//   (i^e X^a Z^b)(i^f X^c Z^h) = i^{e+f} (-1)^{|b & c|} X^{a^c} Z^{b^h};
// blades with a null generator map to 0 (the representation of Cl(p,q,r) that
// kills the nilpotent ideal). (X^a Z^b)[r][c] = [r = c ^ a] (-1)^{|b & c|}, so
// with T_a[b] = sum over blades A labelled (a, b) of i^{e_A} x_A,
//   M(x)[c ^ a][c] = WHT_b(T_a)[c]               (Walsh-Hadamard over b)
// and the inverse map of N = M^{-1} is
//   U_a[b] = WHT_c(N[c ^ a][c])[b] / d,  y_A = Re(i^{-e_A} U_{a_A}[b_A]).
// Even n': one blade per label (M_d(C) carries the algebra). Odd n': two blades
// per label (A and A times the non-null pseudoscalar P); if P's phase is odd
// (P^2 = -1) their phases differ by +-i and the real part separates them; if
// it is even (P^2 = +1) the algebra is two copies of a matrix algebra and a
// second matrix M(x^) of the grade involution is inverted too:
//   y_A = Re(i^{-e_A} (U+ + (-1)^{|A|} U-)) / 2.
// The result is the inverse of the non-null part x0; for a degenerate metric
// the caller completes it with Newton steps y <- y (2 - x y), whose error
// 1 - x y is nilpotent there.
//
// Gauss-Jordan with partial pivoting in LDS: thread j owns column j of the
// d x d complex matrix (d <= 128), in-place elimination, the row swaps undone
// as column swaps at the end. A zero pivot marks the row singular.
#include "clf_common.h"

namespace clf {

constexpr int kInvMaxD = 128;

__host__ __device__ inline void inv_gamma(int t, int np, bool neg, unsigned& a, unsigned& b, int& e) {
    const int m = np / 2;
    if (t < 2 * m) {
        const int k = t >> 1;
        a = 1u << k;
        b = ((1u << k) - 1u) | ((t & 1) ? (1u << k) : 0u);
        e = t & 1;
    } else {
        a = 0u;
        b = (1u << m) - 1u;
        e = 0;
    }
    if (neg) e += 1;
}

// label (a, b) and phase i^e of blade A (A holds no null generator)
__host__ __device__ inline void inv_blade_label(unsigned A, int n, unsigned nonnull, unsigned neg, int np,
                                                unsigned& a, unsigned& b, int& e) {
    a = 0u;
    b = 0u;
    e = 0;
    int t = 0;
    for (int g = 0; g < n; ++g) {
        if (!((nonnull >> g) & 1u)) continue;
        if ((A >> g) & 1u) {
            unsigned ga, gb;
            int ge;
            inv_gamma(t, np, (neg >> g) & 1u, ga, gb, ge);
            e += ge + 2 * (popc_rt(b & ga) & 1);
            a ^= ga;
            b ^= gb;
        }
        ++t;
    }
    e &= 3;
}

__device__ __forceinline__ float2 cmul(float2 u, float2 v) {
    return make_float2(u.x * v.x - u.y * v.y, u.x * v.y + u.y * v.x);
}
__device__ __forceinline__ float2 cadd(float2 u, float2 v) { return make_float2(u.x + v.x, u.y + v.y); }
__device__ __forceinline__ float2 csub(float2 u, float2 v) { return make_float2(u.x - v.x, u.y - v.y); }
// i^e * v
__device__ __forceinline__ float2 iphase(int e, float2 v) {
    switch (e & 3) {
        case 0: return v;
        case 1: return make_float2(-v.y, v.x);
        case 2: return make_float2(-v.x, -v.y);
        default: return make_float2(v.y, -v.x);
    }
}

// In-place WHT over the second index of a D x D complex array (row a, entry b).
template <int D, int BT>
__device__ __forceinline__ void wht_rows(float2* __restrict__ T) {
    for (int h = 1; h < D; h <<= 1) {
        for (int q = threadIdx.x; q < D * D / 2; q += BT) {
            const int a = q / (D / 2), j = q % (D / 2);
            const int b0 = ((j & ~(h - 1)) << 1) | (j & (h - 1));
            float2* row = T + a * D;
            const float2 u = row[b0], v = row[b0 | h];
            row[b0] = cadd(u, v);
            row[b0 | h] = csub(u, v);
        }
        __syncthreads();
    }
}

// Thread c < D swaps entries (i, c) and (i ^ c, c) of its column: the
// relabelling between "row a = r ^ c" and "row r" of every column.
template <int D>
__device__ __forceinline__ void xor_columns(float2* __restrict__ T) {
    const int c = threadIdx.x;
    if (c < D)
        for (int i = 0; i < D; ++i) {
            const int j = i ^ c;
            if (i < j) {
                const float2 u = T[i * D + c];
                T[i * D + c] = T[j * D + c];
                T[j * D + c] = u;
            }
        }
    __syncthreads();
}

// In-place Gauss-Jordan inverse of the D x D complex matrix M (row-major).
// Returns true (in every thread) if a pivot was zero or not finite.
template <int D, int BT>
__device__ bool gauss_jordan(float2* __restrict__ M, int* __restrict__ piv, float* __restrict__ red_v,
                             int* __restrict__ red_i) {
    constexpr int NW = BT / 64;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    bool bad = false;
    for (int k = 0; k < D; ++k) {
        // pivot: the largest |M[i][k]|^2 over rows i >= k (thread t looks at row t)
        float v = -1.f;
        int idx = k;
        if (t < D && t >= k) {
            const float2 z = M[t * D + k];
            v = z.x * z.x + z.y * z.y;
            idx = t;
        }
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(v, off, 64);
            const int oi = __shfl_xor(idx, off, 64);
            if (ov > v || (ov == v && oi < idx)) {
                v = ov;
                idx = oi;
            }
        }
        if (lane == 0) {
            red_v[wave] = v;
            red_i[wave] = idx;
        }
        __syncthreads();
        float bv = red_v[0];
        int p = red_i[0];
        for (int w = 1; w < NW; ++w)
            if (red_v[w] > bv || (red_v[w] == bv && red_i[w] < p)) {
                bv = red_v[w];
                p = red_i[w];
            }
        if (!(bv > 0.f) || !isfinite(bv)) bad = true;
        if (t == 0) piv[k] = p;
        if (p != k && t < D) {
            const float2 u = M[k * D + t];
            M[k * D + t] = M[p * D + t];
            M[p * D + t] = u;
        }
        __syncthreads();
        const float2 pv = M[k * D + k];
        const float den = pv.x * pv.x + pv.y * pv.y;
        const float2 inv = den > 0.f ? make_float2(pv.x / den, -pv.y / den) : make_float2(0.f, 0.f);
        if (t < D && t != k) M[k * D + t] = cmul(M[k * D + t], inv);
        __syncthreads();
        if (t < D && t != k) {
            const float2 mk = M[k * D + t];
            for (int i = 0; i < D; ++i)
                if (i != k) M[i * D + t] = csub(M[i * D + t], cmul(M[i * D + k], mk));
        }
        __syncthreads();
        if (t == k) {
            for (int i = 0; i < D; ++i)
                if (i != k) {
                    const float2 f = M[i * D + k];
                    M[i * D + k] = make_float2(-(f.x * inv.x - f.y * inv.y), -(f.x * inv.y + f.y * inv.x));
                }
            M[k * D + k] = inv;
        }
        __syncthreads();
    }
    for (int k = D - 1; k >= 0; --k) {
        const int p = piv[k];
        if (p != k && t < D) {
            const float2 u = M[t * D + k];
            M[t * D + k] = M[t * D + p];
            M[t * D + p] = u;
        }
        __syncthreads();
    }
    return bad;
}

// One workgroup per row (grid stride). TWO: the second block of a two-copy
// signature. y holds the inverse of the non-null part; singular[row] = 1 if a
// pivot vanished.
template <int D, bool TWO>
__global__ __launch_bounds__(D < 64 ? 64 : D) void inverse_rep_kernel(int n, unsigned nonnull, unsigned neg, int np,
                                                                       unsigned last_bit,
                                                                       const float* __restrict__ X,
                                                                       float* __restrict__ Y,
                                                                       int* __restrict__ singular, long long batch) {
    constexpr int BT = D < 64 ? 64 : D;
    __shared__ float2 buf[TWO ? 2 : 1][D * D];
    __shared__ int piv[D];
    __shared__ float red_v[BT / 64];
    __shared__ int red_i[BT / 64];
    const unsigned nblades = 1u << n;
    for (long long row = blockIdx.x; row < batch; row += gridDim.x) {
        const float* x = X + (row << n);
        for (int e = threadIdx.x; e < D * D; e += BT) {
            buf[0][e] = make_float2(0.f, 0.f);
            if (TWO) buf[TWO ? 1 : 0][e] = make_float2(0.f, 0.f);
        }
        __syncthreads();
        // the two blades of a label differ by the non-null pseudoscalar, so
        // exactly one of them holds the last non-null generator: two passes
        // never write one label twice
        for (int pass = 0; pass < 2; ++pass) {
            for (unsigned A = threadIdx.x; A < nblades; A += BT) {
                if ((A & ~nonnull) != 0u) continue;
                if (((A & last_bit) != 0u) != (pass == 1)) continue;
                unsigned a, b;
                int e;
                inv_blade_label(A, n, nonnull, neg, np, a, b, e);
                const float xa = x[A];
                buf[0][a * D + b] = cadd(buf[0][a * D + b], iphase(e, make_float2(xa, 0.f)));
                if (TWO) {
                    const float xs = (popc_rt(A) & 1) ? -xa : xa;
                    buf[TWO ? 1 : 0][a * D + b] = cadd(buf[TWO ? 1 : 0][a * D + b], iphase(e, make_float2(xs, 0.f)));
                }
            }
            __syncthreads();
        }
        bool bad = false;
#pragma unroll
        for (int blk = 0; blk < (TWO ? 2 : 1); ++blk) {
            wht_rows<D, BT>(buf[blk]);
            xor_columns<D>(buf[blk]);
            bad |= gauss_jordan<D, BT>(buf[blk], piv, red_v, red_i);
            xor_columns<D>(buf[blk]);
            wht_rows<D, BT>(buf[blk]);
        }
        const float scale = 1.f / (float)D;
        float* y = Y + (row << n);
        for (unsigned A = threadIdx.x; A < nblades; A += BT) {
            float out = 0.f;
            if ((A & ~nonnull) == 0u) {
                unsigned a, b;
                int e;
                inv_blade_label(A, n, nonnull, neg, np, a, b, e);
                float2 u = buf[0][a * D + b];
                if (TWO) {
                    const float2 w = buf[TWO ? 1 : 0][a * D + b];
                    u = (popc_rt(A) & 1) ? csub(u, w) : cadd(u, w);
                    u = make_float2(0.5f * u.x, 0.5f * u.y);
                }
                out = iphase(4 - e, u).x * scale;
            }
            y[A] = out;
        }
        if (threadIdx.x == 0 && singular) singular[row] = bad ? 1 : 0;
        __syncthreads();
    }
}

// Versor inverse: xr = x rev(x) (the product kernel's output). Per row:
// s = xr_0, off = max_{k>0} |xr_k|; flags bit 0: off > rtol * max(|s|, off)
// (x rev(x) is not a scalar); bit 1: |s| < 1e-20 (not invertible).
// y = rev(x) / s. One wave per row, grid stride.
__global__ __launch_bounds__(256) void inverse_versor_kernel(int n, const float* __restrict__ X,
                                                             const float* __restrict__ XR, float* __restrict__ Y,
                                                             int* __restrict__ flags, float rtol, long long batch) {
    const int lane = threadIdx.x & 63;
    const long long waves = (long long)gridDim.x * (blockDim.x >> 6);
    const int D = 1 << n;
    for (long long row = (long long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); row < batch; row += waves) {
        const float* xr = XR + (row << n);
        const float s = xr[0];
        float off = 0.f;
        for (int k = 1 + lane; k < D; k += 64) off = fmaxf(off, fabsf(xr[k]));
        for (int o = 32; o > 0; o >>= 1) off = fmaxf(off, __shfl_xor(off, o, 64));
        const float scale = fmaxf(fmaxf(fabsf(s), off), 1e-30f);
        const float* x = X + (row << n);
        float* y = Y + (row << n);
        for (int k = lane; k < D; k += 64) {
            const int g = popc_rt((unsigned)k);
            const float sign = ((g * (g - 1) / 2) & 1) ? -1.f : 1.f;
            y[k] = sign * x[k] / s;
        }
        if (lane == 0) flags[row] = (off > rtol * scale ? 1 : 0) | (fabsf(s) < 1e-20f ? 2 : 0);
    }
}

// ---- host side --------------------------------------------------------------

struct InvPlan {
    unsigned nonnull, last_bit;
    int np, D;
    bool two;
};

static bool inverse_plan(int n, uint32_t neg, uint32_t nul, InvPlan& P) {
    const unsigned full = n >= 32 ? 0xffffffffu : ((1u << n) - 1u);
    P.nonnull = full & ~nul;
    P.np = popc_rt(P.nonnull);
    P.D = 1 << (P.np / 2);
    P.last_bit = 0u;
    for (int g = 0; g < n; ++g)
        if ((P.nonnull >> g) & 1u) P.last_bit = 1u << g;
    P.two = false;
    if (P.np & 1) {
        unsigned a, b;
        int e;
        inv_blade_label(P.nonnull, n, P.nonnull, neg, P.np, a, b, e);
        P.two = (e & 1) == 0;  // pseudoscalar phase +-1: P^2 = +1, two copies
    }
    // at most 14 non-null generators: the reference serves the representation
    // while its (2^n', d, d) complex blade tensor fits 4e9 bytes, i.e. n' <= 14
    if (P.np > 14 || P.D > kInvMaxD) return false;
    if (P.two && P.D > 64) return false;
    return true;
}

int inverse_rep_supported(int n, uint32_t neg, uint32_t nul) {
    if (n < 1 || n > kMaxN) return 0;
    InvPlan P;
    return inverse_plan(n, neg, nul, P) ? 1 : 0;
}

template <int D, bool TWO>
static void launch_inverse_rep(const InvPlan& P, int n, uint32_t neg, const float* x, float* y, int* singular,
                               int64_t batch, hipStream_t s) {
    constexpr int BT = D < 64 ? 64 : D;
    const unsigned grid = resident_grid((const void*)inverse_rep_kernel<D, TWO>, BT, 0, batch);
    hipLaunchKernelGGL((inverse_rep_kernel<D, TWO>), dim3(grid), dim3(BT), 0, s, n, P.nonnull, neg, P.np, P.last_bit,
                       x, y, singular, (long long)batch);
}

int inverse_rep(int n, uint32_t neg, uint32_t nul, const float* x, float* y, int* singular, int64_t batch,
                void* stream) {
    if (n < 1 || n > kMaxN) return set_error(CLF_ERR_ARG, "n must be in [1, " + std::to_string(kMaxN) + "]");
    const uint32_t full = (1u << n) - 1u;
    if ((neg & ~full) || (nul & ~full)) return set_error(CLF_ERR_ARG, "metric masks have bits above n");
    if (neg & nul) return set_error(CLF_ERR_ARG, "neg_mask and null_mask overlap");
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    InvPlan P;
    if (!inverse_plan(n, neg, nul, P))
        return set_error(CLF_ERR_UNSUPPORTED, "no matrix representation of at most 128 x 128 for this signature");
    if (batch == 0) return CLF_OK;
    if (!x || !y) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (x == y) return set_error(CLF_ERR_ARG, "output must not alias the input");
    hipStream_t s = (hipStream_t)stream;
#define CLF_INV(DD)                                                                      \
    case DD:                                                                             \
        if (P.two) launch_inverse_rep<(DD <= 64 ? DD : 64), true>(P, n, neg, x, y, singular, batch, s); \
        else launch_inverse_rep<DD, false>(P, n, neg, x, y, singular, batch, s);         \
        break;
    switch (P.D) {
        CLF_INV(1)
        CLF_INV(2)
        CLF_INV(4)
        CLF_INV(8)
        CLF_INV(16)
        CLF_INV(32)
        CLF_INV(64)
        CLF_INV(128)
        default: return set_error(CLF_ERR_UNSUPPORTED, "representation size out of range");
    }
#undef CLF_INV
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int inverse_versor(int n, const float* x, const float* xr, float* y, int* flags, float rtol, int64_t batch,
                   void* stream) {
    if (n < 1 || n > kMaxN) return set_error(CLF_ERR_ARG, "n must be in [1, " + std::to_string(kMaxN) + "]");
    if (batch < 0) return set_error(CLF_ERR_ARG, "batch must be >= 0");
    if (batch == 0) return CLF_OK;
    if (!x || !xr || !y || !flags) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (y == x || y == xr) return set_error(CLF_ERR_ARG, "output must not alias the inputs");
    hipStream_t s = (hipStream_t)stream;
    const unsigned grid = resident_grid((const void*)inverse_versor_kernel, 256, 0, (batch + 3) / 4);
    hipLaunchKernelGGL(inverse_versor_kernel, dim3(grid), dim3(256), 0, s, n, x, xr, y, flags, rtol,
                       (long long)batch);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
