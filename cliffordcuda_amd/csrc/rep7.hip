// Geometric product of n = 7 signatures (no null generator) on the 16 x 16
// real representation and the matrix cores.
//
// Seven anticommuting real Pauli products gamma_g = P(x_g, z_g) on 4 qubits
// represent every Cl(p, q) with p + q = 7 in M_16(R) (the Pauli algebra and the
// conversion are the ones of the n = 8 kernels in rep.hip). The 128 blade
// labels (x_I, z_I) span a subspace L; the generators are searched so that the
// x parts of L cover all 16 values, and a permutation of the basis,
// P(x, z) -> P(A x, A^-T z), puts V = {z : (0, z) in L} on the low bits of z.
// Lane x of a row then holds the labels (x, zhi(x) << d | v), v < 2^d, and
// W[x][c] = sum_z t[x][z] (-1)^{popc(z & c)} = s_x(c >> d) T[c & (2^d - 1)]
// with T a 2^d-point WHT of the lane's values and s_x(m) = (-1)^{popc(zhi(x) & m)}.
//
// Pair mode (q odd: the pseudoscalar E squares to +1). The generators are
// chosen with product label (0, 0), so phi(E) = +-1, phi is not faithful and
// every label carries one even blade I and one odd blade I E (d = 2). The row
// goes to Phi(a) = (phi(a), phi(a^)), a^ the grade involution: with
// u = s(I) a_I, w = s(IE) a_IE the two matrices take t = u + w and t^ = u - w.
// Phi(ab) = Phi(a) Phi(b) blockwise and Phi^* Phi = 32, so
//   c = Phi^*(Phi(a) Phi(b)) / 32,  ga = Phi^*(Phi(gc) Phi(b)^T) / 32,
//   gb = Phi^*(Phi(a)^T Phi(gc)) / 32,
// with Phi^*(C1, C2)_I = s(I) (Q1 + Q2), Phi^*(C1, C2)_IE = s(IE) (Q1 - Q2),
// Q = sum_c W_C[x][c] (-1)^{popc(z & c)} of each matrix.
// Single mode (q even: E squares to -1 and phi is faithful): one blade per
// label (d = 3), one matrix per row, c = phi^*(phi(a) phi(b)) / 16.
//
// Layout: one wave owns four rows at a time (row b on lanes 16b .. 16b + 15),
// stages them in its LDS slots, converts (lane = x), multiplies with the
// 4-block 16x16x1 MFMA chain of rep_common.h (block b = row b), and brings the
// products back through the stride-20 relayout. Waves walk the batch with a
// grid stride and prefetch the next rows into registers.
#include <algorithm>
#include <map>
#include <mutex>

#include "rep_common.h"

namespace clf {

constexpr int kRep7Dim = 128;          // floats per row
constexpr int kRep7GroupFloats = 512;  // four rows

struct Rep7Table {
    // [x * 8 + k]: blade | 0x80000000 if s(I) = -1 | 0x40000000 if s(I) (-1)^{popc(x & z)} = -1
    // (the transposed conversion). Pair mode: k = 2 * slot + (0: even blade, 1: odd blade);
    // single mode: k = slot.
    unsigned e[16 * 8];
    unsigned zhi[16];  // high z bits of lane x's labels
    unsigned odd_xor;  // multiple of 4 xor-ed into odd rows' blade offsets in LDS
};

// Four rows: lane l moves float4 chunks l and l + 64 of the group (row c >> 5);
// rows past the end re-read the last row and store to it again (their results
// are bit-identical to the last row's).
struct Pre7 {
    float4 v[2];
};

// ld: floats between rows (128 packed; 0 for one row broadcast over the batch)
template <bool NT>
__device__ __forceinline__ Pre7 fetch7(const float* __restrict__ src, long long row0, long long batch, int lane,
                                       long long ld = kRep7Dim) {
    Pre7 p;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c = lane + 64 * j;
        long long row = row0 + (c >> 5);
        row = row < batch ? row : batch - 1;
        const float4* q = reinterpret_cast<const float4*>(src + ((row & row_mask(ld)) << 7)) + (c & 31);
        p.v[j] = NT ? load_stream(q) : *q;
    }
    return p;
}

// row r at [r * 128, (r + 1) * 128), odd rows with chunk index xor oddc
__device__ __forceinline__ int slot7(int c, unsigned oddc) {
    const int r = c >> 5;
    return r * (kRep7Dim / 4) + (int)((unsigned)(c & 31) ^ ((r & 1) ? oddc : 0u));
}

__device__ __forceinline__ void stage7(float* __restrict__ dst, const Pre7& p, int lane, unsigned oddc) {
#pragma unroll
    for (int j = 0; j < 2; ++j) reinterpret_cast<float4*>(dst)[slot7(lane + 64 * j, oddc)] = p.v[j];
}

template <bool NT>
__device__ __forceinline__ void store7(float* __restrict__ dstg, const float* __restrict__ src, long long row0,
                                       long long batch, int lane, unsigned oddc) {
    float4 v[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) v[j] = reinterpret_cast<const float4*>(src)[slot7(lane + 64 * j, oddc)];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c = lane + 64 * j;
        long long row = row0 + (c >> 5);
        row = row < batch ? row : batch - 1;
        float4* q = reinterpret_cast<float4*>(dstg + row * kRep7Dim) + (c & 31);
        if (NT) store_stream(q, v[j]);
        else *q = v[j];
    }
}

__device__ __forceinline__ float sgn7(float v, unsigned e, int shift) {
    return __uint_as_float(__float_as_uint(v) ^ ((e << shift) & 0x80000000u));
}

// Pair mode: the lane's eight blades of the staged row; sign convention by
// SIGNSHIFT (0: s(I), 1: transposed); t = WHT4(u + w), th = WHT4(u - w).
template <int SIGNSHIFT>
__device__ __forceinline__ void gather7_pair(const float* __restrict__ row, const unsigned (&ent)[8], float (&t)[4],
                                             float (&th)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float u = sgn7(row[ent[2 * i] & 0x7fu], ent[2 * i], SIGNSHIFT);
        const float w = sgn7(row[ent[2 * i + 1] & 0x7fu], ent[2 * i + 1], SIGNSHIFT);
        t[i] = u + w;
        th[i] = u - w;
    }
    wht_inplace<4>(t);
    wht_inplace<4>(th);
}

// Single mode: t = WHT8 of the lane's eight blades.
template <int SIGNSHIFT>
__device__ __forceinline__ void gather7_single(const float* __restrict__ row, const unsigned (&ent)[8], float (&t)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = sgn7(row[ent[i] & 0x7fu], ent[i], SIGNSHIFT);
    wht_inplace<8>(t);
}

// Operand k of the chain at lane x is W[x ^ k][k] = s_{x ^ k}(k >> D) T_{x ^ k}[k & (L - 1)]
// with W[x][c] = s_x(c >> D) T[c & (L - 1)]. zhi is linear in x (the labels
// form a subspace), so s_{x ^ k}(m) = s_x(m) s_k(m); the lane-independent
// factor s_k(k >> D) appears in both operands of step k and cancels in the
// product, which leaves op[k] = s_x(k >> D) T[k & (L - 1)] read from lane x ^ k.
// The 16 shuffles come from L source registers, so they share their DPP
// stages, and the sign (sg[m] = s_x(m) as +-1.0) multiplies the last stage,
// which the compiler fuses into one DPP multiply. DPP controls: quad_perm
// xor 1 (0xB1), 2 (0x4E), 3 (0x1B); row_half_mirror = xor 7 (0x141);
// row_mirror = xor 15 (0x140); row_ror:8 = xor 8 (0x128).
template <unsigned J>
__device__ __forceinline__ float quad_xor(float v) {
    if constexpr (J == 1u) return dpp16<0xB1>(v);
    else if constexpr (J == 2u) return dpp16<0x4E>(v);
    else if constexpr (J == 3u) return dpp16<0x1B>(v);
    else return v;
}

template <unsigned J>
__device__ __forceinline__ void operand7_d2(const float (&t)[4], const float (&sg)[4], float (&op)[16]) {
    const float q = quad_xor<J>(t[J]);      // lane x ^ J
    const float r = quad_xor<J ^ 3u>(t[J]);  // lane x ^ J ^ 3
    op[J] = q;
    op[4 + J] = dpp16<0x141>(r) * sg[1];   // x ^ J ^ 3 ^ 7 = x ^ (4 + J)
    op[12 + J] = dpp16<0x140>(r) * sg[3];  // x ^ J ^ 3 ^ 15 = x ^ (12 + J)
    op[8 + J] = dpp16<0x128>(q) * sg[2];   // x ^ J ^ 8
}

template <unsigned J>
__device__ __forceinline__ void operand7_d3(const float (&t)[8], const float (&sg)[2], float (&op)[16]) {
    if constexpr (J < 4u) {
        const float q = quad_xor<J>(t[J]);     // lane x ^ J
        op[J] = q;
        op[8 + J] = dpp16<0x128>(q) * sg[1];  // x ^ J ^ 8
    } else {
        const float q = quad_xor<J ^ 7u>(t[J]);   // lane x ^ J ^ 7
        op[J] = dpp16<0x141>(q);                  // x ^ J
        op[8 + J] = dpp16<0x140>(q) * sg[1];      // x ^ J ^ 7 ^ 15 = x ^ (8 + J)
    }
}

template <int D>
__device__ __forceinline__ void operand7(const float (&t)[1 << D], const float (&sg)[16 >> D], float (&op)[16]) {
    if constexpr (D == 2) {
        operand7_d2<0>(t, sg, op);
        operand7_d2<1>(t, sg, op);
        operand7_d2<2>(t, sg, op);
        operand7_d2<3>(t, sg, op);
    } else {
        operand7_d3<0>(t, sg, op);
        operand7_d3<1>(t, sg, op);
        operand7_d3<2>(t, sg, op);
        operand7_d3<3>(t, sg, op);
        operand7_d3<4>(t, sg, op);
        operand7_d3<5>(t, sg, op);
        operand7_d3<6>(t, sg, op);
        operand7_d3<7>(t, sg, op);
    }
}

// Q[i] = sum_c W_C[x][c] (-1)^{popc((zhi << D | i) & c)} (multiplications by +-1 are exact)
template <int D>
__device__ __forceinline__ void lane_q7(const float (&wc)[16], const float (&sg)[16 >> D], float (&q)[1 << D]) {
    constexpr int L = 1 << D;
#pragma unroll
    for (int j = 0; j < L; ++j) {
        float y = wc[j];
#pragma unroll
        for (int m = 1; m < (16 >> D); ++m) y = __builtin_fmaf(wc[m * L + j], sg[m], y);
        q[j] = y;
    }
    wht_inplace<L>(q);
}

// the product's coefficients into the lane's blade slots of the staged row
__device__ __forceinline__ void scatter7_pair(float* __restrict__ row, const unsigned (&ent)[8], const float (&q)[4],
                                              const float (&qh)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        row[ent[2 * i] & 0x7fu] = sgn7((q[i] + qh[i]) * 0.03125f, ent[2 * i], 0);
        row[ent[2 * i + 1] & 0x7fu] = sgn7((q[i] - qh[i]) * 0.03125f, ent[2 * i + 1], 0);
    }
}

__device__ __forceinline__ void scatter7_single(float* __restrict__ row, const unsigned (&ent)[8], const float (&q)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) row[ent[i] & 0x7fu] = sgn7(q[i] * 0.0625f, ent[i], 0);
}

// per-lane constants: table entries (odd rows' offsets xor-ed) and the sign bits s_x(m)
template <int D>
__device__ __forceinline__ void lane_consts7(const Rep7Table& T, unsigned x, int rb, unsigned (&ent)[8],
                                             float (&sg)[16 >> D]) {
    const unsigned oddx = (rb & 1) ? T.odd_xor : 0u;
#pragma unroll
    for (int k = 0; k < 8; ++k) ent[k] = T.e[x * 8 + k] ^ oddx;
    const unsigned zhi = T.zhi[x];
#pragma unroll
    for (int m = 0; m < (16 >> D); ++m) sg[m] = __uint_as_float(0x3f800000u | ((unsigned)(__popc(zhi & (unsigned)m) & 1) << 31));
}

// product of the converted operands through the relayout; returns Q of the lane's row
template <int D>
__device__ __forceinline__ void product_q7(float* __restrict__ rel, const float (&ta)[1 << D], const float (&tb)[1 << D],
                                           const float (&sg)[16 >> D], int lane, int rb, unsigned x,
                                           float (&q)[1 << D]) {
    float oa[16], ob[16];
    operand7<D>(ta, sg, oa);
    operand7<D>(tb, sg, ob);
    const floatx16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const floatx16 acc = mfma_chain_pre<false, false>(zero, oa, ob, std::make_integer_sequence<unsigned, 16>{});
    relayout_store(rel, acc, lane);
    wave_lds_sync();
    float wc[16];
    relayout_load(rel, rb, x, wc);
    wave_lds_sync();
    lane_q7<D>(wc, sg, q);
}

// Memory pipeline (both n = 7 kernels): a wave's loads and stores share one
// completion counter and the compiler waits for all of them before staged rows
// are used, so each group's results stay in an LDS slot and are stored right
// after the next group's wait, with a full group's time to complete. The wave
// index is wave-uniform, so the row bookkeeping runs on the scalar unit.
// ONE: the grid covers the batch (one group per wave), so no next group is
// prefetched (the same in the backward)
template <bool PAIR, bool NT, bool ONE>
__global__ __launch_bounds__(256) void rep7_fwd_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                        float* __restrict__ C, long long batch, Rep7Table T) {
    constexpr int D = PAIR ? 2 : 3;
    // per wave: staged a | b, later the relayout (over both), then c in the b
    // slot until the next group's stores
    __shared__ float lds[4][kRelayoutFloats];
    static_assert(2 * kRep7GroupFloats <= kRelayoutFloats, "staging must fit the wave's LDS slots");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* sa = &lds[wave][0];
    float* sb = sa + kRep7GroupFloats;
    const unsigned oddc = T.odd_xor >> 2;
    unsigned ent[8];
    float sgn[16 >> D];
    lane_consts7<D>(T, x, rb, ent, sgn);

    const long long stride = (long long)gridDim.x * 16;
    const long long rfirst = ((long long)blockIdx.x * 4 + wave) * 4;
    long long row0 = rfirst;
    Pre7 pa = fetch7<NT>(A, row0, batch, lane);
    Pre7 pb = fetch7<NT>(B, row0, batch, lane);
    for (; row0 < batch; row0 += stride) {
        stage7(sa, pa, lane, oddc);
        if (row0 != rfirst) {  // uniform: the previous group's c leaves the b slot first
            wave_lds_sync();
            store7<NT>(C, sb, row0 - stride, batch, lane, oddc);
            wave_lds_sync();
        }
        stage7(sb, pb, lane, oddc);
        if (!ONE) {
            pa = fetch7<NT>(A, row0 + stride, batch, lane);
            pb = fetch7<NT>(B, row0 + stride, batch, lane);
        }
        wave_lds_sync();
        if constexpr (PAIR) {
            float ta[4], tah[4], tb[4], tbh[4];
            gather7_pair<0>(sa + rb * kRep7Dim, ent, ta, tah);
            gather7_pair<1>(sb + rb * kRep7Dim, ent, tb, tbh);
            wave_lds_sync();
            float q[4], qh[4];
            product_q7<2>(sa, ta, tb, sgn, lane, rb, x, q);
            product_q7<2>(sa, tah, tbh, sgn, lane, rb, x, qh);
            scatter7_pair(sb + rb * kRep7Dim, ent, q, qh);
        } else {
            float ta[8], tb[8];
            gather7_single<0>(sa + rb * kRep7Dim, ent, ta);
            gather7_single<1>(sb + rb * kRep7Dim, ent, tb);
            wave_lds_sync();
            float q[8];
            product_q7<3>(sa, ta, tb, sgn, lane, rb, x, q);
            scatter7_single(sb + rb * kRep7Dim, ent, q);
        }
        wave_lds_sync();
    }
    if (row0 != rfirst) store7<NT>(C, sb, row0 - stride, batch, lane, oddc);
}

// Backward: ga from (gc, b) with gc in the s(I) convention and b in s(I);
// gb from (a, gc) both in the transposed convention. The gradients run one
// after the other: gc and b are staged first (a is loaded meanwhile), then a
// over b, and each gradient's relayout and rows in blade order use a scratch
// slot, so few converted operands are live at once.
template <bool PAIR, bool NT, bool WA, bool WB, bool ONE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void rep7_bwd_kernel(
    const float* __restrict__ A, const float* __restrict__ B, const float* __restrict__ GC, long long ldg,
    float* __restrict__ GA, float* __restrict__ GB, long long batch, Rep7Table T) {
    constexpr int D = PAIR ? 2 : 3;
    constexpr int L = 1 << D;
    __shared__ float lds[4][2 * kRep7GroupFloats + kRelayoutFloats];  // per wave: gc | b, then a | scratch
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* sg = &lds[wave][0];
    float* sx = sg + kRep7GroupFloats;
    float* sr = sx + kRep7GroupFloats;
    const unsigned oddc = T.odd_xor >> 2;
    unsigned ent[8];
    float sgn[16 >> D];
    lane_consts7<D>(T, x, rb, ent, sgn);

    const long long stride = (long long)gridDim.x * 16;
    const long long rfirst = ((long long)blockIdx.x * 4 + wave) * 4;
    long long row0 = rfirst;
    Pre7 pb = fetch7<NT>(B, row0, batch, lane);
    Pre7 pg = fetch7<NT>(GC, row0, batch, lane, ldg);
    for (; row0 < batch; row0 += stride) {
        // the table values are re-derived where they are used rather than kept
        // in registers across the loop (register pressure sets the occupancy)
#pragma unroll
        for (int k = 0; k < 8; ++k) asm volatile("" : "+v"(ent[k]));
        stage7(sg, pg, lane, oddc);
        stage7(sx, pb, lane, oddc);
        const Pre7 pa = fetch7<NT>(A, row0, batch, lane);
        // the previous group's gb leaves the scratch slot (stored after this wait)
        if (WB && row0 != rfirst) store7<NT>(GB, sr, row0 - stride, batch, lane, oddc);  // uniform
        wave_lds_sync();
        if (WA) {
            float q[L];
            if constexpr (PAIR) {
                float tg[4], tgh[4], tb[4], tbh[4], qh[4];
                gather7_pair<0>(sg + rb * kRep7Dim, ent, tg, tgh);
                gather7_pair<0>(sx + rb * kRep7Dim, ent, tb, tbh);
                product_q7<2>(sr, tg, tb, sgn, lane, rb, x, q);
                product_q7<2>(sr, tgh, tbh, sgn, lane, rb, x, qh);
                scatter7_pair(sr + rb * kRep7Dim, ent, q, qh);
            } else {
                float tg[8], tb[8];
                gather7_single<0>(sg + rb * kRep7Dim, ent, tg);
                gather7_single<0>(sx + rb * kRep7Dim, ent, tb);
                product_q7<3>(sr, tg, tb, sgn, lane, rb, x, q);
                scatter7_single(sr + rb * kRep7Dim, ent, q);
            }
        }
        wave_lds_sync();
        stage7(sx, pa, lane, oddc);
        if (!ONE) {
            pg = fetch7<NT>(GC, row0 + stride, batch, lane, ldg);
            pb = fetch7<NT>(B, row0 + stride, batch, lane);
        }
        if (WA) store7<NT>(GA, sr, row0, batch, lane, oddc);  // after this group's second wait
        wave_lds_sync();
        if (WB) {
            float q[L];
            if constexpr (PAIR) {
                float tat[4], tath[4], tgt[4], tgth[4], qh[4];
                gather7_pair<1>(sx + rb * kRep7Dim, ent, tat, tath);
                gather7_pair<1>(sg + rb * kRep7Dim, ent, tgt, tgth);
                product_q7<2>(sr, tat, tgt, sgn, lane, rb, x, q);
                product_q7<2>(sr, tath, tgth, sgn, lane, rb, x, qh);
                scatter7_pair(sr + rb * kRep7Dim, ent, q, qh);
            } else {
                float tat[8], tgt[8];
                gather7_single<1>(sx + rb * kRep7Dim, ent, tat);
                gather7_single<1>(sg + rb * kRep7Dim, ent, tgt);
                product_q7<3>(sr, tat, tgt, sgn, lane, rb, x, q);
                scatter7_single(sr + rb * kRep7Dim, ent, q);
            }
        }
        wave_lds_sync();
    }
    if (WB && row0 != rfirst) store7<NT>(GB, sr, row0 - stride, batch, lane, oddc);
}

// ---- host side --------------------------------------------------------------

static int f2_rank(const unsigned* v, int count) {
    unsigned basis[32];
    int nb = 0;
    for (int i = 0; i < count; ++i) {
        unsigned w = v[i];
        for (int j = 0; j < nb; ++j) w = (w ^ basis[j]) < w ? (w ^ basis[j]) : w;
        if (w) basis[nb++] = w;
    }
    return nb;
}

// Seven anticommuting real Pauli products on 4 qubits with the metric's
// squares and x parts spanning F_2^4; with pair set, their product label must
// be (0, 0). Deterministic depth-first search in a fixed candidate order.
static bool rep7_generators(uint32_t neg, bool pair, unsigned* gx, unsigned* gz) {
    int g = 0;
    unsigned cand[7] = {0};
    while (g >= 0) {
        if (g == 7) {
            unsigned xs[7], tx = 0, tz = 0;
            for (int h = 0; h < 7; ++h) {
                xs[h] = gx[h];
                tx ^= gx[h];
                tz ^= gz[h];
            }
            if (f2_rank(xs, 7) == 4 && (!pair || (tx == 0u && tz == 0u))) return true;
            --g;  // reject: continue the search at the last generator
            continue;
        }
        bool found = false;
        for (unsigned c = cand[g] + 1; c < 256u; ++c) {
            const unsigned cx = c / 16u, cz = c % 16u;
            const int want = ((neg >> g) & 1u) ? 1 : 0;
            if ((host_popc(cx & cz) & 1) != want) continue;
            bool ok = true;
            for (int h = 0; h < g && ok; ++h) ok = ((host_popc(cz & gx[h]) + host_popc(gz[h] & cx)) & 1) == 1;
            if (!ok) continue;
            cand[g] = c;
            gx[g] = cx;
            gz[g] = cz;
            found = true;
            break;
        }
        if (found) {
            ++g;
            if (g < 7) cand[g] = 0;
        } else {
            cand[g] = 0;
            --g;
        }
    }
    return false;
}

static bool rep7_table_build(uint32_t neg, Rep7Table& T) {
    const bool pair = (host_popc(neg & 0x7fu) & 1) != 0;  // q odd: E^2 = +1
    unsigned gx[7], gz[7];
    if (!rep7_generators(neg, pair, gx, gz)) return false;
    // V = {z : (0, z) in span of the labels}, then a basis of F_2^4 starting with V
    unsigned span[128];
    int ns = 1;
    span[0] = 0;
    for (int h = 0; h < 7; ++h) {
        const unsigned v = gx[h] | (gz[h] << 4);
        bool in = false;
        for (int i = 0; i < ns && !in; ++i) in = span[i] == v;
        if (in) continue;
        for (int i = 0, e = ns; i < e; ++i) span[ns++] = span[i] ^ v;
    }
    unsigned cols[4];
    int d = 0;
    for (int i = 0; i < ns && d < 4; ++i) {  // dim V <= 3: the x parts alone have rank 4
        if ((span[i] & 15u) != 0u) continue;
        cols[d] = span[i] >> 4;
        if (f2_rank(cols, d + 1) == d + 1) ++d;
    }
    if (d != (pair ? 2 : 3)) return false;
    for (unsigned e = 1; e < 16u && d < 4; e <<= 1) {
        cols[d] = e;
        if (f2_rank(cols, d + 1) == d + 1) ++d;
    }
    // x' = A x with A = M^T (x'_i = popc(cols[i] & x)), z' = M^{-1} z
    unsigned minv[16];
    for (unsigned v = 0; v < 16u; ++v) {
        unsigned m = 0;
        for (int i = 0; i < 4; ++i)
            if ((v >> i) & 1u) m ^= cols[i];
        minv[m] = v;
    }
    for (int h = 0; h < 7; ++h) {
        unsigned xn = 0;
        for (int i = 0; i < 4; ++i) xn |= (unsigned)(host_popc(cols[i] & gx[h]) & 1) << i;
        gx[h] = xn;
        gz[h] = minv[gz[h]];
    }
    const int dd = pair ? 2 : 3;
    const unsigned low = (1u << dd) - 1u;
    bool seen[16 * 8] = {false};
    bool zset[16] = {false};
    for (unsigned I = 0; I < 128u; ++I) {
        unsigned x = 0, z = 0;
        bool negsign = false;
        for (int g = 0; g < 7; ++g)
            if ((I >> g) & 1u) {
                if (host_popc(z & gx[g]) & 1) negsign = !negsign;
                x ^= gx[g];
                z ^= gz[g];
            }
        const unsigned h = z >> dd;
        if (zset[x] && T.zhi[x] != h) return false;
        zset[x] = true;
        T.zhi[x] = h;
        const int k = pair ? (int)(2u * (z & low) + (host_popc(I) & 1)) : (int)(z & low);
        if (seen[x * 8 + k]) return false;
        seen[x * 8 + k] = true;
        const bool tsign = negsign != ((host_popc(x & z) & 1) != 0);
        T.e[x * 8 + k] = I | (negsign ? 0x80000000u : 0u) | (tsign ? 0x40000000u : 0u);
    }
    // the kernels' operand signs rely on zhi being linear in x
    for (unsigned x = 0; x < 16u; ++x)
        for (unsigned y = 0; y < 16u; ++y)
            if (T.zhi[x ^ y] != (T.zhi[x] ^ T.zhi[y])) return false;
    // odd-row offset xor with the fewest bank collisions over the gathers of a
    // half-wave (two rows)
    int best = 1 << 30;
    T.odd_xor = 0;
    for (unsigned hx = 0; hx < 128u; hx += 4) {
        int worst = 0;
        for (int k = 0; k < 8; ++k) {
            int cnt[32] = {0};
            for (unsigned x = 0; x < 16u; ++x) {
                const unsigned I = T.e[x * 8 + k] & 0x7fu;
                worst = std::max(worst, ++cnt[I % 32]);
                worst = std::max(worst, ++cnt[(128u + (I ^ hx)) % 32]);
            }
        }
        if (worst < best) {
            best = worst;
            T.odd_xor = hx;
        }
    }
    return true;
}

// Tables are built once per signature and kept (immutable after insertion).
static bool rep7_table(uint32_t neg, Rep7Table& T) {
    static TableCache<Rep7Table, 128> cache;
    return cache.get((int)(neg & 0x7fu), T, [&](Rep7Table& t) { return rep7_table_build(neg & 0x7fu, t); });
}

bool rep7_applicable(uint32_t neg) {
    Rep7Table T;
    return rep7_table(neg & 0x7fu, T);
}

// Workgroups: one per 16 rows (one group per wave), so that the kernels run
// their variant without the next-group prefetch; the cap only bounds the grid
// dimension, and the grid-stride loop covers larger batches. (With the
// prefetch, 2048 or 4096 workgroups for C2's 65536 rows measured within 2 %.)
static unsigned rep7_grid(int64_t batch) {
    const long long g = (batch + 15) / 16;
    const long long cap = 1LL << 24;
    return (unsigned)(g < 1 ? 1 : (g > cap ? cap : g));
}

int rep7_fwd(uint32_t neg, const float* a, const float* b, float* c, int64_t batch, void* stream) {
    Rep7Table T;
    if (!rep7_table(neg & 0x7fu, T)) return set_error(CLF_ERR_UNSUPPORTED, "no n = 7 matrix representation found");
    const bool pair = (host_popc(neg & 0x7fu) & 1) != 0;
    hipStream_t s = (hipStream_t)stream;
    const dim3 g(rep7_grid(batch));
    const bool one = (long long)g.x * 16 >= batch;
    const bool nt = stream_nt(3.0 * 512.0 * (double)batch);
#define CLF_REP7_FWD(P, NT)                                                                                        \
    do {                                                                                                          \
        if (one) hipLaunchKernelGGL((rep7_fwd_kernel<P, NT, true>), g, dim3(256), 0, s, a, b, c, (long long)batch, T); \
        else hipLaunchKernelGGL((rep7_fwd_kernel<P, NT, false>), g, dim3(256), 0, s, a, b, c, (long long)batch, T); \
    } while (0)
    if (pair) {
        if (nt) CLF_REP7_FWD(true, true);
        else CLF_REP7_FWD(true, false);
    } else {
        if (nt) CLF_REP7_FWD(false, true);
        else CLF_REP7_FWD(false, false);
    }
#undef CLF_REP7_FWD
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int rep7_bwd(uint32_t neg, const float* a, const float* b, const float* gc, int64_t ldg, float* ga, float* gb,
             int64_t batch, void* stream) {
    Rep7Table T;
    if (!rep7_table(neg & 0x7fu, T)) return set_error(CLF_ERR_UNSUPPORTED, "no n = 7 matrix representation found");
    const bool pair = (host_popc(neg & 0x7fu) & 1) != 0;
    hipStream_t s = (hipStream_t)stream;
    const dim3 g(rep7_grid(batch));
    const bool one = (long long)g.x * 16 >= batch;
    const bool nt = stream_nt((3 + (ga != nullptr) + (gb != nullptr)) * 512.0 * (double)batch);
    if (!ga && !gb) return CLF_OK;
#define CLF_REP7_BWD(P, NT, WA, WB)                                                                        \
    do {                                                                                                  \
        if (one)                                                                                          \
            hipLaunchKernelGGL((rep7_bwd_kernel<P, NT, WA, WB, true>), g, dim3(256), 0, s, a, b, gc,       \
                               (long long)ldg, ga, gb, (long long)batch, T);                              \
        else                                                                                              \
            hipLaunchKernelGGL((rep7_bwd_kernel<P, NT, WA, WB, false>), g, dim3(256), 0, s, a, b, gc,      \
                               (long long)ldg, ga, gb, (long long)batch, T);                              \
    } while (0)
#define CLF_REP7_BWD_W(P, NT)                 \
    do {                                      \
        if (ga && gb) CLF_REP7_BWD(P, NT, true, true);   \
        else if (ga) CLF_REP7_BWD(P, NT, true, false);   \
        else CLF_REP7_BWD(P, NT, false, true);           \
    } while (0)
    if (pair) {
        if (nt) CLF_REP7_BWD_W(true, true);
        else CLF_REP7_BWD_W(true, false);
    } else {
        if (nt) CLF_REP7_BWD_W(false, true);
        else CLF_REP7_BWD_W(false, false);
    }
#undef CLF_REP7_BWD_W
#undef CLF_REP7_BWD
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
