// Binary Clifford products on gfx950: forward and fused backward, all six ops,
// any Cl(p,q,r), bit-pattern layout.
//
// Math. Every product is c[k] = sum_i sigma_op(i, i^k) a[i] b[i^k] (reference
// kernels/ga/geom_prod.cu:17-18). The blocked kernels split a blade index into
// a high part and a 4-bit low part, i = ih*16 + il. Because the reorder sign is
// a bilinear form over GF(2) whose high-by-low cross term is all ones, the sign
// factorises as
//   sigma(i, j) = s_hi(ih, jh) * (-1)^{|ih| |jl|} * s_lo(il, jl)
// s_lo is a compile-time 16x16 pattern (op predicate, low-bit metric), so the
// 256 multiply-adds of one (ih, jh) block pair are straight-line FMAs with the
// sign folded into the instruction's negate modifier. s_hi and the |ih||jl|
// parity flip are applied once per block to the b operand (16 sign-bit XORs).
//
// Layout. One workgroup stages whole rows of a and b (and gc for backward) in
// LDS with float4 loads; each lane owns one 16-blade output block of one row
// and keeps its 16 accumulators in VGPRs. Lanes of a row read their b blocks
// as a permutation of the row, the a block as a broadcast. Inside each 64-byte
// block the four float4 slots are XOR-swizzled so the 16 lanes of a row hit
// distinct LDS banks.
#include <cstdlib>
#include <cstring>
#include <utility>

#include "clf_common.h"
#include "contr5_schedule.h"

namespace clf {

// low-block variants: the op's predicate restricted to the low 4 bits
enum LowVar : int { LV_GEOM = 0, LV_WEDGE = 1, LV_INNER = 2, LV_LC = 3, LV_RC = 4, LV_REGR = 5 };

__host__ __device__ constexpr int low_sign(int var, bool lowneg, unsigned il, unsigned jl) {
    const bool pred = var == LV_GEOM    ? true
                      : var == LV_WEDGE ? ((il & jl) == 0u)
                      : var == LV_INNER ? ((((il & ~jl) & 15u) == 0u) || (((jl & ~il) & 15u) == 0u))
                      : var == LV_LC    ? (((il & ~jl) & 15u) == 0u)
                      : var == LV_RC    ? (((jl & ~il) & 15u) == 0u)
                                        : (((il | jl) & 15u) == 15u);
    if (!pred) return 0;
    int p = creorder(il, jl);
    if (var == LV_REGR)
        p += cbitsum(il) + cbitsum(jl);
    else if (lowneg)
        p += cpopc(il & jl);
    return (p & 1) ? -1 : 1;
}

__device__ __forceinline__ float flip(float x, unsigned m) { return __uint_as_float(__float_as_uint(x) ^ m); }

// XOR swizzle of the float4 slot inside a 64-byte block
__device__ __forceinline__ unsigned swz(unsigned blk) { return ((blk >> 1) ^ (blk >> 3)) & 3u; }

__device__ __forceinline__ void load_blk(const float4* __restrict__ base, unsigned blk, float (&v)[16]) {
    const unsigned s = swz(blk);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 t = base[(blk << 2) + ((unsigned)q ^ s)];
        v[4 * q + 0] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
}

// The balanced kernels' staged groups sit in static LDS arrays aligned to 64
// bytes, so a block's four slots (blk << 2) + (q ^ s) are one slot address
// xor 16 q: one address per block instead of one per slot. rs is the staged
// row's extra slot skew (rows that share a lane set read the same blocks
// at the same step, so their slots differ).
typedef float v4f_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4f_t lds_v4f;
__device__ __forceinline__ unsigned lds_addr4(const float4* p) { return (unsigned)(uintptr_t)(const lds_v4f*)p; }
__device__ __forceinline__ float4 lds_ld4(unsigned a) {
    const v4f_t v = *(const lds_v4f*)(uintptr_t)a;
    return make_float4(v.x, v.y, v.z, v.w);
}

// load_blk / load_blk_rev on a 64-byte aligned staged row (REV: v[y] = block[15 - y])
template <bool REV = false>
__device__ __forceinline__ void load_blk_x(const float4* __restrict__ base, unsigned blk, float (&v)[16],
                                           unsigned rs) {
    const unsigned a0 = lds_addr4(base + ((blk << 2) | (swz(blk) ^ rs)));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 t = lds_ld4(a0 ^ ((unsigned)q << 4));
        v[REV ? 15 - (4 * q + 0) : 4 * q + 0] = t.x;
        v[REV ? 15 - (4 * q + 1) : 4 * q + 1] = t.y;
        v[REV ? 15 - (4 * q + 2) : 4 * q + 2] = t.z;
        v[REV ? 15 - (4 * q + 3) : 4 * q + 3] = t.w;
    }
}

// a block stored by store_blk (no swizzle): the inner product's partial slot
__device__ __forceinline__ void load_blk_plain(const float4* __restrict__ base, unsigned blk, float (&v)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 t = base[(blk << 2) + q];
        v[4 * q + 0] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
}

// reversed element order: v[y] = block[15 - y]
__device__ __forceinline__ void load_blk_rev(const float4* __restrict__ base, unsigned blk, float (&v)[16]) {
    const unsigned s = swz(blk);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 t = base[(blk << 2) + ((unsigned)q ^ s)];
        v[15 - (4 * q + 0)] = t.x;
        v[15 - (4 * q + 1)] = t.y;
        v[15 - (4 * q + 2)] = t.z;
        v[15 - (4 * q + 3)] = t.w;
    }
}

// Blocked kernels (one lane per output block, rows side by side in a wave):
// the float4 slot q of block blk sits at (blk << 2) | (q ^ bslot(blk, t)), with
// t the staged row's skew. ds_read_b128 serves a 32-lane half in two 16-lane
// sets (lane bits 2-4 of even and of odd parity), one cycle per distinct
// address on the busiest 16-byte bank group, so a set's lanes, which read one
// block per row (the broadcast operand) and blocks ih ^ kh (the lane's
// partner), must not put two blocks of one row, or the same block of two rows,
// on one group: (blk >> 2) & 3 spreads the partner blocks of a set, and the row
// skews (host: blocked_row_skew) separate the rows of a set.
__device__ __forceinline__ unsigned bslot(unsigned blk, unsigned t) { return ((blk >> 2) ^ t) & 3u; }

template <bool REV = false>
__device__ __forceinline__ void load_blk_s(const float4* __restrict__ base, unsigned blk, unsigned s,
                                           float (&v)[16]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 t = base[(blk << 2) + ((unsigned)q ^ s)];
        v[REV ? 15 - (4 * q + 0) : 4 * q + 0] = t.x;
        v[REV ? 15 - (4 * q + 1) : 4 * q + 1] = t.y;
        v[REV ? 15 - (4 * q + 2) : 4 * q + 2] = t.z;
        v[REV ? 15 - (4 * q + 3) : 4 * q + 3] = t.w;
    }
}

// The three low-block bodies below are expanded at compile time over all 256
// (il, jl) pairs with a constexpr sign, so each term is one FMA (negate
// modifier for -1, nothing for 0).

// acc[t] += s_lo(il, il^t) a[il] b[il^t]
template <int VAR, bool LOWNEG, int IL, int T>
__device__ __forceinline__ void fwd_term(float (&acc)[16], const float (&a)[16], const float (&b)[16]) {
    constexpr int s = low_sign(VAR, LOWNEG, (unsigned)IL, (unsigned)(IL ^ T));
    if constexpr (s > 0) acc[T] = __builtin_fmaf(a[IL], b[IL ^ T], acc[T]);
    else if constexpr (s < 0) acc[T] = __builtin_fmaf(-a[IL], b[IL ^ T], acc[T]);
}

// acc[il] += s_lo(il, jl) b[jl] g[il^jl]          (gradient w.r.t. the left operand)
template <int VAR, bool LOWNEG, int JL, int IL>
__device__ __forceinline__ void ga_term(float (&acc)[16], const float (&b)[16], const float (&g)[16]) {
    constexpr int s = low_sign(VAR, LOWNEG, (unsigned)IL, (unsigned)JL);
    if constexpr (s > 0) acc[IL] = __builtin_fmaf(b[JL], g[IL ^ JL], acc[IL]);
    else if constexpr (s < 0) acc[IL] = __builtin_fmaf(-b[JL], g[IL ^ JL], acc[IL]);
}

// acc[jl] += s_lo(il, jl) a[il] g[il^jl]          (gradient w.r.t. the right operand)
template <int VAR, bool LOWNEG, int IL, int JL>
__device__ __forceinline__ void gb_term(float (&acc)[16], const float (&a)[16], const float (&g)[16]) {
    constexpr int s = low_sign(VAR, LOWNEG, (unsigned)IL, (unsigned)JL);
    if constexpr (s > 0) acc[JL] = __builtin_fmaf(a[IL], g[IL ^ JL], acc[JL]);
    else if constexpr (s < 0) acc[JL] = __builtin_fmaf(-a[IL], g[IL ^ JL], acc[JL]);
}

template <int VAR, bool LOWNEG, int... Is>
__device__ __forceinline__ void lowblock_fwd_seq(float (&acc)[16], const float (&a)[16], const float (&b)[16],
                                                 std::integer_sequence<int, Is...>) {
    (fwd_term<VAR, LOWNEG, Is / 16, Is % 16>(acc, a, b), ...);
}
template <int VAR, bool LOWNEG, int... Is>
__device__ __forceinline__ void lowblock_ga_seq(float (&acc)[16], const float (&b)[16], const float (&g)[16],
                                                std::integer_sequence<int, Is...>) {
    (ga_term<VAR, LOWNEG, Is / 16, Is % 16>(acc, b, g), ...);
}
template <int VAR, bool LOWNEG, int... Is>
__device__ __forceinline__ void lowblock_gb_seq(float (&acc)[16], const float (&a)[16], const float (&g)[16],
                                                std::integer_sequence<int, Is...>) {
    (gb_term<VAR, LOWNEG, Is / 16, Is % 16>(acc, a, g), ...);
}

template <int VAR, bool LOWNEG>
__device__ __forceinline__ void lowblock_fwd(float (&acc)[16], const float (&a)[16], const float (&b)[16]) {
    lowblock_fwd_seq<VAR, LOWNEG>(acc, a, b, std::make_integer_sequence<int, 256>{});
}
template <int VAR, bool LOWNEG>
__device__ __forceinline__ void lowblock_ga(float (&acc)[16], const float (&b)[16], const float (&g)[16]) {
    lowblock_ga_seq<VAR, LOWNEG>(acc, b, g, std::make_integer_sequence<int, 256>{});
}
template <int VAR, bool LOWNEG>
__device__ __forceinline__ void lowblock_gb(float (&acc)[16], const float (&a)[16], const float (&g)[16]) {
    lowblock_gb_seq<VAR, LOWNEG>(acc, a, g, std::make_integer_sequence<int, 256>{});
}

// The inner product's low pattern split by term class: il = jl (both lc and
// rc), il strictly inside jl (lc only), jl strictly inside il (rc only). The
// operand of an lc-only term comes from xl, of an rc-only term from xr, of a
// shared term from x (xl / xr are x or zero, by the pair's high relation).
template <bool LOWNEG, int IL, int JL>
__device__ __forceinline__ const float (&split_operand(const float (&x)[16], const float (&xl)[16],
                                                        const float (&xr)[16]))[16] {
    if constexpr (IL == JL) return x;
    else if constexpr ((IL & ~JL & 15) == 0) return xl;
    else return xr;
}

template <bool LOWNEG, int JL, int IL>
__device__ __forceinline__ void ga_split_term(float (&acc)[16], const float (&b)[16], const float (&bl)[16],
                                              const float (&br)[16], const float (&g)[16]) {
    constexpr int s = low_sign(LV_INNER, LOWNEG, (unsigned)IL, (unsigned)JL);
    const float (&v)[16] = split_operand<LOWNEG, IL, JL>(b, bl, br);
    if constexpr (s > 0) acc[IL] = __builtin_fmaf(v[JL], g[IL ^ JL], acc[IL]);
    else if constexpr (s < 0) acc[IL] = __builtin_fmaf(-v[JL], g[IL ^ JL], acc[IL]);
}

template <bool LOWNEG, int IL, int JL>
__device__ __forceinline__ void gb_split_term(float (&acc)[16], const float (&a)[16], const float (&al)[16],
                                              const float (&ar)[16], const float (&g)[16]) {
    constexpr int s = low_sign(LV_INNER, LOWNEG, (unsigned)IL, (unsigned)JL);
    const float (&v)[16] = split_operand<LOWNEG, IL, JL>(a, al, ar);
    if constexpr (s > 0) acc[JL] = __builtin_fmaf(v[IL], g[IL ^ JL], acc[JL]);
    else if constexpr (s < 0) acc[JL] = __builtin_fmaf(-v[IL], g[IL ^ JL], acc[JL]);
}

template <bool LOWNEG, int... Is>
__device__ __forceinline__ void lowblock_ga_split_seq(float (&acc)[16], const float (&b)[16], const float (&bl)[16],
                                                      const float (&br)[16], const float (&g)[16],
                                                      std::integer_sequence<int, Is...>) {
    (ga_split_term<LOWNEG, Is / 16, Is % 16>(acc, b, bl, br, g), ...);
}

template <bool LOWNEG, int... Is>
__device__ __forceinline__ void lowblock_gb_split_seq(float (&acc)[16], const float (&a)[16], const float (&al)[16],
                                                      const float (&ar)[16], const float (&g)[16],
                                                      std::integer_sequence<int, Is...>) {
    (gb_split_term<LOWNEG, Is / 16, Is % 16>(acc, a, al, ar, g), ...);
}

// lc: the pair's blocks satisfy ih inside jh; rc: jh inside ih (both: ih = jh)
template <bool LOWNEG>
__device__ __forceinline__ void lowblock_ga_split(float (&acc)[16], const float (&b)[16], bool lc, bool rc,
                                                  const float (&g)[16]) {
    float bl[16], br[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        bl[e] = lc ? b[e] : 0.f;
        br[e] = rc ? b[e] : 0.f;
    }
    lowblock_ga_split_seq<LOWNEG>(acc, b, bl, br, g, std::make_integer_sequence<int, 256>{});
}

template <bool LOWNEG>
__device__ __forceinline__ void lowblock_gb_split(float (&acc)[16], const float (&a)[16], bool lc, bool rc,
                                                  const float (&g)[16]) {
    float al[16], ar[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        al[e] = lc ? a[e] : 0.f;
        ar[e] = rc ? a[e] : 0.f;
    }
    lowblock_gb_split_seq<LOWNEG>(acc, a, al, ar, g, std::make_integer_sequence<int, 256>{});
}

struct HiSign {
    bool valid;
    unsigned mask;  // 0 or 0x80000000
};

// s_hi(ih, jh): the high-part factor of sigma_op, including the op's block
// predicate, the high-bit metric and (regressive) the global and per-operand
// signs. Parameters: negh/nulh = metric masks shifted down by 4 bits,
// fullh = all-ones over the high bits, nm1 = (n-1) & 1, mu = parity of |NEG|.
template <int OP>
__device__ __forceinline__ HiSign hi_sign(unsigned ih, unsigned jh, unsigned negh, unsigned nulh,
                                          unsigned fullh, int nm1, int mu) {
    int par = reorder_parity(ih, jh);
    bool ok = true;
    if (OP == OP_GEOM) {
        ok = (ih & jh & nulh) == 0u;
        par += __popc(ih & jh & negh);
    } else if (OP == OP_WEDGE) {
        ok = (ih & jh) == 0u;
    } else if (OP == OP_INNER) {
        ok = (((ih & ~jh) == 0u) || ((jh & ~ih) == 0u)) && ((ih & jh & nulh) == 0u);
        par += __popc(ih & jh & negh);
    } else if (OP == OP_LC) {
        ok = ((ih & ~jh) == 0u) && ((ih & jh & nulh) == 0u);
        par += __popc(ih & jh & negh);
    } else if (OP == OP_RC) {
        ok = ((jh & ~ih) == 0u) && ((ih & jh & nulh) == 0u);
        par += __popc(ih & jh & negh);
    } else {  // regressive
        ok = (ih | jh) == fullh;
        par += bitsum_parity(ih) + bitsum_parity(jh) + nm1 * __popc(jh) + mu;
    }
    return HiSign{ok, (unsigned)(par & 1) << 31};
}

// parity that multiplies |jl| in the cross term, for left-operand high block x
template <int OP>
__device__ __forceinline__ unsigned cross_pi(unsigned x, int nm1) {
    return (unsigned)((__popc(x) + (OP == OP_REGR ? nm1 : 0)) & 1);
}

// b~[jl] = b[jl] * sign * (-1)^{|jl| pi}
__device__ __forceinline__ void apply_flips(float (&v)[16], unsigned m_even, unsigned m_odd) {
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = flip(v[e], (cpopc((unsigned)e) & 1) ? m_odd : m_even);
}

template <int OP, bool LOWNEG>
__device__ __forceinline__ void fwd_block_dispatch(float (&acc)[16], const float (&av)[16], const float (&bv)[16],
                                                   unsigned ih, unsigned jh) {
    if (OP == OP_GEOM) {
        lowblock_fwd<LV_GEOM, LOWNEG>(acc, av, bv);
    } else if (OP == OP_WEDGE) {
        lowblock_fwd<LV_WEDGE, false>(acc, av, bv);
    } else if (OP == OP_LC) {
        lowblock_fwd<LV_LC, LOWNEG>(acc, av, bv);
    } else if (OP == OP_RC) {
        lowblock_fwd<LV_RC, LOWNEG>(acc, av, bv);
    } else if (OP == OP_REGR) {
        lowblock_fwd<LV_REGR, false>(acc, av, bv);
    } else {  // inner: the block relation picks the low predicate
        const bool l = (ih & ~jh) == 0u, r = (jh & ~ih) == 0u;
        if (l && r) lowblock_fwd<LV_INNER, LOWNEG>(acc, av, bv);
        else if (l) lowblock_fwd<LV_LC, LOWNEG>(acc, av, bv);
        else lowblock_fwd<LV_RC, LOWNEG>(acc, av, bv);
    }
}

template <int OP, bool LOWNEG>
__device__ __forceinline__ void ga_block_dispatch(float (&acc)[16], const float (&bv)[16], const float (&g)[16],
                                                  unsigned ih, unsigned jh) {
    if (OP == OP_GEOM) {
        lowblock_ga<LV_GEOM, LOWNEG>(acc, bv, g);
    } else if (OP == OP_WEDGE) {
        lowblock_ga<LV_WEDGE, false>(acc, bv, g);
    } else if (OP == OP_LC) {
        lowblock_ga<LV_LC, LOWNEG>(acc, bv, g);
    } else if (OP == OP_RC) {
        lowblock_ga<LV_RC, LOWNEG>(acc, bv, g);
    } else if (OP == OP_REGR) {
        lowblock_ga<LV_REGR, false>(acc, bv, g);
    } else {
        const bool l = (ih & ~jh) == 0u, r = (jh & ~ih) == 0u;
        if (l && r) lowblock_ga<LV_INNER, LOWNEG>(acc, bv, g);
        else if (l) lowblock_ga<LV_LC, LOWNEG>(acc, bv, g);
        else lowblock_ga<LV_RC, LOWNEG>(acc, bv, g);
    }
}

template <int OP, bool LOWNEG>
__device__ __forceinline__ void gb_block_dispatch(float (&acc)[16], const float (&av)[16], const float (&g)[16],
                                                  unsigned ih, unsigned jh) {
    if (OP == OP_GEOM) {
        lowblock_gb<LV_GEOM, LOWNEG>(acc, av, g);
    } else if (OP == OP_WEDGE) {
        lowblock_gb<LV_WEDGE, false>(acc, av, g);
    } else if (OP == OP_LC) {
        lowblock_gb<LV_LC, LOWNEG>(acc, av, g);
    } else if (OP == OP_RC) {
        lowblock_gb<LV_RC, LOWNEG>(acc, av, g);
    } else if (OP == OP_REGR) {
        lowblock_gb<LV_REGR, false>(acc, av, g);
    } else {
        const bool l = (ih & ~jh) == 0u, r = (jh & ~ih) == 0u;
        if (l && r) lowblock_gb<LV_INNER, LOWNEG>(acc, av, g);
        else if (l) lowblock_gb<LV_LC, LOWNEG>(acc, av, g);
        else lowblock_gb<LV_RC, LOWNEG>(acc, av, g);
    }
}

struct BlkParams {
    long long batch;
    long long ldg4;  // float4 between the rows of the upstream gradient: 1 << (n - 2), or 0 (one row for all)
    int n;          // algebra dimension, 4 <= n <= kMaxN (20)
    unsigned negh;  // metric masks >> 4
    unsigned nulh;
    int nm1;        // (n - 1) & 1
    int mu;         // parity of popcount(neg) (regressive global sign)
    int lpr_log;    // log2(lanes per row)
    int rows_per_wg;
    int kpl;        // output blocks per lane
    int split_log;  // small-batch kernels: log2 of the partner splits S per output block
    int wpr_log;    // small-batch kernels: log2 of the workgroups per row
    unsigned rskew; // blocked kernels: 2-bit slot skew of staged row r at bits 2 (r & 15)
    unsigned negl;  // metric mask, bits 0-3 (the regressive product's dual signs)
};

// Stage NOPS (2 or 3) row-major operands s0, s1[, s2] for the workgroup's rows
// into LDS (swizzled). Each thread issues all its loads (up to four float4 per
// operand per pass, addresses clamped to the last valid chunk) before any LDS
// write, so a pass costs one memory latency instead of one per chunk.
template <int NOPS, bool BSLOT = false>
__device__ __forceinline__ void stage_rows(float4* __restrict__ lds, const float4* __restrict__ s0,
                                           const float4* __restrict__ s1, const float4* __restrict__ s2,
                                           long long row0, int nrows, int n, long long m2 = -1, unsigned rskew = 0u) {
    // BSLOT: the blocked kernels' slots (bslot with the row skews in rskew), else swz
    // m2 masks s2's float4 index: -1 (packed like s0 and s1) or 2^(n-2) - 1
    // (one row for all rows: the row offset drops out)
    const int d4_log = n - 2;
    const int D4 = 1 << d4_log;
    const int total = nrows << d4_log;
    const long long g0 = row0 << d4_log;
    const int nt = (int)blockDim.x;
    for (int base = (int)threadIdx.x; base < total; base += 4 * nt) {
        const int i0 = base, i1 = base + nt, i2 = base + 2 * nt, i3 = base + 3 * nt;
        const int c1 = i1 < total ? i1 : total - 1, c2 = i2 < total ? i2 : total - 1, c3 = i3 < total ? i3 : total - 1;
        const float4 a0 = s0[g0 + i0], a1 = s0[g0 + c1], a2 = s0[g0 + c2], a3 = s0[g0 + c3];
        const float4 b0 = s1[g0 + i0], b1 = s1[g0 + c1], b2 = s1[g0 + c2], b3 = s1[g0 + c3];
        float4 e0, e1, e2, e3;
        if constexpr (NOPS == 3) {
            e0 = s2[(g0 + i0) & m2];
            e1 = s2[(g0 + c1) & m2];
            e2 = s2[(g0 + c2) & m2];
            e3 = s2[(g0 + c3) & m2];
        }
        auto put = [&](int idx, const float4& x, const float4& y, const float4& z) {
            const int r = idx >> d4_log;
            const unsigned f = (unsigned)(idx & (D4 - 1));
            const unsigned blk = f >> 2, q = f & 3u;
            const unsigned sx = BSLOT ? bslot(blk, rskew >> (2 * (r & 15))) : swz(blk);
            const int dst = r * NOPS * D4 + (int)((blk << 2) + (q ^ sx));
            lds[dst] = x;
            lds[dst + D4] = y;
            if constexpr (NOPS == 3) lds[dst + 2 * D4] = z;
        };
        put(i0, a0, b0, e0);
        if (i1 < total) put(i1, a1, b1, e1);
        if (i2 < total) put(i2, a2, b2, e2);
        if (i3 < total) put(i3, a3, b3, e3);
    }
}

template <int OP, bool LOWNEG>
__global__ __launch_bounds__(256) void prod_fwd_blk(const float* __restrict__ A, const float* __restrict__ B,
                                                     float* __restrict__ C, BlkParams P) {
    extern __shared__ float4 lds[];
    const int n = P.n;
    const int D4 = 1 << (n - 2);
    const unsigned NB = 1u << (n - 4);
    const long long row0 = (long long)blockIdx.x * P.rows_per_wg;
    const int nrows = (int)((P.batch - row0) < P.rows_per_wg ? (P.batch - row0) : P.rows_per_wg);
    stage_rows<2, true>(lds, reinterpret_cast<const float4*>(A), reinterpret_cast<const float4*>(B), nullptr, row0,
                        nrows, n, -1, P.rskew);
    __syncthreads();
    const int r = threadIdx.x >> P.lpr_log;
    if (r >= nrows) return;
    const unsigned t = (P.rskew >> (2 * (r & 15))) & 3u;
    const unsigned lane_blk = threadIdx.x & ((1u << P.lpr_log) - 1u);
    const float4* la = lds + r * 2 * D4;
    const float4* lb = la + D4;
    float4* out = reinterpret_cast<float4*>(C) + ((row0 + r) << (n - 2));
    const unsigned fullh = NB - 1u;

    for (int kk = 0; kk < P.kpl; ++kk) {
        const unsigned kh = lane_blk + ((unsigned)kk << P.lpr_log);
        float acc[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.f;
        for (unsigned ih = 0; ih < NB; ++ih) {
            const unsigned jh = ih ^ kh;
            const HiSign hs = hi_sign<OP>(ih, jh, P.negh, P.nulh, fullh, P.nm1, P.mu);
            if (!hs.valid) continue;
            float av[16], bv[16];
            load_blk_s(la, ih, bslot(ih, t), av);
            load_blk_s(lb, jh, bslot(jh, t), bv);
            apply_flips(bv, hs.mask, hs.mask ^ (cross_pi<OP>(ih, P.nm1) << 31));
            fwd_block_dispatch<OP, LOWNEG>(acc, av, bv, ih, jh);
        }
        if (OP == OP_REGR) {
            const unsigned ob = fullh ^ kh;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                out[(ob << 2) + (3 - q)] = make_float4(acc[4 * q + 3], acc[4 * q + 2], acc[4 * q + 1], acc[4 * q]);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                out[(kh << 2) + q] = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
        }
    }
}

// The inner product's backward for one output block h (one lane per output):
// its partner blocks are walked by relation class, so the lanes of a wave run
// the same low pattern at every step: the strict supersets m of h (ga pairs
// (h, m) in the lc relation, gb pairs (m, h) in the rc relation), the strict
// subsets (the other way round), then m = h (both patterns). A lane whose
// class has fewer partners than another lane's idles for the difference; the
// wave stops a class when no lane has partners left.
template <int CLASS, bool LOWNEG>
__device__ __forceinline__ void inner_pair(const float4* __restrict__ la, const float4* __restrict__ lb,
                                           const float4* __restrict__ lg, unsigned h, unsigned m, unsigned fullh,
                                           bool do_a, bool do_b, float (&ga)[16], float (&gb)[16],
                                           const BlkParams& P, unsigned t) {
    // CLASS 0: m strict superset of h; 1: strict subset; 2: m = h
    constexpr int VA = CLASS == 0 ? LV_LC : CLASS == 1 ? LV_RC : LV_INNER;
    constexpr int VB = CLASS == 0 ? LV_RC : CLASS == 1 ? LV_LC : LV_INNER;
    const HiSign sa = hi_sign<OP_INNER>(h, m, P.negh, P.nulh, fullh, P.nm1, P.mu);
    const HiSign sb = hi_sign<OP_INNER>(m, h, P.negh, P.nulh, fullh, P.nm1, P.mu);
    do_a = do_a && sa.valid;
    do_b = do_b && sb.valid;
    if (!do_a && !do_b) return;
    float g[16];
    load_blk_s(lg, h ^ m, bslot(h ^ m, t), g);
    if (do_a) {
        float bv[16];
        load_blk_s(lb, m, bslot(m, t), bv);
        apply_flips(bv, sa.mask, sa.mask ^ (cross_pi<OP_INNER>(h, P.nm1) << 31));
        lowblock_ga<VA, LOWNEG>(ga, bv, g);
    }
    if (do_b) {
        const unsigned pm = cross_pi<OP_INNER>(m, P.nm1) << 31;
        float av[16], gt[16];
        load_blk_s(la, m, bslot(m, t), av);
        apply_flips(av, sb.mask, sb.mask ^ pm);
#pragma unroll
        for (int e = 0; e < 16; ++e) gt[e] = (cpopc((unsigned)e) & 1) ? flip(g[e], pm) : g[e];
        lowblock_gb<VB, LOWNEG>(gb, av, gt);
    }
}

template <bool LOWNEG>
__device__ __forceinline__ void inner_bwd_blocks(const float4* __restrict__ la, const float4* __restrict__ lb,
                                                 const float4* __restrict__ lg, unsigned h, unsigned fullh,
                                                 bool want_a, bool want_b, float (&ga)[16], float (&gb)[16],
                                                 const BlkParams& P, unsigned t) {
    const unsigned co = fullh & ~h;
    // strict supersets m = h | S, S a nonempty subset of co, in increasing order
    const int nsup = (1 << __popc(co)) - 1;
    unsigned S = 0u;
    for (int k = 0; __any(k < nsup); ++k) {
        S = (S - co) & co;
        inner_pair<0, LOWNEG>(la, lb, lg, h, h | S, fullh, want_a && k < nsup, want_b && k < nsup, ga, gb, P, t);
    }
    // strict subsets m of h (the empty set first)
    const int nsub = (1 << __popc(h)) - 1;
    unsigned T = 0u;
    for (int k = 0; __any(k < nsub); ++k) {
        inner_pair<1, LOWNEG>(la, lb, lg, h, T, fullh, want_a && k < nsub, want_b && k < nsub, ga, gb, P, t);
        T = (T - h) & h;
    }
    inner_pair<2, LOWNEG>(la, lb, lg, h, h, fullh, want_a, want_b, ga, gb, P, t);
}

template <int OP, bool LOWNEG>
__global__ __launch_bounds__(256) void prod_bwd_blk(const float* __restrict__ A, const float* __restrict__ B,
                                                     const float* __restrict__ GC, float* __restrict__ GA,
                                                     float* __restrict__ GB, BlkParams P) {
    extern __shared__ float4 lds[];
    const int n = P.n;
    const int D4 = 1 << (n - 2);
    const unsigned NB = 1u << (n - 4);
    const long long row0 = (long long)blockIdx.x * P.rows_per_wg;
    const int nrows = (int)((P.batch - row0) < P.rows_per_wg ? (P.batch - row0) : P.rows_per_wg);
    stage_rows<3, true>(lds, reinterpret_cast<const float4*>(A), reinterpret_cast<const float4*>(B),
                        reinterpret_cast<const float4*>(GC), row0, nrows, n, P.ldg4 ? -1LL : (1LL << (n - 2)) - 1,
                        P.rskew);
    __syncthreads();
    const int r = threadIdx.x >> P.lpr_log;
    if (r >= nrows) return;
    const unsigned t = (P.rskew >> (2 * (r & 15))) & 3u;
    const unsigned lane_blk = threadIdx.x & ((1u << P.lpr_log) - 1u);
    const float4* la = lds + r * 3 * D4;
    const float4* lb = la + D4;
    const float4* lg = la + 2 * D4;
    const unsigned fullh = NB - 1u;
    const bool want_a = GA != nullptr, want_b = GB != nullptr;

    for (int kk = 0; kk < P.kpl; ++kk) {
        const unsigned h = lane_blk + ((unsigned)kk << P.lpr_log);
        const unsigned pi_h = cross_pi<OP>(h, P.nm1);
        float ga[16], gb[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            ga[e] = 0.f;
            gb[e] = 0.f;
        }
        if constexpr (OP == OP_INNER) {
            inner_bwd_blocks<LOWNEG>(la, lb, lg, h, fullh, want_a, want_b, ga, gb, P, t);
        } else
        for (unsigned m = 0; m < NB; ++m) {
            const unsigned x = h ^ m;
            const HiSign sa = hi_sign<OP>(h, m, P.negh, P.nulh, fullh, P.nm1, P.mu);  // (i, j) = (h, m)
            const HiSign sb = hi_sign<OP>(m, h, P.negh, P.nulh, fullh, P.nm1, P.mu);  // (i, j) = (m, h)
            const bool do_a = want_a && sa.valid, do_b = want_b && sb.valid;
            if (!do_a && !do_b) continue;
            float g[16];
            if (OP == OP_REGR) load_blk_s<true>(lg, fullh ^ x, bslot(fullh ^ x, t), g);
            else load_blk_s(lg, x, bslot(x, t), g);
            if (do_a) {
                float bv[16];
                load_blk_s(lb, m, bslot(m, t), bv);
                apply_flips(bv, sa.mask, sa.mask ^ (pi_h << 31));
                ga_block_dispatch<OP, LOWNEG>(ga, bv, g, h, m);
            }
            if (do_b) {
                const unsigned pm = cross_pi<OP>(m, P.nm1) << 31;
                float av[16], gt[16];
                load_blk_s(la, m, bslot(m, t), av);
                apply_flips(av, sb.mask, sb.mask ^ pm);
#pragma unroll
                for (int e = 0; e < 16; ++e) gt[e] = (cpopc((unsigned)e) & 1) ? flip(g[e], pm) : g[e];
                gb_block_dispatch<OP, LOWNEG>(gb, av, gt, m, h);
            }
        }
        const long long base = (row0 + r) << (n - 2);
        if (want_a) {
            float4* o = reinterpret_cast<float4*>(GA) + base;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                o[(h << 2) + q] = make_float4(ga[4 * q], ga[4 * q + 1], ga[4 * q + 2], ga[4 * q + 3]);
        }
        if (want_b) {
            float4* o = reinterpret_cast<float4*>(GB) + base;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                o[(h << 2) + q] = make_float4(gb[4 * q], gb[4 * q + 1], gb[4 * q + 2], gb[4 * q + 3]);
        }
    }
}

// ---- small-batch kernels (9 <= n <= 12; the forward also at n = 8): the partner loop split over lanes ----
// At batches of a few rows the one-lane-per-output-block kernels run one or
// two waves per row, so a row of n = 12 takes 256 dependent block pairs on one
// lane (0.65 ms at batch 1). Here a workgroup of 256 lanes owns G = 256 / S
// output blocks of one row: lane (o, s) walks partners ih = s, s + S, ... (NB / S
// of them, the pairs the op keeps), then the S partial blocks of each output
// are summed in LDS in a fixed order. S = NB / 4, so every lane walks 4
// partners and a row spreads over NB / G workgroups, each staging the whole
// row (the same row is read NB / G times: small batches only).
__device__ __forceinline__ int split_slot(unsigned o, unsigned s, int split_log) {
    // 20-float slots: the four float4 writes of 16 consecutive slots hit 16 bank groups
    return (int)((o << split_log) + s) * 20;
}

template <int OP, bool LOWNEG>
__global__ __launch_bounds__(256) void prod_fwd_split(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* __restrict__ C, BlkParams P) {
    extern __shared__ float4 lds[];
    const int n = P.n;
    const unsigned NB = 1u << (n - 4);
    const unsigned S = 1u << P.split_log;
    const long long row = (long long)(blockIdx.x >> P.wpr_log);
    const unsigned ogrp = blockIdx.x & ((1u << P.wpr_log) - 1u);
    stage_rows<2>(lds, reinterpret_cast<const float4*>(A), reinterpret_cast<const float4*>(B), nullptr, row, 1, n);
    __syncthreads();
    const unsigned sl = threadIdx.x & (S - 1u), ol = threadIdx.x >> P.split_log;
    const unsigned G = 256u >> P.split_log;
    const unsigned kh = ogrp * G + ol;
    const float4* la = lds;
    const float4* lb = lds + (1 << (n - 2));
    const unsigned fullh = NB - 1u;
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    for (unsigned ih = sl; ih < NB; ih += S) {
        const unsigned jh = ih ^ kh;
        const HiSign hs = hi_sign<OP>(ih, jh, P.negh, P.nulh, fullh, P.nm1, P.mu);
        if (!hs.valid) continue;
        float av[16], bv[16];
        load_blk(la, ih, av);
        load_blk(lb, jh, bv);
        apply_flips(bv, hs.mask, hs.mask ^ (cross_pi<OP>(ih, P.nm1) << 31));
        fwd_block_dispatch<OP, LOWNEG>(acc, av, bv, ih, jh);
    }
    __syncthreads();  // the staged row is no longer read: the partials go over it
    float* red = reinterpret_cast<float*>(lds);
    {
        float4* slot = reinterpret_cast<float4*>(red + split_slot(ol, sl, P.split_log));
#pragma unroll
        for (int q = 0; q < 4; ++q) slot[q] = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
    }
    __syncthreads();
    // lane i: element e = i & 15 of output ol = i >> 4 (G * 16 = 256 values... or fewer lanes busy)
    const unsigned e = threadIdx.x & 15u, o2 = threadIdx.x >> 4;
    for (unsigned o = o2; o < G; o += 16u) {
        float v = 0.f;
        for (unsigned k = 0; k < S; ++k) v += red[split_slot(o, k, P.split_log) + (int)e];
        const unsigned ko = ogrp * G + o;
        float* out = C + (row << n);
        if (OP == OP_REGR) out[((fullh ^ ko) << 4) + (15u - e)] = v;
        else out[(ko << 4) + e] = v;
    }
}

template <int OP, bool LOWNEG>
__global__ __launch_bounds__(256) void prod_bwd_split(const float* __restrict__ A, const float* __restrict__ B,
                                                       const float* __restrict__ GC, float* __restrict__ GA,
                                                       float* __restrict__ GB, BlkParams P) {
    extern __shared__ float4 lds[];
    const int n = P.n;
    const unsigned NB = 1u << (n - 4);
    const unsigned S = 1u << P.split_log;
    const long long row = (long long)(blockIdx.x >> P.wpr_log);
    const unsigned ogrp = blockIdx.x & ((1u << P.wpr_log) - 1u);
    stage_rows<3>(lds, reinterpret_cast<const float4*>(A), reinterpret_cast<const float4*>(B),
                  reinterpret_cast<const float4*>(GC), row, 1, n, P.ldg4 ? -1LL : (1LL << (n - 2)) - 1);
    __syncthreads();
    const unsigned sl = threadIdx.x & (S - 1u), ol = threadIdx.x >> P.split_log;
    const unsigned G = 256u >> P.split_log;
    const unsigned h = ogrp * G + ol;
    const int D4 = 1 << (n - 2);
    const float4* la = lds;
    const float4* lb = lds + D4;
    const float4* lg = lds + 2 * D4;
    const unsigned fullh = NB - 1u;
    const bool want_a = GA != nullptr, want_b = GB != nullptr;
    const unsigned pi_h = cross_pi<OP>(h, P.nm1);
    float ga[16], gb[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        ga[e] = 0.f;
        gb[e] = 0.f;
    }
    for (unsigned m = sl; m < NB; m += S) {
        const unsigned x = h ^ m;
        const HiSign sa = hi_sign<OP>(h, m, P.negh, P.nulh, fullh, P.nm1, P.mu);  // (i, j) = (h, m)
        const HiSign sb = hi_sign<OP>(m, h, P.negh, P.nulh, fullh, P.nm1, P.mu);  // (i, j) = (m, h)
        const bool do_a = want_a && sa.valid, do_b = want_b && sb.valid;
        if (!do_a && !do_b) continue;
        float g[16];
        if (OP == OP_REGR) load_blk_rev(lg, fullh ^ x, g);
        else load_blk(lg, x, g);
        if (do_a) {
            float bv[16];
            load_blk(lb, m, bv);
            apply_flips(bv, sa.mask, sa.mask ^ (pi_h << 31));
            ga_block_dispatch<OP, LOWNEG>(ga, bv, g, h, m);
        }
        if (do_b) {
            const unsigned pm = cross_pi<OP>(m, P.nm1) << 31;
            float av[16], gt[16];
            load_blk(la, m, av);
            apply_flips(av, sb.mask, sb.mask ^ pm);
#pragma unroll
            for (int e = 0; e < 16; ++e) gt[e] = (cpopc((unsigned)e) & 1) ? flip(g[e], pm) : g[e];
            gb_block_dispatch<OP, LOWNEG>(gb, av, gt, m, h);
        }
    }
    __syncthreads();  // the staged row is no longer read: the partials go over it
    float* red = reinterpret_cast<float*>(lds);
    const int half = (int)(256u * 20u);  // gb partials after the ga partials
    {
        float4* sa4 = reinterpret_cast<float4*>(red + split_slot(ol, sl, P.split_log));
        float4* sb4 = reinterpret_cast<float4*>(red + half + split_slot(ol, sl, P.split_log));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            sa4[q] = make_float4(ga[4 * q], ga[4 * q + 1], ga[4 * q + 2], ga[4 * q + 3]);
            sb4[q] = make_float4(gb[4 * q], gb[4 * q + 1], gb[4 * q + 2], gb[4 * q + 3]);
        }
    }
    __syncthreads();
    const unsigned e = threadIdx.x & 15u, o2 = threadIdx.x >> 4;
    for (unsigned o = o2; o < G; o += 16u) {
        float va = 0.f, vb = 0.f;
        for (unsigned k = 0; k < S; ++k) {
            va += red[split_slot(o, k, P.split_log) + (int)e];
            vb += red[half + split_slot(o, k, P.split_log) + (int)e];
        }
        const long long at = (row << n) + (long long)(((ogrp * G + o) << 4) + e);
        if (want_a) GA[at] = va;
        if (want_b) GB[at] = vb;
    }
}

// ---- balanced persistent kernels (4 <= n <= 10) -----------------------------
// For the masked products the work of an output block varies by up to 2^nh
// (wedge: 2^|kh| partner blocks, lc: 2^(nh - |kh|), ...), so one lane per
// output block leaves most lanes idle while the busiest one runs. Here the
// valid (output, partner) block pairs of a row, ordered by output block, are
// dealt out to the row's NB lanes in equal contiguous ranges of
// T = ceil(total / NB) pairs. A lane closes a segment when its output's pairs
// or its own range end: a segment that began in an earlier lane (a "head") is
// written to LDS, one that began and ended here is stored, and a last segment
// that continues in later lanes (a "tail") gets the later lanes' heads added
// after the loop, in lane order (deterministic sums).
// ROLE 0: output kh, partner ih (jh = ih ^ kh); ROLE 1: output ih (gradient
// of the left operand), partner jh; ROLE 2: output jh, partner ih. The
// partners of an output are a family {base | S}: the subsets S of mask in
// increasing order (S <- (S - mask) & mask), from index `first`, `count` of
// them. The inner product's low pattern depends on the pair (lc when ih is
// strictly inside jh, rc when jh is inside ih, both when ih = jh). Its forward
// runs one round (CLS 3): every pair (o, S) computes both the lc half
// (S, S | o) and the rc half (S | o, S), which share the partner family, and
// for o = 0 the terms both halves share (il = jl) are taken off the scalar slot
// once. Its backward (CLS 4) enumerates all partners of an output, the lc side
// then the rc side (two sub-families), and splits the low pattern by term
// class: shared terms always count, lc-only and rc-only terms take their
// operand from a copy zeroed unless the pair's blocks are related that way.
// Layout: a wave owns groups of 1024 floats per operand (R = 1024 / D rows,
// NB lanes per row) in wave-private LDS and walks the groups with a grid
// stride, loading the next group into registers while it computes.
constexpr int kBalMinN = 4, kBalMaxN = 10;
constexpr int kBalGroupF4 = 256;  // float4 per operand per group

struct BalFam {
    unsigned base, mask;
    int first, count;
    // a second sub-family (the inner product's backward round: the lc-side and
    // the rc-side partners of an output), enumerated after the first
    unsigned base2 = 0u, mask2 = 0u;
    int first2 = 0, count2 = 0;
};

__device__ __forceinline__ int fam_total(const BalFam& f) { return f.count + f.count2; }

// number of subsets of onn (= o without its null generators) strictly inside o
__device__ __forceinline__ int strict_sub(unsigned o, unsigned onn) {
    return (1 << __popc(onn)) - (onn == o ? 1 : 0);
}

// nul: the high-part null generators. Pairs whose blocks share one are zero
// for the metric ops and are left out of the families; an output of a stored
// (not added) op whose pairs all vanish keeps one such zero pair, so that it
// is still written.
template <int OP, int ROLE, int CLS>
__device__ __forceinline__ BalFam bal_family(unsigned o, unsigned full, unsigned nul) {
    const unsigned co = ~o & full;
    const int nco = 1 << __popc(co), no = 1 << __popc(o);
    const unsigned con = co & ~nul, onn = o & ~nul;  // partner bits that never meet a null
    const int ncon = 1 << __popc(con), nonn = 1 << __popc(onn);
    const bool onul = (o & nul) != 0u;
    if (OP == OP_GEOM) {
        const unsigned m = ROLE == 0 ? full & ~(nul & ~o) : full & ~(nul & o);
        return BalFam{0u, m, 0, 1 << __popc(m)};
    }
    if (OP == OP_WEDGE) return ROLE == 0 ? BalFam{0u, o, 0, no} : BalFam{0u, co, 0, nco};
    if (OP == OP_LC) {
        if (ROLE == 0) return BalFam{0u, con, 0, ncon};
        if (ROLE == 1) return onul ? BalFam{o, 0u, 0, 1} : BalFam{o, co, 0, nco};
        return BalFam{0u, onn, 0, nonn};
    }
    if (OP == OP_RC) {
        if (ROLE == 0) return BalFam{o, con, 0, ncon};
        if (ROLE == 1) return BalFam{0u, onn, 0, nonn};
        return onul ? BalFam{o, 0u, 0, 1} : BalFam{o, co, 0, nco};
    }
    if (OP == OP_REGR) return BalFam{co, o, 0, no};
    // inner, fused forward round: output o, partners S (ih = S, jh = S | o for the
    // lc half, ih = S | o, jh = S for the rc half)
    if (CLS == 3) return BalFam{0u, con, 0, ncon};
    // inner, backward in two deals: deal A (class 5) takes the partners on the
    // far side of the output (role 1: jh = o | S, lc relation; role 2:
    // ih = o | S, rc relation), deal B (class 6) those on the near side
    // (S inside o, the other relation), both with the pair ih = jh
    if (CLS == 5) return BalFam{o, co, 0, onul ? 0 : nco};
    if (CLS == 6) return BalFam{0u, onn, 0, nonn};
    // inner, backward round: all partners of an output, the lc side (with the
    // pair ih = jh) first, then the rc side
    if (CLS == 4) {
        if (ROLE == 1)  // output ih = o: jh = o | S (S inside co), then jh = S strictly inside o
            return BalFam{o, co, 0, onul ? 0 : nco, 0u, onn, 0, strict_sub(o, onn)};
        // ROLE 2, output jh = o: ih = S inside o, then ih = o | S (S nonempty, inside co)
        return BalFam{0u, onn, 0, nonn, o, co, 1, onul ? 0 : nco - 1};
    }
    return BalFam{0u, 0u, 0, 0};  // not reached: the inner product uses classes 3 and 4
}

// the s-th subset of m in increasing order (bits of s deposited on the bits of m)
__device__ __forceinline__ unsigned deposit_bits(unsigned s, unsigned m) {
    unsigned r = 0u;
    for (unsigned bit = 1u; m != 0u; bit <<= 1) {
        const unsigned low = m & (0u - m);
        if (s & bit) r |= low;
        m ^= low;
    }
    return r;
}

struct BalSched {
    int T;            // pairs per lane (the loop trip count, uniform)
    int p0, p1;       // this lane's pair range [p0, p1)
    unsigned o0;      // output of pair p0
    int s0;           // index of p0 inside o0
    bool cont0;       // o0 began in an earlier lane
    bool tail;        // the last segment continues in later lanes
    unsigned olast;   // output of the last segment
    int last_lane;    // last lane holding pairs of olast
};

// The schedule is the same for every row; the NB lanes of a row compute it
// together: lane lr counts the pairs of output lr, a segmented scan gives the
// output offsets, and binary searches over them (lane shuffles) find the
// outputs holding the lane's first and last pair.
__device__ __forceinline__ int bal_largest_le(int pre, int v, unsigned NB) {
    // largest output o with pre[o] <= v (pre non-decreasing, pre[0] = 0)
    int lo = 0;
    for (int step = (int)NB >> 1; step > 0; step >>= 1) {
        const int cand = __shfl(pre, lo + step, (int)NB);
        if (cand <= v) lo += step;
    }
    return lo;
}

template <int OP, int ROLE, int CLS>
__device__ __forceinline__ BalSched bal_schedule(unsigned lr, unsigned NB, unsigned nul) {
    const unsigned full = NB - 1u;
    const int c = fam_total(bal_family<OP, ROLE, CLS>(lr, full, nul));
    int inc = c;  // inclusive scan of the counts over the row's lanes
    for (int d = 1; d < (int)NB; d <<= 1) {
        const int v = __shfl_up(inc, (unsigned)d, (int)NB);
        if ((int)lr >= d) inc += v;
    }
    const int pre = inc - c;
    const int total = __shfl(inc, (int)NB - 1, (int)NB);
    BalSched sc;
    sc.T = (total + (int)NB - 1) / (int)NB;
    sc.p0 = (int)lr * sc.T;
    sc.p1 = sc.p0 + sc.T < total ? sc.p0 + sc.T : total;
    if (sc.p1 < sc.p0) sc.p1 = sc.p0;
    // every lane takes part in the shuffles; lanes without pairs discard them
    const int o0 = bal_largest_le(pre, sc.p0, NB);
    const int ol = bal_largest_le(pre, sc.p1 - 1, NB);
    const int pre_o0 = __shfl(pre, o0, (int)NB);
    const int end_ol = __shfl(inc, ol, (int)NB);
    const bool has = sc.p1 > sc.p0;
    sc.o0 = has ? (unsigned)o0 : 0u;
    sc.s0 = has ? sc.p0 - pre_o0 : 0;
    sc.olast = has ? (unsigned)ol : 0u;
    const int last_end = has ? end_ol : 0;
    sc.cont0 = sc.s0 > 0;
    sc.tail = has && sc.p1 < last_end && !(sc.olast == sc.o0 && sc.cont0);
    sc.last_lane = sc.T > 0 ? (last_end - 1) / sc.T : 0;
    return sc;
}

__device__ __forceinline__ void store_blk(float4* __restrict__ out, unsigned blk, const float (&acc)[16], bool rev) {
    if (rev) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            out[(blk << 2) + (3 - q)] = make_float4(acc[4 * q + 3], acc[4 * q + 2], acc[4 * q + 1], acc[4 * q]);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            out[(blk << 2) + q] = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
    }
}

// low-block pattern of a pair: the op's; the inner product's rounds pick their
// patterns per half (forward) or per term class (backward)
template <int OP, int CLS>
constexpr int bal_variant() {
    return OP != OP_INNER ? OP : (CLS == 3 ? LV_LC : LV_INNER);
}

// sum_l s_lo(l, l) a[l] b[l]: the terms the lc and rc low patterns share
template <bool LOWNEG, int... L>
__device__ __forceinline__ float lowblock_diag(const float (&a)[16], const float (&b)[16],
                                               std::integer_sequence<int, L...>) {
    float e = 0.f;
    ((e = low_sign(LV_LC, LOWNEG, (unsigned)L, (unsigned)L) > 0 ? __builtin_fmaf(a[L], b[L], e)
                                                                 : __builtin_fmaf(-a[L], b[L], e)),
     ...);
    return e;
}

// One role (and class) over one row: la / lb / lg are the row's staged
// operands, heads the row's head slots (4 float4 per lane). Completed outputs
// are stored to out (the row in global memory, nullptr for a row past the end
// of the batch). The caller syncs the wave's LDS before (staged data) and
// after (heads reused).
template <int OP, int ROLE, int CLS, bool LOWNEG>
__device__ __forceinline__ void bal_role(const BalSched& sc, const float4* __restrict__ la,
                                         const float4* __restrict__ lb, const float4* __restrict__ lg,
                                         float4* __restrict__ heads, unsigned lr, float4* __restrict__ out,
                                         unsigned NB, const BlkParams& P, unsigned rs) {
    const unsigned full = NB - 1u;
    constexpr bool kRev = OP == OP_REGR && ROLE == 0;
    constexpr int VAR = bal_variant<OP, CLS>();
    constexpr bool kLowNeg = VAR == LV_WEDGE || VAR == LV_REGR ? false : LOWNEG;
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    unsigned o = sc.o0;
    BalFam f = bal_family<OP, ROLE, CLS>(o, full, P.nulh);
    int s = sc.s0;
    // S runs over the first sub-family, then (the inner backward round) the second
    unsigned S = s < f.count ? deposit_bits((unsigned)(f.first + s), f.mask)
                             : deposit_bits((unsigned)(f.first2 + s - f.count), f.mask2);
    bool first = true;
    int p = sc.p0;
    for (int t = 0; t < sc.T; ++t) {
        if (p >= sc.p1) break;
        const bool in2 = CLS == 4 && s >= f.count;
        const unsigned part = (in2 ? f.base2 : f.base) | S;
        if (OP == OP_INNER && CLS == 3) {
            // lc half: (S, S | o), lc low pattern; rc half: (S | o, S), rc low
            // pattern. For o = 0 both halves are (S, S) and count the terms with
            // il = jl twice: those are taken off the scalar slot once.
            const HiSign hl = hi_sign<OP>(part, part ^ o, P.negh, P.nulh, full, P.nm1, P.mu);
            const HiSign hr = hi_sign<OP>(part ^ o, part, P.negh, P.nulh, full, P.nm1, P.mu);
            {
                float av[16], bv[16];
                load_blk_x(la, part, av, rs);
                load_blk_x(lb, part ^ o, bv, rs);
                const unsigned m = hl.valid ? hl.mask : 0u;
                apply_flips(bv, m, m ^ (cross_pi<OP>(part, P.nm1) << 31));
                if (hl.valid) {
                    lowblock_fwd<LV_LC, kLowNeg>(acc, av, bv);
                    const float e = lowblock_diag<kLowNeg>(av, bv, std::make_integer_sequence<int, 16>{});
                    acc[0] = __builtin_fmaf(o == 0u ? -1.f : 0.f, e, acc[0]);
                }
            }
            if (hr.valid) {
                float av[16], bv[16];
                load_blk_x(la, part ^ o, av, rs);
                load_blk_x(lb, part, bv, rs);
                apply_flips(bv, hr.mask, hr.mask ^ (cross_pi<OP>(part ^ o, P.nm1) << 31));
                lowblock_fwd<LV_RC, kLowNeg>(acc, av, bv);
            }
        } else if (ROLE == 0) {
            const unsigned ih = part, jh = part ^ o;
            const HiSign hs = hi_sign<OP>(ih, jh, P.negh, P.nulh, full, P.nm1, P.mu);
            if (hs.valid) {
                float av[16], bv[16];
                load_blk_x(la, ih, av, rs);
                load_blk_x(lb, jh, bv, rs);
                apply_flips(bv, hs.mask, hs.mask ^ (cross_pi<OP>(ih, P.nm1) << 31));
                if (OP == OP_INNER) lowblock_fwd<VAR, kLowNeg>(acc, av, bv);
                else fwd_block_dispatch<OP, LOWNEG>(acc, av, bv, ih, jh);
            }
        } else {
            const unsigned h = o, m = part, x = h ^ m;
            const HiSign hs = ROLE == 1 ? hi_sign<OP>(h, m, P.negh, P.nulh, full, P.nm1, P.mu)
                                        : hi_sign<OP>(m, h, P.negh, P.nulh, full, P.nm1, P.mu);
            if (hs.valid) {
                float g[16];
                if (OP == OP_REGR) load_blk_x<true>(lg, full ^ x, g, rs);
                else load_blk_x(lg, x, g, rs);
                if (ROLE == 1) {
                    float bv[16];
                    load_blk_x(lb, m, bv, rs);
                    apply_flips(bv, hs.mask, hs.mask ^ (cross_pi<OP>(h, P.nm1) << 31));
                    if (OP == OP_INNER && CLS == 4)  // ih = h, jh = m
                        lowblock_ga_split<kLowNeg>(acc, bv, (h & ~m) == 0u, (m & ~h) == 0u, g);
                    else if (OP == OP_INNER) lowblock_ga<VAR, kLowNeg>(acc, bv, g);
                    else ga_block_dispatch<OP, LOWNEG>(acc, bv, g, h, m);
                } else {
                    const unsigned pm = cross_pi<OP>(m, P.nm1) << 31;
                    float av[16], gt[16];
                    load_blk_x(la, m, av, rs);
                    apply_flips(av, hs.mask, hs.mask ^ pm);
#pragma unroll
                    for (int e = 0; e < 16; ++e) gt[e] = (cpopc((unsigned)e) & 1) ? flip(g[e], pm) : g[e];
                    if (OP == OP_INNER && CLS == 4)  // ih = m, jh = h
                        lowblock_gb_split<kLowNeg>(acc, av, (m & ~h) == 0u, (h & ~m) == 0u, gt);
                    else if (OP == OP_INNER) lowblock_gb<VAR, kLowNeg>(acc, av, gt);
                    else gb_block_dispatch<OP, LOWNEG>(acc, av, gt, m, h);
                }
            }
        }
        ++p;
        ++s;
        if (CLS == 4 && s == f.count) {
            S = deposit_bits((unsigned)f.first2, f.mask2);
        } else {
            const unsigned msk = in2 ? f.mask2 : f.mask;
            S = (S - msk) & msk;
        }
        const bool done = s == fam_total(f);
        if (done || p == sc.p1) {
            if (first && sc.cont0) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    heads[lr * 4 + q] = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
            } else if (done && out) {
                store_blk(out, kRev ? (full ^ o) : o, acc, kRev);
            }
            if (done) {
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[e] = 0.f;
                first = false;
                // next output with pairs (outputs of a class may have none)
                do {
                    ++o;
                    if (o >= NB) break;
                    f = bal_family<OP, ROLE, CLS>(o, full, P.nulh);
                } while (fam_total(f) == 0);
                s = 0;
                S = f.count > 0 ? deposit_bits((unsigned)f.first, f.mask) : deposit_bits((unsigned)f.first2, f.mask2);
            }
        }
    }
    wave_lds_sync();
    if (sc.tail) {
        for (int l = (int)lr + 1; l <= sc.last_lane; ++l) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = heads[l * 4 + q];
                acc[4 * q] += v.x;
                acc[4 * q + 1] += v.y;
                acc[4 * q + 2] += v.z;
                acc[4 * q + 3] += v.w;
            }
        }
        if (out) store_blk(out, kRev ? (full ^ sc.olast) : sc.olast, acc, kRev);
    }
}

// ---- table-driven rounds (the inner product's deals, n >= 8) --------------
// The schedule of a role is the same for every row, so its per-pair
// bookkeeping (the family walk, the high-part sign, segment ends) is done once
// per workgroup into a table in LDS: one 16-bit entry per (step, lane of the
// row). The round over a row then reads an entry, loads two blocks, applies
// two sign masks and runs the op's low pattern; it carries no family state.
//   bits 0-5   partner block P (role 0: ih; role 1: jh; role 2: ih)
//   bits 6-11  output block O (role 0: ih ^ jh; roles 1 and 2: the gradient's block)
//   bit 12     high-part sign (1: negative)
//   bit 13     compute (the pair's high blocks are related; else the pair adds nothing)
//   bits 14-15 after this step: 0 continue, 1 write the head slot, 2 store the output
// A lane with no pair at a step has the entry 0 (nothing to compute or store).
constexpr unsigned kTabSign = 1u << 12, kTabCompute = 1u << 13;
constexpr int kTabActShift = 14;
constexpr int kBalTMax = 12;  // steps: at most ceil(3^nh / 2^nh) = 12 pairs per lane (nh <= 6)
constexpr int kBalTabEntries = kBalTMax * 64;

// The lane's tail (its last segment continues in later lanes) is packed in a
// header word: bit 0 tail, bits 1-6 the last lane holding pairs of that
// output, bits 7-12 the output.
template <int OP, int ROLE, int CLS = 0>
__device__ __forceinline__ void bal_build_tab(const BalSched& sc, unsigned lr, unsigned NB, const BlkParams& P,
                                              unsigned short* __restrict__ tab, unsigned* __restrict__ hdr) {
    const unsigned full = NB - 1u;
    hdr[lr] = (sc.tail ? 1u : 0u) | ((unsigned)sc.last_lane << 1) | (sc.olast << 7);
    unsigned o = sc.o0;
    BalFam f = bal_family<OP, ROLE, CLS>(o, full, P.nulh);
    int s = sc.s0;
    unsigned S = deposit_bits((unsigned)(f.first + s), f.mask);
    bool first = true;
    int p = sc.p0;
    for (int t = 0; t < sc.T; ++t) {
        unsigned e = 0u;
        if (p < sc.p1) {
            const unsigned part = f.base | S;
            const HiSign hs = ROLE == 0   ? hi_sign<OP>(part, part ^ o, P.negh, P.nulh, full, P.nm1, P.mu)
                              : ROLE == 1 ? hi_sign<OP>(o, part, P.negh, P.nulh, full, P.nm1, P.mu)
                                          : hi_sign<OP>(part, o, P.negh, P.nulh, full, P.nm1, P.mu);
            e = part | (o << 6) | (hs.valid ? kTabCompute : 0u) | (hs.mask ? kTabSign : 0u);
            ++p;
            ++s;
            S = (S - f.mask) & f.mask;
            const bool done = s == f.count;
            if (done || p == sc.p1) {
                if (first && sc.cont0) e |= 1u << kTabActShift;
                else if (done) e |= 2u << kTabActShift;
                if (done) {
                    first = false;
                    do {
                        ++o;
                        if (o >= NB) break;
                        f = bal_family<OP, ROLE, CLS>(o, full, P.nulh);
                    } while (f.count == 0);
                    s = 0;
                    S = deposit_bits((unsigned)f.first, f.mask);
                }
            }
        }
        tab[t * NB + lr] = (unsigned short)e;
    }
}

// sum_e s_lo(e, e) x[e] y0 terms of a pair ih = jh: the terms both deals of
// the inner product's backward count (subtracted once from the output)
template <bool LOWNEG, int... E>
__device__ __forceinline__ void diag_sub(float (&acc)[16], const float (&x)[16], float y0,
                                        std::integer_sequence<int, E...>) {
    ((acc[E] = low_sign(LV_LC, LOWNEG, (unsigned)E, (unsigned)E) > 0 ? __builtin_fmaf(-x[E], y0, acc[E])
                                                                      : __builtin_fmaf(x[E], y0, acc[E])),
     ...);
}

// One role over one row from its table (see bal_role for the arguments; T is
// the table's step count, hdr the lane's tail header). MODE 0 stores completed
// outputs; the inner product's deal A (MODE 1) leaves them in the row's
// partial slot `part`, its deal B (MODE 2) adds the partial (outputs whose
// deal A had pairs), takes off the terms of the pair ih = jh that both deals
// counted, and stores.
template <int OP, int ROLE, bool LOWNEG, int MODE = 0>
__device__ __forceinline__ void bal_role_tab(int T, unsigned hdr, const unsigned short* __restrict__ tab,
                                             const float4* __restrict__ la, const float4* __restrict__ lb,
                                             const float4* __restrict__ lg, float4* __restrict__ heads, unsigned lr,
                                             float4* __restrict__ out, unsigned NB, const BlkParams& P, unsigned rs,
                                             float4* __restrict__ part = nullptr) {
    const unsigned full = NB - 1u;
    constexpr bool kRev = OP == OP_REGR && ROLE == 0;
    // the inner product's deals: role 1 deal A and role 2 deal B pair blocks
    // in the lc relation, the others in the rc relation
    constexpr int VAR = OP != OP_INNER ? OP : ((ROLE == 1) == (MODE == 1) ? LV_LC : LV_RC);
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    // completion of output ob: store (MODE 0), park (MODE 1) or finish (MODE 2)
    auto finish = [&](unsigned ob) {
        if (MODE == 1) {
            store_blk(part, ob, acc, false);
            return;
        }
        if (MODE == 2) {
            const unsigned nul = P.nulh;
            if ((ob & nul) == 0u) {  // deal A had pairs and both deals had the pair (ob, ob)
                float pv[16];
                load_blk_plain(part, ob, pv);
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[e] += pv[e];
                const HiSign hs = hi_sign<OP>(ob, ob, P.negh, P.nulh, full, P.nm1, P.mu);
                const unsigned sm = hs.mask;
                const unsigned pm = cross_pi<OP>(ob, P.nm1) << 31;
                float xv[16];
                load_blk_x(ROLE == 1 ? lb : la, ob, xv, rs);
                apply_flips(xv, sm, sm ^ pm);
                const float g0 = reinterpret_cast<const float*>(lg)[4u * (swz(0u) ^ rs)];  // gc element 0
                diag_sub<LOWNEG>(acc, xv, g0, std::make_integer_sequence<int, 16>{});
            }
        }
        if (out) store_blk(out, kRev ? (full ^ ob) : ob, acc, kRev);
    };
    for (int t = 0; t < T; ++t) {
        const unsigned e = tab[t * NB + lr];
        const unsigned pb = e & 63u, ob = (e >> 6) & 63u;
        if (e & kTabCompute) {
            const unsigned sm = (e & kTabSign) << 19;  // bit 12 -> the float sign bit
            if (ROLE == 0) {  // ih = pb, jh = pb ^ ob
                float av[16], bv[16];
                load_blk_x(la, pb, av, rs);
                load_blk_x(lb, pb ^ ob, bv, rs);
                apply_flips(bv, sm, sm ^ (cross_pi<OP>(pb, P.nm1) << 31));
                fwd_block_dispatch<OP, LOWNEG>(acc, av, bv, pb, pb ^ ob);
            } else {
                const unsigned x = ob ^ pb;
                float g[16];
                if (OP == OP_REGR) load_blk_x<true>(lg, full ^ x, g, rs);
                else load_blk_x(lg, x, g, rs);
                if (ROLE == 1) {  // h = ob, m = pb
                    float bv[16];
                    load_blk_x(lb, pb, bv, rs);
                    apply_flips(bv, sm, sm ^ (cross_pi<OP>(ob, P.nm1) << 31));
                    if (OP == OP_INNER) lowblock_ga<VAR, LOWNEG>(acc, bv, g);
                    else ga_block_dispatch<OP, LOWNEG>(acc, bv, g, ob, pb);
                } else {  // h = ob (jh), m = pb (ih)
                    const unsigned pm = cross_pi<OP>(pb, P.nm1) << 31;
                    float av[16], gt[16];
                    load_blk_x(la, pb, av, rs);
                    apply_flips(av, sm, sm ^ pm);
#pragma unroll
                    for (int k = 0; k < 16; ++k) gt[k] = (cpopc((unsigned)k) & 1) ? flip(g[k], pm) : g[k];
                    if (OP == OP_INNER) lowblock_gb<VAR, LOWNEG>(acc, av, gt);
                    else gb_block_dispatch<OP, LOWNEG>(acc, av, gt, pb, ob);
                }
            }
        }
        const unsigned act = e >> kTabActShift;
        if (act == 1u) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                heads[lr * 4 + q] = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
        } else if (act == 2u) {
            finish(ob);
        }
        if (act != 0u) {
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[k] = 0.f;
        }
    }
    wave_lds_sync();
    if (hdr & 1u) {
        const int last_lane = (int)((hdr >> 1) & 63u);
        for (int l = (int)lr + 1; l <= last_lane; ++l) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = heads[l * 4 + q];
                acc[4 * q] += v.x;
                acc[4 * q + 1] += v.y;
                acc[4 * q + 2] += v.z;
                acc[4 * q + 3] += v.w;
            }
        }
        finish((hdr >> 7) & 63u);
    }
}

// ---- register-held steps (wedge, lc, rc, regressive) ----------------------
// The same schedule as the deals' tables, held per lane in registers (one
// 32-bit word per step) with the staged blocks' LDS byte offsets precomputed,
// so a step decodes two offsets and three bits instead of walking the swizzle:
//   bits 0-11   offset of the first block (role 0: a[ih]; role 1: b[jh]; role 2: a[ih])
//   bits 12-23  offset of the second block (role 0: b[jh]; roles 1 and 2: gc[ih ^ jh],
//               regressive: gc[~(ih ^ jh)])
//   bit 24      high-part sign; bit 25 cross parity (role 0 and 2: the partner's,
//               role 1: the output's); bit 26 compute; bits 27-28 the action at the step's
//               end (as in the tables: continue, write the head slot, store)
// Every output of these ops has at least one pair, so a lane's outputs are
// consecutive from its first one and the output of a step is counted, not
// stored. Each lane builds its own words (its row's slot skew is in the
// offsets) once per kernel.
constexpr unsigned kRegCompute = 1u << 26;
constexpr int kRegActShift = 27;

__device__ __forceinline__ unsigned bal_blk_off(unsigned blk, unsigned rs) {
    return ((blk << 2) | (swz(blk) ^ rs)) << 4;
}

template <int OP, int ROLE>
__device__ __forceinline__ void bal_reg_entries(const BalSched& sc, unsigned NB, const BlkParams& P, unsigned rs,
                                                unsigned (&E)[kBalTMax]) {
    const unsigned full = NB - 1u;
    unsigned o = sc.o0;
    BalFam f = bal_family<OP, ROLE, 0>(o, full, P.nulh);
    int s = sc.s0;
    unsigned S = deposit_bits((unsigned)(f.first + s), f.mask);
    bool first = true;
    int p = sc.p0;
#pragma unroll
    for (int t = 0; t < kBalTMax; ++t) {
        unsigned e = 0u;
        if (p < sc.p1) {
            const unsigned part = f.base | S;
            const HiSign hs = ROLE == 0   ? hi_sign<OP>(part, part ^ o, P.negh, P.nulh, full, P.nm1, P.mu)
                              : ROLE == 1 ? hi_sign<OP>(o, part, P.negh, P.nulh, full, P.nm1, P.mu)
                                          : hi_sign<OP>(part, o, P.negh, P.nulh, full, P.nm1, P.mu);
            const unsigned x = part ^ o;
            const unsigned b2 = ROLE == 0 ? x : (OP == OP_REGR ? full ^ x : x);
            const unsigned cr = cross_pi<OP>(ROLE == 1 ? o : part, P.nm1);
            e = bal_blk_off(part, rs) | (bal_blk_off(b2, rs) << 12) | ((hs.mask >> 31) << 24) | (cr << 25) |
                (hs.valid ? kRegCompute : 0u);
            ++p;
            ++s;
            S = (S - f.mask) & f.mask;
            const bool done = s == f.count;
            if (done || p == sc.p1) {
                if (first && sc.cont0) e |= 1u << kRegActShift;
                else if (done) e |= 2u << kRegActShift;
                if (done) {
                    first = false;
                    ++o;  // every output has pairs
                    f = bal_family<OP, ROLE, 0>(o < NB ? o : 0u, full, P.nulh);
                    s = 0;
                    S = deposit_bits((unsigned)f.first, f.mask);
                }
            }
        }
        E[t] = e;
    }
}

// One role over one row from the lane's words (T: the schedule's step count,
// hdr: the lane's tail header, o0: its first output). b1 / b2: LDS byte
// addresses of the row's first and second staged operand (role 0: a, b;
// role 1: b, gc; role 2: a, gc).
template <int OP, int ROLE, bool LOWNEG>
__device__ __forceinline__ void bal_role_reg(int T, const unsigned (&E)[kBalTMax], unsigned hdr, unsigned o0,
                                             unsigned b1, unsigned b2, float4* __restrict__ heads, unsigned lr,
                                             float4* __restrict__ out, unsigned NB) {
    const unsigned full = NB - 1u;
    constexpr bool kRev = OP == OP_REGR && ROLE == 0;
    T = __builtin_amdgcn_readfirstlane(T);  // the same for every lane of the row's schedule
    unsigned o = o0;
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
    for (int t = 0; t < kBalTMax; ++t) {
        if (t >= T) break;
        unsigned e = E[t];
        asm volatile("" : "+v"(e));  // decoded at its step, not ahead of the loop
        if (e & kRegCompute) {
            const unsigned a1 = b1 + (e & 4095u), a2 = b2 + ((e >> 12) & 4095u);
            const unsigned sm = (e << 7) & 0x80000000u;
            const unsigned cm = (e << 6) & 0x80000000u;
            float v1[16], v2[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 x1 = lds_ld4(a1 ^ ((unsigned)q << 4));
                const float4 x2 = lds_ld4(a2 ^ ((unsigned)q << 4));
                v1[4 * q] = x1.x; v1[4 * q + 1] = x1.y; v1[4 * q + 2] = x1.z; v1[4 * q + 3] = x1.w;
                constexpr bool kR2 = OP == OP_REGR && ROLE != 0;  // regressive gc blocks read reversed
                v2[kR2 ? 15 - 4 * q : 4 * q] = x2.x;
                v2[kR2 ? 14 - 4 * q : 4 * q + 1] = x2.y;
                v2[kR2 ? 13 - 4 * q : 4 * q + 2] = x2.z;
                v2[kR2 ? 12 - 4 * q : 4 * q + 3] = x2.w;
            }
            if (ROLE == 0) {  // v1 = a[ih], v2 = b[jh]
                apply_flips(v2, sm, sm ^ cm);
                fwd_block_dispatch<OP, LOWNEG>(acc, v1, v2, 0u, 0u);
            } else if (ROLE == 1) {  // v1 = b[jh], v2 = gc
                apply_flips(v1, sm, sm ^ cm);
                ga_block_dispatch<OP, LOWNEG>(acc, v1, v2, 0u, 0u);
            } else {  // v1 = a[ih], v2 = gc
                apply_flips(v1, sm, sm ^ cm);
                float gt[16];
#pragma unroll
                for (int k = 0; k < 16; ++k) gt[k] = (cpopc((unsigned)k) & 1) ? flip(v2[k], cm) : v2[k];
                gb_block_dispatch<OP, LOWNEG>(acc, v1, gt, 0u, 0u);
            }
        }
        const unsigned act = e >> kRegActShift;
        if (act == 1u) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                heads[lr * 4 + q] = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
        } else if (act == 2u) {
            if (out) store_blk(out, kRev ? (full ^ o) : o, acc, kRev);
        }
        if (act != 0u) {
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[k] = 0.f;
            ++o;
        }
    }
    wave_lds_sync();
    if (hdr & 1u) {
        const int last_lane = (int)((hdr >> 1) & 63u);
        for (int l = (int)lr + 1; l <= last_lane; ++l) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = heads[l * 4 + q];
                acc[4 * q] += v.x;
                acc[4 * q + 1] += v.y;
                acc[4 * q + 2] += v.z;
                acc[4 * q + 3] += v.w;
            }
        }
        const unsigned ol = (hdr >> 7) & 63u;
        if (out) store_blk(out, kRev ? (full ^ ol) : ol, acc, kRev);
    }
}

// A group's operand: float4 chunk lane + 64 i (i < 4) of R consecutive rows,
// rows past the end clamped to the last row.
struct BalPre {
    float4 v[4];
};

// A lane's share of a group (1024 floats per operand): chunks c = lane + 64 i
// (i < 4), row rr = c >> (n - 2) of the group, float4 ff = c & (D4 - 1), and
// the chunk's staged LDS byte offset (stage_rows' layout: row rr at rr * D4,
// float4 slots swizzled inside a block, with the row's skew rr & 3 xor-ed into
// the slot). Fixed for the kernel, so a group's fetch and staging take no
// per-group index arithmetic.
struct BalLane {
    unsigned rr[4], ff[4], so[4];
};

// RX: the row term of the chunk slots as a 4-entry table of 2-bit values
// (entry r & 3 at bits 2 (r & 3)); 0xE4 is r & 3
template <unsigned RX = 0xE4u>
__device__ __forceinline__ unsigned row_x(unsigned r) { return (RX >> (2u * (r & 3u))) & 3u; }

// SW: the block swizzle as an 8-entry table of 2-bit values (blocks 0..7), or
// 0 for swz()
template <unsigned SW = 0u>
__device__ __forceinline__ unsigned blk_swz(unsigned blk) {
    if constexpr (SW == 0u) return swz(blk);
    else return (SW >> (2u * (blk & 7u))) & 3u;
}

template <unsigned RX = 0xE4u, unsigned SW = 0u>
__device__ __forceinline__ BalLane bal_lane(int n, int lane) {
    BalLane L;
    const int d4_log = n - 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned c = (unsigned)(lane + 64 * i);
        const unsigned r = c >> d4_log, f = c & ((1u << d4_log) - 1u);
        const unsigned blk = f >> 2, q = f & 3u;
        L.rr[i] = r;
        L.ff[i] = f;
        L.so[i] = 16u * ((r << d4_log) + (blk << 2) + (q ^ blk_swz<SW>(blk) ^ row_x<RX>(r)));
    }
    return L;
}

// Where a group's rows come from: the first row's address (wave-uniform) and
// the last row of the group to read; rows past it re-read it (the end of the
// batch; every row is row 0 of an upstream gradient broadcast over the batch;
// a group past the end reads the batch's last row).
struct BalSrc {
    const float4* g0;
    unsigned rlim;
};

__device__ __forceinline__ BalSrc bal_src(const float* __restrict__ src, long long grp, long long batch, int n, int R,
                                          bool bcast = false) {
    const long long row0 = grp * R;
    const bool in = row0 < batch;
    const long long first = bcast ? 0 : (in ? row0 : batch - 1);
    const long long left = (bcast || !in) ? 1 : (batch - row0 < R ? batch - row0 : R);
    return {reinterpret_cast<const float4*>(src) + (first << (n - 2)), (unsigned)(left - 1)};
}

__device__ __forceinline__ BalPre bal_fetch(const BalSrc& s, const BalLane& L, int d4_log) {
    BalPre p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned row = L.rr[i] < s.rlim ? L.rr[i] : s.rlim;
        p.v[i] = s.g0[(row << d4_log) | L.ff[i]];
    }
    return p;
}

__device__ __forceinline__ void lds_st4(unsigned a, float4 v) {
    *(lds_v4f*)(uintptr_t)a = v4f_t{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ void bal_stage(float4* __restrict__ dst, const BalPre& p, const BalLane& L) {
    const unsigned a = lds_addr4(dst);
#pragma unroll
    for (int i = 0; i < 4; ++i) lds_st4(a + L.so[i], p.v[i]);
}

template <int OP, bool LOWNEG>
__global__ __launch_bounds__(256) void prod_fwd_bal(const float* __restrict__ A, const float* __restrict__ B,
                                                     float* __restrict__ C, BlkParams P) {
    // LDS per wave: a | b | heads. The inner product runs its fused round
    // (class 3: lc and rc halves of every pair), so every op stores directly.
    constexpr int kCls = OP == OP_INNER ? 3 : 0;
    __shared__ __attribute__((aligned(64))) float4 lds[4][3 * kBalGroupF4];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int n = P.n;
    const int lpr_log = n - 4;
    const unsigned NB = 1u << lpr_log;
    const unsigned lr = (unsigned)lane & (NB - 1u);
    const int r = lane >> lpr_log;
    const int R = 64 >> lpr_log;
    float4* sa = lds[wave];
    float4* sb = sa + kBalGroupF4;
    float4* heads = sb + kBalGroupF4 + (r << lpr_log) * 4;
    const int roff = r << (n - 2);
    const unsigned rs = (unsigned)r & 3u;  // the row's slot skew
    const BalSched sc = bal_schedule<OP, 0, kCls>(lr, NB, P.nulh);
    // wedge, lc, rc and regressive run from the lane's register-held steps
    constexpr bool kTab = OP != OP_INNER && OP != OP_GEOM;
    unsigned E[kBalTMax];
    if constexpr (kTab) bal_reg_entries<OP, 0>(sc, NB, P, rs, E);
    const unsigned my_hdr = (sc.tail ? 1u : 0u) | ((unsigned)sc.last_lane << 1) | (sc.olast << 7);
    const long long ngrp = (P.batch + R - 1) / R;
    const long long gstride = (long long)gridDim.x * 4;
    long long grp = (long long)blockIdx.x * 4 + wave;
    const BalLane L = bal_lane(n, lane);
    const int d4_log = n - 2;
    BalPre pa = bal_fetch(bal_src(A, grp, P.batch, n, R), L, d4_log);
    BalPre pb = bal_fetch(bal_src(B, grp, P.batch, n, R), L, d4_log);
    for (; grp < ngrp; grp += gstride) {
        bal_stage(sa, pa, L);
        bal_stage(sb, pb, L);
        pa = bal_fetch(bal_src(A, grp + gstride, P.batch, n, R), L, d4_log);
        pb = bal_fetch(bal_src(B, grp + gstride, P.batch, n, R), L, d4_log);
        wave_lds_sync();
        const long long row = grp * R + r;
        float4* out = row < P.batch ? reinterpret_cast<float4*>(C) + (row << (n - 2)) : nullptr;
        if constexpr (kTab)
            bal_role_reg<OP, 0, LOWNEG>(sc.T, E, my_hdr, sc.o0, lds_addr4(sa + roff), lds_addr4(sb + roff), heads, lr,
                                        out, NB);
        else bal_role<OP, 0, kCls, LOWNEG>(sc, sa + roff, sb + roff, nullptr, heads, lr, out, NB, P, rs);
        wave_lds_sync();
    }
}

// Backward: b and gc are staged first and the left-operand gradient runs with
// its heads in the a slot; then a is staged and the right-operand gradient
// runs with its heads in the b slot (12 KB of LDS per wave). The inner product
// runs each gradient in two deals (classes 5 and 6: the lc-relation and the
// rc-relation partners, 81 terms per pair each) whose sums meet in a fourth
// slot (16 KB per wave).
template <int OP, bool LOWNEG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void prod_bwd_bal(const float* __restrict__ A, const float* __restrict__ B,
                                                     const float* __restrict__ GC, float* __restrict__ GA,
                                                     float* __restrict__ GB, BlkParams P) {
    constexpr bool kDeals = OP == OP_INNER;
    constexpr bool kTab = OP != OP_GEOM;  // every op but geom runs from precomputed steps (registers, or
                                          // LDS tables for the inner product's deals)
    constexpr int kTabs = kDeals ? 4 : 2;
    __shared__ __attribute__((aligned(64))) float4 lds[4][(kDeals ? 4 : 3) * kBalGroupF4];  // a | b | gc [| the inner product's partials]
    __shared__ unsigned short tab[kDeals ? kTabs : 1][kDeals ? kBalTabEntries : 1];
    __shared__ unsigned hdr[kDeals ? kTabs : 1][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int n = P.n;
    const int lpr_log = n - 4;
    const unsigned NB = 1u << lpr_log;
    const unsigned lr = (unsigned)lane & (NB - 1u);
    const int r = lane >> lpr_log;
    const int R = 64 >> lpr_log;
    float4* sa = lds[wave];
    float4* sb = sa + kBalGroupF4;
    float4* sg = sb + kBalGroupF4;
    float4* sp = sg + kBalGroupF4;  // inner product only
    const int roff = r << (n - 2);
    const unsigned rs = (unsigned)r & 3u;  // the row's slot skew
    const int hoff = (r << lpr_log) * 4;
    const bool want_a = GA != nullptr, want_b = GB != nullptr;
    // step counts of the roles' tables (deals A, B for the inner product)
    int T[kTabs];
    if constexpr (kDeals) {
        const BalSched s0 = bal_schedule<OP, 1, 5>(lr, NB, P.nulh), s1 = bal_schedule<OP, 1, 6>(lr, NB, P.nulh);
        const BalSched s2 = bal_schedule<OP, 2, 5>(lr, NB, P.nulh), s3 = bal_schedule<OP, 2, 6>(lr, NB, P.nulh);
        if (wave == 0 && lane < (int)NB) {
            bal_build_tab<OP, 1, 5>(s0, lr, NB, P, tab[0], hdr[0]);
            bal_build_tab<OP, 1, 6>(s1, lr, NB, P, tab[1], hdr[1]);
            bal_build_tab<OP, 2, 5>(s2, lr, NB, P, tab[2], hdr[2]);
            bal_build_tab<OP, 2, 6>(s3, lr, NB, P, tab[3], hdr[3]);
        }
        T[0] = s0.T;
        T[1] = s1.T;
        T[2] = s2.T;
        T[3] = s3.T;
    }
    if (kDeals) __syncthreads();
    // wedge, lc, rc and regressive: the lane's register-held steps per role
    unsigned EA[kBalTMax], EB[kBalTMax];
    unsigned hdr_a = 0u, hdr_b = 0u, o0_a = 0u, o0_b = 0u;
    if constexpr (kTab && !kDeals) {
        const BalSched sca = bal_schedule<OP, 1, 0>(lr, NB, P.nulh), scb = bal_schedule<OP, 2, 0>(lr, NB, P.nulh);
        bal_reg_entries<OP, 1>(sca, NB, P, rs, EA);
        bal_reg_entries<OP, 2>(scb, NB, P, rs, EB);
        hdr_a = (sca.tail ? 1u : 0u) | ((unsigned)sca.last_lane << 1) | (sca.olast << 7);
        hdr_b = (scb.tail ? 1u : 0u) | ((unsigned)scb.last_lane << 1) | (scb.olast << 7);
        o0_a = sca.o0;
        o0_b = scb.o0;
        T[0] = sca.T;
        T[1] = scb.T;
    }
    const BalSched sca = bal_schedule<OP, 1, 0>(lr, NB, P.nulh);  // geom only
    const BalSched scb = bal_schedule<OP, 2, 0>(lr, NB, P.nulh);
    const long long ngrp = (P.batch + R - 1) / R;
    const long long gstride = (long long)gridDim.x * 4;
    long long grp = (long long)blockIdx.x * 4 + wave;
    const BalLane L = bal_lane(n, lane);
    const int d4_log = n - 2;
    const bool gbc = P.ldg4 == 0;  // gc: one row for all rows
    BalPre pa, pb;
    if (want_b) pa = bal_fetch(bal_src(A, grp, P.batch, n, R), L, d4_log);
    if (want_a) pb = bal_fetch(bal_src(B, grp, P.batch, n, R), L, d4_log);
    BalPre pg = bal_fetch(bal_src(GC, grp, P.batch, n, R, gbc), L, d4_log);
    for (; grp < ngrp; grp += gstride) {
        const long long row = grp * R + r;
        const bool row_ok = row < P.batch;
        bal_stage(sg, pg, L);
        pg = bal_fetch(bal_src(GC, grp + gstride, P.batch, n, R, gbc), L, d4_log);
        if (want_a) {  // uniform: a kernel argument
            bal_stage(sb, pb, L);
            pb = bal_fetch(bal_src(B, grp + gstride, P.batch, n, R), L, d4_log);
            wave_lds_sync();
            float4* out = row_ok ? reinterpret_cast<float4*>(GA) + (row << (n - 2)) : nullptr;
            if constexpr (kDeals) {
                bal_role_tab<OP, 1, LOWNEG, 1>(T[0], hdr[0][lr], tab[0], nullptr, sb + roff, sg + roff, sa + hoff, lr,
                                               nullptr, NB, P, rs, sp + roff);
                wave_lds_sync();
                bal_role_tab<OP, 1, LOWNEG, 2>(T[1], hdr[1][lr], tab[1], nullptr, sb + roff, sg + roff, sa + hoff, lr,
                                               out, NB, P, rs, sp + roff);
            } else if constexpr (kTab) {
                bal_role_reg<OP, 1, LOWNEG>(T[0], EA, hdr_a, o0_a, lds_addr4(sb + roff), lds_addr4(sg + roff), sa + hoff,
                                            lr, out, NB);
            } else {
                bal_role<OP, 1, 0, LOWNEG>(sca, nullptr, sb + roff, sg + roff, sa + hoff, lr, out, NB, P, rs);
            }
            wave_lds_sync();
        }
        if (want_b) {
            bal_stage(sa, pa, L);
            pa = bal_fetch(bal_src(A, grp + gstride, P.batch, n, R), L, d4_log);
            wave_lds_sync();
            float4* out = row_ok ? reinterpret_cast<float4*>(GB) + (row << (n - 2)) : nullptr;
            if constexpr (kDeals) {
                bal_role_tab<OP, 2, LOWNEG, 1>(T[2], hdr[2][lr], tab[2], sa + roff, nullptr, sg + roff, sb + hoff, lr,
                                               nullptr, NB, P, rs, sp + roff);
                wave_lds_sync();
                bal_role_tab<OP, 2, LOWNEG, 2>(T[3], hdr[3][lr], tab[3], sa + roff, nullptr, sg + roff, sb + hoff, lr,
                                               out, NB, P, rs, sp + roff);
            } else if constexpr (kTab) {
                bal_role_reg<OP, 2, LOWNEG>(T[1], EB, hdr_b, o0_b, lds_addr4(sa + roff), lds_addr4(sg + roff), sb + hoff,
                                            lr, out, NB);
            } else {
                bal_role<OP, 2, 0, LOWNEG>(scb, sa + roff, nullptr, sg + roff, sb + hoff, lr, out, NB, P, rs);
            }
        }
        wave_lds_sync();
    }
}

// ---- inner product backward for 4 <= n <= 8: one lane per output block ------
// Lane h of a row computes both gradient blocks h: ga[h] over the partners
// jh = p of the relation (p inside h: rc pairs; p containing h: lc pairs) and
// gb[h] over ih = p, with the same partner list, so one gc block g[h ^ p]
// serves both. A partner p inside h needs the "sub" low pattern (q inside o),
// one containing h the "sup" pattern (q containing o); lanes of a wave are
// at different points of their lists, so the wave runs one instruction stream
// by turning sub pairs into sup pairs: with o' = ~o, q' = ~q (4-bit
// complements), q inside o is q' containing o', and o ^ q = o' ^ q'. A lane in
// sub mode reads its partner block reversed (element ~q' at position q') and
// accumulates in the reversed frame (position o' holds output ~o'); the
// sign of the reversed pair factors into
//   s_lo(~i, ~j) = s_lo(i, j) (-1)^{w1(i) + w2(j)} [low metric: (-1)^{|i|+|j|}]
// with w1(k) = k1 ^ k3 and w2(k) = k0 ^ k2 (the reorder parities of complemented
// indices), so the partner's flips take the w-term and the frame change takes
// the output's. Every lane walks its sub partners (subsets of h, ascending,
// ending with h) and then its sup partners (h | S, ascending from h), turning
// its accumulators to the normal frame in between (position k <- +-position
// 15 - k; w1, w2 and the parity are invariant under the complement, so the
// turn is its own inverse). The pair (h, h) is walked in both modes; its
// diagonal terms il = jl are the only terms of any pair that read element 0
// of gc block 0, so the sub-mode walk zeroes that element and they count
// once. Lanes have 2^|h| + 2^(nh - |h|) steps (at most 2^nh + 1); a lane
// stores when its list ends and idles (with a repeated partner) until the
// wave's last step.
// The a and b blocks are staged with float4 slot q holding elements
// 4q + (c ^ q) in component c, so the reversed block is the slot order
// reversed (an address xor) with the same element-to-register map.
constexpr int kFrameMinN = 4, kFrameMaxN = 8;

// register of element e of a frame-staged block
__host__ __device__ constexpr int fr_reg(int e) { return (e & 12) | ((e & 3) ^ (e >> 2)); }
__host__ __device__ constexpr int par4(int k) { return (k ^ (k >> 1) ^ (k >> 2) ^ (k >> 3)) & 1; }
__host__ __device__ constexpr int w1b(int k) { return ((k >> 1) ^ (k >> 3)) & 1; }
__host__ __device__ constexpr int w2b(int k) { return (k ^ (k >> 2)) & 1; }

// sup pattern: ca[o] += s_lo(o, q) wa[q] g[o ^ q] (ga: il = o, jl = q) and
// cb[o] += s_lo(q, o) wb[q] gt[o ^ q] (gb: il = q, jl = o), q containing o
template <bool LOWNEG, bool WA, bool WB, int... Is>
__device__ __forceinline__ void frame_sup(float (&ca)[16], float (&cb)[16], const float (&wa)[16],
                                          const float (&wb)[16], const float (&g)[16], const float (&gt)[16],
                                          std::integer_sequence<int, Is...>) {
    auto term = [&](auto oq) {
        constexpr int O = decltype(oq)::value >> 4, Q = decltype(oq)::value & 15;
        if constexpr ((O & ~Q) == 0) {
            constexpr int sa = low_sign(LV_LC, LOWNEG, (unsigned)O, (unsigned)Q);
            constexpr int sb = low_sign(LV_RC, LOWNEG, (unsigned)Q, (unsigned)O);
            if constexpr (WA) ca[O] = __builtin_fmaf(sa > 0 ? wa[fr_reg(Q)] : -wa[fr_reg(Q)], g[O ^ Q], ca[O]);
            if constexpr (WB) cb[O] = __builtin_fmaf(sb > 0 ? wb[fr_reg(Q)] : -wb[fr_reg(Q)], gt[O ^ Q], cb[O]);
        }
    };
    (term(std::integral_constant<int, Is>{}), ...);
}

// Lane-dependent selects of whole accumulators: a mask that is all ones
// where the lane's condition holds, formed once and opaque to the compiler
// (which would turn the bit operations back into conditional moves, twice
// the issue cost of a three-input bit operation on gfx950)
__device__ __forceinline__ unsigned lane_mask(bool c) {
    unsigned m = c ? ~0u : 0u;
    asm volatile("" : "+v"(m));
    return m;
}
__device__ __forceinline__ float bsel(unsigned m, float a, float b) {  // a where m, else b
    return __uint_as_float((__float_as_uint(a) & m) | (__float_as_uint(b) & ~m));
}
__device__ __forceinline__ float bzero(unsigned m, float a) {  // 0 where m, else a
    return __uint_as_float(__float_as_uint(a) & ~m);
}

// turn an accumulator between the reversed and the normal frame where cond
// holds: c[k] <- f(k) c[15 - k], f = w2 (gb) or w1 (ga), times the parity
// for a negative low metric (negated elements: one conditional move with a
// negate modifier; the others a bit select)
template <bool LOWNEG, bool GB>
__device__ __forceinline__ void frame_turn(float (&c)[16], bool cond) {
    const unsigned m = lane_mask(cond);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const bool f = ((GB ? w2b(k) : w1b(k)) ^ (LOWNEG ? par4(k) : 0)) != 0;
        const float x = c[k], y = c[15 - k];
        c[k] = f ? (cond ? -y : x) : bsel(m, y, x);
        c[15 - k] = f ? (cond ? -x : y) : bsel(m, x, y);
    }
}

template <class F, int... Ts>
__device__ __forceinline__ void frame_steps(F&& f, std::integer_sequence<int, Ts...>) {
    (f(std::integral_constant<int, Ts>{}), ...);
}

// At n = 7 and 8 the lanes of outputs 0 and full have 2^nh + 1 steps and
// the others at most 2^(nh-1) + 2, so the last pairs of outputs 0 and full go
// to helper lanes that have finished their own lists, C pairs each in the
// wave's last C steps, and DPP adds merge them after the last step:
//   n = 7 (7 steps, C = 1): quad lanes 1, 2 help output 0 (its sup pairs 6,
//          7), lanes 5, 6 output 7 (its sub pairs 6, 7); quad_perm merges;
//   n = 8 (11 steps, C = 2): lanes 3, 5, 6 help output 0 (sup pairs 10..15),
//          lanes 9, 10, 12 output 15 (sub pairs 10..15); row-shift merges.
// Output full walks its one sup pair (full, full) first, so its last pairs
// are sub pairs like its helpers'. A helper stores its own output when its
// list ends and starts from zero before its first helper step.
template <int NH>
struct FrameSched {
    static constexpr bool kHelp = NH == 3 || NH == 4;
    static constexpr int NB = 1 << NH;
    static constexpr int T = NH == 3 ? 7 : NH == 4 ? 11 : NB + 1;
    static constexpr int C = NH == 3 ? 1 : 2;  // pairs per helper lane
    // a lane may turn its frame before step t / store after step t
    static constexpr bool turn(int t) { return t >= 1 && t <= (kHelp ? NB / 2 : NB) && (t & (t - 1)) == 0; }
    static constexpr bool store(int t) {
        if (kHelp && t == T - 1) return true;
        for (int k = kHelp ? 1 : 0; k <= (kHelp ? NH - 1 : NH); ++k)
            if ((1 << k) + (1 << (NH - k)) == t + 1) return true;
        return false;
    }
    static constexpr bool helper(unsigned h) {
        return NH == 3 ? (h == 1u || h == 2u || h == 5u || h == 6u)
                       : (h == 3u || h == 5u || h == 6u || h == 9u || h == 10u || h == 12u);
    }
    // helper index 0..2 among the helpers of its output (output 0: the first
    // group, output full: the second)
    static constexpr int help_rank(unsigned h) {
        return NH == 3 ? (h == 1u || h == 5u ? 0 : 1) : (h == 3u || h == 9u ? 0 : h == 5u || h == 10u ? 1 : 2);
    }
    static constexpr bool helps_zero(unsigned h) { return NH == 3 ? h < 4u : h < 8u; }
};

// step t of lane h: output block o, partner block p, sub mode
struct FrameStep {
    unsigned o, p;
    bool sub;
    bool idle = false;  // frame_step at n = 7: the step reads blocks X = o, W = p, result unused
};

// n = 7 (NH = 3): the frame schedule as searched for the LDS bank rules of the
// backward kernels (prod_bwd_inner_frame, prod_bwd_contr_frame). Byte h of
// kFrame7Sched[t] is lane h's step t: p (bits 0-2), o (3-5), sub (6), idle
// (7; then o and p name the gc and partner blocks it reads). The lists are
// the ones frame_step builds (sub partners, then sup partners; outputs 0 and
// 7 keep six pairs and helpers 1, 2 and 5, 6 take one each at step 6) in
// searched orders; with the block swizzle kFrame7Swz and the row term
// kFrame7RowX of the LDS slots, the 16 lanes of each bank set read one
// address per 16-byte group at every step of the inner product and the
// contractions (the wedge and regressive products: one extra cycle per two
// steps), and the row-order output stores stay conflict-free.
constexpr unsigned long long kFrame7Sched[7] = {0x3f746d645b504940ull, 0x7972696059524807ull, 0x7a70682758170f05ull,
                                                0x7e766c255a130900ull, 0x7c372f261b120b03ull, 0x7f362d241f160d06ull,
                                                0x7b7d78aea3020104ull};
constexpr unsigned kFrame7RowX = 0x8Du;   // rows 0..3 -> 1, 3, 0, 2
constexpr unsigned kFrame7Swz = 0x50AFu;  // blocks 0..7 -> 3, 3, 2, 2, 0, 0, 1, 1

// LDS slot terms of the frame kernels: the searched ones at n = 7
template <int N>
struct FrameLayout {
    static constexpr unsigned kRowX = N == 7 ? kFrame7RowX : 0xE4u;
    static constexpr unsigned kSwz = N == 7 ? kFrame7Swz : 0u;
};

template <int NH>
__device__ __forceinline__ FrameStep frame_step(unsigned h, int t) {
    using Sch = FrameSched<NH>;
    constexpr unsigned full = (1u << NH) - 1u;
    if constexpr (NH == 3) {
        const unsigned c = (unsigned)(kFrame7Sched[t] >> (8u * h)) & 0xffu;
        return FrameStep{(c >> 3) & 7u, c & 7u, ((c >> 6) & 1u) != 0u, (c >> 7) != 0u};
    }
    if (Sch::kHelp) {
        if (h == 0u) return t == 0 ? FrameStep{0u, 0u, true} : FrameStep{0u, (unsigned)(t - 1), false};
        if (h == full) return t == 0 ? FrameStep{full, full, false} : FrameStep{full, (unsigned)(t - 1), true};
        if (t >= Sch::T - Sch::C && Sch::helper(h)) {  // the last pairs of outputs 0 and full
            const unsigned p = (unsigned)(Sch::T - 1 + Sch::C * Sch::help_rank(h) + (t - (Sch::T - Sch::C)));
            return Sch::helps_zero(h) ? FrameStep{0u, p, false} : FrameStep{full, p, true};
        }
    }
    const int cs = 1 << __popc(h), cnt = cs + (1 << (NH - __popc(h)));
    if (t < cs) return FrameStep{h, deposit_bits((unsigned)t, h), true};
    if (t < cnt) return FrameStep{h, h | deposit_bits((unsigned)(t - cs), full & ~h), false};
    return FrameStep{h, h, false};  // idle
}

// x + x[quad lane 1] + x[quad lane 2] on quad lanes 0 and 3 (other lanes:
// unused sums). Two DPP adds; each s_nop gives the DPP read of x the wait
// states a VALU write of x right before it would need.
__device__ __forceinline__ float quad_merge(float x) {
    float t, y;
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 quad_perm:[1,1,2,1] row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(t) : "v"(x), "v"(x));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 quad_perm:[2,1,2,2] row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(y) : "v"(x), "v"(t));
    return y;
}

// n = 8: x + x[lane + 3] + x[lane + 5] + x[lane + 6] on lane 0 of each row
// of 16 (its helpers 3, 5, 6) and x + x[lane - 6] + x[lane - 5] + x[lane - 3]
// on lane 15 (helpers 9, 10, 12); other lanes keep x. s_nop as in quad_merge.
__device__ __forceinline__ float row16_merge(float x, unsigned h) {
    float a1, a2, a3, b1, b2, b3;
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 row_shl:3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(a1) : "v"(x), "v"(x));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 row_shl:5 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(a2) : "v"(x), "v"(a1));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 row_shl:6 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(a3) : "v"(x), "v"(a2));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 row_shr:6 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(b1) : "v"(x), "v"(x));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 row_shr:5 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(b2) : "v"(x), "v"(b1));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 row_shr:3 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(b3) : "v"(x), "v"(b2));
    return h == 0u ? a3 : (h == 15u ? b3 : x);
}

template <int N, bool LOWNEG, bool WA, bool WB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void prod_bwd_inner_frame(
    const float* __restrict__ A, const float* __restrict__ B, const float* __restrict__ GC, float* __restrict__ GA,
    float* __restrict__ GB, BlkParams P) {
    constexpr int NH = N - 4, NB = 1 << NH, R = 64 >> NH;
    using Sch = FrameSched<NH>;
    using FL = FrameLayout<N>;
    constexpr int T = Sch::T;
    constexpr unsigned full = NB - 1u;
    __shared__ __attribute__((aligned(64))) float4 lds[4][3 * kBalGroupF4];  // a | b | gc
    // the steps of lane (h, row slot skew rs): tab[t][rs * NB + h]
    __shared__ unsigned tab[T][4 * NB];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned h = (unsigned)lane & full;
    const int r = lane >> NH;
    const unsigned rs = (unsigned)r & 3u;
    // the lane's frame turn (before its first sup step) and store steps
    const int kh = __popc(h);
    const int cs = 1 << kh;
    const bool edge = Sch::kHelp && (h == 0u || h == full);
    const int turn_t = edge ? 1 : cs;
    const int store_t = edge ? Sch::T - 1 : cs + (1 << (NH - kh)) - 1;
    // one group of R rows per wave (the host splits batches larger than one grid)
    const long long ngrp = (P.batch + R - 1) / R;
    const long long grp = (long long)blockIdx.x * 4 + wave;
    const BalLane L = bal_lane<FL::kRowX, FL::kSwz>(N, lane);
    const bool gbc = P.ldg4 == 0;
    // the group's loads are in flight while the step table is built
    BalPre pa, pb, pg;
    if (WB) pa = bal_fetch(bal_src(A, grp, P.batch, N, R), L, N - 2);
    if (WA) pb = bal_fetch(bal_src(B, grp, P.batch, N, R), L, N - 2);
    pg = bal_fetch(bal_src(GC, grp, P.batch, N, R, gbc), L, N - 2);
    // entry: block offsets (gc block o ^ p; partner p, its slot order reversed
    // in sub mode), sub flag, the high-part signs, the parities of p and o, and
    // whether the step is the pair (o, o) in sub mode
    if (wave == 0 && lane < 4 * NB) {
        const unsigned th = (unsigned)lane & full, trs = row_x<FL::kRowX>((unsigned)lane >> NH);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const FrameStep st = frame_step<NH>(th, t);
            const unsigned X = st.idle ? st.o : st.o ^ st.p;
            const HiSign sga = hi_sign<OP_INNER>(st.o, st.p, P.negh, P.nulh, full, P.nm1, P.mu);
            const HiSign sgb = hi_sign<OP_INNER>(st.p, st.o, P.negh, P.nulh, full, P.nm1, P.mu);
            const unsigned offg = ((X << 2) | (blk_swz<FL::kSwz>(X) ^ trs)) << 4;
            const unsigned offw = ((st.p << 2) | (blk_swz<FL::kSwz>(st.p) ^ trs ^ (st.sub ? 3u : 0u))) << 4;
            tab[t][lane] = offg | (offw << 10) | ((st.sub ? 1u : 0u) << 20) | ((sga.mask >> 31) << 21) |
                           ((sgb.mask >> 31) << 22) | (((unsigned)__popc(st.p) & 1u) << 23) |
                           (((unsigned)__popc(st.o) & 1u) << 24) | ((st.sub && st.p == st.o ? 1u : 0u) << 25);
        }
    }
    __syncthreads();
    if (grp >= ngrp) return;
    const int tix = (int)(rs * NB + h);
    float4* sa = lds[wave];
    const unsigned base = lds_addr4(sa + (r << (N - 2)));  // the row's a block 0; b at +4 KB, gc at +8 KB
    {
        // a and b in the frame layout: component c of the lane's chunks (block
        // slot fq) goes to component c ^ fq, one dword store each
        const unsigned fq = (unsigned)lane & 3u;
        const unsigned a0 = lds_addr4(sa);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned ad = (a0 + L.so[i]) | (fq << 2);
            const float va[4] = {pa.v[i].x, pa.v[i].y, pa.v[i].z, pa.v[i].w};
            const float vb[4] = {pb.v[i].x, pb.v[i].y, pb.v[i].z, pb.v[i].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const unsigned adc = ad ^ ((unsigned)c << 2);
                if (WB) *(__attribute__((address_space(3))) float*)(uintptr_t)adc = va[c];
                if (WA) *(__attribute__((address_space(3))) float*)(uintptr_t)(adc + 4096u) = vb[c];
            }
            lds_st4(a0 + 8192u + L.so[i], pg.v[i]);
        }
    }
    wave_lds_sync();
    const long long row = grp * R + r;
    const bool row_ok = row < P.batch;
    float ca[16], cb[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        ca[e] = 0.f;
        cb[e] = 0.f;
    }
    // a lane's output blocks wait in ya / yb once complete and leave through
    // LDS in row order after the last step (n = 5, which has no registers to
    // spare, stores each block when it is complete)
    constexpr bool kRowOut = N != 5;
    float ya[16], yb[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        ya[e] = 0.f;
        yb[e] = 0.f;
    }
    auto store = [&]() {
        if constexpr (kRowOut) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                if (WA) ya[e] = ca[e];
                if (WB) yb[e] = cb[e];
            }
        } else if (row_ok) {
            if (WA) store_blk(reinterpret_cast<float4*>(GA) + (row << (N - 2)), h, ca, false);
            if (WB) store_blk(reinterpret_cast<float4*>(GB) + (row << (N - 2)), h, cb, false);
        }
    };
    auto step = [&](auto tc) {
        constexpr int t = decltype(tc)::value;
        // steps do not overlap: two steps' operands (56 registers each) would
        // not fit beside the accumulators at three waves per SIMD
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (Sch::turn(t)) {
            const bool turn = turn_t == t;
            if (WA) frame_turn<LOWNEG, false>(ca, turn);
            if (WB) frame_turn<LOWNEG, true>(cb, turn);
        }
        unsigned e = tab[t][tix];
        asm volatile("" : "+v"(e));  // decoded per step, not kept for every step across the kernel
        const unsigned ga0 = base + 8192u + (e & 1023u);
        const unsigned wa0 = base + ((e >> 10) & 1023u);
        const unsigned subm = (e << 11) & 0x80000000u;
        const unsigned sga = (e << 10) & 0x80000000u, sgb = (e << 9) & 0x80000000u;
        const unsigned podd = (e << 8) & 0x80000000u, oodd = (e << 7) & 0x80000000u;
        const unsigned subln = LOWNEG ? subm : 0u;
        float g[16], wa[16], wb[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 vg = lds_ld4(ga0 ^ ((unsigned)q << 4));
            // the pair (o, o) is walked in both modes and its diagonal terms (the
            // only ones that read gc element 0 of block 0) count in sup mode only
            g[4 * q] = q == 0 && ((e >> 25) & 1u) ? 0.f : vg.x;
            g[4 * q + 1] = vg.y;
            g[4 * q + 2] = vg.z;
            g[4 * q + 3] = vg.w;
            if (WA) {
                const float4 v = lds_ld4((wa0 ^ ((unsigned)q << 4)) + 4096u);
                wa[4 * q] = v.x;
                wa[4 * q + 1] = v.y;
                wa[4 * q + 2] = v.z;
                wa[4 * q + 3] = v.w;
            }
            if (WB) {
                const float4 v = lds_ld4(wa0 ^ ((unsigned)q << 4));
                wb[4 * q] = v.x;
                wb[4 * q + 1] = v.y;
                wb[4 * q + 2] = v.z;
                wb[4 * q + 3] = v.w;
            }
        }
        // partner flips by element class (parity, w-term): pair sign, cross
        // sign (|o| for ga, |p| for gb, on odd elements), sub-mode w-term and
        // (negative low metric) sub-mode parity
        // (the masks are formed once: opaque to the compiler, which would
        // otherwise fold the bit extraction into each element's flip)
        if (WA) {
            unsigned m0 = sga, m1 = sga ^ oodd ^ subln, m2 = sga ^ subm, m3 = m1 ^ subm;
            asm volatile("" : "+v"(m0), "+v"(m1), "+v"(m2), "+v"(m3));
#pragma unroll
            for (int el = 0; el < 16; ++el) {
                const int cl = par4(el) + 2 * w2b(el);
                const unsigned m = cl == 0 ? m0 : cl == 1 ? m1 : cl == 2 ? m2 : m3;
                wa[fr_reg(el)] = flip(wa[fr_reg(el)], m);
            }
        }
        float gt[16];
        if (WB) {
            unsigned m0 = sgb, m1 = sgb ^ podd ^ subln, m2 = sgb ^ subm, m3 = m1 ^ subm, mp = podd;
            asm volatile("" : "+v"(m0), "+v"(m1), "+v"(m2), "+v"(m3), "+v"(mp));
#pragma unroll
            for (int el = 0; el < 16; ++el) {
                const int cl = par4(el) + 2 * w1b(el);
                const unsigned m = cl == 0 ? m0 : cl == 1 ? m1 : cl == 2 ? m2 : m3;
                wb[fr_reg(el)] = flip(wb[fr_reg(el)], m);
            }
#pragma unroll
            for (int x = 0; x < 16; ++x) gt[x] = par4(x) ? flip(g[x], mp) : g[x];
        }
        frame_sup<LOWNEG, WA, WB>(ca, cb, wa, wb, g, gt, std::make_integer_sequence<int, 256>{});
        if constexpr (Sch::kHelp && t == T - 1) {
            // outputs 0 and full add their helpers' sums (the other lanes have
            // stored theirs), then output full turns to the normal frame
#pragma unroll
            for (int el = 0; el < 16; ++el) {
                if constexpr (NH == 3) {
                    if (WA) ca[el] = quad_merge(ca[el]);
                    if (WB) cb[el] = quad_merge(cb[el]);
                } else {
                    if (WA) ca[el] = row16_merge(ca[el], h);
                    if (WB) cb[el] = row16_merge(cb[el], h);
                }
            }
            if (WA) frame_turn<LOWNEG, false>(ca, h == full);
            if (WB) frame_turn<LOWNEG, true>(cb, h == full);
        }
        if constexpr (Sch::store(t)) {
            if constexpr (kRowOut) {  // the lanes whose outputs complete here keep them
                const unsigned ms = lane_mask(store_t == t);
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    if (WA) ya[e] = bsel(ms, ca[e], ya[e]);
                    if (WB) yb[e] = bsel(ms, cb[e], yb[e]);
                }
            } else if (store_t == t) {
                store();
            }
        }
        if constexpr (Sch::kHelp && t == T - Sch::C - 1) {  // the helpers start from zero
            const unsigned mz = lane_mask(Sch::helper(h));
#pragma unroll
            for (int el = 0; el < 16; ++el) {
                if (WA) ca[el] = bzero(mz, ca[el]);
                if (WB) cb[el] = bzero(mz, cb[el]);
            }
        }
    };
    frame_steps(step, std::make_integer_sequence<int, T>{});
    if constexpr (kRowOut) {
        // ga rows over the staged a, gb rows over b, in the staging layout of
        // gc (block h of row r at slots 4h + (q ^ swz(h) ^ row_x(r)), the
        // kernel's swizzle and row term); then row-order stores
        wave_lds_sync();
        const unsigned a0 = lds_addr4(sa);
        const unsigned rowb = a0 + ((unsigned)r << (N + 2));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const unsigned slot = ((h << 2) | ((unsigned)q ^ blk_swz<FL::kSwz>(h) ^ row_x<FL::kRowX>(rs))) << 4;
            if (WA) lds_st4(rowb + slot, make_float4(ya[4 * q], ya[4 * q + 1], ya[4 * q + 2], ya[4 * q + 3]));
            if (WB) lds_st4(rowb + 4096u + slot, make_float4(yb[4 * q], yb[4 * q + 1], yb[4 * q + 2], yb[4 * q + 3]));
        }
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long long rr = grp * R + (long long)L.rr[i];
            if (rr < P.batch) {
                const long long at = (rr << (N - 2)) + (long long)L.ff[i];
                if (WA) reinterpret_cast<float4*>(GA)[at] = lds_ld4(a0 + L.so[i]);
                if (WB) reinterpret_cast<float4*>(GB)[at] = lds_ld4(a0 + 4096u + L.so[i]);
            }
        }
    }
}

// ---- left and right contraction backward for 4 <= n <= 8 -----------------
// The inner product's frame schedule (frame_step, helpers, merges) and layout
// with one accumulator per lane. A contraction's pair is related one way
// only, so a step yields one gradient: the left contraction's sub pairs
// (partner a[p], p inside h) give gb[h] and its sup pairs (b[p], p containing
// h) give ga[h]; the right contraction the other way round. Every step runs
// the ga sup pattern acc[o] += s_lc(o, q) w[q] g[o ^ q] (q containing o); a
// gb step uses s_rc(q, o) = s_lc(o, q) rho(o) rho(q) rho(o ^ q), rho the
// reversion sign (-1)^(|k| (|k| - 1) / 2): its partner block takes rho(q) and
// its gc block rho(x) on top of the inner kernel's flips, and the stored block
// takes rho(o). A lane stores its first output when its first mode ends
// (turned to the normal frame if that mode was sub) and starts from zero, and
// its second output at the end of its list; outputs 0 and full (which walk
// one pair in their first mode) add their helpers' sums first.
__host__ __device__ constexpr int rho4(int k) { return (__builtin_popcount((unsigned)k) >> 1) & 1; }

template <int NH>
struct ContrSched {
    using S = FrameSched<NH>;
    static constexpr int NB = 1 << NH;
    static constexpr bool edge(unsigned h) { return S::kHelp && (h == 0u || h == (unsigned)(NB - 1)); }
    // steps after which lane h stores its first and its second output
    static constexpr int first_t(unsigned h) { return edge(h) ? 0 : (1 << __builtin_popcount(h)) - 1; }
    static constexpr int second_t(unsigned h) {
        return edge(h) ? S::T - 1 : (1 << __builtin_popcount(h)) + (1 << (NH - __builtin_popcount(h))) - 1;
    }
    // the mode of a lane's first output: sub, except output full with helpers
    static constexpr bool first_sub(unsigned h) { return !(edge(h) && h == (unsigned)(NB - 1)); }
    // modes of the outputs stored after step t: bit 0 sub, bit 1 sup
    static constexpr int kinds(int t) {
        int k = 0;
        for (unsigned h = 0; h < (unsigned)NB; ++h) {
            if (first_t(h) == t) k |= first_sub(h) ? 1 : 2;
            if (second_t(h) == t) k |= first_sub(h) ? 2 : 1;
        }
        return k;
    }
    static constexpr bool any_first(int t) {
        for (unsigned h = 0; h < (unsigned)NB; ++h)
            if (first_t(h) == t) return true;
        return false;
    }
    static constexpr bool any_second(int t) {
        for (unsigned h = 0; h < (unsigned)NB; ++h)
            if (second_t(h) == t) return true;
        return false;
    }
};

// y = the stored block of an accumulator whose mode was sub (turned to the
// normal frame) or sup; GBK: the block is a gb block (rho(o) on the
// accumulator's positions)
template <bool LOWNEG, bool GBK>
__device__ __forceinline__ float contr_out_sub(const float (&x)[16], int k) {
    const int src = 15 - k;
    const bool f = (((GBK ? w2b(k) : w1b(k)) ^ (LOWNEG ? par4(k) : 0) ^ (GBK ? rho4(src) : 0)) & 1) != 0;
    return f ? -x[src] : x[src];
}

template <bool GBK>
__device__ __forceinline__ float contr_out_sup(const float (&x)[16], int k) {
    return GBK && rho4(k) ? -x[k] : x[k];
}

// disjoint pattern of the wedge product: acc[o] += s_w(o, q) w[q] g[o | q]
template <int... Is>
__device__ __forceinline__ void frame_disjoint(float (&acc)[16], const float (&w)[16], const float (&g)[16],
                                               std::integer_sequence<int, Is...>) {
    auto term = [&](auto oq) {
        constexpr int O = decltype(oq)::value >> 4, Q = decltype(oq)::value & 15;
        if constexpr ((O & Q) == 0) {
            constexpr int sw = low_sign(LV_WEDGE, false, (unsigned)O, (unsigned)Q);
            acc[O] = __builtin_fmaf(sw > 0 ? w[fr_reg(Q)] : -w[fr_reg(Q)], g[O ^ Q], acc[O]);
        }
    };
    (term(std::integral_constant<int, Is>{}), ...);
}

// The regressive product as a wedge product of duals (the reference's definition,
// c = dual(dual(a) ^ dual(b))): with (D x)[k] = t(~k) x[~k] and
// t(m) = (-1)^{bitsum(m) + |m & NEG| + C(n,2) + |NEG|}, c = D wedge(D a, D b), so its
// backward is the wedge backward on (D a, D b, D^T gc) followed by D^T on both
// gradients ((D^T y)[k] = t(k) y[~k]). On a float4 chunk F (elements 4F + c) the
// complement reverses the chunk order and the components; dual_chunk_mask(F) has
// bit c set where t(4F + c) = -1.
__device__ __forceinline__ unsigned dual_chunk_mask(unsigned F, unsigned neg, unsigned c0) {
    const unsigned b = ((unsigned)bitsum_parity(F) ^ (unsigned)__popc(F & (neg >> 2)) ^ c0) & 1u;
    unsigned m = 0u;
#pragma unroll
    for (unsigned c = 0; c < 4u; ++c) m |= ((b ^ (c >> 1) ^ (unsigned)__popc(c & neg & 3u)) & 1u) << c;
    return m;
}

// out.c = src.(3 - c), negated where bit (3 - c) (SRC: the source element's sign) or bit c
// (the destination element's) of m is set
template <bool SRC>
__device__ __forceinline__ float4 dual_chunk(const float4& v, unsigned m) {
    // the mask bit moved to the sign bit and xor-ed in (no compare and select)
    auto sg = [&](float x, unsigned bit) {
        return __uint_as_float(__float_as_uint(x) ^ ((m << (31u - bit)) & 0x80000000u));
    };
    return SRC ? make_float4(sg(v.w, 3), sg(v.z, 2), sg(v.y, 1), sg(v.x, 0))
               : make_float4(sg(v.w, 0), sg(v.z, 1), sg(v.y, 2), sg(v.x, 3));
}

// The wedge product on the same schedule: lane h takes ga[h] over its sup
// steps (partner b[p ^ h], gc block p) and gb[~h] over its sub steps
// (partner a[p], gc block ~h ^ p); both run the disjoint pattern, a gb step
// through s_w(q, o) = s_w(o, q) rho(o) rho(q) rho(o | q) (o, q disjoint, from
// C(|o| + |q|, 2) = C(|o|, 2) + C(|q|, 2) + |o||q|), and no block is read
// reversed.
template <int OP, int N, bool LOWNEG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void prod_bwd_contr_frame(
    const float* __restrict__ A, const float* __restrict__ B, const float* __restrict__ GC, float* __restrict__ GA,
    float* __restrict__ GB, BlkParams P) {
    static_assert(OP == OP_LC || OP == OP_RC || OP == OP_WEDGE || OP == OP_REGR,
                  "contractions, the wedge product and the regressive product only");
    constexpr bool kRg = OP == OP_REGR;  // the wedge schedule on the duals (dual_chunk_mask)
    constexpr int OPW = kRg ? OP_WEDGE : OP;
    constexpr int NH = N - 4, NB = 1 << NH, R = 64 >> NH;
    using Sch = FrameSched<NH>;
    using Cs = ContrSched<NH>;
    using FL = FrameLayout<N>;
    constexpr int T = Sch::T;
    constexpr unsigned full = NB - 1u;
    constexpr bool kW = OPW == OP_WEDGE;
    constexpr bool kLC = OPW != OP_RC;  // sub steps yield gb (lc, wedge) or ga (rc)
    __shared__ __attribute__((aligned(64))) float4 lds[4][3 * kBalGroupF4];  // a | b | gc
    // the steps of lane (h, row slot skew rs): tab[t][rs * NB + h]
    __shared__ unsigned tab[T][4 * NB];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned h = (unsigned)lane & full;
    const int r = lane >> NH;
    const unsigned rs = (unsigned)r & 3u;
    const int first_t = Cs::first_t(h), second_t = Cs::second_t(h);
    const bool first_sub = Cs::first_sub(h);
    // one group of R rows per wave (the host splits batches larger than one grid)
    const long long ngrp = (P.batch + R - 1) / R;
    const long long grp = (long long)blockIdx.x * 4 + wave;
    const BalLane L = bal_lane<FL::kRowX, FL::kSwz>(N, lane);
    const bool gbc = P.ldg4 == 0;
    constexpr unsigned D4 = 1u << (N - 2);
    // regressive: D a, D b and D^T gc, from the complemented chunks
    auto fetch = [&](const float* src, bool bc, int w) {
        const BalSrc sv = bal_src(src, grp, P.batch, N, R, bc);
        BalPre p;
        if constexpr (!kRg) {
            p = bal_fetch(sv, L, N - 2);
        } else {
            const unsigned neg = (P.negh << 4) | P.negl;
            const unsigned c0 = (unsigned)((N * (N - 1) / 2 + __popc(neg)) & 1);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const unsigned row = L.rr[i] < sv.rlim ? L.rr[i] : sv.rlim;
                const unsigned fr = D4 - 1u - L.ff[i];
                const float4 v = sv.g0[(row << (N - 2)) | fr];
                p.v[i] = w < 2 ? dual_chunk<true>(v, dual_chunk_mask(fr, neg, c0))
                               : dual_chunk<false>(v, dual_chunk_mask(L.ff[i], neg, c0));
            }
        }
        return p;
    };
    const BalPre pa = fetch(A, false, 0);
    const BalPre pb = fetch(B, false, 1);
    const BalPre pg = fetch(GC, gbc, 2);
    // entry: gc block offset (o ^ p), partner offset (a at +0, b at +4 KB; slot
    // order reversed in sub mode), then the step's flip bits: pair sign S,
    // parity term Pm, w1 and w2 terms (sub mode), rho (gb steps), gc parity
    // term Gp (gb steps)
    if (wave == 0 && lane < 4 * NB) {
        const unsigned th = (unsigned)lane & full, trs = row_x<FL::kRowX>((unsigned)lane >> NH);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const FrameStep st = frame_step<NH>(th, t);
            const bool gbs = kLC ? st.sub : !st.sub;
            const unsigned podd = (unsigned)__popc(st.p) & 1u, oodd = (unsigned)__popc(st.o) & 1u;
            const unsigned sub = st.sub ? 1u : 0u, gb = gbs ? 1u : 0u;
            unsigned X, wb, pm, cw;
            HiSign hs;
            if (st.idle) {  // reads only: gc block o, partner block p
                X = st.o;
                wb = st.p;
                hs = hi_sign<OP_INNER>(0u, 0u, P.negh, P.nulh, full, P.nm1, P.mu);
                pm = 0u;
                cw = 0u;
            } else if (kW) {  // gb[~o]: (ih, jh) = (p, ~o), gc block p | ~o; ga[o]: (o, p ^ o), gc block p
                X = gbs ? (full ^ st.o ^ st.p) : st.p;
                wb = gbs ? st.p : (st.p ^ st.o);
                hs = gbs ? hi_sign<OP_WEDGE>(st.p, full ^ st.o, P.negh, P.nulh, full, P.nm1, P.mu)
                         : hi_sign<OP_WEDGE>(st.o, st.p ^ st.o, P.negh, P.nulh, full, P.nm1, P.mu);
                pm = gb ? podd : oodd;
                cw = 0u;
            } else {
                X = st.o ^ st.p;
                wb = st.p;
                hs = gbs ? hi_sign<OP_INNER>(st.p, st.o, P.negh, P.nulh, full, P.nm1, P.mu)
                         : hi_sign<OP_INNER>(st.o, st.p, P.negh, P.nulh, full, P.nm1, P.mu);
                pm = (gb ? podd : oodd) ^ (LOWNEG ? sub : 0u);
                cw = sub;
            }
            const unsigned offg = ((X << 2) | (blk_swz<FL::kSwz>(X) ^ trs)) << 4;
            const unsigned offw = (((wb << 2) | (blk_swz<FL::kSwz>(wb) ^ trs ^ (cw ? 3u : 0u))) << 4) + (gbs ? 0u : 4096u);
            tab[t][lane] = offg | (offw << 10) | ((hs.mask >> 31) << 23) | (pm << 24) | ((gb & cw) << 25) |
                           (((gb ^ 1u) & cw) << 26) | (gb << 27) | ((gb & podd) << 28);
        }
    }
    __syncthreads();
    if (grp >= ngrp) return;
    const int tix = (int)(rs * NB + h);
    float4* sa = lds[wave];
    const unsigned base = lds_addr4(sa + (r << (N - 2)));  // the row's a block 0; b at +4 KB, gc at +8 KB
    {
        // a and b in the frame layout: component c of the lane's chunks (block
        // slot fq) goes to component c ^ fq, one dword store each
        const unsigned fq = (unsigned)lane & 3u;
        const unsigned a0 = lds_addr4(sa);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned ad = (a0 + L.so[i]) | (fq << 2);
            const float va[4] = {pa.v[i].x, pa.v[i].y, pa.v[i].z, pa.v[i].w};
            const float vb[4] = {pb.v[i].x, pb.v[i].y, pb.v[i].z, pb.v[i].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const unsigned adc = ad ^ ((unsigned)c << 2);
                *(__attribute__((address_space(3))) float*)(uintptr_t)adc = va[c];
                *(__attribute__((address_space(3))) float*)(uintptr_t)(adc + 4096u) = vb[c];
            }
            lds_st4(a0 + 8192u + L.so[i], pg.v[i]);
        }
    }
    wave_lds_sync();
    // the lane's two output blocks wait in registers (y1: the first mode's,
    // y2: the second's) and leave through LDS in row order after the last step
    float acc[16], y1[16], y2[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        acc[e] = 0.f;
        y1[e] = 0.f;
        y2[e] = 0.f;
    }
    auto step = [&](auto tc) {
        constexpr int t = decltype(tc)::value;
        __builtin_amdgcn_sched_barrier(0);
        unsigned e = tab[t][tix];
        asm volatile("" : "+v"(e));  // decoded per step, not kept for every step across the kernel
        const unsigned g0 = base + 8192u + (e & 1023u);
        const unsigned w0 = base + ((e >> 10) & 8191u);
        unsigned ms = (e << 8) & 0x80000000u, mp = (e << 7) & 0x80000000u, m1 = (e << 6) & 0x80000000u;
        unsigned m2 = (e << 5) & 0x80000000u, mr = (e << 4) & 0x80000000u, mg = (e << 3) & 0x80000000u;
        asm volatile("" : "+v"(ms), "+v"(mp), "+v"(m1), "+v"(m2), "+v"(mr), "+v"(mg));
        float g[16], w[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 vg = lds_ld4(g0 ^ ((unsigned)q << 4));
            const float4 vw = lds_ld4(w0 ^ ((unsigned)q << 4));
            g[4 * q] = vg.x;
            g[4 * q + 1] = vg.y;
            g[4 * q + 2] = vg.z;
            g[4 * q + 3] = vg.w;
            w[4 * q] = vw.x;
            w[4 * q + 1] = vw.y;
            w[4 * q + 2] = vw.z;
            w[4 * q + 3] = vw.w;
        }
        // partner flips by element class: one mask by (parity, rho) with the
        // pair sign, one by (w1, w2), both xor-ed in one three-input op; gc
        // flips by (parity, rho)
        unsigned x1 = ms ^ mp, x2 = ms ^ mr, x3 = x1 ^ mr, y3 = m1 ^ m2, gpr = mg ^ mr;
        asm volatile("" : "+v"(x1), "+v"(x2), "+v"(x3), "+v"(y3), "+v"(gpr));
#pragma unroll
        for (int el = 0; el < 16; ++el) {
            const unsigned xa = par4(el) ? (rho4(el) ? x3 : x1) : (rho4(el) ? x2 : ms);
            const int wcl = w1b(el) + 2 * w2b(el);
            const unsigned u = __float_as_uint(w[fr_reg(el)]);
            w[fr_reg(el)] = __uint_as_float(wcl == 0 ? u ^ xa : u ^ xa ^ (wcl == 1 ? m1 : wcl == 2 ? m2 : y3));
            if (par4(el) || rho4(el)) g[el] = flip(g[el], par4(el) && rho4(el) ? gpr : par4(el) ? mg : mr);
        }
        if constexpr (kW) frame_disjoint(acc, w, g, std::make_integer_sequence<int, 256>{});
        else frame_sup<LOWNEG, true, false>(acc, acc, w, w, g, g, std::make_integer_sequence<int, 256>{});
        if constexpr (Sch::kHelp && t == T - 1) {  // outputs 0 and full add their helpers' sums
#pragma unroll
            for (int el = 0; el < 16; ++el) {
                if constexpr (NH == 3) acc[el] = quad_merge(acc[el]);
                else acc[el] = row16_merge(acc[el], h);
            }
        }
        constexpr int K = Cs::kinds(t);
        if constexpr (K != 0) {
            const bool first = first_t == t, second = second_t == t;
            const bool sub = first == first_sub;  // the mode of the output completed here
            const unsigned m1 = lane_mask(first), m2 = lane_mask(second), msub = lane_mask(sub);
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                // the wedge product's sub-mode output is gb[~h] in the normal frame
                const float ys = kW ? contr_out_sup<true>(acc, k) : contr_out_sub<LOWNEG, kLC>(acc, k);
                const float yp = contr_out_sup<!kLC>(acc, k);
                const float y = K == 1 ? ys : K == 2 ? yp : bsel(msub, ys, yp);
                if constexpr (Cs::any_first(t)) y1[k] = bsel(m1, y, y1[k]);
                if constexpr (Cs::any_second(t)) y2[k] = bsel(m2, y, y2[k]);
            }
            if constexpr (Cs::any_first(t)) {
#pragma unroll
                for (int el = 0; el < 16; ++el) acc[el] = bzero(m1, acc[el]);
            }
        }
        if constexpr (Sch::kHelp && t == T - Sch::C - 1) {  // the helpers start from zero
            const unsigned mz = lane_mask(Sch::helper(h));
#pragma unroll
            for (int el = 0; el < 16; ++el) acc[el] = bzero(mz, acc[el]);
        }
    };
    frame_steps(step, std::make_integer_sequence<int, T>{});
    // ga rows over the staged a, gb rows over b, in the staging layout (block
    // h of row r at slots 4h + (q ^ swz(h) ^ row_x(r)), the kernel's swizzle
    // and row term); then row-order stores
    wave_lds_sync();
    {
        const bool first_gb = first_sub == kLC;  // the first mode's output is a gb block
        const unsigned rowb = lds_addr4(sa) + ((unsigned)r << (N + 2));
        const unsigned o1 = rowb + (first_gb ? 4096u : 0u), o2 = rowb + (first_gb ? 0u : 4096u);
        // output blocks: ga h; gb h (contractions) or ~h (wedge)
        const unsigned b1 = kW && first_gb ? full ^ h : h, b2 = kW && !first_gb ? full ^ h : h;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const unsigned s1 = ((b1 << 2) | ((unsigned)q ^ blk_swz<FL::kSwz>(b1) ^ row_x<FL::kRowX>(rs))) << 4;
            const unsigned s2 = ((b2 << 2) | ((unsigned)q ^ blk_swz<FL::kSwz>(b2) ^ row_x<FL::kRowX>(rs))) << 4;
            lds_st4(o1 + s1, make_float4(y1[4 * q], y1[4 * q + 1], y1[4 * q + 2], y1[4 * q + 3]));
            lds_st4(o2 + s2, make_float4(y2[4 * q], y2[4 * q + 1], y2[4 * q + 2], y2[4 * q + 3]));
        }
    }
    wave_lds_sync();
    {
        const unsigned a0 = lds_addr4(sa);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const long long rr = grp * R + (long long)L.rr[i];
            if (rr < P.batch) {
                const long long at = (rr << (N - 2)) + (long long)L.ff[i];
                if constexpr (kRg) {  // D^T of the wedge gradients: the complemented chunk, dest signs
                    const unsigned neg = (P.negh << 4) | P.negl;
                    const unsigned c0 = (unsigned)((N * (N - 1) / 2 + __popc(neg)) & 1);
                    const unsigned m = dual_chunk_mask(L.ff[i], neg, c0);
                    const unsigned fr = D4 - 1u - L.ff[i], blk = fr >> 2, r4 = L.rr[i];
                    const unsigned so =
                        16u * ((r4 << (N - 2)) + (blk << 2) + ((fr & 3u) ^ blk_swz<FL::kSwz>(blk) ^ row_x<FL::kRowX>(r4)));
                    if (GA) reinterpret_cast<float4*>(GA)[at] = dual_chunk<false>(lds_ld4(a0 + so), m);
                    if (GB) reinterpret_cast<float4*>(GB)[at] = dual_chunk<false>(lds_ld4(a0 + 4096u + so), m);
                } else {
                    if (GA) reinterpret_cast<float4*>(GA)[at] = lds_ld4(a0 + L.so[i]);
                    if (GB) reinterpret_cast<float4*>(GB)[at] = lds_ld4(a0 + 4096u + L.so[i]);
                }
            }
        }
    }
}

// ---- left and right contraction on 5 high bits ------------------------------
// n = 9, and n = 10 whose only null generator is the top one (C5's Cl(9,0,1)).
// With e9 null and rightmost in every blade, a = a0 + a1 e9 and b = b0 + b1 e9
// (halves of 512 floats), the left contraction's pairs with e9 in the
// contracted blade vanish and those with e9 in b only append e9, so
//   c0 = lc9(a0, b0),  c1 = lc9(a0, b1)
//   ga0 = ga9(b0, gc0) + ga9(b1, gc1),  ga1 = 0,  gb0 = gb9(a0, gc0),  gb1 = gb9(a0, gc1)
// with the n = 9 left contraction of e0..e8: two n = 9 problems sharing a0 (a1
// is never read). A wave runs two problems of 32 lanes (two rows at n = 9, the
// two halves at n = 10). The lane schedules (contr5_schedule.h, written by
// gen_contr5_schedule.py) split every output's block pairs into 4-step pieces:
// in the backward, steps 0-7 are ga pairs and 8-15 gb pairs for every lane, so
// each step's sign pattern is fixed at compile time (the blocked kernels'
// arithmetic, no per-lane mode); a lane's pieces are a full output, two small
// outputs, or part of a larger output whose owner lane adds the other parts
// through LDS after the last step. Every lane starts a fresh accumulator at the
// same steps, so no step zeroes conditionally. The pair order inside pieces,
// the slot of each role and the blocks' LDS slot swizzle were searched on the
// CPU against the measured LDS rules (ds_read_b128: per 32-lane half, two sets
// of 16 lanes by the parity of lane bits 2-4, one cycle per distinct address on
// the busiest 16-byte bank group mod 256 bytes; ds_write_b128: 8 consecutive
// lanes per cycle, groups mod 128 bytes), so the block reads and the result
// traffic of a wave run at one cycle per lane set.
// Finished blocks are staged in LDS and leave in row order.

template <unsigned long long SWZ>
__device__ __forceinline__ unsigned swz5(unsigned blk) { return (unsigned)(SWZ >> (2u * blk)) & 3u; }

template <int OP, bool LOWNEG, bool NULLTOP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void prod_bwd_contr5(
    const float* __restrict__ A, const float* __restrict__ B, const float* __restrict__ GC, float* __restrict__ GA,
    float* __restrict__ GB, BlkParams P) {
    static_assert(OP == OP_LC || OP == OP_RC, "contractions only");
    static_assert(!NULLTOP || OP == OP_LC, "the null-top split is the left contraction's");
    constexpr int N = NULLTOP ? 10 : 9;
    constexpr int R = NULLTOP ? 1 : 2;  // rows per wave
    constexpr bool kLC = OP == OP_LC;
    constexpr int V = kLC ? LV_LC : LV_RC;
    constexpr unsigned long long SW = kLC ? kContr5SwzLc : kContr5SwzRc;
    constexpr unsigned full = 31u;
    // per wave (float4): a at 0 (rows 0, 1 of 128; NULLTOP: a0 in row 0), b at 256, gc at 512, zero block at 768
    __shared__ __attribute__((aligned(64))) float4 lds[4][3 * 256 + 4];
    __shared__ unsigned tab[16][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned slot = (unsigned)lane & 31u, prob = (unsigned)lane >> 5;
    const long long ngrp = (P.batch + R - 1) / R;
    // the grid is resident and a wave walks groups grp, grp + 4 * grid, ..., loading the next
    // group's operands into registers while the steps of the current one run, so the waves of a
    // compute unit do not all wait on memory at the same time
    constexpr bool PF = true;
    const long long gstride = PF ? (long long)gridDim.x * 4 : 0;
    long long grp = (long long)blockIdx.x * 4 + wave;
    BalPre pa, pb, pg;
    auto fetch = [&](long long g) {
        unsigned lo = (unsigned)lane;  // opaque: the loop keeps no lane-derived pointers
        asm volatile("" : "+v"(lo));
        const BalLane L = bal_lane(N, (int)lo);
        const BalSrc sa = bal_src(A, g, P.batch, N, R);
        if constexpr (NULLTOP) {  // a0 only: chunks 0, 1 of the row
            pa.v[0] = sa.g0[L.ff[0]];
            pa.v[1] = sa.g0[L.ff[1]];
        } else {
            pa = bal_fetch(sa, L, N - 2);
        }
        pb = bal_fetch(bal_src(B, g, P.batch, N, R), L, N - 2);
        pg = bal_fetch(bal_src(GC, g, P.batch, N, R, P.ldg4 == 0), L, N - 2);
    };
    fetch(grp < ngrp ? grp : ngrp - 1);
    // step entries: partner byte offset (bits 0-13), gc byte offset (14-27), the pair's high
    // sign (28) and the cross parity of the odd partner elements (29): |o| for ga, |p| for gb
    if (wave == 0) {
        for (int t = 0; t < 16; ++t) {
            const unsigned st = kLC ? kContr5StepsLc[slot][t] : kContr5StepsRc[slot][t];
            unsigned e;
            if (st & 2048u) {  // idle: the zero block for both reads
                e = (768u << 4) | (768u << 18);
            } else {
                const unsigned o = st & 31u, p = (st >> 5) & 31u, x = o ^ p;
                const bool ga = t < 8;
                const HiSign hs = ga ? hi_sign<OP>(o, p, P.negh, 0u, full, 0, 0) : hi_sign<OP>(p, o, P.negh, 0u, full, 0, 0);
                const unsigned par = (unsigned)__popc(ga ? o : p) & 1u;
                const unsigned prow = (NULLTOP && !ga) ? 0u : prob;  // gb partners: a (NULLTOP: a0, row 0)
                const unsigned pw = (ga ? 256u : 0u) + prow * 128u + ((p << 2) | swz5<SW>(p));
                const unsigned pg4 = 512u + prob * 128u + ((x << 2) | swz5<SW>(x));
                e = (pw << 4) | (pg4 << 18) | ((hs.mask >> 31) << 28) | (par << 29);
            }
            tab[t][lane] = e;
        }
    }
    __syncthreads();
    if (grp >= ngrp) return;
    float4* sw = lds[wave];
    const unsigned base = lds_addr4(sw);
    if (lane < 4) lds_st4(base + 16u * (768u + (unsigned)lane), make_float4(0.f, 0.f, 0.f, 0.f));
    for (;;) {
    // lane and base as opaque copies: every address of the body is formed inside the loop
    // instead of being kept in registers across it
    unsigned lane_o = (unsigned)lane, base_o = base;
    asm volatile("" : "+v"(lane_o), "+v"(base_o) :: "memory");
    {
    const int lane = (int)lane_o;
    const unsigned base = base_o, slot = lane_o & 31u, prob = lane_o >> 5;
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // slot q of block blk at (blk << 2) | (q ^ swz(blk))
        const unsigned c = (unsigned)lane + 64u * (unsigned)i;
        const unsigned hr = c >> 7, f = c & 127u, blk = f >> 2;
        const unsigned so = 16u * (hr * 128u + ((blk << 2) | ((f & 3u) ^ swz5<SW>(blk))));
        if (!NULLTOP || i < 2) lds_st4(base + so, pa.v[i]);
        lds_st4(base + 4096u + so, pb.v[i]);
        lds_st4(base + 8192u + so, pg.v[i]);
    }
    wave_lds_sync();
    const long long nxt = grp + gstride;
    if (PF && nxt < ngrp) fetch(nxt);
    float acc[16], y1[16], y2[16], y3[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    auto step = [&](auto tc) {
        constexpr int t = decltype(tc)::value;
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");  // the step's block reads stay in the step
        unsigned e = tab[t][lane];
        asm volatile("" : "+v"(e));
        const unsigned w0 = base + (e & 16383u);
        const unsigned g0 = base + ((e >> 14) & 16383u);
        const unsigned ms = (e << 3) & 0x80000000u, mq = (e << 2) & 0x80000000u;
        float g[16], w[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 vg = lds_ld4(g0 ^ ((unsigned)q << 4));
            const float4 vw = lds_ld4(w0 ^ ((unsigned)q << 4));
            g[4 * q] = vg.x;
            g[4 * q + 1] = vg.y;
            g[4 * q + 2] = vg.z;
            g[4 * q + 3] = vg.w;
            w[4 * q] = vw.x;
            w[4 * q + 1] = vw.y;
            w[4 * q + 2] = vw.z;
            w[4 * q + 3] = vw.w;
        }
        apply_flips(w, ms, ms ^ mq);
        if constexpr (t < 8) {
            lowblock_ga<V, LOWNEG>(acc, w, g);
        } else {
#pragma unroll
            for (int el = 0; el < 16; ++el)
                if (cpopc((unsigned)el) & 1) g[el] = flip(g[el], mq);
            lowblock_gb<V, LOWNEG>(acc, w, g);
        }
#pragma unroll
        for (int el = 0; el < 16; ++el) asm volatile("" : "+v"(acc[el]));  // the step's FMAs end here
        if constexpr ((t & 3) == 3 && t < 15) {  // a piece ends: keep it, start from zero
#pragma unroll
            for (int el = 0; el < 16; ++el) {
                if constexpr (t == 3) y1[el] = acc[el];
                else if constexpr (t == 7) y2[el] = acc[el];
                else y3[el] = acc[el];
                acc[el] = 0.f;
            }
        }
    };
    frame_steps(step, std::make_integer_sequence<int, 16>{});
    // pieces: y1, y2 (ga), y3, acc (gb)
    wave_lds_sync();  // every block read of the wave is done: its LDS takes the results
    const unsigned dA = kLC ? kContr5OutLc[slot][0] : kContr5OutRc[slot][0];
    const unsigned dB = kLC ? kContr5OutLc[slot][1] : kContr5OutRc[slot][1];
    const unsigned part = base + 16u * (512u + prob * 128u);  // 16 partial slots of 4 float4, over the gc rows
    float sA[16], sB[16];
#pragma unroll
    for (int el = 0; el < 16; ++el) {
        sA[el] = y1[el] + y2[el];
        sB[el] = y3[el] + acc[el];
    }
    auto st16 = [&](unsigned a, const float (&x)[16]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) lds_st4(a + 16u * (unsigned)q, make_float4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]));
    };
    auto add16 = [&](unsigned a, float (&x)[16]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = lds_ld4(a + 16u * (unsigned)q);
            x[4 * q] += v.x;
            x[4 * q + 1] += v.y;
            x[4 * q + 2] += v.z;
            x[4 * q + 3] += v.w;
        }
    };
    if ((dA & 3u) == 2u) st16(part + 64u * ((dA >> 12) & 15u), sA);  // helpers' partials
    if ((dB & 3u) == 2u) st16(part + 64u * ((dB >> 12) & 15u), sB);
    wave_lds_sync();
    if ((dA & 3u) == 3u) {  // owners add them, in slot order
        const unsigned p0 = (dA >> 12) & 15u, cnt = (dA >> 16) & 3u;
        for (unsigned k = 0; k < cnt; ++k) add16(part + 64u * (p0 + k), sA);
    }
    if ((dB & 3u) == 3u) {
        const unsigned p0 = (dB >> 12) & 15u, cnt = (dB >> 16) & 3u;
        for (unsigned k = 0; k < cnt; ++k) add16(part + 64u * (p0 + k), sB);
    }
    // results into the staging rows (over the dead inputs): ga over a, gb over b, row = problem
    auto put = [&](unsigned region, unsigned blk, const float (&x)[16]) {
        const unsigned rowb = base + 16u * (region + prob * 128u);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            lds_st4(rowb + 16u * ((blk << 2) | ((unsigned)q ^ swz5<SW>(blk))),
                    make_float4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]));
    };
    {
        const unsigned tA = dA & 3u, tB = dB & 3u;
        if (tA == 1u) {
            put(0u, (dA >> 2) & 31u, y1);
            put(0u, (dA >> 7) & 31u, y2);
        } else if (tA != 2u) {
            put(0u, (dA >> 2) & 31u, sA);
        }
        if (tB == 1u) {
            put(256u, (dB >> 2) & 31u, y3);
            put(256u, (dB >> 7) & 31u, acc);
        } else if (tB != 2u) {
            put(256u, (dB >> 2) & 31u, sB);
        }
    }
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned c = (unsigned)lane + 64u * (unsigned)i;
        const unsigned hr = c >> 7, f = c & 127u, blk = f >> 2;
        const unsigned so = 16u * (hr * 128u + ((blk << 2) | ((f & 3u) ^ swz5<SW>(blk))));
        if constexpr (NULLTOP) {
            const long long at = (grp << 8) + (long long)c;  // float4 of the row: half hr, float4 f
            if (GA) {
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                if (hr == 0u) {  // ga0 = the two problems' ga
                    const float4 p0 = lds_ld4(base + so), p1 = lds_ld4(base + 2048u + so);
                    v = make_float4(p0.x + p1.x, p0.y + p1.y, p0.z + p1.z, p0.w + p1.w);
                }
                reinterpret_cast<float4*>(GA)[at] = v;
            }
            if (GB) reinterpret_cast<float4*>(GB)[at] = lds_ld4(base + 4096u + so);
        } else {
            const long long row = grp * 2 + (long long)hr;
            if (row < P.batch) {
                const long long at = (row << 7) + (long long)f;
                if (GA) reinterpret_cast<float4*>(GA)[at] = lds_ld4(base + so);
                if (GB) reinterpret_cast<float4*>(GB)[at] = lds_ld4(base + 4096u + so);
            }
        }
    }
    if (!PF || nxt >= ngrp) break;
    grp = nxt;
    wave_lds_sync();  // the result reads are done before the next group's staging
    }
    }
}

// ---- inner product backward on the contraction schedules ------------------
// The inner product's block pairs are the left contraction's (ih inside jh)
// and the right contraction's (jh inside ih); the (o, o) pairs belong to both,
// and so does their element diagonal (il = jl), which the two low patterns
// would count twice. prod_bwd_inner5 runs the lc and the rc lane schedules of
// prod_bwd_contr5 (their searched layouts for one shared block swizzle,
// kContr5In*) one after the other on the same staged rows: four sub-phases
// of 8 steps (lc ga, rc ga, lc gb, rc gb), each with its compile-time low
// pattern, each flushed into result rows in LDS by its owners (helpers'
// partials first), then the element diagonal taken off once:
//   ga[i] -= F(i) b[i] gc[0],  gb[i] -= F(i) a[i] gc[0],
//   F((o, il)) = s_hi(o, o) (-1)^{|il| |o|} s_lo(il, il).
// n = 9: two rows per wave, one problem each. n = 10 whose only null
// generator is the top one: with a = a0 + a1 e9, b = b0 + b1 e9 the pairs with
// e9 in both vanish and moving e9 past a blade of b gives (-1)^{|j|} (beta,
// the grade involution), so c0 = inner9(a0, b0), c1 = lc9(a0, b1) +
// rc9(a1, beta b0):
//   ga0 = inner9_ga(b0, gc0) + lc9_ga(b1, gc1),  ga1 = rc9_ga(beta b0, gc1),
//   gb0 = inner9_gb(a0, gc0) + beta rc9_gb(a1, gc1),  gb1 = lc9_gb(a0, gc1);
// problem 0 (lanes 0-31) is the inner9 problem, problem 1 runs the lc
// sub-phases on (a0, b1, gc1) and the rc ones on (a1, beta b0, gc1), beta
// folded into the step signs (rc ga) and into the flush (rc gb).
template <bool LOWNEG, bool NULLTOP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void prod_bwd_inner5(
    const float* __restrict__ A, const float* __restrict__ B, const float* __restrict__ GC, float* __restrict__ GA,
    float* __restrict__ GB, BlkParams P) {
    constexpr int N = NULLTOP ? 10 : 9;
    constexpr int R = NULLTOP ? 1 : 2;
    constexpr unsigned long long SW = kContr5InSwz;
    constexpr unsigned full = 31u;
    // per wave (float4): a at 0 (rows 0, 1 or halves a0, a1), b at 256, gc at 512, the zero block at
    // 768, partial slots at 772 (8 slots of 4 float4 per problem), ga rows at 836; the gb rows go
    // over b once the ga sub-phases are done
    constexpr unsigned kZero = 768u, kPart = 772u, kGa = 836u, kGb = 256u;
    __shared__ __attribute__((aligned(64))) float4 lds[4][1092];
    __shared__ unsigned tab[32][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const long long ngrp = (P.batch + R - 1) / R;
    // resident grid: a wave walks groups grp, grp + 4 * grid, ..., loading the next group's
    // operands into registers while the current group's steps run
    const long long gstride = (long long)gridDim.x * 4;
    long long grp = (long long)blockIdx.x * 4 + wave;
    BalPre pa, pb, pg;
    auto fetch = [&](long long g) {
        unsigned lo = (unsigned)lane;  // opaque: the loop keeps no lane-derived pointers
        asm volatile("" : "+v"(lo));
        const BalLane L = bal_lane(N, (int)lo);
        pa = bal_fetch(bal_src(A, g, P.batch, N, R), L, N - 2);
        pb = bal_fetch(bal_src(B, g, P.batch, N, R), L, N - 2);
        pg = bal_fetch(bal_src(GC, g, P.batch, N, R, P.ldg4 == 0), L, N - 2);
    };
    fetch(grp < ngrp ? grp : ngrp - 1);
    // step entries of sub-phase u (0 lc ga, 1 rc ga, 2 lc gb, 3 rc gb) at tab[8 u + t]: partner
    // byte offset (bits 0-13), gc byte offset (14-27), high sign (28), cross parity (29)
    if (wave == 0) {
        const unsigned slot = (unsigned)lane & 31u, prob = (unsigned)lane >> 5;
        for (int u = 0; u < 4; ++u) {
            const bool lcr = (u & 1) == 0, ga = u < 2;
            for (int t = 0; t < 8; ++t) {
                const int tt = t + (ga ? 0 : 8);
                const unsigned st = lcr ? kContr5InStepsLc[slot][tt] : kContr5InStepsRc[slot][tt];
                unsigned e;
                if (st & 2048u) {
                    e = (kZero << 4) | (kZero << 18);
                } else {
                    const unsigned o = st & 31u, p = (st >> 5) & 31u, x = o ^ p;
                    const HiSign hs = ga ? (lcr ? hi_sign<OP_LC>(o, p, P.negh, 0u, full, 0, 0)
                                                : hi_sign<OP_RC>(o, p, P.negh, 0u, full, 0, 0))
                                         : (lcr ? hi_sign<OP_LC>(p, o, P.negh, 0u, full, 0, 0)
                                                : hi_sign<OP_RC>(p, o, P.negh, 0u, full, 0, 0));
                    unsigned hsb = hs.mask >> 31, par = (unsigned)__popc(ga ? o : p) & 1u;
                    // null-top: rc ga of problem 1 reads b0 (beta b0), lc gb of both problems reads a0
                    const bool row0 = NULLTOP && ((u == 1) || (u == 2));
                    const unsigned prow = row0 ? 0u : prob;
                    if (NULLTOP && u == 1 && prob == 1u) {  // beta b0: (-1)^{|p| + |jl|}
                        hsb ^= (unsigned)__popc(p) & 1u;
                        par ^= 1u;
                    }
                    const unsigned pw = (ga ? 256u : 0u) + prow * 128u + ((p << 2) | swz5<SW>(p));
                    const unsigned pg4 = 512u + prob * 128u + ((x << 2) | swz5<SW>(x));
                    e = (pw << 4) | (pg4 << 18) | (hsb << 28) | (par << 29);
                }
                tab[8 * u + t][lane] = e;
            }
        }
    }
    __syncthreads();
    if (grp >= ngrp) return;
    float4* sw = lds[wave];
    const unsigned base = lds_addr4(sw);
    if (lane < 4) lds_st4(base + 16u * (kZero + (unsigned)lane), make_float4(0.f, 0.f, 0.f, 0.f));
    for (;;) {
    // lane and base as opaque copies: every address of the body is formed inside the loop
    unsigned lane_o = (unsigned)lane, base_o = base;
    asm volatile("" : "+v"(lane_o), "+v"(base_o) :: "memory");
    {
    const int lane = (int)lane_o;
    const unsigned base = base_o, slot = lane_o & 31u, prob = lane_o >> 5;
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // slot q of block blk at (blk << 2) | (q ^ swz(blk))
        const unsigned c = (unsigned)lane + 64u * (unsigned)i;
        const unsigned hr = c >> 7, f = c & 127u, blk = f >> 2;
        const unsigned so = 16u * (hr * 128u + ((blk << 2) | ((f & 3u) ^ swz5<SW>(blk))));
        lds_st4(base + so, pa.v[i]);
        lds_st4(base + 4096u + so, pb.v[i]);
        lds_st4(base + 8192u + so, pg.v[i]);
    }
    wave_lds_sync();
    const long long nxt = grp + gstride;
    if (nxt < ngrp) fetch(nxt);
    auto st16 = [&](unsigned a, const float (&x)[16]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) lds_st4(a + 16u * (unsigned)q, make_float4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]));
    };
    auto add16 = [&](unsigned a, float (&x)[16]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = lds_ld4(a + 16u * (unsigned)q);
            x[4 * q] += v.x;
            x[4 * q + 1] += v.y;
            x[4 * q + 2] += v.z;
            x[4 * q + 3] += v.w;
        }
    };
    // block blk of the result row at rowb (slots swizzled as the staged rows) = x (put) or += x
    auto addblk = [&](unsigned rowb, unsigned blk, const float (&x)[16], bool put) {
        const unsigned s0 = swz5<SW>(blk);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const unsigned at = rowb + 16u * ((blk << 2) | ((unsigned)q ^ s0));
            if (put) {
                lds_st4(at, make_float4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]));
            } else {
                const float4 v = lds_ld4(at);
                lds_st4(at, make_float4(v.x + x[4 * q], v.y + x[4 * q + 1], v.z + x[4 * q + 2], v.w + x[4 * q + 3]));
            }
        }
    };
    auto subphase = [&](auto uc) {
        constexpr int U = decltype(uc)::value;
        constexpr bool kL = (U & 1) == 0, kGA = U < 2;
        constexpr int V = kL ? LV_LC : LV_RC;
        float acc[16], y1[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.f;
        auto step = [&](auto tc) {
            constexpr int t = decltype(tc)::value;
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("" ::: "memory");  // the step's block reads stay in the step
            unsigned e = tab[8 * U + t][lane];
            asm volatile("" : "+v"(e));
            const unsigned w0 = base + (e & 16383u);
            const unsigned g0 = base + ((e >> 14) & 16383u);
            const unsigned ms = (e << 3) & 0x80000000u, mq = (e << 2) & 0x80000000u;
            float g[16], w[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 vg = lds_ld4(g0 ^ ((unsigned)q << 4));
                const float4 vw = lds_ld4(w0 ^ ((unsigned)q << 4));
                g[4 * q] = vg.x;
                g[4 * q + 1] = vg.y;
                g[4 * q + 2] = vg.z;
                g[4 * q + 3] = vg.w;
                w[4 * q] = vw.x;
                w[4 * q + 1] = vw.y;
                w[4 * q + 2] = vw.z;
                w[4 * q + 3] = vw.w;
            }
            apply_flips(w, ms, ms ^ mq);
            if constexpr (kGA) {
                lowblock_ga<V, LOWNEG>(acc, w, g);
            } else {
#pragma unroll
                for (int el = 0; el < 16; ++el)
                    if (cpopc((unsigned)el) & 1) g[el] = flip(g[el], mq);
                lowblock_gb<V, LOWNEG>(acc, w, g);
            }
#pragma unroll
            for (int el = 0; el < 16; ++el) asm volatile("" : "+v"(acc[el]));  // the step's FMAs end here
            if constexpr (t == 3) {  // the first piece ends
#pragma unroll
                for (int el = 0; el < 16; ++el) {
                    y1[el] = acc[el];
                    acc[el] = 0.f;
                }
            }
        };
        frame_steps(step, std::make_integer_sequence<int, 8>{});
        wave_lds_sync();  // every block read of the sub-phase is done
        const unsigned d = kL ? kContr5InOutLc[slot][U >> 1] : kContr5InOutRc[slot][U >> 1];
        const unsigned typ = d & 3u;
        const unsigned part = base + 16u * (kPart + prob * 32u);
        float sv[16];
#pragma unroll
        for (int el = 0; el < 16; ++el) sv[el] = y1[el] + acc[el];
        if (typ == 2u) st16(part + 64u * ((d >> 12) & 7u), sv);  // helpers' partials
        wave_lds_sync();
        if (typ == 3u) {  // owners add them, in slot order
            const unsigned p0 = (d >> 12) & 7u, cnt = (d >> 16) & 3u;
            for (unsigned k = 0; k < cnt; ++k) add16(part + 64u * (p0 + k), sv);
        }
        // the row this problem's results of the sub-phase go to (NULLTOP: lc ga of both problems
        // into ga0, rc gb of both into gb0)
        constexpr bool kShared = NULLTOP && (U == 0 || U == 3);
        const unsigned rowb = base + 16u * ((kGA ? kGa : kGb) + (kShared ? 0u : prob * 128u));
        const unsigned b1 = (d >> 2) & 31u, b2 = (d >> 7) & 31u;
        if constexpr (NULLTOP && U == 3) {  // problem 1: beta rc9_gb(a1, gc1), (-1)^{|o| + |el|}
            const unsigned on = prob == 1u ? 0x80000000u : 0u;
            const unsigned m1 = (((unsigned)__popc(b1) & 1u) << 31) & on, m2 = (((unsigned)__popc(b2) & 1u) << 31) & on;
            apply_flips(y1, m1, m1 ^ on);
            apply_flips(acc, m2, m2 ^ on);
            apply_flips(sv, m1, m1 ^ on);
        }
        // the first contribution to a row block is stored, the later ones added: lc ga puts ga
        // (NULLTOP: problem 0 into ga0, problem 1 adds), rc ga adds (NULLTOP problem 1 puts ga1),
        // lc gb puts, rc gb adds
        const bool put = U == 2 || (U == 0 && (!NULLTOP || prob == 0u)) || (U == 1 && NULLTOP && prob == 1u);
#pragma unroll
        for (unsigned r = 0; r < (kShared ? 2u : 1u); ++r) {  // kShared: problem 0, then problem 1
            if (!kShared || prob == r) {
                if (typ == 1u) {
                    addblk(rowb, b1, y1, put);
                    addblk(rowb, b2, acc, put);
                } else if (typ != 2u) {
                    addblk(rowb, b1, sv, put);
                }
            }
            if (kShared && r == 0u) wave_lds_sync();
        }
        if constexpr (U == 1 || U == 3) {
            // the element diagonal, once: lane slot o takes block o of its problem's row (the
            // inner9 problems: both rows at n = 9, problem 0 at n = 10)
            wave_lds_sync();
            if (!NULLTOP || prob == 0u) {
                const unsigned o = slot;
                const unsigned src = base + 16u * ((kGA ? 256u : 0u) + prob * 128u);  // b (ga) or a (gb)
                const float gc0 = lds_ld4(base + 16u * (512u + prob * 128u + (0u ^ swz5<SW>(0u)))).x;
                const unsigned mh = hi_sign<OP_LC>(o, o, P.negh, 0u, full, 0, 0).mask;
                const unsigned mo = ((unsigned)__popc(o) & 1u) << 31;
                float x[16], corr[16];
                const unsigned s0 = swz5<SW>(o);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 v = lds_ld4(src + 16u * ((o << 2) | ((unsigned)q ^ s0)));
                    x[4 * q] = v.x;
                    x[4 * q + 1] = v.y;
                    x[4 * q + 2] = v.z;
                    x[4 * q + 3] = v.w;
                }
#pragma unroll
                for (int el = 0; el < 16; ++el) {
                    const bool lo_neg = low_sign(LV_LC, LOWNEG, (unsigned)el, (unsigned)el) < 0;
                    const unsigned m = mh ^ ((cpopc((unsigned)el) & 1) ? mo : 0u) ^ (lo_neg ? 0x80000000u : 0u);
                    corr[el] = flip(x[el], m) * -gc0;
                }
                addblk(base + 16u * ((kGA ? kGa : kGb) + prob * 128u), o, corr, false);
            }
        }
    };
    subphase(std::integral_constant<int, 0>{});
    subphase(std::integral_constant<int, 1>{});
    subphase(std::integral_constant<int, 2>{});
    subphase(std::integral_constant<int, 3>{});
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned c = (unsigned)lane + 64u * (unsigned)i;
        const unsigned hr = c >> 7, f = c & 127u, blk = f >> 2;
        const unsigned so = 16u * (hr * 128u + ((blk << 2) | ((f & 3u) ^ swz5<SW>(blk))));
        if constexpr (NULLTOP) {
            const long long at = (grp << 8) + (long long)c;
            if (GA) reinterpret_cast<float4*>(GA)[at] = lds_ld4(base + 16u * kGa + so);
            if (GB) reinterpret_cast<float4*>(GB)[at] = lds_ld4(base + 16u * kGb + so);
        } else {
            const long long row = grp * 2 + (long long)hr;
            if (row < P.batch) {
                const long long at = (row << 7) + (long long)f;
                if (GA) reinterpret_cast<float4*>(GA)[at] = lds_ld4(base + 16u * kGa + so);
                if (GB) reinterpret_cast<float4*>(GB)[at] = lds_ld4(base + 16u * kGb + so);
            }
        }
    }
    if (nxt >= ngrp) break;
    grp = nxt;
    wave_lds_sync();  // the result reads are done before the next group's staging
    }
    }
}

// Forward: lane slot s walks 8 pairs of kContr5Fwd in two pieces, (a[S], b[S | o])
// for lc and (a[S | o], b[S]) for rc; the owner of an output adds the helper
// chunks of its list; the lane's own block leaves through LDS in row order.
template <int OP, bool LOWNEG, bool NULLTOP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void prod_fwd_contr5(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, BlkParams P) {
    static_assert(OP == OP_LC || OP == OP_RC, "contractions only");
    static_assert(!NULLTOP || OP == OP_LC, "the null-top split is the left contraction's");
    constexpr int N = NULLTOP ? 10 : 9;
    constexpr int R = NULLTOP ? 1 : 2;
    constexpr bool kLC = OP == OP_LC;
    constexpr int V = kLC ? LV_LC : LV_RC;
    constexpr unsigned long long SW = kContr5FwdSwz;
    constexpr unsigned full = 31u;
    // per wave (float4): a at 0 (rows 0, 1; NULLTOP: a0 in row 0), b at 256, zero block at 512
    __shared__ __attribute__((aligned(64))) float4 lds[4][2 * 256 + 4];
    __shared__ unsigned tab[8][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned slot = (unsigned)lane & 31u, prob = (unsigned)lane >> 5;
    const long long ngrp = (P.batch + R - 1) / R;
    // resident grid: a wave walks groups grp, grp + 4 * grid, ..., loading the next group's
    // operands into registers while the steps of the current one run
    const long long gstride = (long long)gridDim.x * 4;
    long long grp = (long long)blockIdx.x * 4 + wave;
    BalPre pa, pb;
    auto fetch = [&](long long g) {
        unsigned lo = (unsigned)lane;  // opaque: the loop keeps no lane-derived addresses
        asm volatile("" : "+v"(lo));
        const BalLane L = bal_lane(N, (int)lo);
        const BalSrc sa = bal_src(A, g, P.batch, N, R);
        if constexpr (NULLTOP) {
            pa.v[0] = sa.g0[L.ff[0]];
            pa.v[1] = sa.g0[L.ff[1]];
        } else {
            pa = bal_fetch(sa, L, N - 2);
        }
        pb = bal_fetch(bal_src(B, g, P.batch, N, R), L, N - 2);
    };
    fetch(grp < ngrp ? grp : ngrp - 1);
    // entries: a byte offset (bits 0-13), b byte offset (14-27), high sign (28), cross parity |ih| (29)
    if (wave == 0) {
        for (int t = 0; t < 8; ++t) {
            const unsigned st = kContr5Fwd[slot][t];
            unsigned e;
            if (st & 2048u) {
                e = (512u << 4) | (512u << 18);
            } else {
                const unsigned o = st & 31u, S = (st >> 5) & 31u;
                const unsigned ih = kLC ? S : (S | o), jh = kLC ? (S | o) : S;
                const HiSign hs = hi_sign<OP>(ih, jh, P.negh, 0u, full, 0, 0);
                const unsigned arow = NULLTOP ? 0u : prob;
                const unsigned pa4 = arow * 128u + ((ih << 2) | swz5<SW>(ih));
                const unsigned pb4 = 256u + prob * 128u + ((jh << 2) | swz5<SW>(jh));
                e = (pa4 << 4) | (pb4 << 18) | ((hs.mask >> 31) << 28) | (((unsigned)__popc(ih) & 1u) << 29);
            }
            tab[t][lane] = e;
        }
    }
    __syncthreads();
    if (grp >= ngrp) return;
    float4* sw = lds[wave];
    const unsigned base = lds_addr4(sw);
    if (lane < 4) lds_st4(base + 16u * (512u + (unsigned)lane), make_float4(0.f, 0.f, 0.f, 0.f));
    for (;;) {
    // lane and base as opaque copies: every address of the body is formed inside the loop
    // instead of being kept in registers across it
    unsigned lane_o = (unsigned)lane, base_o = base;
    asm volatile("" : "+v"(lane_o), "+v"(base_o) :: "memory");
    {
    const int lane = (int)lane_o;
    const unsigned base = base_o, slot = lane_o & 31u, prob = lane_o >> 5;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned c = (unsigned)lane + 64u * (unsigned)i;
        const unsigned hr = c >> 7, f = c & 127u, blk = f >> 2;
        const unsigned so = 16u * (hr * 128u + ((blk << 2) | ((f & 3u) ^ swz5<SW>(blk))));
        if (!NULLTOP || i < 2) lds_st4(base + so, pa.v[i]);
        lds_st4(base + 4096u + so, pb.v[i]);
    }
    wave_lds_sync();
    const long long nxt = grp + gstride;
    if (nxt < ngrp) fetch(nxt);
    float acc[16], y1[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    auto step = [&](auto tc) {
        constexpr int t = decltype(tc)::value;
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");  // the step's block reads stay in the step
        unsigned e = tab[t][lane];
        asm volatile("" : "+v"(e));
        const unsigned a0 = base + (e & 16383u);
        const unsigned b0 = base + ((e >> 14) & 16383u);
        const unsigned ms = (e << 3) & 0x80000000u, mq = (e << 2) & 0x80000000u;
        float av[16], bv[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 va = lds_ld4(a0 ^ ((unsigned)q << 4));
            const float4 vb = lds_ld4(b0 ^ ((unsigned)q << 4));
            av[4 * q] = va.x;
            av[4 * q + 1] = va.y;
            av[4 * q + 2] = va.z;
            av[4 * q + 3] = va.w;
            bv[4 * q] = vb.x;
            bv[4 * q + 1] = vb.y;
            bv[4 * q + 2] = vb.z;
            bv[4 * q + 3] = vb.w;
        }
        apply_flips(bv, ms, ms ^ mq);
        lowblock_fwd<V, LOWNEG>(acc, av, bv);
#pragma unroll
        for (int el = 0; el < 16; ++el) asm volatile("" : "+v"(acc[el]));  // the step's FMAs end here
        if constexpr (t == 3) {
#pragma unroll
            for (int el = 0; el < 16; ++el) {
                y1[el] = acc[el];
                acc[el] = 0.f;
            }
        }
    };
    frame_steps(step, std::make_integer_sequence<int, 8>{});
    wave_lds_sync();
    const unsigned d = kContr5FwdOut[slot];
    const unsigned chunks = base + 16u * (256u + prob * 128u);  // 16 chunk slots of 4 float4, over the b rows
    const int cw = (int)(d >> 13) - 1;
    // float4 q of chunk slot c at 4 c + (q ^ ((c >> 1) & 3)): the helpers of a write set and the
    // owners of a read set whose chunks share bank groups differ in the swizzle
    if (cw >= 0) {
        const unsigned cx = ((unsigned)cw >> 1) & 3u;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            lds_st4(chunks + 64u * (unsigned)cw + 16u * ((unsigned)q ^ cx),
                    make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]));
    }
    wave_lds_sync();
    float u[16];
    const bool both = (d >> 5) & 1u;
#pragma unroll
    for (int el = 0; el < 16; ++el) u[el] = both ? y1[el] + acc[el] : y1[el];
    {
        const unsigned c0 = (d >> 6) & 15u, cnt = (d >> 10) & 7u;
        for (unsigned k = 0; k < cnt; ++k) {
            const unsigned cx = ((c0 + k) >> 1) & 3u;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 v = lds_ld4(chunks + 64u * (c0 + k) + 16u * ((unsigned)q ^ cx));
                u[4 * q] += v.x;
                u[4 * q + 1] += v.y;
                u[4 * q + 2] += v.z;
                u[4 * q + 3] += v.w;
            }
        }
    }
    {
        const unsigned blk = d & 31u;
        const unsigned rowb = base + 16u * (prob * 128u);  // over a
#pragma unroll
        for (int q = 0; q < 4; ++q)
            lds_st4(rowb + 16u * ((blk << 2) | ((unsigned)q ^ swz5<SW>(blk))),
                    make_float4(u[4 * q], u[4 * q + 1], u[4 * q + 2], u[4 * q + 3]));
    }
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned c = (unsigned)lane + 64u * (unsigned)i;
        const unsigned hr = c >> 7, f = c & 127u, blk = f >> 2;
        const unsigned so = 16u * (hr * 128u + ((blk << 2) | ((f & 3u) ^ swz5<SW>(blk))));
        if constexpr (NULLTOP) {
            reinterpret_cast<float4*>(C)[(grp << 8) + (long long)c] = lds_ld4(base + so);
        } else {
            const long long row = grp * 2 + (long long)hr;
            if (row < P.batch) reinterpret_cast<float4*>(C)[(row << 7) + (long long)f] = lds_ld4(base + so);
        }
    }
    if (nxt >= ngrp) break;
    grp = nxt;
    wave_lds_sync();  // the result reads are done before the next group's staging
    }
    }
}

// ---- inner, lc and rc forward at n = 7: one lane per output block ---------
// Output block o of a row takes, for every partner S inside ~o, the lc half
// (a[S], b[S | o], il inside jl) and the rc half (a[S | o], b[S], jl inside
// il) of the fused round, so every lane runs the same two patterns at every
// step; for o = 0 both halves are (a[S], b[S]) and the diagonal il = jl,
// counted twice, is taken off the scalar once. The left contraction is the
// lc half alone and the right contraction the rc half alone (the pairs
// (S, S | o) and (S | o, S) are exactly their block pairs), with the same
// schedule and no diagonal correction. Output o has 2^(3 - |o|) partners (27
// per row), so eight lanes cover a row in four steps when the lanes of
// outputs 3 and 7, done after step 1, take four of output 0's eight: lanes
// 3, 5, 6 finish their outputs in steps 0 and 1, lane 7 in step 0 (idle in
// step 1), lanes 3 and 7 then run two o = 0 pairs each, and output 0 adds
// lane 3's sum (quad DPP) and lane 7's (row shift by 7).
// Byte h of kFwd7Sched[t] is lane h's pair (o << 3 | p) at step t, or 0x80 |
// S << 3 | So for an idle step (the blocks read, result discarded); the
// constants keep the lookup in registers (no memory load before the table). The step orders,
// the idle reads and the row term of the LDS slots (kFwd7RowX: rows 0..3 ->
// 3, 0, 2, 1) were searched together so that, under the measured b128 read
// rule, the 16 lanes of each bank set read one address per 16-byte bank group
// at every step of all five ops (inner, lc, rc, wedge, regressive), and the
// row-order output stores stay conflict-free.
constexpr unsigned kFwd7RowX = 0x63u;
constexpr unsigned long long kFwd7Sched[4] = {0x38312a2018100a00ull, 0xb73028231c140e01ull, 0x04a5b32106110803ull, 0x07afa02205150c02ull};

// acc[0] += fac * sum_l s_lo(l, l) a[l] b[l] (the diagonal of an o = 0 pair)
template <bool LOWNEG, int... L>
__device__ __forceinline__ void fwd7_diag(float (&acc)[16], const float (&a)[16], const float (&b)[16], float fac,
                                          std::integer_sequence<int, L...>) {
    float e = 0.f;
    ((e = low_sign(LV_LC, LOWNEG, (unsigned)L, (unsigned)L) > 0 ? __builtin_fmaf(a[L], b[L], e)
                                                                 : __builtin_fmaf(-a[L], b[L], e)),
     ...);
    acc[0] = __builtin_fmaf(fac, e, acc[0]);
}

// x + x[lane 3 of the quad] + x[lane + 7 of the DPP row], the sum wanted on
// lane 0 of each row of eight (other lanes get other sums); s_nop as in
// quad_merge
__device__ __forceinline__ float fwd7_merge(float x) {
    float t, y;
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 quad_perm:[3,1,2,3] row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(t) : "v"(x), "v"(x));
    asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 row_shl:7 row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(y) : "v"(x), "v"(t));
    return y;
}

template <int OP, bool LOWNEG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OP == OP_WEDGE || OP == OP_REGR ? 3 : 4))) void prod_fwd_out7(const float* __restrict__ A, const float* __restrict__ B,
                                                     float* __restrict__ C, BlkParams P) {
    static_assert(OP == OP_INNER || OP == OP_LC || OP == OP_RC || OP == OP_WEDGE || OP == OP_REGR,
                  "lc and rc halves only");
    // the halves this op takes; the wedge product runs the lc half's reads on
    // complemented outputs (below)
    constexpr bool kL = OP != OP_RC, kR = OP == OP_INNER || OP == OP_RC;
    constexpr bool kW = OP == OP_WEDGE || OP == OP_REGR;
    constexpr bool kRg = OP == OP_REGR;
    constexpr int N = 7, R = 8, T = 4;
    constexpr unsigned full = 7u;
    __shared__ __attribute__((aligned(64))) float4 lds[4][2 * kBalGroupF4];  // a | b
    // tab[t][rs * 8 + h]: block offsets of S and S | o, the halves' high signs,
    // the cross parities of S and S | o, o = 0
    __shared__ unsigned tab[T][32];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned h = (unsigned)lane & full;
    const int r = lane >> 3;
    const unsigned rs = (unsigned)r & 3u;
    const long long ngrp = (P.batch + R - 1) / R;
    const long long grp = (long long)blockIdx.x * 4 + wave;
    const BalLane L = bal_lane<kFwd7RowX>(N, lane);
    const BalPre pa = bal_fetch(bal_src(A, grp, P.batch, N, R), L, N - 2);
    const BalPre pb = bal_fetch(bal_src(B, grp, P.batch, N, R), L, N - 2);
    if (wave == 0 && lane < 32) {
        const unsigned th = (unsigned)lane & full, trs = row_x<kFwd7RowX>((unsigned)lane >> 3);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const unsigned code = (unsigned)(kFwd7Sched[t] >> (8u * th)) & 0xffu;
            const bool idle = (code & 0x80u) != 0u;
            const FrameStep st{(code >> 3) & 7u, code & 7u, false, idle};
            // wedge: output ~o takes the pair (S, ~o ^ S) for every S inside ~o;
            // regressive: the pair (o | S, ~S) of xor index ~o, stored reversed
            // at block o; an idle step reads blocks S = o, So = p of its code
            const unsigned S = idle ? st.o : kRg ? (st.o | st.p) : st.p;
            const unsigned So = idle ? st.p : kRg ? (full ^ st.p) : kW ? (full ^ st.o ^ S) : (st.p | st.o);
            const HiSign hl = hi_sign<kRg ? OP_REGR : kW ? OP_WEDGE : OP_INNER>(S, So, P.negh, P.nulh, full, P.nm1,
                                                                                 P.mu);
            const HiSign hr = hi_sign<OP_INNER>(So, S, P.negh, P.nulh, full, P.nm1, P.mu);
            const unsigned offs = ((S << 2) | (swz(S) ^ trs)) << 4;
            const unsigned offo = ((So << 2) | (swz(So) ^ trs)) << 4;
            tab[t][lane] = offs | (offo << 10) | ((hl.mask >> 31) << 20) | ((hr.mask >> 31) << 21) |
                           ((cross_pi<kRg ? OP_REGR : OP_WEDGE>(S, P.nm1) & 1u) << 22) |
                           (((unsigned)__popc(So) & 1u) << 23) |
                           ((!idle && st.o == 0u ? 1u : 0u) << 24);
        }
    }
    __syncthreads();
    if (grp >= ngrp) return;
    const int tix = (int)(rs * 8 + h);
    float4* sa = lds[wave];
    bal_stage(sa, pa, L);
    bal_stage(sa + kBalGroupF4, pb, L);
    wave_lds_sync();
    const unsigned base = lds_addr4(sa + (r << (N - 2)));  // the row's a; b at +4 KB
    // lc and rc: outputs 7 and 3, 5, 6 are complete after steps 0 and 1 and
    // wait in y (lanes 3 and 7 go on with output 0); every output leaves
    // through LDS in row order after the last step. The inner product (twice
    // the operands per step) stores each output block when it is complete:
    // holding y as well would halve its occupancy.
    constexpr bool kRowOut = OP != OP_INNER;
    const long long row = grp * R + r;
    const bool row_ok = row < P.batch;
    float acc[16], y[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        acc[e] = 0.f;
        y[e] = 0.f;
    }
    auto keep = [&](bool done) {
        if constexpr (kRowOut) {
            const unsigned md = lane_mask(done);
#pragma unroll
            for (int el = 0; el < 16; ++el) y[el] = bsel(md, acc[el], y[el]);
        } else if (done && row_ok) {
            store_blk(reinterpret_cast<float4*>(C) + (row << (N - 2)), h, acc, false);
        }
    };
    auto step = [&](auto tc) {
        constexpr int t = decltype(tc)::value;
        __builtin_amdgcn_sched_barrier(0);
        unsigned e = tab[t][tix];
        asm volatile("" : "+v"(e));
        const unsigned as0 = base + (e & 1023u), ao0 = base + ((e >> 10) & 1023u);
        unsigned hl = (e << 11) & 0x80000000u, hr = (e << 10) & 0x80000000u;
        unsigned hlo = hl ^ ((e << 9) & 0x80000000u), hro = hr ^ ((e << 8) & 0x80000000u);
        if (kL) asm volatile("" : "+v"(hl), "+v"(hlo));
        if (kR) asm volatile("" : "+v"(hr), "+v"(hro));
        const float fac = (e >> 24) & 1u ? -1.f : 0.f;
        float av[16], bv[16], av2[16], bv2[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const unsigned xs = as0 ^ ((unsigned)q << 4), xo = ao0 ^ ((unsigned)q << 4);
            if (kL) {
                const float4 v0 = lds_ld4(xs), v1 = lds_ld4(xo + 4096u);
                av[4 * q] = v0.x; av[4 * q + 1] = v0.y; av[4 * q + 2] = v0.z; av[4 * q + 3] = v0.w;
                bv[4 * q] = v1.x; bv[4 * q + 1] = v1.y; bv[4 * q + 2] = v1.z; bv[4 * q + 3] = v1.w;
            }
            if (kR) {
                const float4 v2 = lds_ld4(xo), v3 = lds_ld4(xs + 4096u);
                av2[4 * q] = v2.x; av2[4 * q + 1] = v2.y; av2[4 * q + 2] = v2.z; av2[4 * q + 3] = v2.w;
                bv2[4 * q] = v3.x; bv2[4 * q + 1] = v3.y; bv2[4 * q + 2] = v3.z; bv2[4 * q + 3] = v3.w;
            }
        }
        if (kL) {  // lc half (S, S | o) or the wedge pair (S, ~o ^ S): cross parity |S|
            apply_flips(bv, hl, hlo);
            lowblock_fwd<kRg ? LV_REGR : kW ? LV_WEDGE : LV_LC, LOWNEG>(acc, av, bv);
        }
        if (OP == OP_INNER) fwd7_diag<LOWNEG>(acc, av, bv, fac, std::make_integer_sequence<int, 16>{});
        if (kR) {  // rc half (S | o, S): cross parity |S | o|
            apply_flips(bv2, hr, hro);
            lowblock_fwd<LV_RC, LOWNEG>(acc, av2, bv2);
        }
        if constexpr (t == 0) keep(h == 7u);
        if constexpr (t == 1) {
            keep(h == 3u || h == 5u || h == 6u);
            const unsigned mz = lane_mask(h == 3u || h == 7u);  // lanes 3 and 7 turn to output 0
#pragma unroll
            for (int el = 0; el < 16; ++el) acc[el] = bzero(mz, acc[el]);
        }
        if constexpr (t == 3) {
            const unsigned m0 = lane_mask(h == 0u);
#pragma unroll
            for (int el = 0; el < 16; ++el) acc[el] = bsel(m0, fwd7_merge(acc[el]), acc[el]);
            keep(h == 0u || h == 1u || h == 2u || h == 4u);
        }
    };
    frame_steps(step, std::make_integer_sequence<int, T>{});
    if constexpr (!kRowOut) return;
    // output block ob of row r over the staged a (slots 4 ob + (q ^ swz(ob) ^
    // row_x(r))), then row-order stores
    wave_lds_sync();
    const unsigned a0 = lds_addr4(sa);
    const unsigned ob = kW && !kRg ? full ^ h : h;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const unsigned at = a0 + ((unsigned)r << (N + 2)) + (((ob << 2) | ((unsigned)q ^ swz(ob) ^ row_x<kFwd7RowX>(rs))) << 4);
        if (kRg)  // the regressive output block is the xor product's block reversed
            lds_st4(at, make_float4(y[15 - 4 * q], y[14 - 4 * q], y[13 - 4 * q], y[12 - 4 * q]));
        else lds_st4(at, make_float4(y[4 * q], y[4 * q + 1], y[4 * q + 2], y[4 * q + 3]));
    }
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const long long rr = grp * R + (long long)L.rr[i];
        if (rr < P.batch) reinterpret_cast<float4*>(C)[(rr << (N - 2)) + (long long)L.ff[i]] = lds_ld4(a0 + L.so[i]);
    }
}

// ---- tiled path (rows larger than LDS, n >= 12) -----------------------------
// A workgroup of 256 lanes owns 256 output blocks kh = K0 + lane of one row and
// walks the input blocks in aligned tiles of 256 (I0 = 256 t). Because both
// ranges are aligned, the partner blocks jh = ih ^ kh of a tile form the aligned
// tile starting at I0 ^ K0, so each step stages one 16 KB slab per operand in
// LDS (same 64-byte swizzle as the whole-row kernels) and the lane reads its
// partner at local index (ih & 255) ^ (kh & 255).
constexpr int kTileBlocks = 256;                 // blocks per tile = lanes per workgroup
constexpr int kTileF4 = kTileBlocks * 4;         // float4 per operand tile

// stage tile blocks [blk0, blk0 + 256) of one row into dst (swizzled); all
// loads of a pass are issued before its LDS writes
__device__ __forceinline__ void stage_tile(float4* __restrict__ dst, const float4* __restrict__ row,
                                           unsigned blk0) {
    const float4* src = row + ((size_t)blk0 << 2);
#pragma unroll
    for (int pass = 0; pass < kTileF4 / 256 / 4; ++pass) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = src[(pass * 4 + u) * 256 + threadIdx.x];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const unsigned idx = (unsigned)((pass * 4 + u) * 256 + threadIdx.x);
            const unsigned blk = idx >> 2, q = idx & 3u;
            dst[(blk << 2) + (q ^ swz(blk))] = v[u];
        }
    }
}

// work items: (NB / 256) * batch (row, output chunk) pairs, walked with a
// 64-bit grid stride (the grid is capped, so no batch or n overflows it)
template <int OP, bool LOWNEG>
__global__ __launch_bounds__(256) void prod_fwd_tiled(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* __restrict__ C, BlkParams P) {
    __shared__ float4 la[kTileF4];
    __shared__ float4 lb[kTileF4];
    const int n = P.n;
    const unsigned NB = 1u << (n - 4);
    const unsigned chunks = NB / kTileBlocks;
    const long long items = (long long)chunks * P.batch;
    for (long long w = blockIdx.x; w < items; w += gridDim.x) {
        const long long row = w / chunks;
        const unsigned K0 = (unsigned)(w % chunks) * kTileBlocks;
        const unsigned kh = K0 + threadIdx.x;
        const unsigned kl = kh & (kTileBlocks - 1);
        const unsigned fullh = NB - 1u;
        const float4* arow = reinterpret_cast<const float4*>(A) + (row << (n - 2));
        const float4* brow = reinterpret_cast<const float4*>(B) + (row << (n - 2));
        float acc[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.f;
        for (unsigned I0 = 0; I0 < NB; I0 += kTileBlocks) {
            __syncthreads();  // the previous tile is consumed
            stage_tile(la, arow, I0);
            stage_tile(lb, brow, I0 ^ K0);
            __syncthreads();
            for (unsigned il = 0; il < (unsigned)kTileBlocks; ++il) {
                const unsigned ih = I0 + il, jh = ih ^ kh;
                const HiSign hs = hi_sign<OP>(ih, jh, P.negh, P.nulh, fullh, P.nm1, P.mu);
                if (!hs.valid) continue;
                float av[16], bv[16];
                load_blk(la, il, av);
                load_blk(lb, il ^ kl, bv);
                apply_flips(bv, hs.mask, hs.mask ^ (cross_pi<OP>(ih, P.nm1) << 31));
                fwd_block_dispatch<OP, LOWNEG>(acc, av, bv, ih, jh);
            }
        }
        float4* out = reinterpret_cast<float4*>(C) + (row << (n - 2));
        if (OP == OP_REGR) {
            const unsigned ob = fullh ^ kh;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                out[(ob << 2) + (3 - q)] = make_float4(acc[4 * q + 3], acc[4 * q + 2], acc[4 * q + 1], acc[4 * q]);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                out[(kh << 2) + q] = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
        }
    }
}

// lane owns block h = H0 + lane of ga and gb; tiles over m stage a[m], b[m]
// and gc[h ^ m] (regressive: gc[fullh ^ h ^ m]), an aligned tile as well
template <int OP, bool LOWNEG>
__global__ __launch_bounds__(256) void prod_bwd_tiled(const float* __restrict__ A, const float* __restrict__ B,
                                                       const float* __restrict__ GC, float* __restrict__ GA,
                                                       float* __restrict__ GB, BlkParams P) {
    __shared__ float4 la[kTileF4];
    __shared__ float4 lb[kTileF4];
    __shared__ float4 lg[kTileF4];
    const int n = P.n;
    const unsigned NB = 1u << (n - 4);
    const unsigned chunks = NB / kTileBlocks;
    const long long items = (long long)chunks * P.batch;
    for (long long w = blockIdx.x; w < items; w += gridDim.x) {
        const long long row = w / chunks;
        const unsigned H0 = (unsigned)(w % chunks) * kTileBlocks;
        const unsigned h = H0 + threadIdx.x;
        const unsigned hl = h & (kTileBlocks - 1);
        const unsigned fullh = NB - 1u;
        const bool want_a = GA != nullptr, want_b = GB != nullptr;
        const float4* arow = reinterpret_cast<const float4*>(A) + (row << (n - 2));
        const float4* brow = reinterpret_cast<const float4*>(B) + (row << (n - 2));
        const float4* grow = reinterpret_cast<const float4*>(GC) + row * P.ldg4;
        const unsigned pi_h = cross_pi<OP>(h, P.nm1);
        float ga[16], gb[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            ga[e] = 0.f;
            gb[e] = 0.f;
        }
        for (unsigned M0 = 0; M0 < NB; M0 += kTileBlocks) {
            const unsigned G0 = (OP == OP_REGR) ? ((fullh ^ H0 ^ M0) & ~(unsigned)(kTileBlocks - 1)) : (H0 ^ M0);
            __syncthreads();
            stage_tile(la, arow, M0);
            stage_tile(lb, brow, M0);
            stage_tile(lg, grow, G0);
            __syncthreads();
            for (unsigned ml = 0; ml < (unsigned)kTileBlocks; ++ml) {
                const unsigned m = M0 + ml;
                const HiSign sa = hi_sign<OP>(h, m, P.negh, P.nulh, fullh, P.nm1, P.mu);  // (i, j) = (h, m)
                const HiSign sb = hi_sign<OP>(m, h, P.negh, P.nulh, fullh, P.nm1, P.mu);  // (i, j) = (m, h)
                const bool do_a = want_a && sa.valid, do_b = want_b && sb.valid;
                if (!do_a && !do_b) continue;
                float g[16];
                const unsigned gl = (OP == OP_REGR) ? ((kTileBlocks - 1) ^ hl ^ ml) : (hl ^ ml);
                if (OP == OP_REGR) load_blk_rev(lg, gl, g);
                else load_blk(lg, gl, g);
                if (do_a) {
                    float bv[16];
                    load_blk(lb, ml, bv);
                    apply_flips(bv, sa.mask, sa.mask ^ (pi_h << 31));
                    ga_block_dispatch<OP, LOWNEG>(ga, bv, g, h, m);
                }
                if (do_b) {
                    const unsigned pm = cross_pi<OP>(m, P.nm1) << 31;
                    float av[16], gt[16];
                    load_blk(la, ml, av);
                    apply_flips(av, sb.mask, sb.mask ^ pm);
#pragma unroll
                    for (int e = 0; e < 16; ++e) gt[e] = (cpopc((unsigned)e) & 1) ? flip(g[e], pm) : g[e];
                    gb_block_dispatch<OP, LOWNEG>(gb, av, gt, m, h);
                }
            }
        }
        const long long base = row << (n - 2);
        if (want_a) {
            float4* o = reinterpret_cast<float4*>(GA) + base;
#pragma unroll
            for (int q = 0; q < 4; ++q) o[(h << 2) + q] = make_float4(ga[4 * q], ga[4 * q + 1], ga[4 * q + 2], ga[4 * q + 3]);
        }
        if (want_b) {
            float4* o = reinterpret_cast<float4*>(GB) + base;
#pragma unroll
            for (int q = 0; q < 4; ++q) o[(h << 2) + q] = make_float4(gb[4 * q], gb[4 * q + 1], gb[4 * q + 2], gb[4 * q + 3]);
        }
    }
}

// ---- generic path: one thread per output coefficient, closed-form signs ----
// Used for n < 4 and for metrics whose low four generators are not all +1 or
// all -1 (or contain a null generator).
__global__ __launch_bounds__(256) void prod_fwd_generic(int op, int n, unsigned neg, unsigned nul,
                                                         const float* __restrict__ A, const float* __restrict__ B,
                                                         float* __restrict__ C, long long batch) {
    const unsigned D = 1u << n;
    const long long total = batch << n;
    for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (long long)gridDim.x * blockDim.x) {
        const long long row = idx >> n;
        const unsigned k = (unsigned)(idx & (D - 1));
        const float* a = A + (row << n);
        const float* b = B + (row << n);
        float acc = 0.f;
        for (unsigned i = 0; i < D; ++i) {
            const int s = full_sign(op, n, i, i ^ k, neg, nul);
            if (s) acc = __builtin_fmaf((float)s * a[i], b[i ^ k], acc);
        }
        const unsigned ok = (op == OP_REGR) ? (~k & (D - 1)) : k;
        C[(row << n) + ok] = acc;
    }
}

// ga[k] = sum_j sigma(k, j) b[j] gf[k^j]   (which == 0)
// gb[k] = sum_i sigma(i, k) a[i] gf[i^k]   (which == 1)
__global__ __launch_bounds__(256) void prod_bwd_generic(int op, int n, unsigned neg, unsigned nul, int which,
                                                         const float* __restrict__ X, const float* __restrict__ GC,
                                                         long long ldg, float* __restrict__ OUT, long long batch) {
    const unsigned D = 1u << n;
    const long long total = batch << n;
    for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (long long)gridDim.x * blockDim.x) {
        const long long row = idx >> n;
        const unsigned k = (unsigned)(idx & (D - 1));
        const float* x = X + (row << n);
        const float* gc = GC + row * ldg;  // ldg = 2^n, or 0 for one row broadcast over the batch
        float acc = 0.f;
        for (unsigned u = 0; u < D; ++u) {
            const int s = which == 0 ? full_sign(op, n, k, u, neg, nul) : full_sign(op, n, u, k, neg, nul);
            if (!s) continue;
            const unsigned m = u ^ k;
            const float gv = (op == OP_REGR) ? gc[~m & (D - 1)] : gc[m];
            acc = __builtin_fmaf((float)s * x[u], gv, acc);
        }
        OUT[(row << n) + k] = acc;
    }
}

// ---- host side --------------------------------------------------------------

static int check_common(int op, int n, uint32_t neg, uint32_t nul, int64_t batch) {
    if (op < CLF_OP_GEOM || op > CLF_OP_REGRESSIVE) return set_error(CLF_ERR_ARG, "unknown product op " + std::to_string(op));
    if (n < 1 || n > kMaxN)
        return set_error(CLF_ERR_ARG, "n must be in [1, " + std::to_string(kMaxN) + "], got " + std::to_string(n));
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

// The block factorisation needs the low four generators to share one metric
// value (+1 or -1, not null) for ops whose signs depend on it; wedge and
// regressive signs do not. Sets the low-block sign variant.
static bool blocked_metric(int op, int n, uint32_t neg, uint32_t nul, bool& lowneg) {
    if (n < 4) return false;
    const uint32_t neg4 = neg & 15u, nul4 = nul & 15u;
    if (op == CLF_OP_WEDGE || op == CLF_OP_REGRESSIVE) {
        lowneg = false;  // these signs do not depend on the low-bit metric
        return true;
    }
    if (nul4) return false;
    if (neg4 != 0u && neg4 != 15u) return false;
    lowneg = neg4 == 15u;
    return true;
}

static void block_sign_params(int n, uint32_t neg, uint32_t nul, BlkParams& P) {
    P.n = n;
    P.negh = neg >> 4;
    P.nulh = nul >> 4;
    P.nm1 = (n - 1) & 1;
    P.mu = popc_rt(neg) & 1;
    P.negl = neg & 15u;
}

constexpr size_t kBlockedLdsMax = 48 * 1024;

// Launch shape for the whole-row blocked kernels. Returns false if the rows do
// not fit the LDS budget (tiled path) or the metric needs the generic path.
// Row skews of the blocked kernels' slots (bslot), 2 bits per staged row r at
// bits 2 (r & 15): the rows that share a lane set of a ds_read_b128 (4 at n = 7,
// 2 at n = 8, 4 of the 8 at n <= 6) get distinct skews, chosen on the CPU so
// that neither the broadcast nor the partner reads put two addresses of one
// set on a bank group; at n >= 9 a half-wave holds one row.
static unsigned blocked_row_skew(int n) {
    if (n <= 6) return 0xE4E4E4E4u;  // 0, 1, 2, 3
    if (n == 7) return 0x78787878u;  // 0, 2, 3, 1
    if (n == 8) return 0xCCCCCCCCu;  // 0, 3
    return 0u;
}

static bool blocked_plan(int op, int n, uint32_t neg, uint32_t nul, int nops, BlkParams& P, bool& lowneg,
                         dim3& grid, dim3& block, size_t& lds_bytes) {
    if (!blocked_metric(op, n, neg, nul, lowneg)) return false;
    const int nh = n - 4;
    const int NB = 1 << nh;
    const int lpr = NB < 64 ? NB : 64;
    int lpr_log = 0;
    while ((1 << lpr_log) < lpr) ++lpr_log;
    const int rpw = 64 / lpr;
    const size_t row_bytes = (size_t)nops * ((size_t)4 << n);
    int nwaves = 4;
    while (nwaves > 1 && (size_t)nwaves * rpw * row_bytes > kBlockedLdsMax) nwaves >>= 1;
    if ((size_t)nwaves * rpw * row_bytes > kBlockedLdsMax) return false;
    block_sign_params(n, neg, nul, P);
    P.lpr_log = lpr_log;
    P.rows_per_wg = nwaves * rpw;
    P.kpl = NB / lpr;
    P.rskew = blocked_row_skew(n);
    grid = dim3((unsigned)((P.batch + P.rows_per_wg - 1) / P.rows_per_wg));
    block = dim3(64 * nwaves);
    lds_bytes = (size_t)P.rows_per_wg * row_bytes;
    return true;
}

// Grid cap of the grid-stride kernels (tiled, per-coefficient): well inside
// the 2^32 work-items of one launch dimension.
constexpr long long kMaxGrid = 1LL << 22;

// Tiled kernels: n >= 12 (at least one 256-block tile per row).
static bool tiled_plan(int op, int n, uint32_t neg, uint32_t nul, BlkParams& P, bool& lowneg, dim3& grid) {
    if (n < 12 || !blocked_metric(op, n, neg, nul, lowneg)) return false;
    block_sign_params(n, neg, nul, P);
    const long long items = (1LL << (n - 4)) / kTileBlocks * P.batch;
    grid = dim3((unsigned)(items < kMaxGrid ? items : kMaxGrid));
    return true;
}

// CLF_PRODUCT_PATH (options()) selects a path for comparisons where several
// apply: "tiled" runs n = 12 on the tiled kernels instead of the whole-row
// ones, "generic" runs the per-coefficient kernels for any n.
static bool tiled_forced() { return options().product_path == PATH_TILED; }
static bool generic_forced() { return options().product_path == PATH_GENERIC; }

// The inner product's backward for 4 <= n <= 8 runs on the per-lane frame
// kernel when the low generators share one metric value and no generator is
// null (CLF_PRODUCT_PATH=blocked or =balanced keep it on those kernels).
static bool frame_plan(int op, int n, uint32_t neg, uint32_t nul, BlkParams& P, bool& lowneg) {
    if (op != OP_INNER || n < kFrameMinN || n > kFrameMaxN || nul != 0u) return false;
    if (options().product_path != PATH_DEFAULT) return false;
    if (!blocked_metric(op, n, neg, nul, lowneg)) return false;
    block_sign_params(n, neg, nul, P);
    return true;
}

// the one-lane-per-output forward at n = 7: inner, lc, rc and wedge without a
// null generator (blocked_metric: a uniform low metric for inner, lc and rc)
static bool out7_plan(int op, int n, uint32_t neg, uint32_t nul, BlkParams& P, bool& lowneg) {
    if (n != 7 || nul != 0u || (op != OP_INNER && op != OP_LC && op != OP_RC && op != OP_WEDGE && op != OP_REGR))
        return false;
    if (options().product_path != PATH_DEFAULT) return false;
    if (!blocked_metric(op, n, neg, nul, lowneg)) return false;
    block_sign_params(n, neg, nul, P);
    return true;
}

template <int OP>
static void launch_out7(hipStream_t s, bool ln, const float* a, const float* b, float* c, const BlkParams& P) {
    const long long groups = (P.batch + 7) / 8;
    for (long long g0 = 0; g0 < groups; g0 += kMaxGrid * 4) {  // one group of 8 rows per wave
        const long long gn = groups - g0 < kMaxGrid * 4 ? groups - g0 : kMaxGrid * 4;
        BlkParams Q = P;
        Q.batch = (g0 + gn) * 8 < P.batch ? gn * 8 : P.batch - g0 * 8;
        const long long off = g0 * 8 * 128;
        const dim3 grid((unsigned)((gn + 3) / 4));
        if (ln) hipLaunchKernelGGL((prod_fwd_out7<OP, true>), grid, dim3(256), 0, s, a + off, b + off, c + off, Q);
        else hipLaunchKernelGGL((prod_fwd_out7<OP, false>), grid, dim3(256), 0, s, a + off, b + off, c + off, Q);
    }
}

template <int N, bool LN, bool WA, bool WB>
static void launch_frame3(hipStream_t s, const float* A, const float* B, const float* GCp, float* GA, float* GB,
                          const BlkParams& P) {
    // one wave per group of R rows: batches beyond kMaxGrid workgroups go in
    // several launches over consecutive rows
    const long long R = 64 >> (N - 4);
    const long long chunk = kMaxGrid * 4 * R;
    const long long D = 1LL << N;
    for (long long r0 = 0; r0 < P.batch; r0 += chunk) {
        BlkParams Q = P;
        Q.batch = P.batch - r0 < chunk ? P.batch - r0 : chunk;
        const long long groups = (Q.batch + R - 1) / R;
        const dim3 g((unsigned)((groups + 3) / 4));
        const long long off = r0 * D;
        hipLaunchKernelGGL((prod_bwd_inner_frame<N, LN, WA, WB>), g, dim3(256), 0, s, A + off, B + off,
                           GCp + (P.ldg4 ? off : 0), GA ? GA + off : nullptr, GB ? GB + off : nullptr, Q);
    }
}

template <int N, bool LN>
static void launch_frame2(hipStream_t s, const float* A, const float* B, const float* GCp, float* GA, float* GB,
                          const BlkParams& P) {
    if (GA && GB) launch_frame3<N, LN, true, true>(s, A, B, GCp, GA, GB, P);
    else if (GA) launch_frame3<N, LN, true, false>(s, A, B, GCp, GA, GB, P);
    else launch_frame3<N, LN, false, true>(s, A, B, GCp, GA, GB, P);
}

static void launch_frame(int n, bool ln, hipStream_t s, const float* A, const float* B, const float* GCp, float* GA,
                         float* GB, const BlkParams& P) {
#define CLF_FRAME_N(NV)                                                  \
    case NV:                                                             \
        if (ln) launch_frame2<NV, true>(s, A, B, GCp, GA, GB, P);        \
        else launch_frame2<NV, false>(s, A, B, GCp, GA, GB, P);          \
        break;
    switch (n) {
        CLF_FRAME_N(4)
        CLF_FRAME_N(5)
        CLF_FRAME_N(6)
        CLF_FRAME_N(7)
        CLF_FRAME_N(8)
    }
#undef CLF_FRAME_N
}

// The contractions' backward on the frame schedule: lc and rc for
// 4 <= n <= 8 without a null generator and with a uniform low metric; the
// wedge product, and the regressive product as the wedge of duals, for any
// metric without a null generator.
static bool contr_plan(int op, int n, uint32_t neg, uint32_t nul, BlkParams& P, bool& lowneg) {
    if ((op != OP_LC && op != OP_RC && op != OP_WEDGE && op != OP_REGR) || n < kFrameMinN || n > kFrameMaxN ||
        nul != 0u)
        return false;
    if (options().product_path != PATH_DEFAULT) return false;
    if (!blocked_metric(op, n, neg, nul, lowneg)) return false;
    block_sign_params(n, neg, nul, P);
    return true;
}

template <int OP, int N, bool LN>
static void launch_contr3(hipStream_t s, const float* A, const float* B, const float* GCp, float* GA, float* GB,
                          const BlkParams& P) {
    // one wave per group of R rows, as launch_frame3
    const long long R = 64 >> (N - 4);
    const long long chunk = kMaxGrid * 4 * R;
    const long long D = 1LL << N;
    for (long long r0 = 0; r0 < P.batch; r0 += chunk) {
        BlkParams Q = P;
        Q.batch = P.batch - r0 < chunk ? P.batch - r0 : chunk;
        const long long groups = (Q.batch + R - 1) / R;
        const dim3 g((unsigned)((groups + 3) / 4));
        const long long off = r0 * D;
        hipLaunchKernelGGL((prod_bwd_contr_frame<OP, N, LN>), g, dim3(256), 0, s, A + off, B + off,
                           GCp + (P.ldg4 ? off : 0), GA ? GA + off : nullptr, GB ? GB + off : nullptr, Q);
    }
}

template <int OP>
static void launch_contr(int n, bool ln, hipStream_t s, const float* A, const float* B, const float* GCp, float* GA,
                         float* GB, const BlkParams& P) {
#define CLF_CONTR_N(NV)                                                  \
    case NV:                                                             \
        if (ln) launch_contr3<OP, NV, true>(s, A, B, GCp, GA, GB, P);    \
        else launch_contr3<OP, NV, false>(s, A, B, GCp, GA, GB, P);      \
        break;
    switch (n) {
        CLF_CONTR_N(4)
        CLF_CONTR_N(5)
        CLF_CONTR_N(6)
        CLF_CONTR_N(7)
        CLF_CONTR_N(8)
    }
#undef CLF_CONTR_N
}

// prod_bwd_contr5: lc and rc at n = 9 without null generators, lc at n = 10
// whose only null generator is e9 (low generators of one metric value).
static bool contr5_plan(int op, int n, uint32_t neg, uint32_t nul, BlkParams& P, bool& lowneg, bool& nulltop) {
    if (op != OP_LC && op != OP_RC) return false;
    if (options().product_path != PATH_DEFAULT) return false;
    if (n == 9 && nul == 0u) nulltop = false;
    else if (n == 10 && nul == (1u << 9) && op == OP_LC) nulltop = true;
    else return false;
    if (!blocked_metric(op, n, neg, nul, lowneg)) return false;
    block_sign_params(n, neg, nul, P);
    P.negh = (neg >> 4) & 31u;  // the n = 9 problem's high generators
    P.nulh = 0u;
    return true;
}

// prod_bwd_inner5: the inner product's backward at n = 9 without a null
// generator and at n = 10 whose only null generator is the top one
static bool inner5_plan(int op, int n, uint32_t neg, uint32_t nul, BlkParams& P, bool& lowneg, bool& nulltop) {
    if (op != OP_INNER) return false;
    if (options().product_path != PATH_DEFAULT) return false;
    if (n == 9 && nul == 0u) nulltop = false;
    else if (n == 10 && nul == (1u << 9)) nulltop = true;
    else return false;
    if (!blocked_metric(op, n, neg, nul, lowneg)) return false;
    block_sign_params(n, neg, nul, P);
    P.negh = (neg >> 4) & 31u;  // the n = 9 problems' high generators
    P.nulh = 0u;
    return true;
}

template <bool LN, bool NT>
static void launch_inner5_t(hipStream_t s, const float* A, const float* B, const float* GCp, float* GA, float* GB,
                            const BlkParams& P) {
    const long long R = NT ? 1 : 2;
    const long long chunk = kMaxGrid * 4 * R;
    const long long D = NT ? 1024 : 512;
    for (long long r0 = 0; r0 < P.batch; r0 += chunk) {
        BlkParams Q = P;
        Q.batch = P.batch - r0 < chunk ? P.batch - r0 : chunk;
        const long long groups = (Q.batch + R - 1) / R;
        const dim3 g(resident_grid((const void*)prod_bwd_inner5<LN, NT>, 256, 0, (groups + 3) / 4));
        const long long off = r0 * D;
        hipLaunchKernelGGL((prod_bwd_inner5<LN, NT>), g, dim3(256), 0, s, A + off, B + off,
                           GCp + (P.ldg4 ? off : 0), GA ? GA + off : nullptr, GB ? GB + off : nullptr, Q);
    }
}

static void launch_inner5(bool ln, bool nt, hipStream_t s, const float* A, const float* B, const float* GCp, float* GA,
                          float* GB, const BlkParams& P) {
    if (nt) {
        if (ln) launch_inner5_t<true, true>(s, A, B, GCp, GA, GB, P);
        else launch_inner5_t<false, true>(s, A, B, GCp, GA, GB, P);
    } else {
        if (ln) launch_inner5_t<true, false>(s, A, B, GCp, GA, GB, P);
        else launch_inner5_t<false, false>(s, A, B, GCp, GA, GB, P);
    }
}

template <int OP, bool LN, bool NT>
static void launch_contr5_t(hipStream_t s, const float* A, const float* B, const float* GCp, float* GA, float* GB,
                            const BlkParams& P) {
    const long long R = NT ? 1 : 2;
    const long long chunk = kMaxGrid * 4 * R;
    const long long D = NT ? 1024 : 512;
    for (long long r0 = 0; r0 < P.batch; r0 += chunk) {
        BlkParams Q = P;
        Q.batch = P.batch - r0 < chunk ? P.batch - r0 : chunk;
        const long long groups = (Q.batch + R - 1) / R;
        const dim3 g(resident_grid((const void*)prod_bwd_contr5<OP, LN, NT>, 256, 0, (groups + 3) / 4));
        const long long off = r0 * D;
        hipLaunchKernelGGL((prod_bwd_contr5<OP, LN, NT>), g, dim3(256), 0, s, A + off, B + off,
                           GCp + (P.ldg4 ? off : 0), GA ? GA + off : nullptr, GB ? GB + off : nullptr, Q);
    }
}

template <int OP, bool LN, bool NT>
static void launch_fcontr5_t(hipStream_t s, const float* A, const float* B, float* C, const BlkParams& P) {
    const long long R = NT ? 1 : 2;
    const long long chunk = kMaxGrid * 4 * R;
    const long long D = NT ? 1024 : 512;
    for (long long r0 = 0; r0 < P.batch; r0 += chunk) {
        BlkParams Q = P;
        Q.batch = P.batch - r0 < chunk ? P.batch - r0 : chunk;
        const long long groups = (Q.batch + R - 1) / R;
        const dim3 g(resident_grid((const void*)prod_fwd_contr5<OP, LN, NT>, 256, 0, (groups + 3) / 4));
        const long long off = r0 * D;
        hipLaunchKernelGGL((prod_fwd_contr5<OP, LN, NT>), g, dim3(256), 0, s, A + off, B + off, C + off, Q);
    }
}

static void launch_fcontr5(int op, bool ln, bool nt, hipStream_t s, const float* A, const float* B, float* C,
                           const BlkParams& P) {
    if (nt) {
        if (ln) launch_fcontr5_t<OP_LC, true, true>(s, A, B, C, P);
        else launch_fcontr5_t<OP_LC, false, true>(s, A, B, C, P);
    } else if (op == OP_LC) {
        if (ln) launch_fcontr5_t<OP_LC, true, false>(s, A, B, C, P);
        else launch_fcontr5_t<OP_LC, false, false>(s, A, B, C, P);
    } else {
        if (ln) launch_fcontr5_t<OP_RC, true, false>(s, A, B, C, P);
        else launch_fcontr5_t<OP_RC, false, false>(s, A, B, C, P);
    }
}

static void launch_contr5(int op, bool ln, bool nt, hipStream_t s, const float* A, const float* B, const float* GCp,
                          float* GA, float* GB, const BlkParams& P) {
    if (nt) {
        if (ln) launch_contr5_t<OP_LC, true, true>(s, A, B, GCp, GA, GB, P);
        else launch_contr5_t<OP_LC, false, true>(s, A, B, GCp, GA, GB, P);
    } else if (op == OP_LC) {
        if (ln) launch_contr5_t<OP_LC, true, false>(s, A, B, GCp, GA, GB, P);
        else launch_contr5_t<OP_LC, false, false>(s, A, B, GCp, GA, GB, P);
    } else {
        if (ln) launch_contr5_t<OP_RC, true, false>(s, A, B, GCp, GA, GB, P);
        else launch_contr5_t<OP_RC, false, false>(s, A, B, GCp, GA, GB, P);
    }
}

// Balanced kernels: wedge, lc, rc, regressive and the inner product for
// 4 <= n <= 10 (CLF_PRODUCT_PATH=blocked keeps them on the one-lane-per-output
// kernels). Up to n = 8 the inner product's backward runs on the per-lane
// frame kernels (frame_plan; the blocked kernel when the metric has a null
// generator), and at n = 7 its forward too. The geometric product, whose
// outputs all have the same work, gains nothing; both use the balanced
// kernels only when CLF_PRODUCT_PATH=balanced.
static bool bal_plan(int op, int n, uint32_t neg, uint32_t nul, bool fwd, BlkParams& P, bool& lowneg) {
    if (n < kBalMinN || n > kBalMaxN) return false;
    const bool opt_in = op == OP_GEOM || (op == OP_INNER && !fwd && n < 8);
    if (opt_in ? options().product_path != PATH_BALANCED : options().product_path == PATH_BLOCKED) return false;
    if (!blocked_metric(op, n, neg, nul, lowneg)) return false;
    block_sign_params(n, neg, nul, P);
    return true;
}

static unsigned bal_grid(const void* kernel, const BlkParams& P) {
    const long long R = 1LL << (10 - P.n);
    const long long groups = (P.batch + R - 1) / R;
    return resident_grid(kernel, 256, 0, (groups + 3) / 4);
}

// Small-batch kernels: 9 <= n <= 12 (whole row in LDS) when the one-lane-
// per-output-block kernels would run fewer than 512 waves (batch * NB < 2^15);
// CLF_PRODUCT_PATH=split forces them at any batch, =blocked or =balanced
// turn them off.
static bool split_plan(int op, int n, uint32_t neg, uint32_t nul, BlkParams& P, bool& lowneg, bool fwd, dim3& grid,
                       size_t& lds_bytes) {
    // n = 8: the forward only (one workgroup per row, 16 lanes per output
    // block, one partner each); the backward's one-lane-per-output kernels are
    // short enough at n = 8
    if (n < (fwd ? 8 : 9) || n > 12) return false;
    const int pp = options().product_path;
    if (pp == PATH_BLOCKED || pp == PATH_BALANCED || pp == PATH_TILED || pp == PATH_GENERIC) return false;
    const long long NB = 1LL << (n - 4);
    if (pp != PATH_SPLIT && P.batch * NB >= (1LL << 15)) return false;
    if (!blocked_metric(op, n, neg, nul, lowneg)) return false;
    block_sign_params(n, neg, nul, P);
    P.split_log = n == 8 ? 4 : n - 6;    // S = NB / 4: four partners per lane (n = 8: S = NB, one)
    const int g_log = 8 - P.split_log;   // G = 256 / S output blocks per workgroup
    P.wpr_log = (n - 4) - g_log;
    const long long wgs = P.batch << P.wpr_log;
    if (wgs > kMaxGrid) return false;
    grid = dim3((unsigned)wgs);
    const size_t stage = (size_t)(fwd ? 2 : 3) * ((size_t)4 << n);
    const size_t red = (size_t)(fwd ? 1 : 2) * 256 * 20 * sizeof(float);
    lds_bytes = stage > red ? stage : red;
    return true;
}

template <int OP, bool LN>
static void launch_fwd_bal(hipStream_t s, const float* A, const float* B, float* C, const BlkParams& P) {
    const dim3 g(bal_grid((const void*)prod_fwd_bal<OP, LN>, P));
    hipLaunchKernelGGL((prod_fwd_bal<OP, LN>), g, dim3(256), 0, s, A, B, C, P);
}

template <int OP, bool LN>
static void launch_bwd_bal(hipStream_t s, const float* A, const float* B, const float* GCp, float* GA, float* GB,
                           const BlkParams& P) {
    const dim3 g(bal_grid((const void*)prod_bwd_bal<OP, LN>, P));
    hipLaunchKernelGGL((prod_bwd_bal<OP, LN>), g, dim3(256), 0, s, A, B, GCp, GA, GB, P);
}

template <int OP, bool LN>
static void launch_fwd(dim3 g, dim3 b, size_t lds, hipStream_t s, const float* A, const float* B, float* C,
                       const BlkParams& P) {
    hipLaunchKernelGGL((prod_fwd_blk<OP, LN>), g, b, lds, s, A, B, C, P);
}

template <int OP, bool LN>
static void launch_bwd(dim3 g, dim3 b, size_t lds, hipStream_t s, const float* A, const float* B, const float* GCp,
                       float* GA, float* GB, const BlkParams& P) {
    hipLaunchKernelGGL((prod_bwd_blk<OP, LN>), g, b, lds, s, A, B, GCp, GA, GB, P);
}

bool rep_applicable(int op, int n, uint32_t neg, uint32_t nul);
bool rep_disabled_by_env();
int rep_fwd(int n, uint32_t neg, const float* a, const float* b, float* c, int64_t batch, void* stream);
int rep_bwd(int n, uint32_t neg, const float* a, const float* b, const float* gc, int64_t ldg, float* ga, float* gb,
            int64_t batch, void* stream);

// The geometric product of real-matrix-type signatures goes through the matrix
// representation unless CLF_GEOM_PATH=direct asks for the per-term kernels.
static bool use_rep(int op, int n, uint32_t neg, uint32_t nul) {
    if (rep_disabled_by_env()) return false;
    return rep_applicable(op, n, neg, nul);
}

int product_fwd(int op, int n, uint32_t neg, uint32_t nul, const float* a, const float* b, float* c,
                int64_t batch, void* stream) {
    int rc = check_common(op, n, neg, nul, batch);
    if (rc) return rc;
    if (batch == 0) return CLF_OK;
    if (!a || !b || !c) return set_error(CLF_ERR_ARG, "null pointer argument");
    if (c == a || c == b) return set_error(CLF_ERR_ARG, "output must not alias an input");
    if ((((uintptr_t)a) | ((uintptr_t)b) | ((uintptr_t)c)) & 15u)
        return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    if (use_rep(op, n, neg, nul)) return rep_fwd(n, neg, a, b, c, batch, stream);
    hipStream_t s = (hipStream_t)stream;
    BlkParams P{};
    P.batch = batch;
    bool ln = false, nt5 = false;
    dim3 g, bl;
    size_t lds = 0;
    const bool force_tiled = n >= 12 && tiled_forced(), force_generic = generic_forced();
    if (split_plan(op, n, neg, nul, P, ln, true, g, lds)) {
#define CLF_FWD_SPLIT(OPV, LNV) hipLaunchKernelGGL((prod_fwd_split<OPV, LNV>), g, dim3(256), lds, s, a, b, c, P)
        switch (op) {
            case OP_GEOM: if (ln) CLF_FWD_SPLIT(OP_GEOM, true); else CLF_FWD_SPLIT(OP_GEOM, false); break;
            case OP_INNER: if (ln) CLF_FWD_SPLIT(OP_INNER, true); else CLF_FWD_SPLIT(OP_INNER, false); break;
            case OP_LC: if (ln) CLF_FWD_SPLIT(OP_LC, true); else CLF_FWD_SPLIT(OP_LC, false); break;
            case OP_RC: if (ln) CLF_FWD_SPLIT(OP_RC, true); else CLF_FWD_SPLIT(OP_RC, false); break;
            case OP_WEDGE: CLF_FWD_SPLIT(OP_WEDGE, false); break;
            case OP_REGR: CLF_FWD_SPLIT(OP_REGR, false); break;
        }
#undef CLF_FWD_SPLIT
    } else if (contr5_plan(op, n, neg, nul, P, ln, nt5)) {
        launch_fcontr5(op, ln, nt5, s, a, b, c, P);
    } else if (out7_plan(op, n, neg, nul, P, ln)) {
        if (op == OP_INNER) launch_out7<OP_INNER>(s, ln, a, b, c, P);
        else if (op == OP_LC) launch_out7<OP_LC>(s, ln, a, b, c, P);
        else if (op == OP_RC) launch_out7<OP_RC>(s, ln, a, b, c, P);
        else if (op == OP_WEDGE) launch_out7<OP_WEDGE>(s, ln, a, b, c, P);
        else launch_out7<OP_REGR>(s, ln, a, b, c, P);
    } else if (!force_generic && bal_plan(op, n, neg, nul, true, P, ln)) {
#define CLF_FWD_BAL(OPV)                                               \
    case OPV:                                                          \
        if (ln) launch_fwd_bal<OPV, true>(s, a, b, c, P);              \
        else launch_fwd_bal<OPV, false>(s, a, b, c, P);                \
        break;
        switch (op) {
            CLF_FWD_BAL(OP_GEOM)
            CLF_FWD_BAL(OP_INNER)
            CLF_FWD_BAL(OP_LC)
            CLF_FWD_BAL(OP_RC)
            case OP_WEDGE: launch_fwd_bal<OP_WEDGE, false>(s, a, b, c, P); break;
            case OP_REGR: launch_fwd_bal<OP_REGR, false>(s, a, b, c, P); break;
        }
#undef CLF_FWD_BAL
    } else if (!force_generic && !force_tiled && blocked_plan(op, n, neg, nul, 2, P, ln, g, bl, lds)) {
#define CLF_FWD_CASE(OPV)                                              \
    case OPV:                                                          \
        if (ln) launch_fwd<OPV, true>(g, bl, lds, s, a, b, c, P);      \
        else launch_fwd<OPV, false>(g, bl, lds, s, a, b, c, P);        \
        break;
        switch (op) {
            CLF_FWD_CASE(OP_GEOM)
            CLF_FWD_CASE(OP_INNER)
            CLF_FWD_CASE(OP_LC)
            CLF_FWD_CASE(OP_RC)
            case OP_WEDGE: launch_fwd<OP_WEDGE, false>(g, bl, lds, s, a, b, c, P); break;
            case OP_REGR: launch_fwd<OP_REGR, false>(g, bl, lds, s, a, b, c, P); break;
        }
#undef CLF_FWD_CASE
    } else if (!force_generic && tiled_plan(op, n, neg, nul, P, ln, g)) {
#define CLF_FWD_TILED(OPV, LNV) hipLaunchKernelGGL((prod_fwd_tiled<OPV, LNV>), g, dim3(256), 0, s, a, b, c, P)
        switch (op) {
            case OP_GEOM: if (ln) CLF_FWD_TILED(OP_GEOM, true); else CLF_FWD_TILED(OP_GEOM, false); break;
            case OP_INNER: if (ln) CLF_FWD_TILED(OP_INNER, true); else CLF_FWD_TILED(OP_INNER, false); break;
            case OP_LC: if (ln) CLF_FWD_TILED(OP_LC, true); else CLF_FWD_TILED(OP_LC, false); break;
            case OP_RC: if (ln) CLF_FWD_TILED(OP_RC, true); else CLF_FWD_TILED(OP_RC, false); break;
            case OP_WEDGE: CLF_FWD_TILED(OP_WEDGE, false); break;
            case OP_REGR: CLF_FWD_TILED(OP_REGR, false); break;
        }
#undef CLF_FWD_TILED
    } else {
        const long long total = batch << n;
        const long long want = (total + 255) / 256;
        const unsigned blocks = (unsigned)(want < kMaxGrid ? want : kMaxGrid);
        hipLaunchKernelGGL(prod_fwd_generic, dim3(blocks), dim3(256), 0, s, op, n, neg, nul, a, b, c,
                           (long long)batch);
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

// gc's rows are ldg floats apart: 2^n (packed) or 0 (one row broadcast over
// the batch, e.g. the gradient of a sum)
int product_bwd(int op, int n, uint32_t neg, uint32_t nul, const float* a, const float* b, const float* gc,
                int64_t ldg, float* ga, float* gb, int64_t batch, void* stream) {
    int rc = check_common(op, n, neg, nul, batch);
    if (rc) return rc;
    if (ldg != 0 && ldg != (1LL << n)) return set_error(CLF_ERR_ARG, "gc row stride must be 0 or 2^n");
    if (batch == 0 || (!ga && !gb)) return CLF_OK;
    if (!a || !b || !gc) return set_error(CLF_ERR_ARG, "null pointer argument");
    if ((ga && (ga == a || ga == b || ga == gc)) || (gb && (gb == a || gb == b || gb == gc)) || (ga && ga == gb))
        return set_error(CLF_ERR_ARG, "gradient outputs must not alias inputs or each other");
    if ((((uintptr_t)a) | ((uintptr_t)b) | ((uintptr_t)gc) | ((uintptr_t)ga) | ((uintptr_t)gb)) & 15u)
        return set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    if (use_rep(op, n, neg, nul)) return rep_bwd(n, neg, a, b, gc, ldg, ga, gb, batch, stream);
    hipStream_t s = (hipStream_t)stream;
    BlkParams P{};
    P.batch = batch;
    P.ldg4 = ldg >> 2;
    bool ln = false, nt5 = false;
    dim3 g, bl;
    size_t lds = 0;
    const bool force_tiled = n >= 12 && tiled_forced(), force_generic = generic_forced();
    if (split_plan(op, n, neg, nul, P, ln, false, g, lds)) {
#define CLF_BWD_SPLIT(OPV, LNV) \
    hipLaunchKernelGGL((prod_bwd_split<OPV, LNV>), g, dim3(256), lds, s, a, b, gc, ga, gb, P)
        switch (op) {
            case OP_GEOM: if (ln) CLF_BWD_SPLIT(OP_GEOM, true); else CLF_BWD_SPLIT(OP_GEOM, false); break;
            case OP_INNER: if (ln) CLF_BWD_SPLIT(OP_INNER, true); else CLF_BWD_SPLIT(OP_INNER, false); break;
            case OP_LC: if (ln) CLF_BWD_SPLIT(OP_LC, true); else CLF_BWD_SPLIT(OP_LC, false); break;
            case OP_RC: if (ln) CLF_BWD_SPLIT(OP_RC, true); else CLF_BWD_SPLIT(OP_RC, false); break;
            case OP_WEDGE: CLF_BWD_SPLIT(OP_WEDGE, false); break;
            case OP_REGR: CLF_BWD_SPLIT(OP_REGR, false); break;
        }
#undef CLF_BWD_SPLIT
    } else if (frame_plan(op, n, neg, nul, P, ln)) {
        launch_frame(n, ln, s, a, b, gc, ga, gb, P);
    } else if (contr5_plan(op, n, neg, nul, P, ln, nt5)) {
        launch_contr5(op, ln, nt5, s, a, b, gc, ga, gb, P);
    } else if (inner5_plan(op, n, neg, nul, P, ln, nt5)) {
        launch_inner5(ln, nt5, s, a, b, gc, ga, gb, P);
    } else if (contr_plan(op, n, neg, nul, P, ln)) {
        if (op == OP_LC) launch_contr<OP_LC>(n, ln, s, a, b, gc, ga, gb, P);
        else if (op == OP_RC) launch_contr<OP_RC>(n, ln, s, a, b, gc, ga, gb, P);
        else if (op == OP_REGR) launch_contr<OP_REGR>(n, false, s, a, b, gc, ga, gb, P);
        else launch_contr<OP_WEDGE>(n, false, s, a, b, gc, ga, gb, P);
    } else if (!force_generic && bal_plan(op, n, neg, nul, false, P, ln)) {
#define CLF_BWD_BAL(OPV)                                                       \
    case OPV:                                                                  \
        if (ln) launch_bwd_bal<OPV, true>(s, a, b, gc, ga, gb, P);             \
        else launch_bwd_bal<OPV, false>(s, a, b, gc, ga, gb, P);               \
        break;
        switch (op) {
            CLF_BWD_BAL(OP_GEOM)
            CLF_BWD_BAL(OP_INNER)
            CLF_BWD_BAL(OP_LC)
            CLF_BWD_BAL(OP_RC)
            case OP_WEDGE: launch_bwd_bal<OP_WEDGE, false>(s, a, b, gc, ga, gb, P); break;
            case OP_REGR: launch_bwd_bal<OP_REGR, false>(s, a, b, gc, ga, gb, P); break;
        }
#undef CLF_BWD_BAL
    } else if (!force_generic && !force_tiled && blocked_plan(op, n, neg, nul, 3, P, ln, g, bl, lds)) {
#define CLF_BWD_CASE(OPV)                                                      \
    case OPV:                                                                  \
        if (ln) launch_bwd<OPV, true>(g, bl, lds, s, a, b, gc, ga, gb, P);     \
        else launch_bwd<OPV, false>(g, bl, lds, s, a, b, gc, ga, gb, P);       \
        break;
        switch (op) {
            CLF_BWD_CASE(OP_GEOM)
            CLF_BWD_CASE(OP_INNER)
            CLF_BWD_CASE(OP_LC)
            CLF_BWD_CASE(OP_RC)
            case OP_WEDGE: launch_bwd<OP_WEDGE, false>(g, bl, lds, s, a, b, gc, ga, gb, P); break;
            case OP_REGR: launch_bwd<OP_REGR, false>(g, bl, lds, s, a, b, gc, ga, gb, P); break;
        }
#undef CLF_BWD_CASE
    } else if (!force_generic && tiled_plan(op, n, neg, nul, P, ln, g)) {
#define CLF_BWD_TILED(OPV, LNV) \
    hipLaunchKernelGGL((prod_bwd_tiled<OPV, LNV>), g, dim3(256), 0, s, a, b, gc, ga, gb, P)
        switch (op) {
            case OP_GEOM: if (ln) CLF_BWD_TILED(OP_GEOM, true); else CLF_BWD_TILED(OP_GEOM, false); break;
            case OP_INNER: if (ln) CLF_BWD_TILED(OP_INNER, true); else CLF_BWD_TILED(OP_INNER, false); break;
            case OP_LC: if (ln) CLF_BWD_TILED(OP_LC, true); else CLF_BWD_TILED(OP_LC, false); break;
            case OP_RC: if (ln) CLF_BWD_TILED(OP_RC, true); else CLF_BWD_TILED(OP_RC, false); break;
            case OP_WEDGE: CLF_BWD_TILED(OP_WEDGE, false); break;
            case OP_REGR: CLF_BWD_TILED(OP_REGR, false); break;
        }
#undef CLF_BWD_TILED
    } else {
        const long long total = batch << n;
        const long long want = (total + 255) / 256;
        const unsigned blocks = (unsigned)(want < kMaxGrid ? want : kMaxGrid);
        if (ga)
            hipLaunchKernelGGL(prod_bwd_generic, dim3(blocks), dim3(256), 0, s, op, n, neg, nul, 0, b, gc,
                               (long long)ldg, ga, (long long)batch);
        if (gb)
            hipLaunchKernelGGL(prod_bwd_generic, dim3(blocks), dim3(256), 0, s, op, n, neg, nul, 1, a, gc,
                               (long long)ldg, gb, (long long)batch);
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
