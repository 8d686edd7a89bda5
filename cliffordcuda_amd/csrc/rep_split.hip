// Geometric product through the split matrix representation, for
//   n = 9,  Cl(p, q) with p - q = 1 (mod 8):       M_16(R) + M_16(R)
//   n = 10, the same 9 generators plus a null e_9:  three such products
// (the C5 signature Cl(9,0,1) is the second case).
//
// Split representation. Generators 0..7 form a real-type signature and use the
// real Pauli tables of the m = 16 path; e_8 maps to +-phi(E_8), E_8 = e_0...e_7
// (phi(E_8) anticommutes with the other generators and phi(E_8)^2 = e_8^2 holds
// for every such signature). Each label (x, z) is the image of one blade I0
// without e_8 and one blade I1 with it, so the conversion of a row a is
//   t_+-[x][z] = s(I0) a_I0 +- s(I1) a_I1,  W_+- = WHT_z(t_+-),  phi_+-[r][c] = W_+-[r ^ c][c]
// and the inverse is a_I0 = s(I0) (t_+ + t_-) / 2, a_I1 = s(I1) (t_+ - t_-) / 2
// after the inverse WHT (1/16). T(a) = (phi_+(a), phi_-(a)) is an algebra
// isomorphism onto block-diagonal pairs and orthogonal up to 32, so every
// forward and backward term is a pair sum
//   out = T^-1( sum_p opA(T(X_p)) opB(T(Y_p)) ),  op = identity or transpose,
// with the grade involution of an operand folded into its gather signs.
// The null generator on bit 9 (e_9 rightmost in every blade) gives
//   (L0 + L1 e9)(R0 + R1 e9) = L0 R0 + (L0 R1 + L1 R0^) e9
// and the backward terms
//   gL0 = G0 R0^T + G1 R1^T, gL1 = G1 (R0^)^T,
//   gR0 = L0^T G0 + (L1^)^T G1^, gR1 = L0^T G1
// (the grade involution commutes with the adjoint of left multiplication).
//
// Kernel. One wave takes two rows; lanes 16b .. 16b + 15 with b = 2r + s hold
// row r's block s (+ or -). The 4-block 16x16x1 MFMA then multiplies all four
// (row, sign) blocks at once with the operands built by xor shuffles; the pair
// sum continues the same accumulator. The two halves of the output are combined
// through one ds_swizzle (lane ^ 16) before the scatter to blade order.
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>

#include "rep_common.h"

namespace clf {

// Entry [x * 16 + z] for the label (x, z):
//   bits 0..8 blade I0 (without e_8), bits 9..17 blade I1 (with e_8),
//   bit 18 s(I0) = -1, bit 19 s(I1) = -1, bit 20 |I0| odd, bit 21 |I1| odd,
//   bit 22 popc(x & z) odd (the sign of the transposed conversion).
struct SplitTable {
    unsigned e[256];
};

constexpr int kPairMax = 2;
constexpr unsigned kTransA = 1u, kTransB = 2u, kHatX = 4u, kHatY = 8u;

// out[row] = T^-1( sum_p opA(T(X_p[row])) opB(T(Y_p[row])) ) for row < batch;
// X_p, Y_p, out are rows of 512 floats at the given strides (floats).
struct PairSum {
    const float* X[kPairMax];
    const float* Y[kPairMax];
    long long ldx[kPairMax];
    long long ldy[kPairMax];
    unsigned flags[kPairMax];
    int npairs;
    float* out;
    long long ldo;
    long long batch;
};

// bit 2z: sign of the I0 term, bit 2z + 1: sign of the I1 term of gather z
__device__ __forceinline__ unsigned gather_signs(const unsigned (&ent)[16], bool hat, bool tr, unsigned s) {
    const unsigned hm = hat ? ~0u : 0u, tm = tr ? ~0u : 0u;
    unsigned m = 0;
#pragma unroll
    for (int z = 0; z < 16; ++z) {
        const unsigned e = ent[z];
        const unsigned b0 = ((e >> 18) ^ ((e >> 20) & hm) ^ ((e >> 22) & tm)) & 1u;
        const unsigned b1 = ((e >> 19) ^ ((e >> 21) & hm) ^ ((e >> 22) & tm) ^ s) & 1u;
        m |= (b0 << (2 * z)) | (b1 << (2 * z + 1));
    }
    return m;
}

// t[z] = +-row[I0] +- row[I1] with the signs of m, then the WHT over z
__device__ __forceinline__ void gather_pair(const float* __restrict__ row, const unsigned (&ent)[16], unsigned m,
                                            float (&w)[16]) {
#pragma unroll
    for (int z = 0; z < 16; ++z) {
        const float v0 = row[ent[z] & 511u];
        const float v1 = row[(ent[z] >> 9) & 511u];
        const unsigned s0 = (m << (31 - 2 * z)) & 0x80000000u;
        const unsigned s1 = (m << (30 - 2 * z)) & 0x80000000u;
        w[z] = __uint_as_float(__float_as_uint(v0) ^ s0) + __uint_as_float(__float_as_uint(v1) ^ s1);
    }
    wht_inplace<16>(w);
}

// Two rows of 512 floats per operand: lane l moves float4 chunk (l + 64 j) & 127
// of row j >> 1 (j = 0..3) into named registers (an array here would be
// demoted to scratch across the loop).
#define CLF_SPLIT_FETCH(V0, V1, V2, V3, SRC, LD, ROW0)                                      \
    do {                                                                                   \
        long long r0_ = (ROW0), r1_ = (ROW0) + 1;                                          \
        r0_ = r0_ < batch ? r0_ : batch - 1; /* past the end: the last row, never stored */ \
        r1_ = r1_ < batch ? r1_ : batch - 1;                                               \
        const float4* p0_ = reinterpret_cast<const float4*>((SRC) + r0_ * (LD));          \
        const float4* p1_ = reinterpret_cast<const float4*>((SRC) + r1_ * (LD));          \
        V0 = p0_[lane];                                                                    \
        V1 = p0_[lane + 64];                                                               \
        V2 = p1_[lane];                                                                    \
        V3 = p1_[lane + 64];                                                               \
    } while (0)

#define CLF_SPLIT_STAGE(DST, V0, V1, V2, V3)                \
    do {                                                    \
        float4* d_ = reinterpret_cast<float4*>(DST);        \
        d_[lane] = V0;                                      \
        d_[lane + 64] = V1;                                 \
        d_[lane + 128] = V2;                                \
        d_[lane + 192] = V3;                                \
    } while (0)

// Stages of one wave: (group g, pair 0), [(g, pair 1)], (g + stride, pair 0) ...
// Each stage stages the prefetched rows in LDS, prefetches the next stage, and
// gathers + converts; the last pair of a group finishes the group's output.
template <int NP>
__device__ __forceinline__ void split_pairs_body(const PairSum& P, const SplitTable& T) {
    __shared__ float lds[4][2048];  // per wave: staged X rows | staged Y rows; later the relayout, then out rows
    static_assert(2048 >= kRelayoutFloats, "relayout must fit the wave's LDS slots");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = lane >> 4, r = b >> 1;
    const unsigned s = (unsigned)b & 1u, x = lane & 15u;
    float* sx = &lds[wave][0];
    float* sy = sx + 1024;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z];
    // A operand: W of X (W' if transposed); B operand (lane x gives column x of
    // opB): W' of Y unless opB transposes, then W
    const unsigned f0 = P.flags[0], f1 = P.flags[1];
    const unsigned mx0 = gather_signs(ent, f0 & kHatX, f0 & kTransA, s);
    const unsigned my0 = gather_signs(ent, f0 & kHatY, !(f0 & kTransB), s);
    const unsigned mx1 = gather_signs(ent, f1 & kHatX, f1 & kTransA, s);
    const unsigned my1 = gather_signs(ent, f1 & kHatY, !(f1 & kTransB), s);
    // output: lane + writes I0, lane - writes I1, each with its blade sign
    unsigned mo = 0;
#pragma unroll
    for (int z = 0; z < 16; ++z) mo |= ((ent[z] >> (18 + s)) & 1u) << z;
    const float pm = s ? -1.f : 1.f;

    const long long batch = P.batch;
    const long long ngroups = (batch + 1) / 2;
    const long long gstride = (long long)gridDim.x * 4;
    const float* X0 = P.X[0];
    const float* Y0 = P.Y[0];
    const float* X1 = P.X[1];
    const float* Y1 = P.Y[1];
    const long long lx0 = P.ldx[0], ly0 = P.ldy[0], lx1 = P.ldx[1], ly1 = P.ldy[1];
    long long g = (long long)blockIdx.x * 4 + wave;
    float4 ax0, ax1, ax2, ax3, ay0, ay1, ay2, ay3;
    CLF_SPLIT_FETCH(ax0, ax1, ax2, ax3, X0, lx0, 2 * g);
    CLF_SPLIT_FETCH(ay0, ay1, ay2, ay3, Y0, ly0, 2 * g);
    for (; g < ngroups; g += gstride) {
        // opaque per-group copies of the sign masks: otherwise the shifted
        // sign words of every gather are hoisted out of the loop into VGPRs
        unsigned m0x = mx0, m0y = my0, m1x = mx1, m1y = my1, mout = mo;
        asm volatile("" : "+v"(m0x), "+v"(m0y), "+v"(m1x), "+v"(m1y), "+v"(mout));
        // and of the table entries, so that the gather and scatter addresses
        // are formed where they are used instead of living across the loop
        unsigned en[16];
#pragma unroll
        for (int z = 0; z < 16; ++z) {
            en[z] = ent[z];
            asm volatile("" : "+v"(en[z]));
        }
        // pair 0
        CLF_SPLIT_STAGE(sx, ax0, ax1, ax2, ax3);
        CLF_SPLIT_STAGE(sy, ay0, ay1, ay2, ay3);
        if constexpr (NP == 2) {
            CLF_SPLIT_FETCH(ax0, ax1, ax2, ax3, X1, lx1, 2 * g);
            CLF_SPLIT_FETCH(ay0, ay1, ay2, ay3, Y1, ly1, 2 * g);
        } else {
            CLF_SPLIT_FETCH(ax0, ax1, ax2, ax3, X0, lx0, 2 * (g + gstride));
            CLF_SPLIT_FETCH(ay0, ay1, ay2, ay3, Y0, ly0, 2 * (g + gstride));
        }
        wave_lds_sync();
        floatx16 acc;
        {
            float wx[16], wy[16];
            gather_pair(sx + r * 512, en, m0x, wx);
            gather_pair(sy + r * 512, en, m0y, wy);
            wave_lds_sync();
            acc = mfma_chain(wx, wy);
        }
        if constexpr (NP == 2) {
            CLF_SPLIT_STAGE(sx, ax0, ax1, ax2, ax3);
            CLF_SPLIT_STAGE(sy, ay0, ay1, ay2, ay3);
            CLF_SPLIT_FETCH(ax0, ax1, ax2, ax3, X0, lx0, 2 * (g + gstride));
            CLF_SPLIT_FETCH(ay0, ay1, ay2, ay3, Y0, ly0, 2 * (g + gstride));
            wave_lds_sync();
            float wx[16], wy[16];
            gather_pair(sx + r * 512, en, m1x, wx);
            gather_pair(sy + r * 512, en, m1y, wy);
            wave_lds_sync();
            acc = mfma_chain_acc(acc, wx, wy, std::make_integer_sequence<unsigned, 16>{});
        }
        relayout_store(sx, acc, lane);
        wave_lds_sync();
        float w[16];
        relayout_load(sx, b, x, w);
        wave_lds_sync();
        wht_inplace<16>(w);
#pragma unroll
        for (int z = 0; z < 16; ++z) {
            const float other = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(w[z]), 0x401F));
            const float v = __builtin_fmaf(pm, w[z], other) * (1.f / 32.f);
            const unsigned blade = s ? ((en[z] >> 9) & 511u) : (en[z] & 511u);
            sx[r * 512 + blade] = __uint_as_float(__float_as_uint(v) ^ (((mout >> z) & 1u) << 31));
        }
        wave_lds_sync();
        // rows past the end were computed from clamped copies of the last row:
        // bit-identical, stored to the last row again
        {
            const float4* src = reinterpret_cast<const float4*>(sx);
            const float4 o0 = src[lane], o1 = src[lane + 64], o2 = src[lane + 128], o3 = src[lane + 192];
            long long r0 = 2 * g, r1 = 2 * g + 1;
            r0 = r0 < batch ? r0 : batch - 1;
            r1 = r1 < batch ? r1 : batch - 1;
            float4* d0 = reinterpret_cast<float4*>(P.out + r0 * P.ldo);
            float4* d1 = reinterpret_cast<float4*>(P.out + r1 * P.ldo);
            d0[lane] = o0;
            d0[lane + 64] = o1;
            d1[lane] = o2;
            d1[lane + 64] = o3;
        }
        wave_lds_sync();
    }
}

// ---- fused kernels for n = 10 with the null e_9 ------------------------------
// The pair sums of one direction read each operand half once (the separate
// pair-sum launches read the shared halves once per sum):
//   KIND 0 (forward): out0 = L0 R0,                   out1 = L0 R1 + L1 R0^
//   KIND 1 (dL):      out0 = G0 R0^T + G1 R1^T,       out1 = G1 (R0^)^T
//   KIND 2 (dR):      out0 = L0^T G0 + (L1^)^T G1^,   out1 = L0^T G1
// with X = (L, G, L) and Y = (R, R, G) for KIND 0, 1, 2 and out0 / out1 the
// halves of one output row. Stage 0 stages (X0, Y0), stage 1 (X1, Y1); the
// operand forms both stages use stay in registers; two sign variants of one
// half come from one gather.
struct FusedSplit {
    const float* X;  // rows of 1024 floats (halves at +0, +512)
    const float* Y;
    float* out;
    long long batch;
    long long ldx, ldy;  // floats between rows: 1024, or 0 for one row broadcast over the batch
};

// The fused kernels' gathers and scatters at LDS byte addresses formed once per
// lane: pa0[z] / pa1[z] = the lane's row in region 0 plus blade I0 / I1 of
// entry z, po[z] the one of the lane's output half; a region's offset
// (REG * 4096 bytes) goes into the instruction's immediate offset, so a
// gather or scatter element needs no address arithmetic.
// Blade I1 of every entry is I0 ^ 511 (the host table checks it), so pa1[z] =
// c1 - pa0[z] with c1 = 2 * row + 4 * 511: the kernel with the fewest free
// registers (PICK) keeps c1 instead of pa1.
template <unsigned REG, bool PICK>
__device__ __forceinline__ void gather_pair_at(const unsigned (&pa0)[16], const unsigned (&pa1)[16], unsigned c1,
                                               unsigned m, float (&w)[16]) {
#pragma unroll
    for (int z = 0; z < 16; ++z) {
        const float v0 = lds_load(pa0[z] + REG * 4096u);
        const float v1 = lds_load((PICK ? c1 - pa0[z] : pa1[z]) + REG * 4096u);
        const unsigned s0 = (m << (31 - 2 * z)) & 0x80000000u;
        const unsigned s1 = (m << (30 - 2 * z)) & 0x80000000u;
        w[z] = __uint_as_float(__float_as_uint(v0) ^ s0) + __uint_as_float(__float_as_uint(v1) ^ s1);
    }
    wht_inplace<16>(w);
}

// the output half's row, the inverse conversion of acc through the relayout
// at rel, written at po[z] + ROWS * 4096 bytes (PICK: po is chosen per
// element from pa0 and c1 - pa0 by the lane mask ms, which keeps 32 fewer
// registers live)
template <unsigned ROWS, bool PICK>
__device__ __forceinline__ void split_finish_at(const floatx16& acc, float* __restrict__ rel, const unsigned (&po)[16],
                                                const unsigned (&pa0)[16], unsigned c1, unsigned ms, unsigned mout,
                                                int lane) {
    const int b = lane >> 4;
    const unsigned s = (unsigned)b & 1u, x = lane & 15u;
    const float pm = s ? -1.f : 1.f;
    relayout_store(rel, acc, lane);
    wave_lds_sync();
    float w[16];
    relayout_load(rel, b, x, w);
    wave_lds_sync();
    wht_inplace<16>(w);
#pragma unroll
    for (int z = 0; z < 16; ++z) {
        const float other = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(w[z]), 0x401F));
        const float v = __builtin_fmaf(pm, w[z], other) * (1.f / 32.f);
        const unsigned at = PICK ? (((c1 - pa0[z]) & ms) | (pa0[z] & ~ms)) : po[z];
        lds_store(at + ROWS * 4096u, __uint_as_float(__float_as_uint(v) ^ (((mout >> z) & 1u) << 31)));
    }
    wave_lds_sync();
}

// the two half rows of group g (rows 2g, 2g + 1 at dst, row stride 1024)
__device__ __forceinline__ void split_emit(const float* __restrict__ rows, float* __restrict__ dst, long long g,
                                           long long batch, int lane) {
    const float4* src = reinterpret_cast<const float4*>(rows);
    const float4 o0 = src[lane], o1 = src[lane + 64], o2 = src[lane + 128], o3 = src[lane + 192];
    long long r0 = 2 * g, r1 = 2 * g + 1;
    r0 = r0 < batch ? r0 : batch - 1;  // clamped rows repeat the last row's values
    r1 = r1 < batch ? r1 : batch - 1;
    float4* d0 = reinterpret_cast<float4*>(dst + r0 * 1024);
    float4* d1 = reinterpret_cast<float4*>(dst + r1 * 1024);
    d0[lane] = o0;
    d0[lane + 64] = o1;
    d1[lane] = o2;
    d1[lane + 64] = o3;
}

// LDS per wave: four regions of two half rows (1024 floats each) so that the
// stage-0 halves stay staged through stage 1 and are gathered again where a
// sum needs them (instead of holding their operands in registers). Each
// output's relayout (1280 floats) uses regions whose halves are consumed by
// then, and its rows wait in a region the next stage does not overwrite: a
// wave's loads and stores share one completion counter that is drained before
// staged rows are used, so the rows are stored right after the next stage's
// wait rather than just before it (the forward, whose first half is complete
// before stage 1, keeps its rows in a fifth region).
template <int KIND>
struct FusedRegions {
    // offsets (in units of 1024 floats) of X0, Y0, X1, Y1
    static constexpr int x0 = 0;
    static constexpr int y0 = KIND == 1 ? 3 : 1;
    static constexpr int x1 = 2;
    static constexpr int y1 = KIND == 1 ? 1 : 3;
    // relayout areas and row slots of out0 / out1
    static constexpr int rel0 = KIND == 0 ? 2 : (KIND == 1 ? 0 : 1);
    static constexpr int rows0 = KIND == 0 ? 4 : (KIND == 1 ? 1 : 2);
    static constexpr int rel1 = KIND == 0 ? 0 : (KIND == 1 ? 2 : 0);
    static constexpr int rows1 = KIND == 0 ? 4 : (KIND == 1 ? 2 : 3);
    static constexpr int regions = KIND == 0 ? 5 : 4;
};

// waves per workgroup of the fused kernels
constexpr int kFusedWaves = 4;

template <int KIND>
__global__ __launch_bounds__(64 * kFusedWaves) __attribute__((amdgpu_waves_per_eu(2))) void split_fused_kernel(FusedSplit P, SplitTable T) {
    using RG = FusedRegions<KIND>;
    __shared__ float lds[kFusedWaves][RG::regions * 1024];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int b = lane >> 4, r = b >> 1;
    const unsigned s = (unsigned)b & 1u, x = lane & 15u;
    float* base = &lds[wave][0];
    float* sx0 = base + RG::x0 * 1024;
    float* sy0 = base + RG::y0 * 1024;
    float* sx1 = base + RG::x1 * 1024;
    float* sy1 = base + RG::y1 * 1024;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z];
    // sign masks of the operand forms: A operand (W of X, W' if transposed),
    // B operand (W' of Y unless transposed, then W); hats folded in
    unsigned mx0, my0, my0b, mx1, my1, my1b;
    if (KIND == 0) {
        mx0 = gather_signs(ent, false, false, s);   // L0
        my0 = gather_signs(ent, false, true, s);    // R0
        my0b = gather_signs(ent, true, true, s);    // R0^
        mx1 = gather_signs(ent, false, false, s);   // L1
        my1 = gather_signs(ent, false, true, s);    // R1
        my1b = 0u;
    } else if (KIND == 1) {
        mx0 = gather_signs(ent, false, false, s);   // G0
        my0 = gather_signs(ent, false, false, s);   // R0^T
        my0b = gather_signs(ent, true, false, s);   // (R0^)^T
        mx1 = gather_signs(ent, false, false, s);   // G1
        my1 = gather_signs(ent, false, false, s);   // R1^T
        my1b = 0u;
    } else {
        mx0 = gather_signs(ent, false, true, s);    // L0^T
        my0 = gather_signs(ent, false, true, s);    // G0
        my0b = 0u;
        mx1 = gather_signs(ent, true, true, s);     // (L1^)^T
        my1 = gather_signs(ent, true, true, s);     // G1^
        my1b = gather_signs(ent, false, true, s);   // G1
    }
    unsigned mo = 0;
#pragma unroll
    for (int z = 0; z < 16; ++z) mo |= ((ent[z] >> (18 + s)) & 1u) << z;
    // LDS byte addresses of the lane's blades in its row of region 0 (kept:
    // opaque, so they are not re-derived from the entries in the loop)
    // (the forward, whose registers are fullest, picks the output half's
    // addresses per element instead of keeping them)
    constexpr bool kPick = KIND == 0;
    unsigned pa0[16], pa1[16], po[16];
    unsigned ms = s ? ~0u : 0u;
    const unsigned lb = lds_byte_addr(base) + (unsigned)r * 2048u;
    unsigned c1 = 2u * lb + 4u * 511u;
    asm volatile("" : "+v"(ms), "+v"(c1));
#pragma unroll
    for (int z = 0; z < 16; ++z) {
        pa0[z] = lb + 4u * (ent[z] & 511u);
        asm volatile("" : "+v"(pa0[z]));
        if constexpr (!kPick) {
            pa1[z] = lb + 4u * ((ent[z] >> 9) & 511u);
            po[z] = s ? pa1[z] : pa0[z];
            asm volatile("" : "+v"(pa1[z]), "+v"(po[z]));
        }
    }

    const long long batch = P.batch;
    const long long ngroups = (batch + 1) / 2;
    const long long gstride = (long long)gridDim.x * kFusedWaves;
    const float* X0 = P.X;
    const float* Y0 = P.Y;
    const float* X1 = P.X + 512;
    const float* Y1 = P.Y + 512;
    const long long g0 = (long long)blockIdx.x * kFusedWaves + wave;
    long long g = g0;
    float4 ax0, ax1, ax2, ax3, ay0, ay1, ay2, ay3;
    CLF_SPLIT_FETCH(ax0, ax1, ax2, ax3, X0, P.ldx, 2 * g);
    CLF_SPLIT_FETCH(ay0, ay1, ay2, ay3, Y0, P.ldy, 2 * g);
    for (; g < ngroups; g += gstride) {
        unsigned m_x0 = mx0, m_y0 = my0, m_y0b = my0b, m_x1 = mx1, m_y1 = my1, m_y1b = my1b, mout = mo;
        asm volatile("" : "+v"(m_x0), "+v"(m_y0), "+v"(m_y0b), "+v"(m_x1), "+v"(m_y1), "+v"(m_y1b), "+v"(mout));
        // stage 0: X0, Y0 (staged until the group ends)
        CLF_SPLIT_STAGE(sx0, ax0, ax1, ax2, ax3);
        CLF_SPLIT_STAGE(sy0, ay0, ay1, ay2, ay3);
        CLF_SPLIT_FETCH(ax0, ax1, ax2, ax3, X1, P.ldx, 2 * g);
        CLF_SPLIT_FETCH(ay0, ay1, ay2, ay3, Y1, P.ldy, 2 * g);
        if (g != g0) {  // uniform: the previous group's rows wait in regions stage 0 does not touch
            if (KIND != 0) split_emit(base + RG::rows0 * 1024, P.out, g - gstride, batch, lane);
            split_emit(base + RG::rows1 * 1024, P.out + 512, g - gstride, batch, lane);
        }
        wave_lds_sync();
        floatx16 acc0;
        {
            float wx[16], wy[16];
            gather_pair_at<RG::x0, kPick>(pa0, pa1, c1, m_x0, wx);
            gather_pair_at<RG::y0, kPick>(pa0, pa1, c1, m_y0, wy);
            acc0 = mfma_chain(wx, wy);
        }
        if constexpr (KIND == 0) {  // C0 = L0 R0 is complete; X1 / Y1 regions are still free
            split_finish_at<RG::rows0, kPick>(acc0, base + RG::rel0 * 1024, po, pa0, c1, ms, mout, lane);
        }
        // stage 1: X1, Y1
        CLF_SPLIT_STAGE(sx1, ax0, ax1, ax2, ax3);
        CLF_SPLIT_STAGE(sy1, ay0, ay1, ay2, ay3);
        CLF_SPLIT_FETCH(ax0, ax1, ax2, ax3, X0, P.ldx, 2 * (g + gstride));
        CLF_SPLIT_FETCH(ay0, ay1, ay2, ay3, Y0, P.ldy, 2 * (g + gstride));
        if constexpr (KIND == 0) split_emit(base + RG::rows0 * 1024, P.out, g, batch, lane);
        wave_lds_sync();
        if constexpr (KIND == 0) {
            // C1 = L0 R1 + L1 R0^
            floatx16 acc1;
            {
                float wx[16], wy[16];
                gather_pair_at<RG::x0, kPick>(pa0, pa1, c1, m_x0, wx);
                gather_pair_at<RG::y1, kPick>(pa0, pa1, c1, m_y1, wy);
                acc1 = mfma_chain(wx, wy);
            }
            {
                float wx[16], wy[16];
                gather_pair_at<RG::x1, kPick>(pa0, pa1, c1, m_x1, wx);
                gather_pair_at<RG::y0, kPick>(pa0, pa1, c1, m_y0b, wy);
                acc1 = mfma_chain_acc(acc1, wx, wy, std::make_integer_sequence<unsigned, 16>{});
            }
            wave_lds_sync();
            split_finish_at<RG::rows1, kPick>(acc1, base + RG::rel1 * 1024, po, pa0, c1, ms, mout, lane);
        } else if constexpr (KIND == 1) {
            // out0 += G1 R1^T; out1 = G1 (R0^)^T
            float wx[16];
            gather_pair_at<RG::x1, kPick>(pa0, pa1, c1, m_x1, wx);
            {
                float wy[16];
                gather_pair_at<RG::y1, kPick>(pa0, pa1, c1, m_y1, wy);
                acc0 = mfma_chain_acc(acc0, wx, wy, std::make_integer_sequence<unsigned, 16>{});
            }
            wave_lds_sync();
            split_finish_at<RG::rows0, kPick>(acc0, base + RG::rel0 * 1024, po, pa0, c1, ms, mout, lane);
            floatx16 acc1;
            {
                float wy[16];
                gather_pair_at<RG::y0, kPick>(pa0, pa1, c1, m_y0b, wy);
                acc1 = mfma_chain(wx, wy);
            }
            wave_lds_sync();
            split_finish_at<RG::rows1, kPick>(acc1, base + RG::rel1 * 1024, po, pa0, c1, ms, mout, lane);
        } else {
            // out0 += (L1^)^T G1^; out1 = L0^T G1
            {
                float wx[16], wy[16];
                gather_pair_at<RG::x1, kPick>(pa0, pa1, c1, m_x1, wx);
                gather_pair_at<RG::y1, kPick>(pa0, pa1, c1, m_y1, wy);
                acc0 = mfma_chain_acc(acc0, wx, wy, std::make_integer_sequence<unsigned, 16>{});
            }
            wave_lds_sync();
            split_finish_at<RG::rows0, kPick>(acc0, base + RG::rel0 * 1024, po, pa0, c1, ms, mout, lane);
            floatx16 acc1;
            {
                float wx[16], wy[16];
                gather_pair_at<RG::x0, kPick>(pa0, pa1, c1, m_x0, wx);
                gather_pair_at<RG::y1, kPick>(pa0, pa1, c1, m_y1b, wy);
                acc1 = mfma_chain(wx, wy);
            }
            wave_lds_sync();
            split_finish_at<RG::rows1, kPick>(acc1, base + RG::rel1 * 1024, po, pa0, c1, ms, mout, lane);
        }
    }
    if (g != g0) {
        if (KIND != 0) split_emit(base + RG::rows0 * 1024, P.out, g - gstride, batch, lane);
        split_emit(base + RG::rows1 * 1024, P.out + 512, g - gstride, batch, lane);
    }
}

#undef CLF_SPLIT_FETCH
#undef CLF_SPLIT_STAGE

// One pair fits three waves per SIMD without spilling; two pairs keep the
// accumulator live across both and run at the compiler's default (two).
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void split_pairs1_kernel(PairSum P,
                                                                                                  SplitTable T) {
    split_pairs_body<1>(P, T);
}

__global__ __launch_bounds__(256) void split_pairs2_kernel(PairSum P, SplitTable T) { split_pairs_body<2>(P, T); }

// ---- host side --------------------------------------------------------------

// Table for a 9-generator signature (bit g of neg9: e_g^2 = -1), or false if it
// is not p - q = 1 (mod 8).
static bool split_table_build(uint32_t neg9, SplitTable& T) {
    const int q = host_popc(neg9 & 511u), p = 9 - q;
    if ((((p - q) % 8) + 8) % 8 != 1) return false;
    unsigned gx[16], gz[16];
    if (!rep_generators(8, neg9 & 255u, gx, gz)) return false;
    unsigned lab[256], sg[256];  // label x << 4 | z and sign bit of the 8-generator blades
    for (unsigned I = 0; I < 256; ++I) {
        unsigned x = 0, z = 0;
        bool neg = false;
        for (int g = 0; g < 8; ++g)
            if ((I >> g) & 1u) {
                if (host_popc(z & gx[g]) & 1) neg = !neg;
                x ^= gx[g];
                z ^= gz[g];
            }
        lab[I] = (x << 4) | z;
        sg[I] = neg ? 1u : 0u;
    }
    const unsigned xE = lab[255] >> 4, zE = lab[255] & 15u, sE = sg[255];
    unsigned i0[256], i1[256], s0[256], s1[256];
    for (unsigned I = 0; I < 512; ++I) {
        const unsigned Il = I & 255u;
        unsigned x = lab[Il] >> 4, z = lab[Il] & 15u, sgn = sg[Il];
        if (I >> 8) {  // phi(e_I') phi(E_8)
            if (host_popc(z & xE) & 1) sgn ^= 1u;
            sgn ^= sE;
            x ^= xE;
            z ^= zE;
        }
        const unsigned key = x * 16 + z;
        if (I >> 8) {
            i1[key] = I;
            s1[key] = sgn;
        } else {
            i0[key] = I;
            s0[key] = sgn;
        }
    }
    for (unsigned key = 0; key < 256; ++key) {
        // the kernels address blade I1 as I0 ^ 511 (the label of I | e_8 is
        // the label of I times that of the Cl(8) pseudoscalar)
        if (i1[key] != (i0[key] ^ 511u)) return false;
        const unsigned x = key >> 4, z = key & 15u;
        T.e[key] = i0[key] | (i1[key] << 9) | (s0[key] << 18) | (s1[key] << 19) |
                   ((unsigned)(host_popc(i0[key]) & 1) << 20) | ((unsigned)(host_popc(i1[key]) & 1) << 21) |
                   ((unsigned)(host_popc(x & z) & 1) << 22);
    }
    return true;
}

static bool split_table(uint32_t neg9, SplitTable& T) {
    static TableCache<SplitTable, 512> cache;
    return cache.get((int)(neg9 & 0x1ffu), T, [&](SplitTable& t) { return split_table_build(neg9 & 0x1ffu, t); });
}

// n = 9 without null generators, or n = 10 whose only null generator is e_9
bool split_applicable(int op, int n, uint32_t neg, uint32_t nul) {
    if (op != CLF_OP_GEOM) return false;
    if (!((n == 9 && nul == 0u) || (n == 10 && nul == (1u << 9)))) return false;
    SplitTable T;
    return split_table(neg & 511u, T);
}

// ldx / ldy: floats between rows of X / Y (0: one row broadcast over the batch;
// -1: the launch's ld_in)
struct PairSpec {
    const float* X;
    const float* Y;
    unsigned flags;
    long long ldx = -1, ldy = -1;
};

static int launch_pairs(const SplitTable& T, const PairSpec* ps, int npairs, long long ld_in, float* out,
                        long long ld_out, int64_t batch, hipStream_t s) {
    PairSum P{};
    for (int p = 0; p < kPairMax; ++p) {
        const PairSpec& q = ps[p < npairs ? p : 0];
        P.X[p] = q.X;
        P.Y[p] = q.Y;
        P.ldx[p] = q.ldx < 0 ? ld_in : q.ldx;
        P.ldy[p] = q.ldy < 0 ? ld_in : q.ldy;
        P.flags[p] = q.flags;
    }
    P.npairs = npairs;
    P.out = out;
    P.ldo = ld_out;
    P.batch = batch;
    // at most the resident grid, then the waves walk the batch and each wave's
    // next group is prefetched during its current one (16384 rows at n = 10:
    // ~10 % faster than a grid of four times the resident workgroups)
    const long long groups = (batch + 1) / 2;
    const void* k = npairs == 2 ? (const void*)split_pairs2_kernel : (const void*)split_pairs1_kernel;
    const dim3 grid(resident_grid(k, 256, 0, (groups + 3) / 4));
    if (npairs == 2) hipLaunchKernelGGL(split_pairs2_kernel, grid, dim3(256), 0, s, P, T);
    else hipLaunchKernelGGL(split_pairs1_kernel, grid, dim3(256), 0, s, P, T);
    return CLF_OK;
}

// n = 10: one launch per direction and gradient reads each operand half once
// (CLF_SPLIT_PATH=pairs runs the separate pair-sum launches instead).
static bool split_fused_enabled() { return !options().split_pairs; }

template <int KIND>
static void launch_fused(const SplitTable& T, const float* X, const float* Y, float* out, int64_t batch,
                         hipStream_t s, long long ldx = 1024, long long ldy = 1024) {
    FusedSplit P{X, Y, out, (long long)batch, ldx, ldy};
    const long long groups = (batch + 1) / 2;
    // grid rule of the pair sums: at most the resident workgroups
    const dim3 grid(resident_grid((const void*)split_fused_kernel<KIND>, 64 * kFusedWaves, 0,
                                  (groups + kFusedWaves - 1) / kFusedWaves));
    hipLaunchKernelGGL(split_fused_kernel<KIND>, grid, dim3(64 * kFusedWaves), 0, s, P, T);
}

int split_fwd(int n, uint32_t neg, const float* a, const float* b, float* c, int64_t batch, void* stream) {
    SplitTable T;
    if (!split_table(neg & 511u, T)) return set_error(CLF_ERR_UNSUPPORTED, "signature has no split representation");
    hipStream_t s = (hipStream_t)stream;
    if (n == 9) {
        const PairSpec ab[1] = {{a, b, 0u}};
        launch_pairs(T, ab, 1, 512, c, 512, batch, s);
    } else if (split_fused_enabled()) {
        launch_fused<0>(T, a, b, c, batch, s);
    } else {
        const PairSpec c0[1] = {{a, b, 0u}};
        const PairSpec c1[2] = {{a, b + 512, 0u}, {a + 512, b, kHatY}};
        launch_pairs(T, c0, 1, 1024, c, 1024, batch, s);
        launch_pairs(T, c1, 2, 1024, c + 512, 1024, batch, s);
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

// gc's rows are ldg floats apart: 2^n, or 0 for one row broadcast over the batch
int split_bwd(int n, uint32_t neg, const float* a, const float* b, const float* gc, int64_t ldg, float* ga,
              float* gb, int64_t batch, void* stream) {
    SplitTable T;
    if (!split_table(neg & 511u, T)) return set_error(CLF_ERR_UNSUPPORTED, "signature has no split representation");
    hipStream_t s = (hipStream_t)stream;
    const long long lg = (long long)ldg;
    if (n == 9) {
        if (ga) {
            const PairSpec p[1] = {{gc, b, kTransB, lg, -1}};
            launch_pairs(T, p, 1, 512, ga, 512, batch, s);
        }
        if (gb) {
            const PairSpec p[1] = {{a, gc, kTransA, -1, lg}};
            launch_pairs(T, p, 1, 512, gb, 512, batch, s);
        }
    } else if (split_fused_enabled()) {
        if (ga) launch_fused<1>(T, gc, b, ga, batch, s, lg, 1024);
        if (gb) launch_fused<2>(T, a, gc, gb, batch, s, 1024, lg);
    } else {
        const float *L0 = a, *L1 = a + 512, *R0 = b, *R1 = b + 512, *G0 = gc, *G1 = gc + 512;
        if (ga) {
            const PairSpec l0[2] = {{G0, R0, kTransB, lg, -1}, {G1, R1, kTransB, lg, -1}};
            const PairSpec l1[1] = {{G1, R0, kTransB | kHatY, lg, -1}};
            launch_pairs(T, l0, 2, 1024, ga, 1024, batch, s);
            launch_pairs(T, l1, 1, 1024, ga + 512, 1024, batch, s);
        }
        if (gb) {
            const PairSpec r0[2] = {{L0, G0, kTransA, -1, lg}, {L1, G1, kTransA | kHatX | kHatY, -1, lg}};
            const PairSpec r1[1] = {{L0, G1, kTransA, -1, lg}};
            launch_pairs(T, r0, 2, 1024, gb, 1024, batch, s);
            launch_pairs(T, r1, 1, 1024, gb + 512, 1024, batch, s);
        }
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
