// Rotor sandwich for n = 8 on the matrix cores.
//
// y = ~R x R of a Euclidean rotor is the outermorphism Lambda(Q) of its
// rotation Q, which acts on bit-pattern blade coefficients independently of the
// algebra's metric (reference: the composite of src/cliffordcuda/algebra.py:343-373
// applies the Euclidean rotor whatever the metric). For n = 8 it is computed in
// the real 16 x 16 representation phi of Cl(8,0):
//   phi(y)  = U^T phi(x) U,   U = phi(R)           (forward)
//   phi(gx) = U phi(gy) U^T                          (transpose, the x gradient)
// two 16 x 16 x 16 products per row instead of the 28 plane rotations of the
// register chain (rotor.hip). U is built by the compile kernel from the
// half-angle factors of the Givens chain and stored in the rotor state.
//
// Bivector gradient. The chain kernels accumulate per plane
//   K_pq = sum_rows sum_pairs sig (x_J gx_I - x_I gx_J);
// in the representation the same sums are
//   K_pq = -(1/32) < sum_rows phi(x)^T phi(gx) + phi(x) phi(gx)^T, phi(e_p e_q) >,
// a 16 x 16 matrix accumulated in the MFMA registers over a wave's rows and
// contracted with the 28 signed permutations phi(e_p e_q) once per workgroup,
// which writes the same per-workgroup partial K as the chain kernel; the
// gamma finalize and the compile backward are shared.
//
// Layout per wave: four rows (one per 16-lane block of the 4-block MFMA), the
// conversions and LDS relayout of the geometric-product kernels (rep.hip).
// The product of the first factor comes out with its row index in the
// registers; transpose_blocks moves it, with permlane swaps, to the operand
// layout of the second product, so the two products of a sandwich need no LDS
// round trip between them.
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "rep_common.h"

namespace clf {

// op[k] = U[x][k] (ROWS) or U[k][x] for lane x; U row-major 16 x 16
template <bool ROWS>
__device__ __forceinline__ void load_spin_operand(const float* __restrict__ U, unsigned x, float (&op)[16]) {
    // once per kernel: plain loads, so the state needs no 16-byte alignment
#pragma unroll
    for (int k = 0; k < 16; ++k) op[k] = ROWS ? U[x * 16 + k] : U[k * 16 + x];
}

// phi(y) = V^T phi(x) V with V = U (forward, TRANS = false) or V = U^T (the
// transpose of the action). vop[k] = V[k][x] is both the B operand of
// phi(x) V and the A operand of V^T (phi(x) V).
//
// Memory pipeline (both rotor16 kernels). A wave's global loads and stores
// share one completion counter, and the compiler waits for all of them before
// the staged rows are used, so a group's results are stored from their own LDS
// slot halfway through the next group's work, not at the end of their own:
// when the wave next waits, those stores have had half a group's time to
// complete. The wave index is made wave-uniform (readfirstlane), so the row
// bookkeeping runs on the scalar unit and the row clamps need no branches.
constexpr int kApplyWaveFloats = kRelayoutFloats + 4 * 256;  // staged x, then the relayout | the previous group's y

// ldx: floats between the input's rows (256, or 0 for one row broadcast over
// the batch: the transposed action on the gradient of a sum)
template <bool TRANS, bool NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void rotor16_apply_kernel(
    const float* __restrict__ U, const float* __restrict__ X, float* __restrict__ Y, long long batch, RepTable T,
    long long ldx) {
    __shared__ float lds[4][kApplyWaveFloats];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* sx = &lds[wave][0];
    float* su = sx + kRelayoutFloats;
    const unsigned oddx = (rb & 1) ? T.odd_xor : 0u, oddc = T.odd_xor >> 2;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z] ^ oddx;
    float vop[16];
    load_spin_operand<TRANS>(U, x, vop);
    // V / 4 on both sides: phi(y) comes out with the 1/16 of the inverse
    // conversion already applied (exact: a power of two)
#pragma unroll
    for (int k = 0; k < 16; ++k) vop[k] *= 0.25f;
    const floatx16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

    const long long stride = (long long)gridDim.x * 4 * 4;
    const long long rfirst = ((long long)blockIdx.x * 4 + wave) * 4;
    long long row0 = rfirst;
    Pre16 px = fetch16<NT>(X, row0, batch, lane, ldx);
    for (; row0 < batch; row0 += stride) {
        // the table values are re-derived where they are used rather than kept
        // in registers across the loop (register pressure sets the occupancy)
#pragma unroll
        for (int z = 0; z < 16; ++z) asm volatile("" : "+v"(ent[z]));
        stage16(sx, px, lane, oddc);
        px = fetch16<NT>(X, row0 + stride, batch, lane, ldx);
        wave_lds_sync();
        float wx[16];
        gather16<0>(sx + rb * 256, ent, wx);
        wave_lds_sync();
        wht_inplace<16>(wx);
        const floatx16 p = mfma_chain_pre<true, false>(zero, wx, vop, std::make_integer_sequence<unsigned, 16>{});
        float pop[16];
        transpose_blocks(p, pop);
        const floatx16 acc = mfma_chain_pre<false, false>(zero, vop, pop, std::make_integer_sequence<unsigned, 16>{});
        if (row0 != rfirst) store16<NT>(Y, su, row0 - stride, batch, lane, oddc);  // uniform
        relayout_store(sx, acc, lane);
        wave_lds_sync();
        float wc[16];
        relayout_load(sx, rb, x, wc);
        unconvert16_prescaled(wc, su + rb * 256, ent);
        wave_lds_sync();
    }
    if (row0 != rfirst) store16<NT>(Y, su, row0 - stride, batch, lane, oddc);
}

// gx = Lambda(Q)^T gy (if GX) and the workgroup's partial K (C(8,2) floats at
// gamma_ws[blockIdx.x * 28]). uop[k] = U[x][k] / 4 is the B operand of
// phi(gy) U^T and the A operand of U (phi(gy) U^T), so phi(gx) comes out with
// the 1/16 of the inverse conversion already applied (exact: a power of two).
//
// The kernel is issue-bound: on gfx950 the fp32 MFMA chains and the VALU work
// of the conversions do not overlap, so the design removes VALU work.
// phi(x) is converted once: its W rows are written to LDS transposed (block
// rb, element (r, c) at float 256 rb + 16 (c ^ rb) + r), and both statistic
// products read their A operands from there, one ds_read per operand with a
// loop-invariant address: operand K of phi(x)^T (product phi(x)^T phi(gx)) is
// W_x[l ^ K][l], because the transposed conversion of x is W_x with its
// columns xor-ed by the lane's row (W_xt[c] = W_x[c ^ x]); operand K of
// phi(x) (product phi(x) phi(gx)^T) is W_x[l ^ K][K]. Both patterns, and the
// transposed writes, hit 64 distinct banks per instruction. This replaces the
// second conversion of x (gather, signs, WHT) and 32 DPP shuffles.
// staged x, then W_x^T | staged gy, then the relayout | the previous group's gx
constexpr int kRotorBwdWaveFloats = 4 * 256 + kRelayoutFloats + 4 * 256;

template <bool NT, bool WGX>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void rotor16_bwd_kernel(
    const float* __restrict__ U, const float* __restrict__ X, const float* __restrict__ GY, long long ldg,
    float* __restrict__ GX, float* __restrict__ gamma_ws, long long batch, RepTable T, SpinTable S) {
    // the W_x^T address forms below need the wave slots 1024-byte aligned
    static_assert((kRotorBwdWaveFloats * 4) % 1024 == 0, "wave slots stay 1024-byte aligned");
    __shared__ __attribute__((aligned(1024))) float lds[4][kRotorBwdWaveFloats];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* sx = &lds[wave][0];
    float* sg = sx + 4 * 256;
    float* su = sg + kRelayoutFloats;
    const unsigned oddx = (rb & 1) ? T.odd_xor : 0u, oddc = T.odd_xor >> 2;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z] ^ oddx;
    float uop[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) uop[k] = 0.25f * U[x * 16 + k];
    // byte addresses in the W_x^T layout: element (r, c) of block rb at
    // xb + 1024 rb + 64 (c ^ rb) + 4 r; the xor forms need xb 1024-aligned
    const unsigned xb = lds_byte_addr(sx);
    const unsigned wbase = xb + 1024u * rb + 64u * rb + 4u * x;                // element (x ^ .., ..) writes
    const unsigned tbase = xb + 1024u * rb + 64u * (x ^ (unsigned)rb) + 4u * x;  // element (x ^ K, x)
    const floatx16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    floatx16 accm = zero;

    const long long stride = (long long)gridDim.x * 4 * 4;
    const long long rfirst = ((long long)blockIdx.x * 4 + wave) * 4;
    long long row0 = rfirst;
    Pre16 px = fetch16<NT>(X, row0, batch, lane);
    Pre16 pg = fetch16<NT>(GY, row0, batch, lane, ldg);
    for (; row0 < batch; row0 += stride) {
        stage16(sx, px, lane, oddc);
        stage16(sg, pg, lane, oddc);
        px = fetch16<NT>(X, row0 + stride, batch, lane);
        pg = fetch16<NT>(GY, row0 + stride, batch, lane, ldg);
        wave_lds_sync();
        float wg[16], wx[16];
        gather16<0>(sg + rb * 256, ent, wg);
        gather16<0>(sx + rb * 256, ent, wx);
        wave_lds_sync();
        wht_inplace<16>(wg);
        // phi(gx) / 16 = (U / 4) (phi(gy) (U / 4)^T)
        const floatx16 p = mfma_chain_pre<true, false>(zero, wg, uop, std::make_integer_sequence<unsigned, 16>{});
        wht_inplace<16>(wx);
        if (row0 + 3 >= batch) {  // uniform; a block whose row is past the end (a clamped copy) adds nothing
            const bool keep = row0 + rb < batch;
#pragma unroll
            for (int k = 0; k < 16; ++k) wx[k] = keep ? wx[k] : 0.f;
        }
#pragma unroll
        for (int c = 0; c < 16; ++c) lds_store(wbase ^ (64u * c), wx[c]);
        wave_lds_sync();
        float at[16], an[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) at[k] = lds_load(tbase ^ (4u * k));
#pragma unroll
        for (int k = 0; k < 16; ++k) an[k] = lds_load(wbase ^ (68u * k));
        float pop[16];
        transpose_blocks(p, pop);
        const floatx16 g = mfma_chain_pre<false, false>(zero, uop, pop, std::make_integer_sequence<unsigned, 16>{});
        if (WGX && row0 != rfirst) store16<NT>(GX, su, row0 - stride, batch, lane, oddc);  // uniform
        relayout_store(sg, g, lane);
        // phi(x)^T phi(gx): B operand phi(gx)[k][j] from the block transpose
        float gop[16];
        transpose_blocks(g, gop);
        accm = mfma_chain_pre<false, false>(accm, at, gop, std::make_integer_sequence<unsigned, 16>{});
        wave_lds_sync();
        // phi(x) phi(gx)^T: B operand phi(gx)[j][k] = W_gx[j ^ k][k] after the relayout
        float wgx[16];
        relayout_load(sg, rb, x, wgx);
        accm = mfma_chain_pre<false, true>(accm, an, wgx, std::make_integer_sequence<unsigned, 16>{});
        if (WGX) unconvert16_prescaled(wgx, su + rb * 256, ent);
        wave_lds_sync();
    }
    if (WGX && row0 != rfirst) store16<NT>(GX, su, row0 - stride, batch, lane, oddc);
    // M = sum of the four blocks and four waves; lane (g, j) holds M[4g + t][j] in m[t]
    __syncthreads();
    float* red = &lds[0][0];
    {
        const unsigned gq = (unsigned)lane >> 4, j = (unsigned)lane & 15u;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            red[wave * 256 + (4 * gq + t) * 16 + j] = (accm[t] + accm[4 + t]) + (accm[8 + t] + accm[12 + t]);
    }
    __syncthreads();
    const int tid = threadIdx.x;
    static_assert(1024 + 256 <= kRotorBwdWaveFloats, "reduction fits wave 0's slot");
    red[1024 + tid] = (red[tid] + red[256 + tid]) + (red[512 + tid] + red[768 + tid]);
    __syncthreads();
    if (tid < kSpinPlanes) {
        const unsigned pl = S.plane[tid];
        const unsigned px = pl & 15u, mask = pl >> 16;
        float acc = 0.f;
#pragma unroll
        for (unsigned r = 0; r < 16; ++r) {
            const float v = red[1024 + r * 16 + (r ^ px)];
            acc += ((mask >> r) & 1u) ? -v : v;
        }
        gamma_ws[(long long)blockIdx.x * kSpinPlanes + tid] = acc * (-16.f / 32.f);  // phi(gx) carries 1/16
    }
}

// ---- host side --------------------------------------------------------------

bool spin_tables(RepTable& T, SpinTable& S) {
    static std::once_flag once;
    static bool ok = false;
    static RepTable t{};
    static SpinTable s{};
    std::call_once(once, [] {
        if (!rep_table(kSpinN, 0u, t)) return;
        // label of blade e_p e_q: the entry whose blade index is 2^p + 2^q
        int k = 0;
        for (int p = 0; p < kSpinN; ++p)
            for (int q = p + 1; q < kSpinN; ++q, ++k) {
                const unsigned I = (1u << p) | (1u << q);
                bool found = false;
                for (unsigned lab = 0; lab < 256 && !found; ++lab)
                    if ((t.e[lab] & 0xffffu) == I) {
                        const unsigned px = lab >> 4, pz = lab & 15u;
                        const bool neg = (t.e[lab] >> 31) != 0u;
                        unsigned mask = 0;
                        for (unsigned r = 0; r < 16; ++r)
                            if (neg != ((host_popc(pz & (r ^ px)) & 1) != 0)) mask |= 1u << r;
                        s.plane[k] = px | (mask << 16);
                        found = true;
                    }
                if (!found) return;
            }
        ok = true;
    });
    if (ok) {
        T = t;
        S = s;
    }
    return ok;
}

// Environment override CLF_ROTOR_PATH=chain keeps n = 8 on the register chain.
bool rotor16_enabled(int n) {
    if (n != kSpinN) return false;
    if (options().rotor_chain) return false;
    RepTable T;
    SpinTable S;
    return spin_tables(T, S);
}

static unsigned rotor16_grid(int64_t batch) {
    long long g = (batch + 15) / 16;
    const long long cap = 256LL * 8;
    return (unsigned)(g < 1 ? 1 : (g > cap ? cap : g));
}

int rotor16_apply(bool fwd, const float* U, const float* x, float* y, int64_t batch, void* stream, long long ldx) {
    RepTable T;
    SpinTable S;
    if (!spin_tables(T, S)) return set_error(CLF_ERR_UNSUPPORTED, "Cl(8,0) representation tables unavailable");
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(rotor16_grid(batch));
    const bool nt = stream_nt(2.0 * 1024.0 * (double)batch);
#define CLF_ROTOR16(TR, NT) \
    hipLaunchKernelGGL((rotor16_apply_kernel<TR, NT>), grid, dim3(256), 0, s, U, x, y, (long long)batch, T, ldx)
    if (fwd) {
        if (nt) CLF_ROTOR16(false, true);
        else CLF_ROTOR16(false, false);
    } else {
        if (nt) CLF_ROTOR16(true, true);
        else CLF_ROTOR16(true, false);
    }
#undef CLF_ROTOR16
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

// Workgroups for the backward: at most `wanted` (the workspace bound), at most
// the resident ones (the kernel is persistent). The gamma finalize reads this
// many partials.
unsigned rotor16_bwd_grid(long long wanted) {
    // every instantiation has the same register and LDS footprint
    return resident_grid((const void*)rotor16_bwd_kernel<false, true>, 256, 0, wanted);
}

// grid = the number of partials the gamma finalize reads (<= the workspace bound)
int rotor16_bwd(const float* U, const float* x, const float* gy, long long ldg, float* gx, float* gamma_ws,
                int64_t batch, unsigned grid, void* stream) {
    RepTable T;
    SpinTable S;
    if (!spin_tables(T, S)) return set_error(CLF_ERR_UNSUPPORTED, "Cl(8,0) representation tables unavailable");
    hipStream_t s = (hipStream_t)stream;
    const bool nt = stream_nt((2 + (gx != nullptr)) * 1024.0 * (double)batch);
#define CLF_ROTOR16_BWD(NT, WGX)                                                                                 \
    hipLaunchKernelGGL((rotor16_bwd_kernel<NT, WGX>), dim3(grid), dim3(256), 0, s, U, x, gy, ldg, gx, gamma_ws,  \
                       (long long)batch, T, S)
    if (gx) {
        if (nt) CLF_ROTOR16_BWD(true, true);
        else CLF_ROTOR16_BWD(false, true);
    } else {
        if (nt) CLF_ROTOR16_BWD(true, false);
        else CLF_ROTOR16_BWD(false, false);
    }
#undef CLF_ROTOR16_BWD
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
