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
template <bool TRANS, bool NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void rotor16_apply_kernel(
    const float* __restrict__ U, const float* __restrict__ X, float* __restrict__ Y, long long batch, RepTable T) {
    // per wave: staged x rows (1024 floats); later the relayout (1280), then y rows
    __shared__ float lds[4][kRelayoutFloats];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* sx = &lds[wave][0];
    const unsigned oddx = (rb & 1) ? T.odd_xor : 0u, oddc = T.odd_xor >> 2;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z] ^ oddx;
    float vop[16];
    load_spin_operand<TRANS>(U, x, vop);
    const floatx16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};

    const long long stride = (long long)gridDim.x * 4 * 4;
    long long row0 = ((long long)blockIdx.x * 4 + wave) * 4;
    Pre16 px = fetch16<NT>(X, row0, batch, lane);
    for (; row0 < batch; row0 += stride) {
        // the table values are re-derived where they are used rather than kept
        // in registers across the loop (register pressure sets the occupancy)
#pragma unroll
        for (int z = 0; z < 16; ++z) asm volatile("" : "+v"(ent[z]));
        stage16(sx, px, lane, oddc);
        px = fetch16<NT>(X, row0 + stride, batch, lane);
        wave_lds_sync();
        float wx[16];
        gather16<0>(sx + rb * 256, ent, wx);
        wave_lds_sync();
        wht_inplace<16>(wx);
        const floatx16 p = mfma_chain_pre<true, false>(zero, wx, vop, std::make_integer_sequence<unsigned, 16>{});
        float pop[16];
        transpose_blocks(p, pop);
        const floatx16 acc = mfma_chain_pre<false, false>(zero, vop, pop, std::make_integer_sequence<unsigned, 16>{});
        relayout_store(sx, acc, lane);
        wave_lds_sync();
        float wc[16];
        relayout_load(sx, rb, x, wc);
        wave_lds_sync();
        unconvert16(wc, sx + rb * 256, ent);
        wave_lds_sync();
        store16<NT>(Y, sx, row0, batch, lane, oddc);
        wave_lds_sync();
    }
}

// gx = Lambda(Q)^T gy (if GX) and the workgroup's partial K (C(8,2) floats at
// gamma_ws[blockIdx.x * 28]). uop[k] = U[x][k] is the B operand of
// phi(gy) U^T and the A operand of U (phi(gy) U^T). The steps are ordered so
// that few operand sets are live at once (phi(gy), then the two products,
// then phi(x)^T, then phi(x)); the scheduling barriers keep the compiler from
// hoisting the later gathers, which would cost occupancy.
constexpr int kRotorBwdWaveFloats = 4 * 256 + kRelayoutFloats;  // staged x | staged gy, then the relayout

template <bool NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void rotor16_bwd_kernel(const float* __restrict__ U, const float* __restrict__ X,
                                                           const float* __restrict__ GY, float* __restrict__ GX,
                                                           float* __restrict__ gamma_ws, long long batch, RepTable T,
                                                           SpinTable S) {
    // per wave: staged x rows [0, 1024), staged gy rows [1024, 2048); the
    // relayout of phi(gx) reuses the gy slot [1024, 2304) once gy is gathered;
    // the gx rows reuse the x slot once x is gathered
    __shared__ float lds[4][kRotorBwdWaveFloats];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* sx = &lds[wave][0];
    float* sg = sx + 4 * 256;
    const unsigned oddx = (rb & 1) ? T.odd_xor : 0u, oddc = T.odd_xor >> 2;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z] ^ oddx;
    float uop[16];
    load_spin_operand<true>(U, x, uop);
    const floatx16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    floatx16 accm = zero;

    const long long stride = (long long)gridDim.x * 4 * 4;
    long long row0 = ((long long)blockIdx.x * 4 + wave) * 4;
    Pre16 px = fetch16<NT>(X, row0, batch, lane);
    Pre16 pg = fetch16<NT>(GY, row0, batch, lane);
    for (; row0 < batch; row0 += stride) {
#pragma unroll
        for (int z = 0; z < 16; ++z) asm volatile("" : "+v"(ent[z]));  // as in rotor16_apply_kernel
        stage16(sx, px, lane, oddc);
        stage16(sg, pg, lane, oddc);
        px = fetch16<NT>(X, row0 + stride, batch, lane);
        pg = fetch16<NT>(GY, row0 + stride, batch, lane);
        wave_lds_sync();
        // a block whose row is past the end (a clamped copy of the last row)
        // adds nothing to the sums: its phi(x) operands are zeroed
        const bool keep = row0 + rb < batch;
        float wg[16];
        gather16<0>(sg + rb * 256, ent, wg);
        wave_lds_sync();
        wht_inplace<16>(wg);
        // phi(gx) = U (phi(gy) U^T)
        const floatx16 p = mfma_chain_pre<true, false>(zero, wg, uop, std::make_integer_sequence<unsigned, 16>{});
        float pop[16];
        transpose_blocks(p, pop);
        const floatx16 g = mfma_chain_pre<false, false>(zero, uop, pop, std::make_integer_sequence<unsigned, 16>{});
        relayout_store(sg, g, lane);
        __builtin_amdgcn_sched_barrier(0);
        // phi(x)^T phi(gx): B operand phi(gx)[k][j] from the block transpose
        float gop[16];
        transpose_blocks(g, gop);
        float wxt[16];
        gather16<1>(sx + rb * 256, ent, wxt);
        wht_inplace<16>(wxt);
#pragma unroll
        for (int k = 0; k < 16; ++k) wxt[k] = keep ? wxt[k] : 0.f;
        accm = mfma_chain_pre<true, false>(accm, wxt, gop, std::make_integer_sequence<unsigned, 16>{});
        __builtin_amdgcn_sched_barrier(0);
        // phi(x) phi(gx)^T: B operand phi(gx)[j][k] = W_gx[j ^ k][k] after the relayout
        float wx[16];
        gather16<0>(sx + rb * 256, ent, wx);
        wave_lds_sync();
        float wgx[16];
        relayout_load(sg, rb, x, wgx);
        wht_inplace<16>(wx);
#pragma unroll
        for (int k = 0; k < 16; ++k) wx[k] = keep ? wx[k] : 0.f;
        accm = mfma_chain_pre<true, true>(accm, wx, wgx, std::make_integer_sequence<unsigned, 16>{});
        if (GX) {  // uniform: a kernel argument
            unconvert16(wgx, sx + rb * 256, ent);
            wave_lds_sync();
            store16<NT>(GX, sx, row0, batch, lane, oddc);
        }
        wave_lds_sync();
    }
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
        gamma_ws[(long long)blockIdx.x * kSpinPlanes + tid] = acc * (-1.f / 32.f);
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

int rotor16_apply(bool fwd, const float* U, const float* x, float* y, int64_t batch, void* stream) {
    RepTable T;
    SpinTable S;
    if (!spin_tables(T, S)) return set_error(CLF_ERR_UNSUPPORTED, "Cl(8,0) representation tables unavailable");
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(rotor16_grid(batch));
    const bool nt = stream_nt(2.0 * 1024.0 * (double)batch);
#define CLF_ROTOR16(TR, NT) \
    hipLaunchKernelGGL((rotor16_apply_kernel<TR, NT>), grid, dim3(256), 0, s, U, x, y, (long long)batch, T)
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
    return resident_grid((const void*)rotor16_bwd_kernel<false>, 256, 0, wanted);
}

// grid = the number of partials the gamma finalize reads (<= the workspace bound)
int rotor16_bwd(const float* U, const float* x, const float* gy, float* gx, float* gamma_ws, int64_t batch,
                unsigned grid, void* stream) {
    RepTable T;
    SpinTable S;
    if (!spin_tables(T, S)) return set_error(CLF_ERR_UNSUPPORTED, "Cl(8,0) representation tables unavailable");
    hipStream_t s = (hipStream_t)stream;
    if (stream_nt((2 + (gx != nullptr)) * 1024.0 * (double)batch))
        hipLaunchKernelGGL(rotor16_bwd_kernel<true>, dim3(grid), dim3(256), 0, s, U, x, gy, gx, gamma_ws,
                           (long long)batch, T, S);
    else
        hipLaunchKernelGGL(rotor16_bwd_kernel<false>, dim3(grid), dim3(256), 0, s, U, x, gy, gx, gamma_ws,
                           (long long)batch, T, S);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
