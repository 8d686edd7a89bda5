// Geometric product through the real matrix representation, for the
// signatures where Cl(p,q) is the full real matrix algebra M_m(R), m = 2^(n/2)
// (p - q = 0 or 2 mod 8, no null generator). The product of two rows is then
// one m x m matrix product (m^3 multiply-adds) instead of the 4^n terms of the
// XOR-indexed sum; forward and backward give the same values as the per-term
// kernels up to fp32 rounding.
//
// Representation. Generators are real Pauli products gamma_g = P(x_g, z_g),
//   P(x, z)[r][c] = [c == r ^ x] (-1)^{popc(z & c)},
//   P(x1, z1) P(x2, z2) = (-1)^{popc(z1 & x2)} P(x1 ^ x2, z1 ^ z2),
// chosen on the host so that they anticommute and square to the metric. Blade I
// maps to phi(e_I) = s(I) P(x_I, z_I). A host table gives, for every label
// (x, z), the blade and its sign. Conversion a -> phi(a): gather
// t[x][z] = s(I) a_I, Walsh-Hadamard transform over z for each x,
// W[x][c] = sum_z t[x][z] (-1)^{popc(z & c)}, and phi(a)[r][c] = W[r ^ c][c].
// The inverse runs the same steps backwards with a factor 1/m.
// Backward: ga = phi^{-1}(phi(gc) phi(b)^T), gb = phi^{-1}(phi(a)^T phi(gc))
// (phi is orthogonal up to the factor m).
//
// Layout. One row is handled by m lanes of one wave (lane = x for the
// conversions, lane = matrix row r for the products), so all exchanges are
// wave-local through the row's LDS slots and need no workgroup barrier. Waves
// walk row groups with a grid stride and prefetch the next group's rows into
// registers while the current group is computed.
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>

#include "rep_common.h"

namespace clf {


// gather t[z] = s * row[blade] from the staged row, WHT over z, and write the
// standard-layout matrix phi[r][c] = W[r ^ c][c] (lane holds x) into mat
template <int M>
__device__ __forceinline__ void row_to_matrix(const float* __restrict__ row, float* __restrict__ mat,
                                              const unsigned (&ent)[M], unsigned x) {
    float w[M];
#pragma unroll
    for (int z = 0; z < M; ++z) {
        const float v = row[ent[z] & 0xffffu];
        w[z] = __uint_as_float(__float_as_uint(v) ^ (ent[z] & 0x80000000u));
    }
    wht_inplace<M>(w);
#pragma unroll
    for (int c = 0; c < M; ++c) mat[((x ^ (unsigned)c) * M) + c] = w[c];
}

// inverse: read W[x][c] = mat[x ^ c][c], inverse WHT, scatter s * t[z] / m into row
template <int M>
__device__ __forceinline__ void matrix_to_row(const float* __restrict__ mat, float* __restrict__ row,
                                              const unsigned (&ent)[M], unsigned x) {
    float w[M];
#pragma unroll
    for (int c = 0; c < M; ++c) w[c] = mat[((x ^ (unsigned)c) * M) + c];
    wht_inplace<M>(w);
    constexpr float inv = 1.0f / (float)M;
#pragma unroll
    for (int z = 0; z < M; ++z)
        row[ent[z] & 0xffffu] = __uint_as_float(__float_as_uint(w[z] * inv) ^ (ent[z] & 0x80000000u));
}

template <int M>
__device__ __forceinline__ void load_mrow(const float* __restrict__ mat, unsigned r, float (&v)[M]) {
    const float4* p = reinterpret_cast<const float4*>(mat + r * M);
#pragma unroll
    for (int q = 0; q < M / 4; ++q) {
        const float4 t = p[q];
        v[4 * q] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
}

template <int M>
__device__ __forceinline__ void store_mrow(float* __restrict__ mat, unsigned r, const float (&v)[M]) {
    float4* p = reinterpret_cast<float4*>(mat + r * M);
#pragma unroll
    for (int q = 0; q < M / 4; ++q) p[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

// out[c] = sum_k arow[k] * B[k][c]
template <int M>
__device__ __forceinline__ void row_times_mat(const float (&arow)[M], const float* __restrict__ B, float (&out)[M]) {
#pragma unroll
    for (int c = 0; c < M; ++c) out[c] = 0.f;
#pragma unroll
    for (int k = 0; k < M; ++k) {
        float bk[M];
        load_mrow<M>(B, (unsigned)k, bk);
#pragma unroll
        for (int c = 0; c < M; ++c) out[c] = __builtin_fmaf(arow[k], bk[c], out[c]);
    }
}

// out[c] = sum_k arow[k] * B[c][k]   (row times B^T)
template <int M>
__device__ __forceinline__ void row_times_matT(const float (&arow)[M], const float* __restrict__ B, float (&out)[M]) {
#pragma unroll
    for (int c = 0; c < M; ++c) {
        float bc[M];
        load_mrow<M>(B, (unsigned)c, bc);
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < M; ++k) t = __builtin_fmaf(arow[k], bc[k], t);
        out[c] = t;
    }
}

// Per-wave row-group staging: rows row0 .. row0 + RPW - 1 (RPW = 64 / M), each
// D = M*M floats; lane l moves float4 chunks l, l + 64, ... of the group.
template <int M>
struct RowGroup {
    static constexpr int D = M * M;
    static constexpr int RPW = 64 / M;
    static constexpr int CH = RPW * D / 4 / 64;  // float4 chunks per lane
};

// Prefetch registers of one operand's row group: CH float4 per lane.
template <int CH>
struct Pre {
    float4 v[CH];
};

template <int M>
__device__ __forceinline__ Pre<RowGroup<M>::CH> fetch_group(const float* __restrict__ src, long long row0,
                                                            long long batch, int lane,
                                                            long long ld = RowGroup<M>::D) {
    constexpr int D = RowGroup<M>::D, CH = RowGroup<M>::CH;
    Pre<CH> p;
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const int f = lane + 64 * j;          // float4 index inside the group
        const int rl = (f * 4) / D;           // row inside the group
        long long row = row0 + rl;
        row = row < batch ? row : batch - 1;  // rows past the end re-read the last row; never stored
        p.v[j] = reinterpret_cast<const float4*>(src + (row & row_mask(ld)) * D)[(f * 4 - rl * D) / 4];
    }
    return p;
}

template <int CH>
__device__ __forceinline__ void stage_group(float* __restrict__ dst, const Pre<CH>& p, int lane) {
#pragma unroll
    for (int j = 0; j < CH; ++j) reinterpret_cast<float4*>(dst)[lane + 64 * j] = p.v[j];
}

template <int LOGM>
__global__ __launch_bounds__(256) void rep_fwd_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                       float* __restrict__ C, long long batch, RepTable T) {
    constexpr int M = 1 << LOGM;
    constexpr int D = M * M;
    constexpr int RPW = RowGroup<M>::RPW;
    constexpr int CH = RowGroup<M>::CH;
    __shared__ float lds[4][2][RPW * D];  // per wave: staged a (then phi(a), then c), staged b (then phi(b))
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const unsigned x = lane & (M - 1);
    const int rl = lane >> LOGM;
    float* sa = &lds[wave][0][0];
    float* sb = &lds[wave][1][0];
    unsigned ent[M];
#pragma unroll
    for (int z = 0; z < M; ++z) ent[z] = T.e[x * M + z];

    const long long waves_total = (long long)gridDim.x * 4;
    long long row0 = ((long long)blockIdx.x * 4 + wave) * RPW;
    Pre<CH> pa = fetch_group<M>(A, row0, batch, lane);
    Pre<CH> pb = fetch_group<M>(B, row0, batch, lane);
    for (; row0 < batch; row0 += waves_total * RPW) {
        // stage the prefetched rows, then prefetch the next group (past the end
        // it re-reads clamped rows: no branch)
        stage_group<CH>(sa, pa, lane);
        stage_group<CH>(sb, pb, lane);
        pa = fetch_group<M>(A, row0 + waves_total * RPW, batch, lane);
        pb = fetch_group<M>(B, row0 + waves_total * RPW, batch, lane);
        wave_lds_sync();
        float* ra = sa + rl * D;
        float* rb = sb + rl * D;
        // conversions: gather + WHT in registers; matrices overwrite the staged rows
        float wa[M], wb[M];
#pragma unroll
        for (int z = 0; z < M; ++z) {
            wa[z] = __uint_as_float(__float_as_uint(ra[ent[z] & 0xffffu]) ^ (ent[z] & 0x80000000u));
            wb[z] = __uint_as_float(__float_as_uint(rb[ent[z] & 0xffffu]) ^ (ent[z] & 0x80000000u));
        }
        wht_inplace<M>(wa);
        wht_inplace<M>(wb);
        wave_lds_sync();
#pragma unroll
        for (int c = 0; c < M; ++c) {
            ra[((x ^ (unsigned)c) * M) + c] = wa[c];
            rb[((x ^ (unsigned)c) * M) + c] = wb[c];
        }
        wave_lds_sync();
        // product: lane r = x computes row r of phi(a) phi(b)
        float arow[M], crow[M];
        load_mrow<M>(ra, x, arow);
        row_times_mat<M>(arow, rb, crow);
        wave_lds_sync();
        store_mrow<M>(ra, x, crow);
        wave_lds_sync();
        // inverse conversion into the b slot (blade order), then a coalesced store
        matrix_to_row<M>(ra, rb, ent, x);
        wave_lds_sync();
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int f = lane + 64 * j;
            const int rr = (f * 4) / D;
            if (row0 + rr < batch)
                reinterpret_cast<float4*>(C + (row0 + rr) * D)[(f * 4 - rr * D) / 4] = reinterpret_cast<const float4*>(sb)[f];
        }
        wave_lds_sync();
    }
}

template <int LOGM>
__global__ __launch_bounds__(256) void rep_bwd_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                       const float* __restrict__ GC, long long ldg,
                                                       float* __restrict__ GA, float* __restrict__ GB, long long batch,
                                                       RepTable T) {
    constexpr int M = 1 << LOGM;
    constexpr int D = M * M;
    constexpr int RPW = RowGroup<M>::RPW;
    constexpr int CH = RowGroup<M>::CH;
    __shared__ float lds[4][3][RPW * D];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const unsigned x = lane & (M - 1);
    const int rl = lane >> LOGM;
    float* sa = &lds[wave][0][0];
    float* sb = &lds[wave][1][0];
    float* sg = &lds[wave][2][0];
    unsigned ent[M];
#pragma unroll
    for (int z = 0; z < M; ++z) ent[z] = T.e[x * M + z];
    const bool want_a = GA != nullptr, want_b = GB != nullptr;

    const long long waves_total = (long long)gridDim.x * 4;
    long long row0 = ((long long)blockIdx.x * 4 + wave) * RPW;
    Pre<CH> pa = fetch_group<M>(A, row0, batch, lane);
    Pre<CH> pb = fetch_group<M>(B, row0, batch, lane);
    Pre<CH> pg = fetch_group<M>(GC, row0, batch, lane, ldg);
    for (; row0 < batch; row0 += waves_total * RPW) {
        stage_group<CH>(sa, pa, lane);
        stage_group<CH>(sb, pb, lane);
        stage_group<CH>(sg, pg, lane);
        pa = fetch_group<M>(A, row0 + waves_total * RPW, batch, lane);
        pb = fetch_group<M>(B, row0 + waves_total * RPW, batch, lane);
        pg = fetch_group<M>(GC, row0 + waves_total * RPW, batch, lane, ldg);
        wave_lds_sync();
        float* ra = sa + rl * D;
        float* rb = sb + rl * D;
        float* rg = sg + rl * D;
        float wa[M], wb[M], wg[M];
#pragma unroll
        for (int z = 0; z < M; ++z) {
            const unsigned bi = ent[z] & 0xffffu, sgn = ent[z] & 0x80000000u;
            wa[z] = __uint_as_float(__float_as_uint(ra[bi]) ^ sgn);
            wb[z] = __uint_as_float(__float_as_uint(rb[bi]) ^ sgn);
            wg[z] = __uint_as_float(__float_as_uint(rg[bi]) ^ sgn);
        }
        wht_inplace<M>(wa);
        wht_inplace<M>(wb);
        wht_inplace<M>(wg);
        wave_lds_sync();
#pragma unroll
        for (int c = 0; c < M; ++c) {
            const unsigned o = ((x ^ (unsigned)c) * M) + c;
            ra[o] = wa[c];
            rb[o] = wb[c];
            rg[o] = wg[c];
        }
        wave_lds_sync();
        // lane r = x: dA[r][.] = G[r][.] B^T, dB[r][.] = (column r of A) G
        float grow[M], dA[M], dB[M];
        if (want_a) {
            load_mrow<M>(rg, x, grow);
            row_times_matT<M>(grow, rb, dA);
        }
        if (want_b) {
            float acol[M];
#pragma unroll
            for (int k = 0; k < M; ++k) acol[k] = ra[k * M + x];
            row_times_mat<M>(acol, rg, dB);
        }
        wave_lds_sync();
        if (want_a) store_mrow<M>(ra, x, dA);
        if (want_b) store_mrow<M>(rb, x, dB);
        wave_lds_sync();
        // inverse conversions: dA -> blade order in the g slot, dB -> the a slot... done in two passes
        if (want_a) matrix_to_row<M>(ra, rg, ent, x);
        wave_lds_sync();
        if (want_a) {
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int f = lane + 64 * j;
                const int rr = (f * 4) / D;
                if (row0 + rr < batch)
                    reinterpret_cast<float4*>(GA + (row0 + rr) * D)[(f * 4 - rr * D) / 4] =
                        reinterpret_cast<const float4*>(sg)[f];
            }
        }
        wave_lds_sync();
        if (want_b) matrix_to_row<M>(rb, ra, ent, x);
        wave_lds_sync();
        if (want_b) {
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int f = lane + 64 * j;
                const int rr = (f * 4) / D;
                if (row0 + rr < batch)
                    reinterpret_cast<float4*>(GB + (row0 + rr) * D)[(f * 4 - rr * D) / 4] =
                        reinterpret_cast<const float4*>(sa)[f];
            }
        }
        wave_lds_sync();
    }
}

// ---- m = 16 (n = 8) on the matrix cores -------------------------------------
// The 4-block v_mfma_f32_16x16x1f32 multiplies four independent 16x16 matrices,
// block b taking its operands from lanes 16b .. 16b + 15 -- exactly the lanes
// that convert row b. Operand k of lane (b, x):
//   A[x][k] = phi(a)[x][k] = W_a[x ^ k][k]   (xor shuffle of register k)
//   B[k][x] = phi(b)^T[x][k] = W'_b[x ^ k][k]
// where W' is the conversion with the extra signs (-1)^{popc(x & z)}, because
// P(x, z)^T = (-1)^{popc(x & z)} P(x, z). The shuffles are DPP moves
// (quad_perm for xor 1..3, row_half_mirror = xor 7, row_mirror = xor 15).
// The product C_b[4g + t][j] lands in lane 16g + j, register 4b + t; it goes
// back through LDS as W_c[i ^ j][j] at row stride 20 floats, which keeps both
// the scattered b32 writes and the b128 row reads free of bank conflicts.

// Memory pipeline. A wave's global loads and stores share one completion
// counter and the compiler waits for all of them before staged rows are used,
// so results are not stored at the end of their own group (the next group's
// wait would take the whole store latency) but from their LDS slot right after
// the next wait: they then have a full group's time to complete. The wave index
// is wave-uniform (readfirstlane), so the row bookkeeping and the clamps run on
// the scalar unit.
template <bool NT, bool ONE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void rep16_fwd_kernel(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C, long long batch, RepTable T) {
    // per wave: staged a | staged b; later the relayout (over a and the start
    // of b), then c in the b slot until the next group's stores
    __shared__ float lds[4][2 * 4 * 256];
    static_assert(2 * 4 * 256 >= kRelayoutFloats, "relayout must fit the wave's LDS slots");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* sa = &lds[wave][0];
    float* sb = sa + 4 * 256;
    const unsigned oddx = (rb & 1) ? T.odd_xor : 0u, oddc = T.odd_xor >> 2;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z] ^ oddx;

    const long long stride = (long long)gridDim.x * 4 * 4;
    const long long rfirst = ((long long)blockIdx.x * 4 + wave) * 4;
    long long row0 = rfirst;
    Pre16 pa = fetch16<NT>(A, row0, batch, lane);
    Pre16 pb = fetch16<NT>(B, row0, batch, lane);
    for (; row0 < batch; row0 += stride) {
        // the table values are re-derived where they are used rather than kept
        // in registers across the loop (register pressure sets the occupancy)
#pragma unroll
        for (int z = 0; z < 16; ++z) asm volatile("" : "+v"(ent[z]));
        stage16(sa, pa, lane, oddc);
        if (row0 != rfirst) {  // uniform: the previous group's c leaves its slot before b is staged there
            wave_lds_sync();
            store16<NT>(C, sb, row0 - stride, batch, lane, oddc);
            wave_lds_sync();
        }
        stage16(sb, pb, lane, oddc);
        if (!ONE) pa = fetch16<NT>(A, row0 + stride, batch, lane);
        wave_lds_sync();
        float wa[16], wb[16];
        gather16<0>(sa + rb * 256, ent, wa);
        gather16<1>(sb + rb * 256, ent, wb);
        wave_lds_sync();
        wht_inplace<16>(wa);
        wht_inplace<16>(wb);
        const floatx16 acc = mfma_chain(wa, wb);
        // b's next rows are requested once the operands are consumed (fewer
        // registers live across the product)
        if (!ONE) pb = fetch16<NT>(B, row0 + stride, batch, lane);
        relayout_store(sa, acc, lane);
        wave_lds_sync();
        float wc[16];
        relayout_load(sa, rb, x, wc);
        wave_lds_sync();
        unconvert16(wc, sb + rb * 256, ent);
        wave_lds_sync();
    }
    if (row0 != rfirst) store16<NT>(C, sb, row0 - stride, batch, lane, oddc);
}

// GA and GB are compile-time flags (a gradient that is not wanted has no
// branch around its stores). dA of a group is stored right after the group's
// second wait, dB right after the next group's first wait. ONE: the grid covers
// the batch (one group per wave), so no next group is prefetched.
template <bool NT, bool WA, bool WB, bool ONE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void rep16_bwd_kernel(
    const float* __restrict__ A, const float* __restrict__ B, const float* __restrict__ GC, long long ldg,
    float* __restrict__ GA, float* __restrict__ GB, long long batch, RepTable T) {
    // per wave: gc | b, then a over b | scratch for each gradient's relayout and
    // its rows in blade order; only two converted operands are live at a time
    __shared__ float lds[4][2 * 4 * 256 + kRelayoutFloats];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* s0 = &lds[wave][0];
    float* s1 = s0 + 4 * 256;
    float* sr = s1 + 4 * 256;
    const unsigned oddx = (rb & 1) ? T.odd_xor : 0u, oddc = T.odd_xor >> 2;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z] ^ oddx;

    const long long stride = (long long)gridDim.x * 4 * 4;
    const long long rfirst = ((long long)blockIdx.x * 4 + wave) * 4;
    long long row0 = rfirst;
    // gc and b of a group are loaded while the previous group's dB runs, a
    // while the group's dA runs
    Pre16 pb = fetch16<NT>(B, row0, batch, lane);
    Pre16 pg = fetch16<NT>(GC, row0, batch, lane, ldg);
    for (; row0 < batch; row0 += stride) {
        // the table values are re-derived where they are used rather than kept
        // in registers across the loop (register pressure sets the occupancy)
#pragma unroll
        for (int z = 0; z < 16; ++z) asm volatile("" : "+v"(ent[z]));
        // dA = G B^T: operands W_g, W_b.  dB = A^T G: operands W'_a, W'_g.
        stage16(s0, pg, lane, oddc);
        stage16(s1, pb, lane, oddc);
        const Pre16 pa = fetch16<NT>(A, row0, batch, lane);
        if (WB && row0 != rfirst) store16<NT>(GB, sr, row0 - stride, batch, lane, oddc);  // uniform
        wave_lds_sync();
        if (WA) {
            float wg[16], wb[16];
            gather16<0>(s0 + rb * 256, ent, wg);
            gather16<0>(s1 + rb * 256, ent, wb);
            wht_inplace<16>(wg);
            wht_inplace<16>(wb);
            const floatx16 acc = mfma_chain(wg, wb);
            relayout_store(sr, acc, lane);
            wave_lds_sync();
            float da[16];
            relayout_load(sr, rb, x, da);
            wave_lds_sync();
            unconvert16(da, sr + rb * 256, ent);
        }
        wave_lds_sync();
        stage16(s1, pa, lane, oddc);
        if (!ONE) {
            pg = fetch16<NT>(GC, row0 + stride, batch, lane, ldg);
            pb = fetch16<NT>(B, row0 + stride, batch, lane);
        }
        if (WA) store16<NT>(GA, sr, row0, batch, lane, oddc);
        wave_lds_sync();
        if (WB) {
            float wat[16], wgt[16];
            gather16<1>(s1 + rb * 256, ent, wat);
            gather16<1>(s0 + rb * 256, ent, wgt);
            wht_inplace<16>(wat);
            wht_inplace<16>(wgt);
            const floatx16 acc = mfma_chain(wat, wgt);
            relayout_store(sr, acc, lane);
            wave_lds_sync();
            float db[16];
            relayout_load(sr, rb, x, db);
            wave_lds_sync();
            unconvert16(db, sr + rb * 256, ent);
        }
        wave_lds_sync();
    }
    if (WB && row0 != rfirst) store16<NT>(GB, sr, row0 - stride, batch, lane, oddc);
}

// ---- broadcast weight (the product layers), m = 16 --------------------------
// y = x w (side 0) or y = w x (side 1) with one weight row w for the whole
// batch: phi(y) = phi(x) phi(w) or phi(w) phi(x), 16^3 multiply-adds per row
// instead of the (2^n)^2 of the dense weight matrix. The weight's MFMA operand
// is the same for the four blocks of every wave, so each lane builds its 16
// shuffled values once per kernel and keeps them in registers.
// Backward (side 0): gx = phi^-1(phi(gy) phi(w)^T), gw = phi^-1(sum_rows phi(x)^T phi(gy));
//          (side 1): gx = phi^-1(phi(w)^T phi(gy)), gw = phi^-1(sum_rows phi(gy) phi(x)^T).
// The weight-gradient sum runs in the MFMA accumulators across a wave's rows;
// workgroups write 16x16 partials that one small kernel sums and converts.

// the weight's conversion for lane x (sign bit 31 - SIGNSHIFT of the entries:
// 0 = phi(w), 1 = the transposed conversion), shuffled into operand order
template <int SIGNSHIFT>
__device__ __forceinline__ void weight_operand(const float* __restrict__ w, const RepTable& T, unsigned x,
                                               float (&op)[16]) {
    float t[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) {
        const unsigned e = T.e[x * 16 + z];
        t[z] = __uint_as_float(__float_as_uint(w[e & 0xffffu]) ^ ((e << SIGNSHIFT) & 0x80000000u));
    }
    wht_inplace<16>(t);
    shuffle_operand(t, op, std::make_integer_sequence<unsigned, 16>{});
}

// Each group's y rows wait in their own LDS slot and are stored after the next
// group's loads have been waited for (the loads and stores of a wave share one
// completion counter, so stores at the end of an iteration would hold up the
// next group's prefetched loads); the wave index is wave-uniform.
constexpr int kBcastFwdWaveFloats = kRelayoutFloats + 4 * 256;  // staged x, then the relayout | the previous group's y

template <int SIDE, bool NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void rep16_bcast_fwd_kernel(const float* __restrict__ X, const float* __restrict__ W,
                                                               float* __restrict__ Y, long long batch, RepTable T) {
    __shared__ float lds[4][kBcastFwdWaveFloats];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* sx = &lds[wave][0];
    float* sy = sx + kRelayoutFloats;
    const unsigned oddx = (rb & 1) ? T.odd_xor : 0u, oddc = T.odd_xor >> 2;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z] ^ oddx;
    // side 0: B = column x of phi(w) (transposed signs); side 1: A = row x of phi(w)
    float wop[16];
    weight_operand<SIDE == 0 ? 1 : 0>(W, T, x, wop);

    const long long stride = (long long)gridDim.x * 4 * 4;
    const long long rfirst = ((long long)blockIdx.x * 4 + wave) * 4;
    long long row0 = rfirst;
    Pre16 px = fetch16<NT>(X, row0, batch, lane);
    for (; row0 < batch; row0 += stride) {
#pragma unroll
        for (int z = 0; z < 16; ++z) asm volatile("" : "+v"(ent[z]));
        stage16(sx, px, lane, oddc);
        px = fetch16<NT>(X, row0 + stride, batch, lane);
        wave_lds_sync();
        float wx[16];
        // side 0: A = row x of phi(x); side 1: B = column x of phi(x) (transposed signs)
        gather16<SIDE == 0 ? 0 : 1>(sx + rb * 256, ent, wx);
        wave_lds_sync();
        wht_inplace<16>(wx);
        const floatx16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        floatx16 acc;
        if constexpr (SIDE == 0)
            acc = mfma_chain_pre<true, false>(zero, wx, wop, std::make_integer_sequence<unsigned, 16>{});
        else
            acc = mfma_chain_pre<false, true>(zero, wop, wx, std::make_integer_sequence<unsigned, 16>{});
        if (row0 != rfirst) store16<NT>(Y, sy, row0 - stride, batch, lane, oddc);  // uniform
        relayout_store(sx, acc, lane);
        wave_lds_sync();
        float wc[16];
        relayout_load(sx, rb, x, wc);
        unconvert16(wc, sy + rb * 256, ent);
        wave_lds_sync();
    }
    if (row0 != rfirst) store16<NT>(Y, sy, row0 - stride, batch, lane, oddc);
}

// parts[blockIdx.x * 256 + r * 16 + c]: the workgroup's sum of the 16x16 weight-gradient products.
// WX / WW: gx / the weight gradient wanted (compile-time, so no branch runs
// around a load or a store). A group's gx rows wait in their own LDS slot and
// are stored after the next group's first wait; the wave index is wave-uniform.
template <int SIDE, bool NT, bool WX, bool WW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void rep16_bcast_bwd_kernel(
    const float* __restrict__ X, const float* __restrict__ W, const float* __restrict__ GY, long long ldg,
    float* __restrict__ GX, float* __restrict__ parts, long long batch, RepTable T) {
    // per wave: staged x | staged gy (the relayout over x and the start of gy) | the previous group's gx rows
    __shared__ float lds[4][3 * 4 * 256];
    static_assert(2 * 4 * 256 >= kRelayoutFloats, "relayout must fit the wave's staging slots");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const unsigned x = lane & 15u;
    const int rb = lane >> 4;
    float* sx = &lds[wave][0];
    float* sg = sx + 4 * 256;
    float* so = sg + 4 * 256;
    const unsigned oddx = (rb & 1) ? T.odd_xor : 0u, oddc = T.odd_xor >> 2;
    unsigned ent[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) ent[z] = T.e[x * 16 + z] ^ oddx;
    // gx operand of the weight: side 0: B = column x of phi(w)^T = row x of phi(w);
    // side 1: A = row x of phi(w)^T (transposed signs)
    float wop[16];
    if (WX) weight_operand<SIDE == 0 ? 0 : 1>(W, T, x, wop);
    const floatx16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    floatx16 accw = zero;

    const long long stride = (long long)gridDim.x * 4 * 4;
    const long long rfirst = ((long long)blockIdx.x * 4 + wave) * 4;
    long long row0 = rfirst;
    Pre16 px = fetch16<NT>(X, row0, batch, lane);
    Pre16 pg = fetch16<NT>(GY, row0, batch, lane, ldg);
    for (; row0 < batch; row0 += stride) {
        // the table values are re-derived where they are used rather than kept
        // in registers across the loop (register pressure sets the occupancy)
#pragma unroll
        for (int z = 0; z < 16; ++z) asm volatile("" : "+v"(ent[z]));
        stage16(sx, px, lane, oddc);
        stage16(sg, pg, lane, oddc);
        px = fetch16<NT>(X, row0 + stride, batch, lane);
        wave_lds_sync();
        // weight gradient first (x as its operand: side 0: A = row of phi(x)^T,
        // transposed signs, with gy in transposed signs; side 1: B = column of
        // phi(x)^T = row of phi(x), with gy in plain signs), then gx from gy in
        // the other convention; one converted pair is live at a time
        if (WW) {
            float wx[16], wgw[16];
            gather16<SIDE == 0 ? 1 : 0>(sx + rb * 256, ent, wx);
            gather16<SIDE == 0 ? 1 : 0>(sg + rb * 256, ent, wgw);
            wht_inplace<16>(wx);
            wht_inplace<16>(wgw);
            // rows past the end are clamped copies of the last row: zero their
            // contribution to the sum (whole 16-lane blocks, so every lane's
            // operand is zero for those blocks)
            if (row0 + rb >= batch) {
#pragma unroll
                for (int k = 0; k < 16; ++k) wx[k] = 0.f;
            }
            if constexpr (SIDE == 0)
                accw = mfma_chain_pre<true, true>(accw, wx, wgw, std::make_integer_sequence<unsigned, 16>{});
            else
                accw = mfma_chain_pre<true, true>(accw, wgw, wx, std::make_integer_sequence<unsigned, 16>{});
        }
        pg = fetch16<NT>(GY, row0 + stride, batch, lane, ldg);
        if (WX && row0 != rfirst) store16<NT>(GX, so, row0 - stride, batch, lane, oddc);  // uniform
        wave_lds_sync();
        if (WX) {
            float wgx[16];
            gather16<SIDE == 0 ? 0 : 1>(sg + rb * 256, ent, wgx);
            wht_inplace<16>(wgx);
            floatx16 acc;
            if constexpr (SIDE == 0)
                acc = mfma_chain_pre<true, false>(zero, wgx, wop, std::make_integer_sequence<unsigned, 16>{});
            else
                acc = mfma_chain_pre<false, true>(zero, wop, wgx, std::make_integer_sequence<unsigned, 16>{});
            relayout_store(sx, acc, lane);
            wave_lds_sync();
            float wc[16];
            relayout_load(sx, rb, x, wc);
            unconvert16(wc, so + rb * 256, ent);
        }
        wave_lds_sync();
    }
    if (WX && row0 != rfirst) store16<NT>(GX, so, row0 - stride, batch, lane, oddc);
    if (!WW) return;
    // sum the four blocks (rows) of the wave: lane (g, j) holds S[4g + t][j]
    __syncthreads();  // every wave is done with its LDS slots
    float* red = &lds[0][0];  // [4 waves][256]
    const unsigned g = (unsigned)lane >> 4, j = (unsigned)lane & 15u;
#pragma unroll
    for (int t = 0; t < 4; ++t)
        red[wave * 256 + (4 * g + t) * 16 + j] = accw[t] + accw[4 + t] + accw[8 + t] + accw[12 + t];
    __syncthreads();
    const int e = threadIdx.x;
    parts[(long long)blockIdx.x * 256 + e] = red[e] + red[256 + e] + red[512 + e] + red[768 + e];
}

// Deterministic sums of the 16x16 partials, in two stages so that every
// thread has few dependent loads: out[k * 256 + e] = sum of partials
// 32k .. 32k + 31 (element e); one workgroup per 32 partials.
constexpr int kPartsPerSum = 32;

__global__ __launch_bounds__(256) void rep16_parts_sum_kernel(const float* __restrict__ parts, int nparts,
                                                               float* __restrict__ out) {
    const int e = threadIdx.x;
    const int p0 = blockIdx.x * kPartsPerSum;
    const int p1 = p0 + kPartsPerSum < nparts ? p0 + kPartsPerSum : nparts;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int p = p0;
    // sixteen loads in flight per batch: a full group of 32 partials is two round trips
    for (; p + 16 <= p1; p += 16) {
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) t[u] = parts[(long long)(p + u) * 256 + e];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[u] += t[u] + t[u + 8];
    }
    for (; p < p1; ++p) acc[0] += parts[(long long)p * 256 + e];
    out[(long long)blockIdx.x * 256 + e] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

// gw = phi^-1(sum of the first-stage sums); one workgroup of 1024 threads.
// Thread (q, e) sums the first-stage sums q, q + 4, q + 8, ... of element e
// (sixteen loads in flight per batch: the usual 64 sums are one round trip),
// and the four quarters are added in a fixed order.
__global__ __launch_bounds__(1024) void rep16_bcast_gw_kernel(const float* __restrict__ sums, int nsums,
                                                               float* __restrict__ gw, RepTable T) {
    __shared__ double Q[1024];
    __shared__ float S[256];
    const int e = threadIdx.x & 255, q = threadIdx.x >> 8;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    int p = q;
    for (; p + 60 < nsums; p += 64) {
        float t[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) t[u] = sums[(long long)(p + 4 * u) * 256 + e];
#pragma unroll
        for (int u = 0; u < 16; ++u) acc[u & 3] += (double)t[u];
    }
    for (; p < nsums; p += 4) acc[0] += (double)sums[(long long)p * 256 + e];
    Q[threadIdx.x] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    __syncthreads();
    if (threadIdx.x < 256) S[e] = (float)((Q[e] + Q[256 + e]) + (Q[512 + e] + Q[768 + e]));
    __syncthreads();
    if (threadIdx.x >= 256) return;  // no barrier follows
    // thread (x, z): t[x][z] = (1/16) sum_c W[x][c] (-1)^{popc(z & c)}, W[x][c] = S[(x ^ c) * 16 + c]
    const unsigned xx = (unsigned)e >> 4, z = (unsigned)e & 15u;
    float t = 0.f;
#pragma unroll
    for (unsigned c = 0; c < 16; ++c) {
        const float v = S[((xx ^ c) * 16) + c];
        t += (__popc(z & c) & 1) ? -v : v;
    }
    const unsigned ent = T.e[xx * 16 + z];
    gw[ent & 0xffffu] = __uint_as_float(__float_as_uint(t * 0.0625f) ^ (ent & 0x80000000u));
}

// ---- host side --------------------------------------------------------------

static bool rep_table_build(int n, uint32_t neg, RepTable& T) {
    unsigned gx[16], gz[16];
    if (!rep_generators(n, neg, gx, gz)) return false;
    const int m = 1 << (n / 2);
    for (unsigned I = 0; I < (1u << n); ++I) {
        unsigned x = 0, z = 0;
        bool negsign = false;
        for (int g = 0; g < n; ++g)
            if ((I >> g) & 1u) {
                if (host_popc(z & gx[g]) & 1) negsign = !negsign;
                x ^= gx[g];
                z ^= gz[g];
            }
        const bool tsign = negsign != ((host_popc(x & z) & 1) != 0);
        T.e[x * m + z] = I | (negsign ? 0x80000000u : 0u) | (tsign ? 0x40000000u : 0u);
    }
    T.odd_xor = 0;
    if (m == 16) {
        // smallest multiple of 4 for which, for every z, the 16 gathers of an
        // even row (blade offsets I) and of the next odd row (256 + (I ^ h))
        // fall on 32 distinct LDS banks
        for (unsigned h = 4; h < 256 && T.odd_xor == 0; h += 4) {
            bool ok = true;
            for (unsigned z = 0; z < 16 && ok; ++z) {
                unsigned used = 0;
                for (unsigned xx = 0; xx < 16 && ok; ++xx) {
                    const unsigned I = T.e[xx * 16 + z] & 0xffffu;
                    const unsigned b0 = I % 32, b1 = (256 + (I ^ h)) % 32;
                    if ((used >> b0) & 1u) ok = false;
                    used |= 1u << b0;
                    if ((used >> b1) & 1u) ok = false;
                    used |= 1u << b1;
                }
            }
            if (ok) T.odd_xor = h;
        }
    }
    return true;
}

// Tables are built once per (n, neg) and kept (immutable after insertion);
// n is even and at most 2 kRepMaxLogM, so (n / 2, neg) indexes a small array.
bool rep_table(int n, uint32_t neg, RepTable& T) {
    constexpr int kNegs = 1 << (2 * kRepMaxLogM);  // neg has at most n <= 8 bits
    static TableCache<RepTable, (kRepMaxLogM + 1) * kNegs> cache;
    if (n < 0 || (n & 1) || n > 2 * kRepMaxLogM || neg >= (unsigned)kNegs) return rep_table_build(n, neg, T);
    return cache.get((n / 2) * kNegs + (int)neg, T, [&](RepTable& t) { return rep_table_build(n, neg, t); });
}

bool split_applicable(int op, int n, uint32_t neg, uint32_t nul);
bool rep7_applicable(uint32_t neg);
int rep7_fwd(uint32_t neg, const float* a, const float* b, float* c, int64_t batch, void* stream);
int rep7_bwd(uint32_t neg, const float* a, const float* b, const float* gc, int64_t ldg, float* ga, float* gb,
             int64_t batch, void* stream);
int split_fwd(int n, uint32_t neg, const float* a, const float* b, float* c, int64_t batch, void* stream);
int split_bwd(int n, uint32_t neg, const float* a, const float* b, const float* gc, int64_t ldg, float* ga,
              float* gb, int64_t batch, void* stream);

// The matrix path serves the geometric product when the signature allows it
// (real type, n = 4, 6, 8; every non-degenerate n = 7 signature; split type
// n = 9, and n = 10 with e_9 null); returns false otherwise (the caller uses
// the per-term kernels).
bool rep_applicable(int op, int n, uint32_t neg, uint32_t nul) {
    if (n == 9 || n == 10) return split_applicable(op, n, neg, nul);
    if (n == 7) return op == CLF_OP_GEOM && nul == 0u && rep7_applicable(neg);
    if (op != CLF_OP_GEOM || nul != 0u || n < 4 || n > 2 * kRepMaxLogM) return false;
    RepTable T;
    return rep_table(n, neg, T);
}

// Workgroups: one per 4 * (64 / m) rows, at most 2048 (8 per CU); the waves
// walk the batch with a grid stride. More workgroups than are resident at once
// measured faster than a grid of exactly the resident count.
static long long rep_blocks(int n, int64_t batch) {
    const int m = 1 << (n / 2);
    const long long rows_per_block = 4LL * (64 / m);
    const long long g = (batch + rows_per_block - 1) / rows_per_block;
    const long long cap = 256LL * 8;
    return g < 1 ? 1 : (g > cap ? cap : g);
}

// The n = 8 backward launches one workgroup per 16 rows (each wave one group
// of four rows) instead of walking a capped grid: at the headline shape
// (262144 rows) 213 against 224 us with the 2048-workgroup cap (4096 and 8192
// workgroups: 221 and 217 us). The cap only bounds the grid dimension; the
// kernel's grid-stride loop covers any batch.
static long long rep16_bwd_blocks(int64_t batch) {
    const long long g = (batch + 15) / 16;
    const long long cap = 1LL << 24;
    return g < 1 ? 1 : (g > cap ? cap : g);
}

int rep_fwd(int n, uint32_t neg, const float* a, const float* b, float* c, int64_t batch, void* stream) {
    if (n == 9 || n == 10) return split_fwd(n, neg, a, b, c, batch, stream);
    if (n == 7) return rep7_fwd(neg, a, b, c, batch, stream);
    RepTable T;
    if (!rep_table(n, neg, T)) return set_error(CLF_ERR_UNSUPPORTED, "signature has no real matrix representation");
    hipStream_t s = (hipStream_t)stream;
    const long long want = rep_blocks(n, batch);
#define CLF_REP_GRID(K) dim3((unsigned)want)
    switch (n) {
        case 4: hipLaunchKernelGGL((rep_fwd_kernel<2>), CLF_REP_GRID(rep_fwd_kernel<2>), dim3(256), 0, s, a, b, c,
                                   (long long)batch, T); break;
        case 6: hipLaunchKernelGGL((rep_fwd_kernel<3>), CLF_REP_GRID(rep_fwd_kernel<3>), dim3(256), 0, s, a, b, c,
                                   (long long)batch, T); break;
        case 8: {
            const long long nb = rep16_bwd_blocks(batch);
            const bool one = nb * 16 >= batch;
#define CLF_REP16_FWD(NT)                                                                                     \
    do {                                                                                                     \
        if (one)                                                                                             \
            hipLaunchKernelGGL((rep16_fwd_kernel<NT, true>), dim3((unsigned)nb), dim3(256), 0, s, a, b, c,     \
                               (long long)batch, T);                                                         \
        else                                                                                                 \
            hipLaunchKernelGGL((rep16_fwd_kernel<NT, false>), dim3((unsigned)nb), dim3(256), 0, s, a, b, c,    \
                               (long long)batch, T);                                                         \
    } while (0)
            if (stream_nt(3.0 * 1024.0 * (double)batch)) CLF_REP16_FWD(true);
            else CLF_REP16_FWD(false);
#undef CLF_REP16_FWD
            break;
        }
        default: return set_error(CLF_ERR_UNSUPPORTED, "matrix path supports n = 4, 6, 8");
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int rep_bwd(int n, uint32_t neg, const float* a, const float* b, const float* gc, int64_t ldg, float* ga, float* gb,
            int64_t batch, void* stream) {
    if (n == 9 || n == 10) return split_bwd(n, neg, a, b, gc, ldg, ga, gb, batch, stream);
    if (n == 7) return rep7_bwd(neg, a, b, gc, ldg, ga, gb, batch, stream);
    RepTable T;
    if (!rep_table(n, neg, T)) return set_error(CLF_ERR_UNSUPPORTED, "signature has no real matrix representation");
    hipStream_t s = (hipStream_t)stream;
    const long long want = rep_blocks(n, batch);
    switch (n) {
        case 4: hipLaunchKernelGGL((rep_bwd_kernel<2>), CLF_REP_GRID(rep_bwd_kernel<2>), dim3(256), 0, s, a, b, gc,
                                   (long long)ldg, ga, gb, (long long)batch, T); break;
        case 6: hipLaunchKernelGGL((rep_bwd_kernel<3>), CLF_REP_GRID(rep_bwd_kernel<3>), dim3(256), 0, s, a, b, gc,
                                   (long long)ldg, ga, gb, (long long)batch, T); break;
        case 8:
            if (!ga && !gb) break;
            {
                const bool nt = stream_nt((3 + (ga != nullptr) + (gb != nullptr)) * 1024.0 * (double)batch);
                const long long nb = rep16_bwd_blocks(batch);
                const bool one = nb * 16 >= batch;
#define CLF_REP16_BWD(NT, WA, WB)                                                                               \
    do {                                                                                                       \
        if (one)                                                                                               \
            hipLaunchKernelGGL((rep16_bwd_kernel<NT, WA, WB, true>), dim3((unsigned)nb), dim3(256), 0, s, a, b, \
                               gc, (long long)ldg, ga, gb, (long long)batch, T);                               \
        else                                                                                                   \
            hipLaunchKernelGGL((rep16_bwd_kernel<NT, WA, WB, false>), dim3((unsigned)nb), dim3(256), 0, s, a,   \
                               b, gc, (long long)ldg, ga, gb, (long long)batch, T);                            \
    } while (0)
                if (ga && gb) {
                    if (nt) CLF_REP16_BWD(true, true, true);
                    else CLF_REP16_BWD(false, true, true);
                } else if (ga) {
                    if (nt) CLF_REP16_BWD(true, true, false);
                    else CLF_REP16_BWD(false, true, false);
                } else {
                    if (nt) CLF_REP16_BWD(true, false, true);
                    else CLF_REP16_BWD(false, false, true);
                }
#undef CLF_REP16_BWD
            }
            break;
        default: return set_error(CLF_ERR_UNSUPPORTED, "matrix path supports n = 4, 6, 8");
    }
#undef CLF_REP_GRID
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf

namespace clf {

// CLF_GEOM_PATH=direct in the environment (read at each call) turns the
// matrix-representation paths off, for comparisons against the per-term and
// GEMM kernels.
bool rep_disabled_by_env() { return options().geom_direct; }

// Broadcast-weight geometric product on the m = 16 path (n = 8, real type).
bool rep_bcast_applicable(int op, int n, uint32_t neg, uint32_t nul) {
    if (op != CLF_OP_GEOM || n != 8 || nul != 0u || rep_disabled_by_env()) return false;
    RepTable T;
    return rep_table(n, neg, T);
}

static long long rep_bcast_grid(int64_t batch) {
    long long g = (batch + 15) / 16;
    const long long cap = 256LL * 8;
    return g < 1 ? 1 : (g > cap ? cap : g);
}

// floats of workspace the backward's weight-gradient partials and their
// first-stage sums need
size_t rep_bcast_ws_floats(int64_t batch) {
    const long long nb = rep_bcast_grid(batch);
    return (size_t)(nb + (nb + kPartsPerSum - 1) / kPartsPerSum) * 256;
}

int rep_bcast_fwd(int side, int n, uint32_t neg, const float* x, const float* w, float* y, int64_t batch,
                  void* stream) {
    RepTable T;
    if (n != 8 || !rep_table(n, neg, T)) return set_error(CLF_ERR_UNSUPPORTED, "no m = 16 matrix representation");
    hipStream_t s = (hipStream_t)stream;
    // a capped grid: each wave builds the weight's operand once and walks
    // several groups (one workgroup per 16 rows measured 110 against 93 us at C3)
    const dim3 grid((unsigned)rep_bcast_grid(batch));
    const bool nt = stream_nt(2.0 * 1024.0 * (double)batch);
#define CLF_BCAST_FWD(SIDE, NT) \
    hipLaunchKernelGGL((rep16_bcast_fwd_kernel<SIDE, NT>), grid, dim3(256), 0, s, x, w, y, (long long)batch, T)
    if (side == 0) {
        if (nt) CLF_BCAST_FWD(0, true);
        else CLF_BCAST_FWD(0, false);
    } else {
        if (nt) CLF_BCAST_FWD(1, true);
        else CLF_BCAST_FWD(1, false);
    }
#undef CLF_BCAST_FWD
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

// ws: at least rep_bcast_ws_floats(batch) floats when gw != nullptr
int rep_bcast_bwd(int side, int n, uint32_t neg, const float* x, const float* w, const float* gy, int64_t ldg,
                  float* gx, float* gw, int64_t batch, float* ws, void* stream) {
    RepTable T;
    if (n != 8 || !rep_table(n, neg, T)) return set_error(CLF_ERR_UNSUPPORTED, "no m = 16 matrix representation");
    hipStream_t s = (hipStream_t)stream;
    const long long nb = rep_bcast_grid(batch);
    float* parts = gw ? ws : nullptr;
    if (batch > 0) {
        const bool nt = stream_nt((1 + (gw != nullptr) + (gx != nullptr)) * 1024.0 * (double)batch);
#define CLF_BCAST_BWD3(SIDE, NT, WX, WW)                                                                        \
    hipLaunchKernelGGL((rep16_bcast_bwd_kernel<SIDE, NT, WX, WW>), dim3((unsigned)nb), dim3(256), 0, s, x, w, gy,   \
                       (long long)ldg, gx, parts, (long long)batch, T)
#define CLF_BCAST_BWD(SIDE, NT)                              \
    do {                                                     \
        if (gx && gw) CLF_BCAST_BWD3(SIDE, NT, true, true);  \
        else if (gx) CLF_BCAST_BWD3(SIDE, NT, true, false);  \
        else if (gw) CLF_BCAST_BWD3(SIDE, NT, false, true);  \
    } while (0)
        if (side == 0) {
            if (nt) CLF_BCAST_BWD(0, true);
            else CLF_BCAST_BWD(0, false);
        } else {
            if (nt) CLF_BCAST_BWD(1, true);
            else CLF_BCAST_BWD(1, false);
        }
#undef CLF_BCAST_BWD
#undef CLF_BCAST_BWD3
    }
    if (gw) {
        int nsums = 0;
        float* sums = parts + nb * 256;
        if (batch > 0) {
            nsums = (int)((nb + kPartsPerSum - 1) / kPartsPerSum);
            hipLaunchKernelGGL(rep16_parts_sum_kernel, dim3((unsigned)nsums), dim3(256), 0, s, parts, (int)nb, sums);
        }
        hipLaunchKernelGGL(rep16_bcast_gw_kernel, dim3(1), dim3(1024), 0, s, sums, nsums, gw, T);
    }
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

}  // namespace clf
