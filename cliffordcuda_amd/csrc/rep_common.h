// Shared pieces of the matrix-representation kernels (rep.hip, rep_split.hip,
// rotor_rep.hip): wave-local LDS ordering, the in-register Walsh-Hadamard
// transform, the DPP xor shuffles that build MFMA operands, the 4-block 16x16
// MFMA chain with its LDS relayout and block transpose, the conversion tables
// and row-group staging of m = 16, and the host search for real Pauli
// generators.
#pragma once

#include <utility>

#include "clf_common.h"

namespace clf {

constexpr int kRepMaxLogM = 4;  // m <= 16: the tables fit the kernel arguments

template <int M>
__device__ __forceinline__ void wht_inplace(float (&v)[M]) {
#pragma unroll
    for (int h = 1; h < M; h <<= 1)
#pragma unroll
        for (int i = 0; i < M; ++i)
            if (!(i & h)) {
                const float a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
}

// ---- 16 x 16 blocks on the matrix cores -------------------------------------
// The 4-block v_mfma_f32_16x16x1f32 multiplies four independent 16x16 matrices,
// block b taking its operands from lanes 16b .. 16b + 15. With lane x holding
// W[x][.] of a conversion (phi[r][c] = W[r ^ c][c]), operand k of lane x is
// W[x ^ k][k]: an xor shuffle inside the 16-lane row, done with DPP moves
// (quad_perm for xor 1..3, row_half_mirror = xor 7, row_mirror = xor 15,
// row_ror:8 = xor 8).
// The product C_b[4g + t][j] lands in lane 16g + j, register 4b + t; it goes
// back through LDS as W_c[i ^ j][j] at row stride 20 floats, which keeps both
// the scattered b32 writes and the b128 row reads free of bank conflicts.

typedef float floatx16 __attribute__((ext_vector_type(16)));

template <unsigned CTRL>
__device__ __forceinline__ float dpp16(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// value of v at lane (lane ^ K) of the same 16-lane row: row_ror:8 (a
// rotation by 8 inside the row is xor 8) for K = 8..11, else row_mirror (xor
// 15) and row_half_mirror (xor 7); then a quad_perm for the low bits
template <unsigned K>
__device__ __forceinline__ float xor16(float v) {
    constexpr bool ror8 = (K & 12u) == 8u;
    constexpr unsigned k1 = ror8 ? (K ^ 8u) : (K & 8u) ? (K ^ 15u) : K;
    constexpr unsigned k2 = (k1 & 4u) ? (k1 ^ 7u) : k1;
    if constexpr (ror8) v = dpp16<0x128>(v);
    else if constexpr ((K & 8u) != 0u) v = dpp16<0x140>(v);
    if constexpr ((k1 & 4u) != 0u) v = dpp16<0x141>(v);
    if constexpr (k2 == 1u) v = dpp16<0xB1>(v);       // quad_perm [1,0,3,2]
    else if constexpr (k2 == 2u) v = dpp16<0x4E>(v);  // quad_perm [2,3,0,1]
    else if constexpr (k2 == 3u) v = dpp16<0x1B>(v);  // quad_perm [3,2,1,0]
    return v;
}

template <unsigned... K>
__device__ __forceinline__ floatx16 mfma_chain_acc(floatx16 acc, const float (&wa)[16], const float (&wb)[16],
                                                   std::integer_sequence<unsigned, K...>) {
    ((acc = __builtin_amdgcn_mfma_f32_16x16x1f32(xor16<K>(wa[K]), xor16<K>(wb[K]), acc, 0, 0, 0)), ...);
    return acc;
}

// acc = sum_k A_b[.][k] B_b[k][.] for the four blocks, operands as above
__device__ __forceinline__ floatx16 mfma_chain(const float (&wa)[16], const float (&wb)[16]) {
    const floatx16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    return mfma_chain_acc(zero, wa, wb, std::make_integer_sequence<unsigned, 16>{});
}

constexpr int kRelayoutStride = 20;
constexpr int kRelayoutBlock = 16 * kRelayoutStride;  // floats per row of the group
constexpr int kRelayoutFloats = 4 * kRelayoutBlock;   // LDS a wave's relayout writes (1280 floats)

// lane (g, j) writes C_b[4g + t][j] (register 4b + t) to W_c[(4g + t) ^ j][j]
__device__ __forceinline__ void relayout_store(float* __restrict__ dst, const floatx16& acc, int lane) {
    const unsigned g = (unsigned)lane >> 4, j = (unsigned)lane & 15u;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int t = 0; t < 4; ++t)
            dst[b * kRelayoutBlock + (((4u * g + t) ^ j) * kRelayoutStride) + j] = acc[4 * b + t];
}

// lane (b, x) reads W_c[x][0..15] of row b
__device__ __forceinline__ void relayout_load(const float* __restrict__ src, int b, unsigned x, float (&w)[16]) {
    const float4* p = reinterpret_cast<const float4*>(src + b * kRelayoutBlock + x * kRelayoutStride);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 t = p[q];
        w[4 * q] = t.x;
        w[4 * q + 1] = t.y;
        w[4 * q + 2] = t.z;
        w[4 * q + 3] = t.w;
    }
}

// ---- conversion tables and the 16 x 16 row-group helpers ------------------

struct RepTable {
    // entry [x * m + z]: blade index | 0x80000000 if the sign s(I) is -1
    //                    | 0x40000000 if s(I) (-1)^{popc(x & z)} is -1 (transposed conversion)
    unsigned e[1 << (2 * kRepMaxLogM)];
    // m = 16: multiple of 4 xor-ed into the blade offsets of odd rows in LDS so
    // that the gathers of two rows in one half-wave use distinct banks (0: none found)
    unsigned odd_xor;
};

// The table for (n, neg), built once and cached; false if the signature has
// no real matrix representation of size 2^(n/2) <= 16.
bool rep_table(int n, uint32_t neg, RepTable& T);

// Group of four rows: lane l moves float4 chunk l of row j (j = 0..3); rows
// past the end re-read the last row and are never stored.
struct Pre16 {
    float4 v[4];
};

// Row strides here are the row length (packed) or 0 (one row read for every
// batch row): (row & row_mask(ld)) * length is then the row's offset, two
// 32-bit ANDs instead of a 64-bit multiply per fetch.
__device__ __forceinline__ long long row_mask(long long ld) { return ld ? -1LL : 0LL; }

// NT: nontemporal accesses (stream_nt decides per launch). ld: floats between
// rows (256 packed; 0 for one row broadcast over the batch, an upstream
// gradient of a sum)
template <bool NT>
__device__ __forceinline__ Pre16 fetch16(const float* __restrict__ src, long long row0, long long batch, int lane,
                                         long long ld = 256) {
    Pre16 p;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        long long row = row0 + j;
        row = row < batch ? row : batch - 1;
        const float4* q = reinterpret_cast<const float4*>(src + ((row & row_mask(ld)) << 8)) + lane;
        p.v[j] = NT ? load_stream(q) : *q;
    }
    return p;
}

// staged row j at [j * 256, (j + 1) * 256), odd rows with chunk index lane ^ oddc
__device__ __forceinline__ void stage16(float* __restrict__ dst, const Pre16& p, int lane, unsigned oddc) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
        reinterpret_cast<float4*>(dst + j * 256)[(j & 1) ? (lane ^ oddc) : lane] = p.v[j];
}

// Rows past the end were computed from clamped copies of the last row, so
// their results are bit-identical to it: they are stored to the last row again
// instead of branching around the stores.
template <bool NT>
__device__ __forceinline__ void store16(float* __restrict__ dstg, const float* __restrict__ src, long long row0,
                                        long long batch, int lane, unsigned oddc) {
    float4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = reinterpret_cast<const float4*>(src + j * 256)[(j & 1) ? (lane ^ oddc) : lane];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        long long row = row0 + j;
        row = row < batch ? row : batch - 1;
        float4* q = reinterpret_cast<float4*>(dstg + row * 256) + lane;
        if (NT) store_stream(q, v[j]);
        else *q = v[j];
    }
}

// gather t[z] of the lane's row with the sign bit selected by SIGNSHIFT
// (0: s(I), 1: the transposed conversion's sign), then WHT
template <int SIGNSHIFT>
__device__ __forceinline__ void gather16(const float* __restrict__ row, const unsigned (&ent)[16], float (&w)[16]) {
#pragma unroll
    for (int z = 0; z < 16; ++z)
        w[z] = __uint_as_float(__float_as_uint(row[ent[z] & 0xffffu]) ^ ((ent[z] << SIGNSHIFT) & 0x80000000u));
}

// inverse WHT of W_c[x][.], scale 1/16, scatter s(I) t[z] into the row's blade slots
__device__ __forceinline__ void unconvert16(float (&w)[16], float* __restrict__ row, const unsigned (&ent)[16]) {
    wht_inplace<16>(w);
#pragma unroll
    for (int z = 0; z < 16; ++z)
        row[ent[z] & 0xffffu] = __uint_as_float(__float_as_uint(w[z] * 0.0625f) ^ (ent[z] & 0x80000000u));
}

// the same for a W that already carries the factor 1/16
__device__ __forceinline__ void unconvert16_prescaled(float (&w)[16], float* __restrict__ row,
                                                      const unsigned (&ent)[16]) {
    wht_inplace<16>(w);
#pragma unroll
    for (int z = 0; z < 16; ++z)
        row[ent[z] & 0xffffu] = __uint_as_float(__float_as_uint(w[z]) ^ (ent[z] & 0x80000000u));
}

// LDS accesses at byte addresses computed by the kernel (xor-swizzled layouts
// whose addresses are one xor away from a per-lane base)
typedef __attribute__((address_space(3))) float lds_f32;
__device__ __forceinline__ unsigned lds_byte_addr(float* p) { return (unsigned)(uintptr_t)(lds_f32*)p; }
__device__ __forceinline__ float lds_load(unsigned a) { return *(lds_f32*)(uintptr_t)a; }
__device__ __forceinline__ void lds_store(unsigned a, float v) { *(lds_f32*)(uintptr_t)a = v; }

// 16 x 16 x 16 product: operand k of A (B) is xor16<k>(a[k]) if SA (SB), else
// a[k] as given (already shuffled)
template <bool SA, bool SB, unsigned... K>
__device__ __forceinline__ floatx16 mfma_chain_pre(floatx16 acc, const float (&a)[16], const float (&b)[16],
                                                   std::integer_sequence<unsigned, K...>) {
    ((acc = __builtin_amdgcn_mfma_f32_16x16x1f32(SA ? xor16<K>(a[K]) : a[K], SB ? xor16<K>(b[K]) : b[K], acc, 0, 0,
                                                  0)),
     ...);
    return acc;
}

template <unsigned... K>
__device__ __forceinline__ void shuffle_operand(const float (&w)[16], float (&op)[16],
                                                std::integer_sequence<unsigned, K...>) {
    ((op[K] = xor16<K>(w[K])), ...);
}


// Block transpose of a product for the next product. C_b[4g + t][j] sits in
// lane 16g + j, register 4b + t; after the swaps, register k = 4g + t of lane
// (b, j) holds C_b[k][j], the B operand of a following 4-block product (and,
// read as C_b^T, its A operand). For each t the four registers 4b + t form a
// 4 x 4 transpose between the register block b and the 16-lane row g: one
// 32-lane swap (bit 1 of b and g), then one 16-lane swap (bit 0).
__device__ __forceinline__ void permlane_swap32(float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

__device__ __forceinline__ void permlane_swap16(float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

__device__ __forceinline__ void transpose_blocks(const floatx16& acc, float (&op)[16]) {
#pragma unroll
    for (int k = 0; k < 16; ++k) op[k] = acc[k];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        permlane_swap32(op[t], op[8 + t]);
        permlane_swap32(op[4 + t], op[12 + t]);
        permlane_swap16(op[t], op[4 + t]);
        permlane_swap16(op[8 + t], op[12 + t]);
    }
}

// ---- rotors through the representation of Cl(8,0) ------------------------
// The sandwich y = ~R x R of a Euclidean rotor acts on blade coefficients the
// same way whatever the algebra's metric (it is the outermorphism of a
// rotation), so for n = 8 it runs through the real 16 x 16 representation of
// Cl(8,0): phi(y) = U^T phi(x) U with U = phi(R). Plane k = (p, q) (lex order)
// has phi(e_p e_q) = sign P(x, z), a signed permutation taking row r to row
// r ^ x with the factor f(r) = sign (-1)^{popc(z & (r ^ x))}; the table packs
// x (bits 0-3) and the mask of rows with f(r) = -1 (bits 16-31).
constexpr int kSpinN = 8;
constexpr int kSpinPlanes = kSpinN * (kSpinN - 1) / 2;
struct SpinTable {
    unsigned plane[kSpinPlanes];
};

// The Cl(8,0) conversion table and the plane table, built once.
bool spin_tables(RepTable& T, SpinTable& S);

// ---- host: generators -------------------------------------------------------

inline int host_popc(unsigned v) { return __builtin_popcount(v); }

// Generators for the metric (bit g of neg set: e_g^2 = -1), or false if the
// signature is not a real matrix algebra of size 2^(n/2).
inline bool rep_generators(int n, uint32_t neg, unsigned* gx, unsigned* gz) {
    if (n % 2 || n < 2 || n > 2 * kRepMaxLogM) return false;
    const int q = host_popc(neg), p = n - q;
    const int d = ((p - q) % 8 + 8) % 8;
    if (d != 0 && d != 2) return false;
    const int k = n / 2;
    const unsigned span = 1u << k;
    // depth-first search in a fixed order (deterministic)
    int g = 0;
    unsigned cand[16] = {0};
    while (g >= 0 && g < n) {
        bool found = false;
        for (unsigned c = cand[g] + 1; c < span * span; ++c) {
            const unsigned cx = c / span, cz = c % span;
            const int want = ((neg >> g) & 1u) ? 1 : 0;  // square -1 <=> popc(z & x) odd
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
            if (g < n) cand[g] = 0;
        } else {
            cand[g] = 0;
            --g;
        }
    }
    return g == n;
}

}  // namespace clf
