// Shared helpers of the gfx950 Clifford library: error state, argument checks,
// and the blade-sign arithmetic used by every kernel.
//
// Blade sign convention (bit-pattern blades, generators e_0..e_{n-1}):
//   e_i e_j = sigma(i, j) e_{i^j},
//   sigma(i, j) = (-1)^{ #{(a,b): a > b, i_a = 1, j_b = 1} + |i & j & NEG| } * [i & j & NULL == 0]
// which is the table the reference builds in
// src/cliffordcuda/extensions/ga/geom_prod.py:44-74, in closed form.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>
#include <string>

#include "../../include/clifford_hip.h"

namespace clf {

constexpr int kMaxN = 20;          // largest n the product kernels accept (tiled above 12)
constexpr int kMaxNGraded = 20;    // graded ops are elementwise; bound rows * 2^n only

int set_error(int code, const std::string& msg);
void clear_error();

// Grid for a persistent (grid-stride) kernel: min(wanted, the number of
// workgroups of `kernel` that are resident at once on the current device),
// from the runtime occupancy query, cached per (device, kernel, dynamic LDS).
unsigned resident_grid(const void* kernel, int block_threads, size_t dyn_lds, long long wanted);

// Streaming global accesses with the nontemporal hint. When a kernel's rows
// (read once, written once) exceed the 256 MB last-level cache, keeping them
// out of the caches raises the sustained HBM rate (a 3-stream row copy of
// 768 MB: 5.5 TB/s plain, 6.3 TB/s nontemporal); when they fit, plain accesses
// keep cache hits for the next kernel. stream_nt() decides per launch from the
// launch's row bytes (CLF_STREAM_NT=on / off forces it).
bool stream_nt(double footprint_bytes);

// Path switches for comparisons and measurements, read from the environment
// once per process (at the first launch) and again only by
// clf_options_reload(); a running model's kernels never change under it.
//   CLF_STREAM_NT=on|off         nontemporal row streaming (default: by size)
//   CLF_PRODUCT_PATH=blocked|balanced|tiled|generic   per-term kernel family
//   CLF_GEOM_PATH=direct         geometric product on the per-term kernels
//   CLF_SPLIT_PATH=pairs         n = 10 split path as separate pair sums
//   CLF_ROTOR_PATH=chain         n = 8 rotor on the register plane chain
enum ProductPath { PATH_DEFAULT = 0, PATH_BLOCKED, PATH_BALANCED, PATH_TILED, PATH_GENERIC, PATH_SPLIT };
struct Options {
    int stream_nt;  // -1 by size, 0 off, 1 on
    int product_path;
    bool geom_direct, split_pairs, rotor_chain;
};
const Options& options();
void options_reload();

// A cache of per-signature tables indexed by a small key (0 <= key < N):
// built once under a lock, read without one afterwards (the ready flag is
// published with release order after the entry is written).
template <class T, int N>
struct TableCache {
    std::atomic<int> ready[N];
    bool ok[N];
    T tab[N];
    std::mutex mu;
    template <class Build>
    bool get(int key, T& out, Build build) {
        if (key < 0 || key >= N) return false;
        if (ready[key].load(std::memory_order_acquire) != 1) {
            std::lock_guard<std::mutex> lock(mu);
            if (ready[key].load(std::memory_order_relaxed) != 1) {
                T t{};
                ok[key] = build(t);
                tab[key] = t;
                ready[key].store(1, std::memory_order_release);
            }
        }
        if (ok[key]) out = tab[key];
        return ok[key];
    }
};
typedef float clf_fvec4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 load_stream(const float4* p) {
    const clf_fvec4 v = __builtin_nontemporal_load(reinterpret_cast<const clf_fvec4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void store_stream(float4* p, const float4& v) {
    const clf_fvec4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<clf_fvec4*>(p));
}

// Orders a wave's LDS accesses (writes by some lanes, reads by others) for the
// compiler; the hardware executes one wave's LDS instructions in order.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

#define CLF_HIP_CHECK(expr)                                                       \
    do {                                                                          \
        hipError_t _e = (expr);                                                   \
        if (_e != hipSuccess)                                                     \
            return ::clf::set_error(CLF_ERR_HIP, std::string(#expr ": ") +        \
                                    hipGetErrorString(_e));                       \
    } while (0)

// ---- compile-time blade arithmetic (low 4-bit register block) -------------
__host__ __device__ constexpr int cpopc(unsigned x) { return x ? (int)(x & 1u) + cpopc(x >> 1) : 0; }

// sum_{a > b} i_a j_b (Euclidean reorder count)
__host__ __device__ constexpr int creorder(unsigned i, unsigned j) {
    int p = 0;
    for (int b = 0; b < 16; ++b)
        if ((j >> b) & 1u) p += cpopc(i >> (b + 1));
    return p;
}

// sum of the set bit positions
__host__ __device__ constexpr int cbitsum(unsigned x) {
    int s = 0;
    for (int a = 0; a < 16; ++a)
        if ((x >> a) & 1u) s += a;
    return s;
}

// ---- run-time blade arithmetic ---------------------------------------------
// bit b of the result = parity of the bits of x strictly above b
__host__ __device__ inline unsigned suffix_parity(unsigned x) {
    unsigned y = x >> 1;
    y ^= y >> 1;
    y ^= y >> 2;
    y ^= y >> 4;
    y ^= y >> 8;
    y ^= y >> 16;
    return y;
}

__host__ __device__ inline int popc_rt(unsigned x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __popc(x);
#else
    return __builtin_popcount(x);
#endif
}

// parity of sum_{a > b} i_a j_b
__host__ __device__ inline int reorder_parity(unsigned i, unsigned j) {
    return popc_rt(j & suffix_parity(i)) & 1;
}

// parity of the sum of set bit positions = number of set bits at odd positions
__host__ __device__ inline int bitsum_parity(unsigned x) { return popc_rt(x & 0xAAAAAAAAu) & 1; }

enum Op : int {
    OP_GEOM = CLF_OP_GEOM,
    OP_WEDGE = CLF_OP_WEDGE,
    OP_INNER = CLF_OP_INNER,
    OP_LC = CLF_OP_LC,
    OP_RC = CLF_OP_RC,
    OP_REGR = CLF_OP_REGRESSIVE,
};

// Full sign sigma_op(i, j) in {-1, 0, +1} for any op, any n (the generic path
// and the host-side checks). For the regressive product the sign is
//   mu(full) * (-1)^{sum_{a in i} a + sum_{b in j} (n-1-b)} * sigma_E(i, j) * [i | j == full],
// which is dual(dual(a) ^ dual(b)) (reference _shared/_einsum_refs.py:86-124)
// written as one XOR-indexed product whose output index is ~k.
__host__ __device__ inline int full_sign(int op, int n, unsigned i, unsigned j, unsigned neg,
                                         unsigned nul) {
    const unsigned full = (n >= 32) ? 0xFFFFFFFFu : ((1u << n) - 1u);
    int par = reorder_parity(i, j);
    switch (op) {
        case OP_GEOM:
            if (i & j & nul) return 0;
            par += popc_rt(i & j & neg);
            break;
        case OP_WEDGE:
            if (i & j) return 0;
            break;
        case OP_INNER:
            if ((i & ~j) && (j & ~i)) return 0;
            if (i & j & nul) return 0;
            par += popc_rt(i & j & neg);
            break;
        case OP_LC:
            if (i & ~j) return 0;
            if (i & j & nul) return 0;
            par += popc_rt(i & j & neg);
            break;
        case OP_RC:
            if (j & ~i) return 0;
            if (i & j & nul) return 0;
            par += popc_rt(i & j & neg);
            break;
        case OP_REGR:
            if ((i | j) != full) return 0;
            par += bitsum_parity(i) + bitsum_parity(j) + ((n - 1) & 1) * popc_rt(j) + popc_rt(neg);
            break;
        default:
            return 0;
    }
    return (par & 1) ? -1 : 1;
}

}  // namespace clf
