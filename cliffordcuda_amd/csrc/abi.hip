// extern "C" entry points of libclifford_hip.so (declared in include/clifford_hip.h).
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include <mutex>

#include "clf_common.h"

namespace clf {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

void clear_error() { g_last_error.clear(); }

// Nontemporal streaming pays when a kernel's rows clearly exceed the 256 MB
// last-level cache (measured on the m = 16 kernels: 400 MB and more gain 5-10 %,
// about 270 MB is neutral; working sets of 100-400 MB that other kernels of a
// step re-read lose their cache hits).
constexpr double kStreamNtBytes = 320.0 * 1024 * 1024;

// ---- options: the environment, read once --------------------------------

static Options read_options() {
    Options o{};
    const char* e = std::getenv("CLF_STREAM_NT");
    o.stream_nt = (e && std::strcmp(e, "on") == 0) ? 1 : ((e && std::strcmp(e, "off") == 0) ? 0 : -1);
    e = std::getenv("CLF_PRODUCT_PATH");
    o.product_path = PATH_DEFAULT;
    if (e) {
        if (std::strcmp(e, "blocked") == 0) o.product_path = PATH_BLOCKED;
        else if (std::strcmp(e, "balanced") == 0) o.product_path = PATH_BALANCED;
        else if (std::strcmp(e, "tiled") == 0) o.product_path = PATH_TILED;
        else if (std::strcmp(e, "generic") == 0) o.product_path = PATH_GENERIC;
        else if (std::strcmp(e, "split") == 0) o.product_path = PATH_SPLIT;
    }
    e = std::getenv("CLF_GEOM_PATH");
    o.geom_direct = e && std::strcmp(e, "direct") == 0;
    e = std::getenv("CLF_SPLIT_PATH");
    o.split_pairs = e && std::strcmp(e, "pairs") == 0;
    e = std::getenv("CLF_ROTOR_PATH");
    o.rotor_chain = e && std::strcmp(e, "chain") == 0;
    return o;
}

// Published snapshots; a reload publishes a new one and keeps the old ones
// alive (readers may still hold them), so a few bytes per reload stay.
static std::atomic<const Options*> g_options{nullptr};
static std::mutex g_options_mu;

const Options& options() {
    const Options* o = g_options.load(std::memory_order_acquire);
    if (o) return *o;
    std::lock_guard<std::mutex> lock(g_options_mu);
    o = g_options.load(std::memory_order_relaxed);
    if (!o) {
        o = new Options(read_options());
        g_options.store(o, std::memory_order_release);
    }
    return *o;
}

void options_reload() {
    std::lock_guard<std::mutex> lock(g_options_mu);
    g_options.store(new Options(read_options()), std::memory_order_release);
}

bool stream_nt(double footprint_bytes) {
    const int f = options().stream_nt;
    if (f >= 0) return f == 1;
    return footprint_bytes > kStreamNtBytes;
}

// ---- resident grid: occupancy per (device, kernel, dynamic LDS) ------------
// Open-addressed table with lock-free reads: a slot's key is published (release)
// after its value; a lookup that finds the key reads the value it guards.
constexpr int kGridSlots = 4096;
struct GridSlot {
    std::atomic<uintptr_t> key;
    long long cap;
};
static GridSlot g_grid[kGridSlots];
static std::mutex g_grid_mu;

static uintptr_t grid_key(int dev, const void* kernel, size_t dyn_lds) {
    // distinct for distinct (dev, kernel, lds) in practice: kernels are code
    // addresses, dev < 256 and the dynamic LDS is below 2^20 bytes
    uintptr_t k = (uintptr_t)kernel;
    k ^= ((uintptr_t)dyn_lds << 40) ^ ((uintptr_t)(dev & 0xff) << 32) ^ ((uintptr_t)(dev >> 8) << 60);
    return k | 1u;  // never 0 (empty)
}

unsigned resident_grid(const void* kernel, int block_threads, size_t dyn_lds, long long wanted) {
    if (wanted < 1) return 1;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const uintptr_t key = grid_key(dev, kernel, dyn_lds);
    const unsigned h0 = (unsigned)((key >> 4) ^ (key >> 17) ^ (key >> 33)) & (kGridSlots - 1);
    long long cap = 0;
    for (unsigned probe = 0; probe < kGridSlots; ++probe) {
        GridSlot& sl = g_grid[(h0 + probe) & (kGridSlots - 1)];
        const uintptr_t k = sl.key.load(std::memory_order_acquire);
        if (k == key) {
            cap = sl.cap;
            break;
        }
        if (k == 0) break;  // not cached yet
    }
    if (cap == 0) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block_threads, dyn_lds) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
            (void)hipGetLastError();  // clear the query's error; fall back to a fixed cap
            per_cu = 2;
            cus = 256;
        }
        cap = (long long)(per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
        std::lock_guard<std::mutex> lock(g_grid_mu);
        for (unsigned probe = 0; probe < kGridSlots; ++probe) {
            GridSlot& sl = g_grid[(h0 + probe) & (kGridSlots - 1)];
            const uintptr_t k = sl.key.load(std::memory_order_relaxed);
            if (k == key) break;  // another thread inserted it meanwhile
            if (k == 0) {
                sl.cap = cap;
                sl.key.store(key, std::memory_order_release);
                break;
            }
        }
    }
    return (unsigned)(wanted < cap ? wanted : cap);
}

int product_fwd(int op, int n, uint32_t neg, uint32_t nul, const float* a, const float* b, float* c,
                int64_t batch, void* stream);
int product_bwd(int op, int n, uint32_t neg, uint32_t nul, const float* a, const float* b, const float* gc,
                int64_t ldg, float* ga, float* gb, int64_t batch, void* stream);
int graded(int kind, int n, uint32_t neg, uint32_t nul, int grade, const float* x, float* y, int64_t batch,
           void* stream);
int norm_sq_fwd(int n, uint32_t neg, uint32_t nul, const float* x, float* out, int64_t batch, void* stream);
int norm_sq_bwd(int n, uint32_t neg, uint32_t nul, const float* x, const float* gout, float* gx, int64_t batch,
                void* stream);

int rotor_state_floats(int n);
size_t rotor_apply_ws_bytes(int n, int64_t batch);
int rotor_compile_fwd(int n, const float* biv, float* state, float* cs, void* stream);
int rotor_compile_bwd(int n, const float* biv, const float* g_state, float* g_biv, void* stream);
int rotor_apply_fwd(int n, const float* state, const float* x, float* y, int64_t batch, void* stream);
int rotor_apply_bwd(int n, const float* state, const float* x, const float* gy, int64_t ldg, float* gx,
                    float* g_state, int64_t batch, void* ws, size_t ws_bytes, void* stream);
size_t rotor_biv_apply_ws_bytes(int n, int64_t batch);
int rotor_biv_apply_bwd(int n, const float* biv, const float* state, const float* x, const float* gy, int64_t ldg,
                        float* gx, float* g_biv, int64_t batch, void* ws, size_t ws_bytes, void* stream);
size_t rotor_cs_apply_ws_bytes(int n, int64_t batch);
int rotor_cs_apply_fwd(int n, const float* cs, const float* x, float* y, int64_t batch, void* stream);
int rotor_cs_apply_bwd(int n, const float* cs, const float* y, const float* gy, int64_t ldg, float* gx,
                       float* g_cs, int64_t batch, void* ws, size_t ws_bytes, void* stream);
int rotor_cs_compile_bwd(int n, const float* biv, const float* g_cs, float* g_biv, void* stream);

size_t bcast_ws_bytes(int n, int64_t batch);
int bcast_fwd(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w, float* y,
              int64_t batch, void* ws, size_t ws_bytes, void* stream);
int bcast_bwd(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w, const float* gy,
              int64_t ldg, float* gx, float* gw, int64_t batch, void* ws, size_t ws_bytes, void* stream);
int inverse_rep_supported(int n, uint32_t neg, uint32_t nul);
int inverse_rep(int n, uint32_t neg, uint32_t nul, const float* x, float* y, int* singular, int64_t batch,
                void* stream);
int inverse_versor(int n, const float* x, const float* xr, float* y, int* flags, float rtol, int64_t batch,
                   void* stream);
size_t bcast_scratch_bytes();
int bcast_bwd_noalloc(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w,
                      const float* gy, int64_t ldg, float* gx, float* gw, int64_t batch, void* stream);

// Floats between the rows of a dense batch of n-dimensional multivectors; an
// out-of-range n maps to 0 and is rejected by the callee's own check on n.
inline int64_t dense_ld(int n) { return (n >= 0 && n <= kMaxN) ? (int64_t(1) << n) : 0; }

// One wave per workgroup: where it runs (XCD index, and the compute unit,
// shader array and shader engine fields of the hardware id) and the two clock
// counters, read back to back (the real-time counter right after the
// shader-clock counter, which is not synchronised across compute units).
__global__ __launch_bounds__(64) void clock_sample_kernel(int64_t* out) {
    if (threadIdx.x != 0) return;
    const unsigned xcc = __builtin_amdgcn_s_getreg(0xf814) & 15u;   // hwreg(HW_REG_XCC_ID)
    const unsigned hw = __builtin_amdgcn_s_getreg(0xf804);          // hwreg(HW_REG_HW_ID)
    const int64_t cyc = (int64_t)__builtin_readcyclecounter();     // s_memtime
    const int64_t rt = (int64_t)__builtin_amdgcn_s_memrealtime();
    out[3 * (int64_t)blockIdx.x] = (int64_t)(xcc | (hw & 0xff00u));
    out[3 * (int64_t)blockIdx.x + 1] = cyc;
    out[3 * (int64_t)blockIdx.x + 2] = rt;
}

// Streaming calibration: out0 = in0 (+ in1 (+ in2)), out1 = in0 - out0, four
// floats per lane and four float4 per lane per pass, grid-stride. The byte
// pattern of a product launch without its arithmetic: its time is the rate
// the memory system gives that pattern (3 reads + 2 writes: the backward,
// 2 + 1: the forward, 1 + 1: a copy).
template <int NIN, int NOUT, bool NT>
__global__ __launch_bounds__(256) void stream_probe_kernel(const float4* __restrict__ a,
                                                           const float4* __restrict__ b,
                                                           const float4* __restrict__ c, float4* __restrict__ o0,
                                                           float4* __restrict__ o1, int64_t n4) {
    constexpr int U = 4;
    const int64_t stride = (int64_t)gridDim.x * 256 * U;
    for (int64_t base = (int64_t)blockIdx.x * 256 * U + threadIdx.x; base < n4; base += stride) {
        float4 x[U], y[U], z[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = base + (int64_t)u * 256;
            if (i < n4) {
                x[u] = NT ? load_stream(a + i) : a[i];
                if (NIN > 1) y[u] = NT ? load_stream(b + i) : b[i];
                if (NIN > 2) z[u] = NT ? load_stream(c + i) : c[i];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = base + (int64_t)u * 256;
            if (i < n4) {
                float4 s = x[u];
                if (NIN > 1) s = make_float4(s.x + y[u].x, s.y + y[u].y, s.z + y[u].z, s.w + y[u].w);
                if (NIN > 2) s = make_float4(s.x + z[u].x, s.y + z[u].y, s.z + z[u].z, s.w + z[u].w);
                if (NT) store_stream(o0 + i, s); else o0[i] = s;
                if (NOUT > 1) {
                    const float4 t = make_float4(x[u].x - s.x, x[u].y - s.y, x[u].z - s.z, x[u].w - s.w);
                    if (NT) store_stream(o1 + i, t); else o1[i] = t;
                }
            }
        }
    }
}

}  // namespace clf

extern "C" {

int clf_abi_version(void) { return CLF_ABI_VERSION; }

void clf_options_reload(void) { clf::options_reload(); }

const char* clf_last_error(void) { return clf::g_last_error.c_str(); }

int clf_device_info_get(int device, clf_device_info* out) {
    clf::clear_error();
    if (!out) return clf::set_error(CLF_ERR_ARG, "out must not be NULL");
    if (device < 0) return clf::set_error(CLF_ERR_ARG, "device must be >= 0");
    hipDeviceProp_t p;
    CLF_HIP_CHECK(hipGetDeviceProperties(&p, device));
    std::memset(out, 0, sizeof(*out));
    out->device = device;
    out->compute_units = p.multiProcessorCount;
    out->lds_bytes_per_block = (int)p.sharedMemPerBlock;
    out->clock_khz = p.clockRate;
    out->memory_clock_khz = p.memoryClockRate;
    out->memory_bus_width_bits = p.memoryBusWidth;
    std::strncpy(out->arch_name, p.gcnArchName, sizeof(out->arch_name) - 1);
    int wall = 0;
    CLF_HIP_CHECK(hipDeviceGetAttribute(&wall, hipDeviceAttributeWallClockRate, device));
    out->wall_clock_khz = wall;
    return CLF_OK;
}

int clf_clock_sample(int64_t* out, int slots, void* stream) {
    clf::clear_error();
    if (!out) return clf::set_error(CLF_ERR_ARG, "out must not be NULL");
    if (slots < 1 || slots > 4096) return clf::set_error(CLF_ERR_ARG, "slots must be in [1, 4096]");
    hipLaunchKernelGGL(clf::clock_sample_kernel, dim3(slots), dim3(64), 0, (hipStream_t)stream, out);
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int clf_stream_probe(int n_in, int n_out, const float* in0, const float* in1, const float* in2, float* out0,
                     float* out1, int64_t n_floats, int nontemporal, void* stream) {
    clf::clear_error();
    if (n_in < 1 || n_in > 3) return clf::set_error(CLF_ERR_ARG, "n_in must be 1, 2 or 3");
    if (n_out < 1 || n_out > 2) return clf::set_error(CLF_ERR_ARG, "n_out must be 1 or 2");
    if (n_floats < 0 || (n_floats & 3)) return clf::set_error(CLF_ERR_ARG, "n_floats must be a multiple of 4, >= 0");
    const void* ptrs[5] = {in0, n_in > 1 ? in1 : in0, n_in > 2 ? in2 : in0, out0, n_out > 1 ? out1 : out0};
    for (const void* q : ptrs) {
        if (!q) return clf::set_error(CLF_ERR_ARG, "null pointer argument");
        if (((uintptr_t)q) & 15u) return clf::set_error(CLF_ERR_ARG, "pointers must be 16-byte aligned");
    }
    if (n_floats == 0) return CLF_OK;
    const int64_t n4 = n_floats / 4;
    const int64_t wgs = std::min<int64_t>((n4 + 1023) / 1024, (int64_t)1 << 20);
    const float4* a = (const float4*)ptrs[0];
    const float4* b = (const float4*)ptrs[1];
    const float4* c = (const float4*)ptrs[2];
    float4* o0 = (float4*)out0;
    float4* o1 = (float4*)ptrs[4];
    hipStream_t s = (hipStream_t)stream;
#define CLF_STREAM_PROBE(NI, NO, NTV)                                                                     \
    hipLaunchKernelGGL((clf::stream_probe_kernel<NI, NO, NTV>), dim3((unsigned)wgs), dim3(256), 0, s, a, b, c, o0, \
                       o1, n4)
#define CLF_STREAM_PROBE_NT(NI, NO) \
    do { if (nontemporal) CLF_STREAM_PROBE(NI, NO, true); else CLF_STREAM_PROBE(NI, NO, false); } while (0)
    switch (n_in * 4 + n_out) {
        case 5: CLF_STREAM_PROBE_NT(1, 1); break;
        case 6: CLF_STREAM_PROBE_NT(1, 2); break;
        case 9: CLF_STREAM_PROBE_NT(2, 1); break;
        case 10: CLF_STREAM_PROBE_NT(2, 2); break;
        case 13: CLF_STREAM_PROBE_NT(3, 1); break;
        default: CLF_STREAM_PROBE_NT(3, 2); break;
    }
#undef CLF_STREAM_PROBE_NT
#undef CLF_STREAM_PROBE
    CLF_HIP_CHECK(hipGetLastError());
    return CLF_OK;
}

int clf_product_max_n(void) { return clf::kMaxN; }

int clf_product_fwd(int op, int n, uint32_t neg_mask, uint32_t null_mask, const float* a, const float* b, float* c,
                    int64_t batch, void* stream) {
    clf::clear_error();
    return clf::product_fwd(op, n, neg_mask, null_mask, a, b, c, batch, stream);
}

int clf_product_bwd(int op, int n, uint32_t neg_mask, uint32_t null_mask, const float* a, const float* b,
                    const float* gc, float* ga, float* gb, int64_t batch, void* stream) {
    clf::clear_error();
    return clf::product_bwd(op, n, neg_mask, null_mask, a, b, gc, clf::dense_ld(n), ga, gb, batch, stream);
}

int clf_product_bwd_ld(int op, int n, uint32_t neg_mask, uint32_t null_mask, const float* a, const float* b,
                       const float* gc, int64_t ldg, float* ga, float* gb, int64_t batch, void* stream) {
    clf::clear_error();
    return clf::product_bwd(op, n, neg_mask, null_mask, a, b, gc, ldg, ga, gb, batch, stream);
}

int clf_graded(int kind, int n, uint32_t neg_mask, uint32_t null_mask, int grade, const float* x, float* y,
               int64_t batch, void* stream) {
    clf::clear_error();
    return clf::graded(kind, n, neg_mask, null_mask, grade, x, y, batch, stream);
}

int clf_norm_sq_fwd(int n, uint32_t neg_mask, uint32_t null_mask, const float* x, float* out, int64_t batch,
                    void* stream) {
    clf::clear_error();
    return clf::norm_sq_fwd(n, neg_mask, null_mask, x, out, batch, stream);
}

int clf_norm_sq_bwd(int n, uint32_t neg_mask, uint32_t null_mask, const float* x, const float* gout, float* gx,
                    int64_t batch, void* stream) {
    clf::clear_error();
    return clf::norm_sq_bwd(n, neg_mask, null_mask, x, gout, gx, batch, stream);
}

int clf_rotor_state_floats(int n) { return clf::rotor_state_floats(n); }

int clf_rotor_compile_fwd(int n, const float* biv, float* state, float* cs, void* stream) {
    clf::clear_error();
    return clf::rotor_compile_fwd(n, biv, state, cs, stream);
}

int clf_rotor_compile_bwd(int n, const float* biv, const float* g_state, float* g_biv, void* stream) {
    clf::clear_error();
    return clf::rotor_compile_bwd(n, biv, g_state, g_biv, stream);
}

int clf_rotor_apply_fwd(int n, const float* state, const float* x, float* y, int64_t batch, void* stream) {
    clf::clear_error();
    return clf::rotor_apply_fwd(n, state, x, y, batch, stream);
}

size_t clf_rotor_apply_ws_bytes(int n, int64_t batch) { return clf::rotor_apply_ws_bytes(n, batch); }

int clf_rotor_apply_bwd(int n, const float* state, const float* x, const float* gy, float* gx, float* g_state,
                        int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    clf::clear_error();
    return clf::rotor_apply_bwd(n, state, x, gy, clf::dense_ld(n), gx, g_state, batch, ws, ws_bytes, stream);
}

int clf_rotor_apply_bwd_ld(int n, const float* state, const float* x, const float* gy, int64_t ldg, float* gx,
                           float* g_state, int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    clf::clear_error();
    return clf::rotor_apply_bwd(n, state, x, gy, ldg, gx, g_state, batch, ws, ws_bytes, stream);
}

size_t clf_rotor_bivector_apply_ws_bytes(int n, int64_t batch) { return clf::rotor_biv_apply_ws_bytes(n, batch); }

int clf_rotor_bivector_apply_bwd(int n, const float* biv, const float* state, const float* x, const float* gy,
                                 int64_t ldg, float* gx, float* g_biv, int64_t batch, void* ws, size_t ws_bytes,
                                 void* stream) {
    clf::clear_error();
    return clf::rotor_biv_apply_bwd(n, biv, state, x, gy, ldg, gx, g_biv, batch, ws, ws_bytes, stream);
}

int clf_rotor_cs_apply_fwd(int n, const float* cs, const float* x, float* y, int64_t batch, void* stream) {
    clf::clear_error();
    return clf::rotor_cs_apply_fwd(n, cs, x, y, batch, stream);
}

size_t clf_rotor_cs_apply_ws_bytes(int n, int64_t batch) { return clf::rotor_cs_apply_ws_bytes(n, batch); }

int clf_rotor_cs_apply_bwd(int n, const float* cs, const float* y, const float* gy, float* gx, float* g_cs,
                           int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    clf::clear_error();
    return clf::rotor_cs_apply_bwd(n, cs, y, gy, clf::dense_ld(n), gx, g_cs, batch, ws, ws_bytes, stream);
}

int clf_rotor_cs_apply_bwd_ld(int n, const float* cs, const float* y, const float* gy, int64_t ldg, float* gx,
                              float* g_cs, int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    clf::clear_error();
    return clf::rotor_cs_apply_bwd(n, cs, y, gy, ldg, gx, g_cs, batch, ws, ws_bytes, stream);
}

int clf_rotor_cs_compile_bwd(int n, const float* biv, const float* g_cs, float* g_biv, void* stream) {
    clf::clear_error();
    return clf::rotor_cs_compile_bwd(n, biv, g_cs, g_biv, stream);
}

int clf_inverse_rep_supported(int n, uint32_t neg_mask, uint32_t null_mask) {
    return clf::inverse_rep_supported(n, neg_mask, null_mask);
}

int clf_inverse_rep(int n, uint32_t neg_mask, uint32_t null_mask, const float* x, float* y, int* singular,
                    int64_t batch, void* stream) {
    clf::clear_error();
    return clf::inverse_rep(n, neg_mask, null_mask, x, y, singular, batch, stream);
}

int clf_inverse_versor(int n, const float* x, const float* xr, float* y, int* flags, float rtol, int64_t batch,
                       void* stream) {
    clf::clear_error();
    return clf::inverse_versor(n, x, xr, y, flags, rtol, batch, stream);
}

size_t clf_product_bcast_ws_bytes(int n, int64_t batch) { return clf::bcast_ws_bytes(n, batch); }

int clf_product_bcast_fwd(int op, int side, int n, uint32_t neg_mask, uint32_t null_mask, const float* x,
                          const float* w, float* y, int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    clf::clear_error();
    return clf::bcast_fwd(op, side, n, neg_mask, null_mask, x, w, y, batch, ws, ws_bytes, stream);
}

int clf_product_bcast_bwd(int op, int side, int n, uint32_t neg_mask, uint32_t null_mask, const float* x,
                          const float* w, const float* gy, float* gx, float* gw, int64_t batch, void* ws,
                          size_t ws_bytes, void* stream) {
    clf::clear_error();
    return clf::bcast_bwd(op, side, n, neg_mask, null_mask, x, w, gy, clf::dense_ld(n), gx, gw, batch, ws, ws_bytes,
                          stream);
}

int clf_product_bcast_bwd_ld(int op, int side, int n, uint32_t neg_mask, uint32_t null_mask, const float* x,
                             const float* w, const float* gy, int64_t ldg, float* gx, float* gw, int64_t batch,
                             void* ws, size_t ws_bytes, void* stream) {
    clf::clear_error();
    return clf::bcast_bwd(op, side, n, neg_mask, null_mask, x, w, gy, ldg, gx, gw, batch, ws, ws_bytes, stream);
}

size_t clf_product_bcast_bwd_noalloc_scratch_bytes(void) { return clf::bcast_scratch_bytes(); }

int clf_product_bcast_bwd_noalloc(int op, int side, int n, uint32_t neg_mask, uint32_t null_mask, const float* x,
                                  const float* w, const float* gy, float* gx, float* gw, int64_t batch,
                                  void* stream) {
    clf::clear_error();
    return clf::bcast_bwd_noalloc(op, side, n, neg_mask, null_mask, x, w, gy, clf::dense_ld(n), gx, gw, batch,
                                  stream);
}

}  // extern "C"
