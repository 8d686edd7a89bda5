// extern "C" entry points of libclifford_hip.so (declared in include/clifford_hip.h).
#include <cstdlib>
#include <cstring>

#include <map>
#include <mutex>
#include <tuple>

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

bool stream_nt(double footprint_bytes) {
    const char* e = std::getenv("CLF_STREAM_NT");
    if (e && std::strcmp(e, "on") == 0) return true;
    if (e && std::strcmp(e, "off") == 0) return false;
    return footprint_bytes > kStreamNtBytes;
}

unsigned resident_grid(const void* kernel, int block_threads, size_t dyn_lds, long long wanted) {
    static std::mutex mu;
    static std::map<std::tuple<int, const void*, size_t>, long long> cache;
    if (wanted < 1) return 1;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    long long cap = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        auto key = std::make_tuple(dev, kernel, dyn_lds);
        auto it = cache.find(key);
        if (it != cache.end()) {
            cap = it->second;
        } else {
            int per_cu = 0, cus = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block_threads, dyn_lds) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
                (void)hipGetLastError();  // clear the query's error; fall back to a fixed cap
                per_cu = 2;
                cus = 256;
            }
            cap = (long long)(per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
            cache.emplace(key, cap);
        }
    }
    return (unsigned)(wanted < cap ? wanted : cap);
}

int product_fwd(int op, int n, uint32_t neg, uint32_t nul, const float* a, const float* b, float* c,
                int64_t batch, void* stream);
int product_bwd(int op, int n, uint32_t neg, uint32_t nul, const float* a, const float* b, const float* gc,
                float* ga, float* gb, int64_t batch, void* stream);
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
int rotor_apply_bwd(int n, const float* state, const float* x, const float* gy, float* gx, float* g_state,
                    int64_t batch, void* ws, size_t ws_bytes, void* stream);
size_t rotor_cs_apply_ws_bytes(int n, int64_t batch);
int rotor_cs_apply_fwd(int n, const float* cs, const float* x, float* y, int64_t batch, void* stream);
int rotor_cs_apply_bwd(int n, const float* cs, const float* y, const float* gy, float* gx, float* g_cs,
                       int64_t batch, void* ws, size_t ws_bytes, void* stream);
int rotor_cs_compile_bwd(int n, const float* biv, const float* g_cs, float* g_biv, void* stream);

size_t bcast_ws_bytes(int n, int64_t batch);
int bcast_fwd(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w, float* y,
              int64_t batch, void* ws, size_t ws_bytes, void* stream);
int bcast_bwd(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w, const float* gy,
              float* gx, float* gw, int64_t batch, void* ws, size_t ws_bytes, void* stream);
int inverse_rep_supported(int n, uint32_t neg, uint32_t nul);
int inverse_rep(int n, uint32_t neg, uint32_t nul, const float* x, float* y, int* singular, int64_t batch,
                void* stream);
int inverse_versor(int n, const float* x, const float* xr, float* y, int* flags, float rtol, int64_t batch,
                   void* stream);
size_t bcast_scratch_bytes();
int bcast_bwd_noalloc(int op, int side, int n, uint32_t neg, uint32_t nul, const float* x, const float* w,
                      const float* gy, float* gx, float* gw, int64_t batch, void* stream);

}  // namespace clf

extern "C" {

int clf_abi_version(void) { return CLF_ABI_VERSION; }

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
    return clf::product_bwd(op, n, neg_mask, null_mask, a, b, gc, ga, gb, batch, stream);
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
    return clf::rotor_apply_bwd(n, state, x, gy, gx, g_state, batch, ws, ws_bytes, stream);
}

int clf_rotor_cs_apply_fwd(int n, const float* cs, const float* x, float* y, int64_t batch, void* stream) {
    clf::clear_error();
    return clf::rotor_cs_apply_fwd(n, cs, x, y, batch, stream);
}

size_t clf_rotor_cs_apply_ws_bytes(int n, int64_t batch) { return clf::rotor_cs_apply_ws_bytes(n, batch); }

int clf_rotor_cs_apply_bwd(int n, const float* cs, const float* y, const float* gy, float* gx, float* g_cs,
                           int64_t batch, void* ws, size_t ws_bytes, void* stream) {
    clf::clear_error();
    return clf::rotor_cs_apply_bwd(n, cs, y, gy, gx, g_cs, batch, ws, ws_bytes, stream);
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
    return clf::bcast_bwd(op, side, n, neg_mask, null_mask, x, w, gy, gx, gw, batch, ws, ws_bytes, stream);
}

size_t clf_product_bcast_bwd_noalloc_scratch_bytes(void) { return clf::bcast_scratch_bytes(); }

int clf_product_bcast_bwd_noalloc(int op, int side, int n, uint32_t neg_mask, uint32_t null_mask, const float* x,
                                  const float* w, const float* gy, float* gx, float* gw, int64_t batch,
                                  void* stream) {
    clf::clear_error();
    return clf::bcast_bwd_noalloc(op, side, n, neg_mask, null_mask, x, w, gy, gx, gw, batch, stream);
}

}  // extern "C"
