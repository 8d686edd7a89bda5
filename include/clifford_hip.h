/*
 * clifford_hip.h — C ABI of the MI355X (gfx950) Clifford product & rotor library.
 *
 * This is the native boundary that replaces the reference's per-kernel pybind11
 * modules (the PYBIND11_MODULE blocks of src/cliffordcuda/kernels/ga/ and kernels/rotor/, loaded by
 * src/cliffordcuda/_config.py:29-38). Everything here takes plain device
 * pointers and sizes; nothing allocates device memory except where a function
 * says so, and nothing synchronises the host. Every call is asynchronous on the
 * given HIP stream (pass the caller's current stream; NULL = legacy default).
 *
 * Conventions
 *   - Multivectors are fp32, row-major (batch, 2^n), bit-pattern blade order:
 *     blade index i has generator k iff bit k of i is set.
 *   - The metric is passed as two bit masks over the n generators:
 *     neg_mask bit k = 1 iff e_k^2 = -1, null_mask bit k = 1 iff e_k^2 = 0
 *     (all other generators square to +1). The two masks must be disjoint.
 *   - Row counts and offsets are 64-bit.
 *   - Every argument is validated before any HIP call, so error paths run on a
 *     host without a GPU. Return value: CLF_OK or a CLF_ERR_* code; the text of
 *     the last error on the calling thread is clf_last_error().
 */
#ifndef CLIFFORD_HIP_H
#define CLIFFORD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CLF_ABI_VERSION 3

/* status codes */
#define CLF_OK               0
#define CLF_ERR_ARG          1   /* invalid argument (null pointer, bad n, bad masks, ...) */
#define CLF_ERR_UNSUPPORTED  2   /* valid but not supported (e.g. regressive on a degenerate metric) */
#define CLF_ERR_HIP          3   /* a HIP runtime call failed */
#define CLF_ERR_WORKSPACE    4   /* workspace missing or too small */

/* binary products: c[k] = sum_i sigma_op(i, i^k) a[i] b[i^k] */
#define CLF_OP_GEOM        0   /* geometric product                    (ref extensions/ga/geom_prod.py:253)      */
#define CLF_OP_WEDGE       1   /* outer product, i&j == 0               (ref extensions/ga/wedge_prod/chunk.py:105) */
#define CLF_OP_INNER       2   /* Hestenes inner incl. scalars          (ref extensions/ga/inner_prod/chunk.py:101) */
#define CLF_OP_LC          3   /* left contraction, i subset j          (ref extensions/ga/left_contract.py:121)  */
#define CLF_OP_RC          4   /* right contraction, j subset i         (ref extensions/ga/right_contract.py:110) */
#define CLF_OP_REGRESSIVE  5   /* dual(dual a ^ dual b), non-degenerate (ref extensions/ga/regressive_prod.py:186) */

/* graded (sign / mask / permutation) ops */
#define CLF_GRADED_REVERSE      0  /* (-1)^{k(k-1)/2}                    (ref algebra.py:195-205) */
#define CLF_GRADED_INVOLUTION   1  /* (-1)^k                             (ref algebra.py:278-286) */
#define CLF_GRADED_CONJUGATION  2  /* (-1)^{k(k+1)/2}                    (ref algebra.py:288-296) */
#define CLF_GRADED_PROJECTION   3  /* keep grade == `grade`              (ref algebra.py:298-306) */
#define CLF_GRADED_DUAL         4  /* y[m] = x[~m] s[m], x I^{-1}        (ref algebra.py:208-265) */
#define CLF_GRADED_DUAL_ADJ     5  /* adjoint of DUAL: y[k] = x[~k] s[~k] (backward of dual)      */

typedef struct clf_device_info {
    int    device;
    int    compute_units;
    int    lds_bytes_per_block;   /* max shared memory per workgroup */
    int    clock_khz;
    int    memory_clock_khz;
    int    memory_bus_width_bits;
    char   arch_name[64];
    int    wall_clock_khz;        /* rate of the s_memrealtime counter (clf_clock_sample) */
} clf_device_info;

/* ABI version (CLF_ABI_VERSION). */
int clf_abi_version(void);

/* Text of the last error on the calling thread ("" if none). Never NULL. */
const char* clf_last_error(void);

/* Re-read the CLF_* path switches from the environment. The library reads
 * them once, at its first launch; this lets a test or benchmark switch paths
 * inside one process. No counterpart in the reference (it has no such switches). */
void clf_options_reload(void);

/* Device properties used for launch shaping and the roofline report.
 * Replaces the reference's shared-memory probe
 * (src/cliffordcuda/extensions/ga/geom_prod_tiled.py:88-117,
 *  kernels/ga/geom_prod_tiled.cu:169-175). */
int clf_device_info_get(int device, clf_device_info* out);

/* Engine-clock sample for the roofline report: launches `slots` one-wave
 * workgroups on `stream`; workgroup w writes out[3w] = where it ran (bits 0..3:
 * XCD index; bits 8..15: compute-unit, shader-array and shader-engine fields
 * of the hardware id), out[3w+1] = that compute unit's shader-clock counter
 * (s_memtime) and out[3w+2] = the constant-rate counter (s_memrealtime,
 * wall_clock_khz). Two samples on one stream around a timed region give, per
 * compute unit seen in both, the mean engine clock over that region:
 * (cycles delta) / (real-time delta). `out` is device memory of 3 * slots
 * int64; 1 <= slots <= 4096 (4096 covers every compute unit in practice).
 * No counterpart in the reference (its harness warms the clock up instead,
 * benchmark/_harness.py:41-50, and records none). */
int clf_clock_sample(int64_t* out, int slots, void* stream);

/* Streaming calibration for the roofline report: the byte pattern of a
 * product launch without its arithmetic. Over n_floats floats (a multiple of
 * 4), out0 = in0 (+ in1 (+ in2)) for 1 <= n_in <= 3 inputs and, when
 * n_out == 2, out1 = in0 - out0; nontemporal != 0 streams with the
 * nontemporal hint, as the product kernels do past the last-level cache. All
 * pointers used are device memory, 16-byte aligned. The launch's time is the
 * rate the memory system gives that pattern (n_in = 3, n_out = 2 is a product
 * backward's, 2 + 1 a forward's). No counterpart in the reference. */
int clf_stream_probe(int n_in, int n_out, const float* in0, const float* in1, const float* in2, float* out0,
                     float* out1, int64_t n_floats, int nontemporal, void* stream);

/* Largest n the product kernels accept (20; rows past the LDS budget, n >= 13,
 * run tiled kernels, as the reference's geom_prod_tiled_fused does,
 * src/cliffordcuda/extensions/ga/geom_prod_tiled.py:370-398, which has no
 * fixed ceiling; a row of n = 20 is 4 MiB and its geometric product 2^40
 * multiply-adds). */
int clf_product_max_n(void);

/* Forward of a binary product on `batch` rows.
 * Replaces geom_prod_fwd (kernels/ga/geom_prod.cu:281-291), wedge_prod_fwd
 * (kernels/ga/wedge_prod.cu:181-217), inner_prod_fwd (kernels/ga/inner_prod.cu:171-230),
 * contract_fwd (kernels/ga/contract.cu:159-200) and the regressive forward
 * (extensions/ga/regressive_prod.py:143-170, GP kernel + index_select).
 * For CLF_OP_REGRESSIVE the output is written in final blade order (index ~k
 * already applied). a, b, c: device pointers to batch * 2^n floats; c must not
 * alias a or b. batch == 0 is a no-op. */
int clf_product_fwd(int op, int n, uint32_t neg_mask, uint32_t null_mask,
                    const float* a, const float* b, float* c,
                    int64_t batch, void* stream);

/* Fused backward of a binary product: one pass over gc produces
 *   ga[k] = sum_j sigma_op(k, j) b[j] gf[k^j],  gb[k] = sum_i sigma_op(i, k) a[i] gf[i^k]
 * (gf = gc, or gc[~.] for regressive). Replaces the reference's two forward-
 * kernel launches per backward (extensions/ga/geom_prod.py:242-250 and the
 * per-product backward wrappers). ga or gb may be NULL (that gradient is not
 * needed). */
int clf_product_bwd(int op, int n, uint32_t neg_mask, uint32_t null_mask,
                    const float* a, const float* b, const float* gc,
                    float* ga, float* gb, int64_t batch, void* stream);

/* clf_product_bwd with gc's row stride given: ldg = 2^n (packed rows, what
 * clf_product_bwd uses) or 0 (one gc row read for every batch row: the
 * gradient of a sum, which autograd hands over as a stride-0 expansion).
 * Any other stride returns CLF_ERR_ARG. Same route and kernels as the packed
 * call; no counterpart entry in the reference, whose wrappers make gc
 * contiguous first (extensions/ga/geom_prod.py:242-250). */
int clf_product_bwd_ld(int op, int n, uint32_t neg_mask, uint32_t null_mask,
                       const float* a, const float* b, const float* gc, int64_t ldg,
                       float* ga, float* gb, int64_t batch, void* stream);

/* Single-pass graded op: y = kind(x). `grade` is used by PROJECTION only.
 * DUAL / DUAL_ADJ need a non-degenerate metric. y must not alias x for the
 * dual kinds (they permute). Replaces the eager torch passes of
 * algebra.py:195-306. */
int clf_graded(int kind, int n, uint32_t neg_mask, uint32_t null_mask, int grade,
               const float* x, float* y, int64_t batch, void* stream);

/* norm_sq: out[r] = sum_b x[r,b]^2 w[b], w[b] = prod_{k in b} metric[k]
 * (ref algebra.py:309-334). */
int clf_norm_sq_fwd(int n, uint32_t neg_mask, uint32_t null_mask,
                    const float* x, float* out, int64_t batch, void* stream);

/* Backward of norm_sq: gx[r,b] = 2 w[b] x[r,b] gout[r]. */
int clf_norm_sq_bwd(int n, uint32_t neg_mask, uint32_t null_mask,
                    const float* x, const float* gout, float* gx,
                    int64_t batch, void* stream);


/* ---- rotor: bivector -> rotation -> Givens cs chain -> sandwich ~R x R ----
 * Euclidean semantics, like the reference: y = ~R x R, R = exp(sum_m b_m e_{i_m} e_{j_m}),
 * bivector slots in triu_indices(n, n, 1) order. Supported n: 2..12.
 *
 * cs is the reference's (C(n,2), 2) tensor (src/cliffordcuda/algebra.py:343-369):
 * the Givens factors of R = expm(2 (M - M^T)) (kernels/rotor/givens_factor.cu:23-38),
 * planes (p, q) in lex order, plane k's (c, s) at row C(n,2) - 1 - k. The chain
 * applies the planes lex-first, mapping each blade pair (I with p not q,
 * J = I ^ {p,q}) as y_I = c x_I + s sig x_J, y_J = c x_J - s sig x_I
 * (kernels/rotor/givens_apply_mb_perm_packed.cu:33-64).
 *
 * Rotor state (clf_rotor_state_floats(n) floats, the library's own cache of a
 * compiled bivector): the n x n rotation Q = expm(-2 (M - M^T)) acting on grade-1
 * coefficients (row-major), the cs pairs and, for n = 8, the 16 x 16 matrix
 * U = phi(R) of the rotor in the real representation of Cl(8,0) (row-major),
 * which the n = 8 state kernels use (phi(y) = U^T phi(x) U). */

/* Number of floats of the rotor state for n, or -1 if n is unsupported. */
int clf_rotor_state_floats(int n);

/* state = compile(biv) and, if cs != NULL, cs (2 C(n,2) floats) = the reference's
 * compile_bivector output. biv: C(n,2) floats. One single-workgroup launch, no
 * host sync. Replaces eigh_exp_fwd (kernels/rotor/eigh_exp.cu:270-322) and
 * givens_factor_fwd_v2 (kernels/rotor/givens_factor.cu:176-199). */
int clf_rotor_compile_fwd(int n, const float* biv, float* state, float* cs, void* stream);

/* g_biv = d/d(biv) of <g_state, compile(biv)>, reading only the Q block of
 * g_state (the cs and spin blocks are derived caches and carry no gradient).
 * The backward of the state path (apply_bivector, RotorLayer). */
int clf_rotor_compile_bwd(int n, const float* biv, const float* g_state, float* g_biv, void* stream);

/* y = ~R x R from a compiled state, for `batch` rows. y must not alias x. */
int clf_rotor_apply_fwd(int n, const float* state, const float* x, float* y,
                        int64_t batch, void* stream);

/* Bytes of device workspace clf_rotor_apply_bwd needs when g_state != NULL. */
size_t clf_rotor_apply_ws_bytes(int n, int64_t batch);

/* Backward of the state sandwich: gx = R gy ~R (the transpose of the action),
 * g_state: the Q block holds the component of dL/dQ tangent to SO(n)
 * (Q skew(Gamma), which is all clf_rotor_compile_bwd needs), the cs and spin
 * blocks are 0. gx or g_state may be NULL. x is read only when g_state != NULL. */
int clf_rotor_apply_bwd(int n, const float* state, const float* x, const float* gy,
                        float* gx, float* g_state, int64_t batch,
                        void* ws, size_t ws_bytes, void* stream);

/* clf_rotor_apply_bwd with gy's row stride given: 2^n (packed) or 0 (one gy
 * row for the whole batch); other strides return CLF_ERR_ARG. */
int clf_rotor_apply_bwd_ld(int n, const float* state, const float* x, const float* gy, int64_t ldg,
                           float* gx, float* g_state, int64_t batch,
                           void* ws, size_t ws_bytes, void* stream);

/* Bytes of device workspace clf_rotor_bivector_apply_bwd needs when g_biv != NULL. */
size_t clf_rotor_bivector_apply_ws_bytes(int n, int64_t batch);

/* Backward of y = apply(compile(biv), x) straight to the bivector: gx = the
 * transposed sandwich of gy, g_biv = dL/dbiv (C(n,2) floats, summed over the
 * batch), from the state clf_rotor_compile_fwd made of biv. One call for what
 * clf_rotor_apply_bwd + clf_rotor_compile_bwd do in two (for n <= 8 the batch
 * sum and the compile backward share one launch and g_state never goes
 * through memory). gy's rows are ldg floats apart (2^n, or 0 for one row read
 * for every batch row). gx or g_biv may be NULL. Replaces the backward of the
 * reference's apply_rotor(compile_bivector(b), x) chain
 * (extensions/rotor/givens_apply/mb_perm_packed.py:20-42 with
 * kernels/rotor/givens_factor.cu:202-231 and kernels/rotor/eigh_exp.cu:325-361). */
int clf_rotor_bivector_apply_bwd(int n, const float* biv, const float* state, const float* x,
                                 const float* gy, int64_t ldg, float* gx, float* g_biv,
                                 int64_t batch, void* ws, size_t ws_bytes, void* stream);

/* y = chain(cs) x for a caller's cs (any pairs, unit or not), `batch` rows.
 * Replaces givens_mb_perm_packed_fwd (kernels/rotor/givens_apply_mb_perm_packed.cu:250-267). */
int clf_rotor_cs_apply_fwd(int n, const float* cs, const float* x, float* y,
                           int64_t batch, void* stream);

/* Bytes of device workspace clf_rotor_cs_apply_bwd needs when g_cs != NULL. */
size_t clf_rotor_cs_apply_ws_bytes(int n, int64_t batch);

/* Backward of the cs chain from its output y: g_cs (2 C(n,2) floats, summed over
 * the batch) by the reference's rule (each plane's input rebuilt with the
 * transposed pair map: the exact gradient for unit pairs), and gx = the
 * transposed chain of gy (the exact gradient for any pairs; the reference
 * returns none). gx or g_cs may be NULL; y is read only when g_cs != NULL.
 * Replaces givens_mb_perm_packed_bwd (kernels/rotor/givens_apply_mb_perm_packed.cu:270-285). */
int clf_rotor_cs_apply_bwd(int n, const float* cs, const float* y, const float* gy,
                           float* gx, float* g_cs, int64_t batch,
                           void* ws, size_t ws_bytes, void* stream);

/* clf_rotor_cs_apply_bwd with gy's row stride given: 2^n or 0. */
int clf_rotor_cs_apply_bwd_ld(int n, const float* cs, const float* y, const float* gy, int64_t ldg,
                              float* gx, float* g_cs, int64_t batch,
                              void* ws, size_t ws_bytes, void* stream);

/* g_biv = d/d(biv) of <g_cs, cs(biv)> through the Givens factorisation and
 * expm (fp64, one single-workgroup launch). Replaces givens_factor_bwd_v2
 * (kernels/rotor/givens_factor.cu:202-231) and eigh_exp_bwd
 * (kernels/rotor/eigh_exp.cu:325-361). */
int clf_rotor_cs_compile_bwd(int n, const float* biv, const float* g_cs, float* g_biv, void* stream);

/* ---- multivector inverse ---------------------------------------------------
 * The native parts of the reference's inverse (src/cliffordcuda/extensions/ga/
 * inverse.py:139-194, inverse_rep.py:126-255). */

/* 1 if clf_inverse_rep serves this signature: the non-null generators (n' of
 * them) have a complex matrix representation of side 2^floor(n'/2) <= 128
 * (<= 64 when two copies are needed, odd n' with pseudoscalar^2 = +1). */
int clf_inverse_rep_supported(int n, uint32_t neg_mask, uint32_t null_mask);

/* y = inverse of the non-null part of each row of x (blades with a null
 * generator are 0 in y), through the matrix representation, one workgroup per
 * row; singular[r] = 1 if row r's matrix had a zero pivot (singular may be
 * NULL). For a metric without null generators y is x^-1. Replaces
 * rep_inverse / the first step of degenerate_rep_inverse (inverse_rep.py:182-255). */
int clf_inverse_rep(int n, uint32_t neg_mask, uint32_t null_mask, const float* x, float* y,
                    int* singular, int64_t batch, void* stream);

/* Versor inverse from xr = x rev(x): y = rev(x) / xr_0 per row, and
 * flags[r] bit 0 = xr is not a scalar (max |xr_k|, k > 0, above
 * rtol * max |xr|), bit 1 = |xr_0| < 1e-20. Replaces _versor_inverse
 * (inverse.py:70-78). */
int clf_inverse_versor(int n, const float* x, const float* xr, float* y, int* flags,
                       float rtol, int64_t batch, void* stream);

/* ---- broadcast-weight products (the product layers) ---------------------
 * y = op(x, w) (side 0, x on the left, as the reference layers compute it,
 * src/cliffordcuda/layers.py:43-47) or y = op(w, x) (side 1), with one weight
 * multivector w (2^n floats) shared by all `batch` rows of x. Replaces the
 * layer path expand -> per-row kernel -> autograd batch sum. Implemented as
 * fp32 MFMA GEMMs against the signed 2^n x 2^n matrix of w. Supported n: 7..10.
 * ws: device workspace of clf_product_bcast_ws_bytes(n, batch) bytes, 16-byte
 * aligned, owned by the caller; calls that share a workspace must not overlap. */
size_t clf_product_bcast_ws_bytes(int n, int64_t batch);

int clf_product_bcast_fwd(int op, int side, int n, uint32_t neg_mask, uint32_t null_mask,
                          const float* x, const float* w, float* y, int64_t batch,
                          void* ws, size_t ws_bytes, void* stream);

/* gx = dL/dx (batch x 2^n) and gw = dL/dw (2^n, summed over the batch); either
 * may be NULL. */
int clf_product_bcast_bwd(int op, int side, int n, uint32_t neg_mask, uint32_t null_mask,
                          const float* x, const float* w, const float* gy,
                          float* gx, float* gw, int64_t batch,
                          void* ws, size_t ws_bytes, void* stream);

/* clf_product_bcast_bwd with gy's row stride given: 2^n or 0. */
int clf_product_bcast_bwd_ld(int op, int side, int n, uint32_t neg_mask, uint32_t null_mask,
                             const float* x, const float* w, const float* gy, int64_t ldg,
                             float* gx, float* gw, int64_t batch,
                             void* ws, size_t ws_bytes, void* stream);

/* Allocation-free variant of clf_product_bcast_bwd. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and results as clf_product_bcast_bwd without ws / ws_bytes:
 * the workspace is a fixed device array of the library
 * (clf_product_bcast_bwd_noalloc_scratch_bytes() bytes, 32 MiB), held on each
 * device it runs on until the process ends. The call allocates nothing (no
 * hipMalloc, no library allocation); the GEMM path caps its split-K count so
 * its partials fit the array, and a call that would need more returns
 * CLF_ERR_WORKSPACE. All calls on one device share the array: calls that
 * overlap on a device (several streams or threads at once) race and must be
 * serialised by the caller. */
size_t clf_product_bcast_bwd_noalloc_scratch_bytes(void);

int clf_product_bcast_bwd_noalloc(int op, int side, int n, uint32_t neg_mask, uint32_t null_mask,
                                  const float* x, const float* w, const float* gy,
                                  float* gx, float* gw, int64_t batch, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CLIFFORD_HIP_H */
