// Internal definitions shared by the libom_hip.so translation units: the context, the arena, error handling and
// small device helpers. Everything here is gfx950 (CDNA4): 64-wide wavefronts, fp32 MFMA, 160 KB LDS per CU.
#pragma once

#include <hip/hip_runtime.h>
#ifdef OM_CHECKED
#include <hsa/hsa.h>
#endif

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../include/om.h"

struct om_slab {
    char *base = nullptr;
    uint64_t size = 0;
};

struct om_region {
    std::vector<om_slab> slabs;
    size_t cur = 0;       // slab being filled
    uint64_t off = 0;     // bytes used in slabs[cur]
    uint64_t used = 0;    // bytes handed out in this region since the last reset
    uint64_t default_slab = 0;
    uint64_t limit = 0;   // om_arena_set_limit: at most this many bytes handed out (0: no limit)
};

// A max pool that a 3x3 convolution's split-sum pass can do in the same pass: kh x kw windows, stride kh, kw, no
// padding, tiling the convolution's output exactly; y and idx as om_maxpool_fwd's.
struct Conv3Pool {
    float *y;
    int32_t *idx;
    int kh, kw;
};

struct om_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    om_region region[2];
    // Device scratch owned by the context (split-K partials, per-row statistics); grown on demand between steps.
    float *scratch = nullptr;
    uint64_t scratch_bytes = 0;
    // Second slot for callers that launch GEMMs while holding their own scratch (attention's score recompute).
    float *scratch2 = nullptr;
    uint64_t scratch2_bytes = 0;
    // Device address of the fixed scratch array the allocation-free entry point uses on this context's device
    // (looked up once per device at context creation; NULL if that failed), and the slot of it this context holds
    // (claimed by its first allocation-free call, released by om_ctx_destroy; -1 while it holds none).
    void *noalloc_scratch = nullptr;
    int noalloc_slot = -1;
    // How the GELU epilogues of products evaluate erf and exp (om_ctx_set_gelu).
    int gelu_mode = OM_GELU_FAST;
    int num_cus = 256;
    // The step graph being captured on the stream (om_graph_capture_begin .. _end), else NULL.
    struct om_graph *cap = nullptr;
    // Launch timing probe (om_ctx_probe): events [2 i] / [2 i + 1] bracket the i-th recorded om_param_grads_group call.
    bool probe_on = false;
    int probe_n = 0;
    std::vector<hipEvent_t> probe_ev;
};

// The per-step values a step graph's kernels read (om_step_values plus the readback's sequence number and the
// launch number), 32 bytes.
struct om_step_block {
    float lr, step_size, sqrt_bc2, pad;
    uint64_t seq, id;
};
static_assert(sizeof(om_step_block) == 32 && offsetof(om_step_block, id) == 24, "k_step_begin reads it as 2 x 16 B");

struct om_graph {
    om_ctx *ctx = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // Pinned, fine-grained host memory: [entry the host writes before a launch][ack the graph's first node writes
    // after reading the entry]. `dev` is device memory the first node copies the entry into for the later nodes.
    char *host = nullptr;
    om_step_block *dev = nullptr;
    uint64_t launches = 0;
    om_readback *rb = nullptr;  // the capture's readback post, if any
    uint64_t rb_bytes = 0;
};

// Checked builds (compiled with -DOM_CHECKED; the reference's Checked configuration fills rented memory with 0xFF,
// "a NaN for floats, so a read of memory nobody wrote is visible", BufferPool.cs:21-22): every workgroup fills its
// whole LDS allocation (static and dynamic: the dispatch packet's group segment size) with 0xFF before the kernel's
// own code runs (OM_LDS_POISON, the first statement of every kernel), and om_alloc and the context scratch hand out
// memory filled with 0xFF, so a value computed from LDS or scratch that nothing wrote in this launch or call becomes
// NaN. Product builds compile OM_LDS_POISON to nothing.
#ifdef OM_CHECKED
__device__ __forceinline__ void om_poison_lds() {
    const hsa_kernel_dispatch_packet_t *pk = (const hsa_kernel_dispatch_packet_t *)__builtin_amdgcn_dispatch_ptr();
    const unsigned words = pk->group_segment_size / 4u;
    const unsigned nt = blockDim.x * blockDim.y * blockDim.z;
    const unsigned t = threadIdx.x + blockDim.x * (threadIdx.y + blockDim.y * threadIdx.z);
    typedef __attribute__((address_space(3))) unsigned lds_u32;
    lds_u32 *lds = reinterpret_cast<lds_u32 *>(static_cast<uintptr_t>(0));  // LDS address 0, not the null pointer
    for (unsigned i = t; i < words; i += nt) lds[i] = 0xFFFFFFFFu;
    __syncthreads();
}
#define OM_LDS_POISON() om_poison_lds()
#else
#define OM_LDS_POISON() \
    do {                \
    } while (0)
#endif

namespace om {

om_status fail(om_ctx *ctx, om_status code, const char *fmt, ...);
om_status check_hip(om_ctx *ctx, hipError_t e, const char *what);
// Returns device scratch of at least `bytes` (kept by the context; valid until the next call that grows it, which
// first synchronises the stream so no in-flight kernel still reads the old buffer).
om_status scratch(om_ctx *ctx, uint64_t bytes, float **out);
// The same for the second slot (never used by the GEMM engine itself).
om_status scratch2(om_ctx *ctx, uint64_t bytes, float **out);
// The MSE loss of pred against target over n elements, with the gradient for a unit upstream gradient in unit and
// the value posted to rb when given (om_mse_fwd_unit / om_mse_fwd_post); mse_final finishes it from per-wavefront
// fp64 partials of the squared differences (the fused epilogue of om_linear_fwd_resid_mse).
om_status mse_of(om_ctx *ctx, const float *pred, const float *target, float *unit, float *loss, int64_t n,
                 om_readback *rb);
om_status mse_final(om_ctx *ctx, const double *part, int np, float *loss, int64_t n, om_readback *rb);
// Checked builds: fills [p, p + bytes) with 0xFF on the context's stream (nothing otherwise).
om_status poison(om_ctx *ctx, void *p, uint64_t bytes);
// Sets ctx->noalloc_scratch to the device address of the fixed scratch array on ctx->device (the current device),
// looking it up on the first call for that device only.
om_status noalloc_init(om_ctx *ctx);
// The context's own slot of that array (OM_NOALLOC_SCRATCH_BYTES bytes), claimed on the first call: no two live
// contexts on one device share a slot, so their calls cannot overwrite each other's partials. OM_E_STATE when every
// slot of the device is held by another live context.
om_status noalloc_slot(om_ctx *ctx, double **out);
void noalloc_release(om_ctx *ctx);
// Comparison knobs: environment variables that force a tile, a kernel family or a code path for A/B runs. They are
// read only in a tuning build (compiled with -DOM_TUNING_KNOBS); the product build's choices depend on the shapes
// alone, so its results repeat bit for bit for a given shape whatever the environment.
inline const char *tuning_env(const char *name) {
#ifdef OM_TUNING_KNOBS
    return std::getenv(name);
#else
    (void)name;
    return nullptr;
#endif
}
// OM_E_STATE with a message when a step graph is being captured on ctx's stream (for calls a graph cannot hold).
om_status refuse_in_capture(om_ctx *ctx, const char *what);
// The launch timing probe around one call: probe_begin records the start event and returns the call's slot (-1 when
// the probe is off, full or the stream is being captured); probe_end records the end event of that slot.
int probe_begin(om_ctx *ctx);
void probe_end(om_ctx *ctx, int slot);
// The stream every launch of the context goes to.
inline hipStream_t cur_stream(const om_ctx *ctx) { return ctx->stream; }
// A readback post written by another entry point's kernel: checks that r belongs to ctx and holds `bytes`, waits for
// the previous post's copy (the pinned buffer is reused), and returns the device addresses of the buffer and of its
// sequence word with the sequence number the post carries; readback_posted records the launched post. Inside a
// step-graph capture nothing is waited for, *seq_dev is the device word the kernel must read the number from (else
// NULL), and the post is registered with the graph, whose launches advance the readback.
om_status readback_target(om_ctx *ctx, om_readback *r, uint64_t bytes, char **dst, uint64_t **seq_at, uint64_t *seq,
                          const uint64_t **seq_dev);
void readback_posted(om_readback *r, uint64_t seq, uint64_t bytes);
// out[col] (+)= (float) sum over c < chunks of part[c * cols + col], in double, a wavefront per column; a second
// (part2, out2) pair of the same shape is reduced in the same launch when given.
om_status chunk_final(om_ctx *ctx, const double *part, int chunks, int cols, float *out, int acc,
                      const double *part2 = nullptr, float *out2 = nullptr);

inline unsigned grid1d(int64_t n, int block, int64_t max_blocks = 1 << 20) {
    int64_t g = (n + block - 1) / block;
    if (g < 1) g = 1;
    if (g > max_blocks) g = max_blocks;
    return (unsigned)g;
}

}  // namespace om

#define OM_CHECK_CTX(ctx)                     \
    do {                                      \
        if (!(ctx)) return OM_E_ARG;          \
    } while (0)
#define OM_REQUIRE(ctx, cond, ...)                                   \
    do {                                                             \
        if (!(cond)) return om::fail((ctx), OM_E_ARG, __VA_ARGS__);  \
    } while (0)
#define OM_LAUNCH_CHECK(ctx, what) om::check_hip((ctx), hipGetLastError(), (what))

// ------------------------------------------------------------------------------------------------ device helpers
namespace omd {

__device__ __forceinline__ float canon(float x) { return x == x ? x : __int_as_float(0x7FC00000); }

// Wavefront (64 lanes) sum of a double by butterfly shuffles; every lane gets the total. The combine order is fixed
// (xor 32, 16, ..., 1), so the result depends only on the lane values.
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float w = __shfl_xor(v, o, 64);
        v = w > v ? w : v;
    }
    return v;
}

// Block sum of a double over `nw` wavefronts through LDS; all threads get the total (fixed order: wave 0..nw-1).
template <int NW>
__device__ __forceinline__ double block_sum(double v, double *sh) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) sh[w] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < NW; i++) t += sh[i];
    return t;
}

// The reference's canonical 16-partial sum (RowReduce.Sum16, Softmax.cs:139-179) over one row held by a 16-lane group:
// lane t holds p[t] = sum of the row's elements j = t, t+16, ... in increasing j; the halving combine p[t]+p[t+8],
// +4, +2, +1 runs as shuffles inside the group, so the bits equal the reference's; every lane gets the total.
__device__ __forceinline__ float sum16(float p) {
    p = p + __shfl_down(p, 8, 16);
    p = p + __shfl_down(p, 4, 16);
    p = p + __shfl_down(p, 2, 16);
    p = p + __shfl_down(p, 1, 16);
    return __shfl(p, 0, 16);
}
// Row maximum over a 16-lane group ignoring NaN (RowReduce.Max, Softmax.cs:181-212); exact, so order-free.
__device__ __forceinline__ float max16(float v) {
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
        float w = __shfl_xor(v, o, 16);
        v = w > v ? w : v;
    }
    return v;
}

// One column of a two-stage column reduction, by one wavefront: lanes add the chunk partials c = lane, lane + 64, ...
// of part[c * cols + col] in increasing c, then the fixed butterfly; lane 0 writes out[col] (+)= the float of the sum.
__device__ __forceinline__ void column_sum_wave(const double *part, float *out, int chunks, int cols, int col, int acc,
                                                int lane) {
    // eight of a lane's loads in flight before their adds (same order: c = lane, lane + 64, ...)
    double s = 0.0;
    for (int c0 = 0; c0 < chunks; c0 += 64 * 8) {
        double v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int c = c0 + 64 * u + lane;
            v[u] = c < chunks ? part[(int64_t)c * cols + col] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (c0 + 64 * u + lane < chunks) s += v[u];
    }
    s = wave_sum(s);
    if (lane == 0) {
        float v = (float)s;
        out[col] = acc ? out[col] + v : v;
    }
}

// The reference's fp32 polynomials (Transcendental.cs:39-263), restated with one IEEE rounding per operation; the
// library is built with -ffp-contract=off so no multiply-add is fused behind our back.
__device__ __forceinline__ float exp_poly(float x) {
    const float magic = 12582912.0f;
    float t = x * 1.44269502f + magic;
    float nf = t - magic;
    float r = (x - nf * 0.693145751953125f) - nf * 1.4286068e-6f;
    float q = 0.0013814613f;
    q = 0.00836871f + q * r;
    q = 0.04166839f + q * r;
    q = 0.16666521f + q * r;
    q = 0.49999994f + q * r;
    float p = 1.0f + (r + (r * r) * q);
    int n = __float_as_int(t) - __float_as_int(magic);
    int a = n >> 1, b = n - a;
    float res = (p * __int_as_float((a + 127) << 23)) * __int_as_float((b + 127) << 23);
    if (x > 88.72283172607422f) res = __int_as_float(0x7F800000);
    if (x < -103.97207641601562f) res = 0.0f;
    return canon(x == x ? res : x);
}
__device__ __forceinline__ float exp_nonpos(float x) {
    const float magic = 12582912.0f;
    float t = x * 1.44269502f + magic;
    float nf = t - magic;
    float r = (x - nf * 0.693145751953125f) - nf * 1.4286068e-6f;
    float q = 0.0013814613f;
    q = 0.00836871f + q * r;
    q = 0.04166839f + q * r;
    q = 0.16666521f + q * r;
    q = 0.49999994f + q * r;
    float p = 1.0f + (r + (r * r) * q);
    int n = __float_as_int(t) - __float_as_int(magic);
    float res = p * __int_as_float((n + 127) << 23);
    if (x < -87.33654f) res = 0.0f;
    return x == x ? res : __int_as_float(0x7FC00000);
}
__device__ __forceinline__ void erf_parts(float x, float &erf, float &ope) {
    unsigned sign = __float_as_uint(x) & 0x80000000u;
    float ax = __uint_as_float(__float_as_uint(x) & 0x7FFFFFFFu);
    float z = ax * ax;
    float p = -0.0007692853f;
    p = 0.0052003083f + p * z;
    p = -0.02686312f + p * z;
    p = 0.11283774f + p * z;
    p = -0.37612638f + p * z;
    p = 1.1283792f + p * z;
    float small = ax * p;
    float t = 1.0f / ax;
    float s = t - 1.0f;
    float g = -0.00057763467f;
    g = 0.0017893383f + g * s;
    g = -0.00010074016f + g * s;
    g = -0.004373198f + g * s;
    g = 0.0034639547f + g * s;
    g = 0.0015023724f + g * s;
    g = -0.0009413088f + g * s;
    g = -0.0018891813f + g * s;
    g = -0.0002586738f + g * s;
    g = 0.0052144383f + g * s;
    g = -0.0103428485f + g * s;
    g = 0.015788378f + g * s;
    g = -0.018338649f + g * s;
    g = 0.008167262f + g * s;
    g = 0.035529688f + g * s;
    g = -0.1543716f + g * s;
    g = 0.42758358f + g * s;
    float split = ax * 4097.0f;
    float axHi = split - (split - ax);
    float axLo = ax - axHi;
    float zLo = ((axHi * axHi - z) + 2.0f * (axHi * axLo)) + axLo * axLo;
    if (!(ax < 64.0f)) zLo = 0.0f;
    float expNegZ = exp_poly(0.0f - z) * (1.0f - zLo);
    float erfc = expNegZ * (t * g);
    bool isSmall = ax < 0.5f;
    float erfAbs = isSmall ? small : 1.0f - erfc;
    float erfSigned = __uint_as_float(__float_as_uint(erfAbs) | sign);
    float opeLarge = x < 0.0f ? erfc : 2.0f - erfc;
    float opeSmall = 1.0f + __uint_as_float(__float_as_uint(small) | sign);
    bool ok = x == x;
    erf = canon(ok ? erfSigned : x);
    ope = canon(ok ? (isSmall ? opeSmall : opeLarge) : x);
}

// GELU, erf form (Ops.Gelu, Ops.Nn.cs:86-112; Transcendental.GeluErf, Transcendental.cs:252): 0.5 x (1 + erf(x/sqrt2)).
__device__ __forceinline__ float gelu(float x) {
    float e, ope;
    erf_parts(x * 0.70710677f, e, ope);
    float res = (0.5f * x) * ope;
    if (x == -__int_as_float(0x7F800000)) res = -0.0f;
    return canon(x == x ? res : x);
}
// GELU's slope at v, the factor GeluGradBin multiplies the incoming gradient by (TrainElementwise.cs:59-85):
// 0.5 (1 + erf(v/sqrt2)) + v exp(-v^2/2) / sqrt(2 pi), rounded as the reference rounds it, from erf_parts' erf.
__device__ __forceinline__ float slope_from_erf(float v, float e) {
    float cdf = 0.5f * (1.0f + e);
    float pdf = exp_poly((-0.5f * v) * v) * 0.3989423f;
    return cdf + v * pdf;
}
// GeluGradBin: g * slope(v). A slope saved by the forward and multiplied in later gives the same bits.
__device__ __forceinline__ float gelu_grad(float g, float v) {
    float e, ope;
    erf_parts(v * 0.70710677f, e, ope);
    return canon(g * slope_from_erf(v, e));
}
// gelu(x) and its slope from one erf evaluation.
__device__ __forceinline__ void gelu_and_slope(float x, float &a, float &s) {
    float e, ope;
    erf_parts(x * 0.70710677f, e, ope);
    float res = (0.5f * x) * ope;
    if (x == -__int_as_float(0x7F800000)) res = -0.0f;
    a = canon(x == x ? res : x);
    s = slope_from_erf(x, e);
}


// GELU and its slope with erf and exp of stated error, for products whose epilogue would otherwise spend about 180
// vector instructions per element on the reference's polynomials (om_ctx_set_gelu, OM_GELU_FAST). With u = x/sqrt2:
// erfc(|u|) = t exp(P(t) - u^2), t = 1 / (1 + |u|/2), P the degree-9 Chebyshev fit of Numerical Recipes (Press,
// Teukolsky, Vetterling, Flannery, 2nd ed., section 6.2, erfcc: fractional error below 1.2e-7 for every argument),
// evaluated by fused multiply-adds, with the hardware's reciprocal and base-2 exponential (v_rcp_f32, v_exp_f32).
// cdf = erfc(|u|)/2 for u < 0, else 1 - erfc(|u|)/2; gelu = x cdf; slope = cdf + x exp(-u^2) / sqrt(2 pi).
// Against double precision on [-12, 12] (fp32 emulation of these steps): |gelu error| <= 1.2e-7 max(1, |x|),
// |slope error| <= 2.2e-7. Special values as the reference's: gelu(-inf) = -0, gelu(+inf) = +inf, NaN stays NaN.
__device__ __forceinline__ float erfc_abs_fast(float u, float z) {
    const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.5f, __builtin_fabsf(u), 1.0f));
    float p = 0.17087277f;
    p = __builtin_fmaf(t, p, -0.82215223f);
    p = __builtin_fmaf(t, p, 1.48851587f);
    p = __builtin_fmaf(t, p, -1.13520398f);
    p = __builtin_fmaf(t, p, 0.27886807f);
    p = __builtin_fmaf(t, p, -0.18628806f);
    p = __builtin_fmaf(t, p, 0.09678418f);
    p = __builtin_fmaf(t, p, 0.37409196f);
    p = __builtin_fmaf(t, p, 1.00002368f);
    p = __builtin_fmaf(t, p, -1.26551223f);
    return t * __builtin_amdgcn_exp2f((p - z) * 1.44269504f);
}
__device__ __forceinline__ void gelu_and_slope_fast(float x, float &a, float &s) {
    const float u = x * 0.70710677f, z = u * u;
    const float hc = 0.5f * erfc_abs_fast(u, z);
    const float cdf = u < 0.0f ? hc : 1.0f - hc;
    const float pdf = __builtin_amdgcn_exp2f(z * -1.44269504f) * 0.3989423f;
    a = x == -__int_as_float(0x7F800000) ? -0.0f : x * cdf;
    s = cdf + x * pdf;
}
__device__ __forceinline__ float gelu_fast(float x) {
    const float u = x * 0.70710677f, z = u * u;
    const float hc = 0.5f * erfc_abs_fast(u, z);
    const float cdf = u < 0.0f ? hc : 1.0f - hc;
    return x == -__int_as_float(0x7F800000) ? -0.0f : x * cdf;
}
__device__ __forceinline__ float gelu_grad_fast(float g, float v) {
    float a, s;
    gelu_and_slope_fast(v, a, s);
    return g * s;
}

}  // namespace omd
