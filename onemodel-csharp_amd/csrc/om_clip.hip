// Gradient clipping on the device: GradClip.ClipNorm and GradClip.ClipValue (Schedules.cs:9-150).
//
// ClipNorm over a list of gradient segments runs as three launches on the context's stream and never blocks the host:
//   1. k_norm_partial: one workgroup per 8192-element chunk of a segment writes the chunk's fp64 partial (sum of
//      squares, or largest |g|) to scratch. Inside a chunk, thread t takes the float4 groups t, t+256, ... in
//      increasing order and the 256 per-thread values are combined by a fixed butterfly and wave order.
//   2. k_norm_final: one workgroup sums the partials in a fixed order (thread t takes partials t, t+256, ... with
//      sixteen loads in flight, then the block's fixed tree), takes the square root, and writes
//      the norm (float) and the clip coefficient min-tested by the consumers: coef = (float)(maxNorm / (norm + 1e-6)),
//      or 1 when the norm is not finite (the reference scales nothing then).
//   3. k_scale_segs: every element g *= coef when coef < 1 (skipped by the whole grid otherwise) — or nothing, when the
//      caller folds the coefficient into the optimizer's read of g instead (om_adam_step_scaled).
// Chunking depends only on the segment lengths, never on alignment or device, so the norm is reproducible bit for
// bit. Each square (double)g*g is exact in double; the sum differs from the reference's serial running sum only by
// fp64 rounding (relative error below count * 2^-53), far inside the float the norm is returned as.
#include "om_internal.hpp"

#include <cmath>

namespace {

constexpr int kBlock = 256;
constexpr int kPer = 8;                                  // float4 groups per thread per chunk
constexpr int64_t kChunk = (int64_t)kBlock * 4 * kPer;  // 8192 floats per workgroup
constexpr int kMaxSeg = 32;                              // segments per launch (kernel-argument table)

struct Segs {
    float *ptr[kMaxSeg];
    int64_t len[kMaxSeg];
    int64_t first[kMaxSeg + 1];  // first chunk of each segment within this launch; first[n] = chunks in the launch
    int n;
};

// The segment holding chunk c of the launch, the chunk's first element and its length.
__device__ __forceinline__ float *chunk_of(const Segs &s, int64_t c, int64_t &len, bool &vec) {
    int i = 0;
    while (i + 1 < s.n && s.first[i + 1] <= c) i++;
    float *g = s.ptr[i];
    const int64_t base = (c - s.first[i]) * kChunk;
    const int64_t rest = s.len[i] - base;
    len = rest < kChunk ? rest : kChunk;
    vec = ((uintptr_t)g & 15) == 0;
    return g + base;
}

// Four consecutive elements e..e+3 of a chunk (zeros past its end; a zero adds nothing to either norm).
__device__ __forceinline__ float4 load4(const float *g, int64_t e, int64_t len, bool vec) {
    if (vec && e + 4 <= len) return *reinterpret_cast<const float4 *>(g + e);
    float4 v;
    v.x = e < len ? g[e] : 0.0f;
    v.y = e + 1 < len ? g[e + 1] : 0.0f;
    v.z = e + 2 < len ? g[e + 2] : 0.0f;
    v.w = e + 3 < len ? g[e + 3] : 0.0f;
    return v;
}

// The reference's infinity-norm step: a larger value or a NaN replaces the running value, so a NaN sticks.
__device__ __forceinline__ double take_max(double acc, double a) { return (a > acc || a != a) ? a : acc; }

template <bool INF>
__device__ __forceinline__ double combine(double a, double b) {
    return INF ? take_max(a, b) : a + b;
}

template <bool INF>
__device__ __forceinline__ double accumulate(double acc, float v) {
    if (INF) return take_max(acc, fabs((double)v));
    return acc + (double)v * (double)v;
}

// Fixed-order block combine of 256 per-thread values (butterfly inside each wavefront, then waves 0..3).
template <bool INF>
__device__ __forceinline__ double block_combine(double v, double *sh) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = combine<INF>(v, __shfl_xor(v, o, 64));
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) sh[w] = v;
    __syncthreads();
    double t = sh[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; i++) t = combine<INF>(t, sh[i]);
    return t;
}

template <bool INF>
__global__ void __launch_bounds__(kBlock) k_norm_partial(Segs s, double *__restrict__ part) {
    OM_LDS_POISON();
    __shared__ double sh[kBlock / 64];
    int64_t len;
    bool vec;
    const float *g = chunk_of(s, blockIdx.x, len, vec);
    float4 v[kPer];
#pragma unroll
    for (int j = 0; j < kPer; j++) v[j] = load4(g, 4 * ((int64_t)j * kBlock + threadIdx.x), len, vec);
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        acc = accumulate<INF>(acc, v[j].x);
        acc = accumulate<INF>(acc, v[j].y);
        acc = accumulate<INF>(acc, v[j].z);
        acc = accumulate<INF>(acc, v[j].w);
    }
    acc = block_combine<INF>(acc, sh);
    if (threadIdx.x == 0) part[blockIdx.x] = acc;
}

template <bool INF>
__global__ void __launch_bounds__(kBlock) k_norm_final(const double *__restrict__ part, int64_t nparts,
                                                       float max_norm, float *__restrict__ total,
                                                       float *__restrict__ coef) {
    OM_LDS_POISON();
    __shared__ double sh[kBlock / 64];
    double acc = 0.0;
    // thread t combines part[t], part[t + 256], ... in that order, sixteen loads in flight before their combines
    constexpr int R = 16;
    for (int64_t base = 0; base < nparts; base += (int64_t)kBlock * R) {
        double v[R];
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int64_t i = base + (int64_t)u * kBlock + threadIdx.x;
            v[u] = i < nparts ? part[i] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < R; u++)
            if (base + (int64_t)u * kBlock + threadIdx.x < nparts) acc = combine<INF>(acc, v[u]);
    }
    acc = block_combine<INF>(acc, sh);
    if (threadIdx.x == 0) {
        const double norm = INF ? acc : sqrt(acc);
        if (total) *total = (float)norm;
        // Schedules.cs:62-68: nothing is scaled when the norm is NaN or infinite; consumers scale iff coef < 1.
        *coef = isfinite(norm) ? (float)((double)max_norm / (norm + 1e-6)) : 1.0f;
    }
}

__global__ void __launch_bounds__(kBlock) k_scale_segs(Segs s, const float *__restrict__ coef) {
    OM_LDS_POISON();
    const float c = *coef;
    if (!(c < 1.0f)) return;
    int64_t len;
    bool vec;
    float *g = chunk_of(s, blockIdx.x, len, vec);
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const int64_t e = 4 * ((int64_t)j * kBlock + threadIdx.x);
        if (vec && e + 4 <= len) {
            float4 v = *reinterpret_cast<float4 *>(g + e);
            v.x = v.x * c;
            v.y = v.y * c;
            v.z = v.z * c;
            v.w = v.w * c;
            *reinterpret_cast<float4 *>(g + e) = v;
        } else {
            for (int r = 0; r < 4; r++)
                if (e + r < len) g[e + r] = g[e + r] * c;
        }
    }
}

__device__ __forceinline__ float clamp_value(float v, float c) { return v > c ? c : v < -c ? -c : v; }

__global__ void __launch_bounds__(kBlock) k_clip_value(Segs s, float c) {
    OM_LDS_POISON();
    int64_t len;
    bool vec;
    float *g = chunk_of(s, blockIdx.x, len, vec);
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const int64_t e = 4 * ((int64_t)j * kBlock + threadIdx.x);
        if (vec && e + 4 <= len) {
            float4 v = *reinterpret_cast<float4 *>(g + e);
            v.x = clamp_value(v.x, c);
            v.y = clamp_value(v.y, c);
            v.z = clamp_value(v.z, c);
            v.w = clamp_value(v.w, c);
            *reinterpret_cast<float4 *>(g + e) = v;
        } else {
            for (int r = 0; r < 4; r++)
                if (e + r < len) g[e + r] = clamp_value(g[e + r], c);
        }
    }
}

// Splits the non-empty segments into launch tables of at most kMaxSeg entries; returns the total chunk count.
om_status tables(om_ctx *ctx, const char *what, int count, float *const *grads, const int64_t *lens,
                 std::vector<Segs> &out, int64_t &chunks) {
    OM_REQUIRE(ctx, count >= 0, "%s: negative segment count", what);
    OM_REQUIRE(ctx, count == 0 || (grads && lens), "%s: NULL segment table", what);
    out.clear();
    chunks = 0;
    for (int i = 0; i < count; i++) {
        OM_REQUIRE(ctx, lens[i] >= 0, "%s: segment %d has negative length", what, i);
        if (!grads[i] || lens[i] == 0) continue;  // a parameter without a gradient is skipped
        if (out.empty() || out.back().n == kMaxSeg) {
            out.emplace_back();
            out.back().n = 0;
            out.back().first[0] = 0;
        }
        Segs &s = out.back();
        s.ptr[s.n] = grads[i];
        s.len[s.n] = lens[i];
        const int64_t c = (lens[i] + kChunk - 1) / kChunk;
        s.first[s.n + 1] = s.first[s.n] + c;
        s.n++;
        chunks += c;
    }
    for (auto &s : out) OM_REQUIRE(ctx, s.first[s.n] < (int64_t)1 << 31, "%s: segments too large", what);
    return OM_OK;
}

}  // namespace

extern "C" {

om_status om_clip_grad_norm(om_ctx *ctx, int count, float *const *grads, const int64_t *lens, float max_norm,
                            int infinity_norm, int scale_in_place, float *total, float *coef) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, max_norm > 0.0f, "om_clip_grad_norm: the maximum norm must be positive (got %g)", (double)max_norm);
    OM_REQUIRE(ctx, scale_in_place || coef, "om_clip_grad_norm: coef is required when scale_in_place is 0");
    std::vector<Segs> segs;
    int64_t chunks = 0;
    om_status st = tables(ctx, "om_clip_grad_norm", count, grads, lens, segs, chunks);
    if (st) return st;
    // Scratch: [coefficient slot (when the caller keeps none) | one fp64 partial per chunk].
    float *sc = nullptr;
    st = om::scratch(ctx, 16 + 8 * (uint64_t)(chunks > 0 ? chunks : 1), &sc);
    if (st) return st;
    double *part = reinterpret_cast<double *>(sc) + 2;
    float *coef_p = coef ? coef : sc;
    int64_t base = 0;
    for (const Segs &s : segs) {
        const unsigned grid = (unsigned)s.first[s.n];
        if (infinity_norm)
            hipLaunchKernelGGL(k_norm_partial<true>, dim3(grid), dim3(kBlock), 0, ctx->stream, s, part + base);
        else
            hipLaunchKernelGGL(k_norm_partial<false>, dim3(grid), dim3(kBlock), 0, ctx->stream, s, part + base);
        base += grid;
    }
    if (infinity_norm)
        hipLaunchKernelGGL(k_norm_final<true>, dim3(1), dim3(kBlock), 0, ctx->stream, part, chunks, max_norm, total,
                           coef_p);
    else
        hipLaunchKernelGGL(k_norm_final<false>, dim3(1), dim3(kBlock), 0, ctx->stream, part, chunks, max_norm, total,
                           coef_p);
    if (scale_in_place)
        for (const Segs &s : segs)
            hipLaunchKernelGGL(k_scale_segs, dim3((unsigned)s.first[s.n]), dim3(kBlock), 0, ctx->stream, s,
                               (const float *)coef_p);
    return OM_LAUNCH_CHECK(ctx, "om_clip_grad_norm");
}

om_status om_clip_grad_value(om_ctx *ctx, int count, float *const *grads, const int64_t *lens, float clip_value) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, clip_value >= 0.0f, "om_clip_grad_value: the bound must not be negative (got %g)",
               (double)clip_value);
    std::vector<Segs> segs;
    int64_t chunks = 0;
    om_status st = tables(ctx, "om_clip_grad_value", count, grads, lens, segs, chunks);
    if (st) return st;
    for (const Segs &s : segs)
        hipLaunchKernelGGL(k_clip_value, dim3((unsigned)s.first[s.n]), dim3(kBlock), 0, ctx->stream, s, clip_value);
    return OM_LAUNCH_CHECK(ctx, "om_clip_grad_value");
}

}  // extern "C"
