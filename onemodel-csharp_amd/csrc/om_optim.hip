// Fused optimizer steps over the contiguous parameter/gradient/moment arena: one read of p, g, m, v and one write
// of p, m, v per element (28 bytes per parameter for AdamW), float4 wide, grid-stride.
//
// Arithmetic is the reference's Adam.UpdateRange (Optimizers.cs:554-589) operation for operation, with one IEEE
// rounding each: the library is compiled with -ffp-contract=off and correctly rounded fp32 division and square root,
// so a parameter update is bit-identical to the reference's CPU update for the same gradient.
#include "om_internal.hpp"

#include <cmath>

namespace {

constexpr int kBlock = 256;

struct AdamArgs {
    float lr, b1, b2, omb1, omb2, eps, wd, decay, step_size, sqrt_bc2;
    int decoupled;
};

__device__ __forceinline__ void adam_one(float &p, float g, float &m, float &v, float *vmax_i, const AdamArgs &a) {
    float pi = p;
    if (a.wd != 0.0f) {
        if (a.decoupled) pi = pi * a.decay;
        else g = g + a.wd * pi;
    }
    float mi = a.b1 * m + a.omb1 * g;
    float vi = a.b2 * v + (a.omb2 * g) * g;
    m = mi;
    v = vi;
    float vd = vi;
    if (vmax_i) {
        vd = *vmax_i > vi ? *vmax_i : vi;
        *vmax_i = vd;
    }
    float denom = sqrtf(vd) / a.sqrt_bc2 + a.eps;
    p = pi - (a.step_size * mi) / denom;
}

// gs (may be NULL): a device-side gradient coefficient, applied as g * c when c < 1 — GradClip.ClipNorm's in-place
// scaling (Schedules.cs:70-76) folded into the update's read of g, with the same single float rounding.
// step (may be NULL): inside a step graph, the step's rate and bias-correction scalars, read when the kernel runs;
// the decoupled decay factor is then formed here with the host's float rounding, 1 - lr * wd.
__global__ void __launch_bounds__(kBlock) k_adam(float *__restrict__ p, const float *__restrict__ g,
                                                 float *__restrict__ m, float *__restrict__ v,
                                                 float *__restrict__ vmax, int64_t n, AdamArgs a,
                                                 const float *__restrict__ gs,
                                                 const om_step_block *__restrict__ step) {
    OM_LDS_POISON();
    if (step) {
        a.lr = step->lr;
        a.step_size = step->step_size;
        a.sqrt_bc2 = step->sqrt_bc2;
        a.decay = 1.0f - a.lr * a.wd;
    }
    const float c = gs ? *gs : 1.0f;
    const bool sc = c < 1.0f;
    int64_t stride = (int64_t)gridDim.x * kBlock;
    int64_t n4 = (vmax == nullptr) ? (n >> 2) : 0;
    float4 *p4 = reinterpret_cast<float4 *>(p);
    const float4 *g4 = reinterpret_cast<const float4 *>(g);
    float4 *m4 = reinterpret_cast<float4 *>(m);
    float4 *v4 = reinterpret_cast<float4 *>(v);
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
        float4 pp = p4[i], gg = g4[i], mm = m4[i], vv = v4[i];
        if (sc) {
            gg.x = gg.x * c;
            gg.y = gg.y * c;
            gg.z = gg.z * c;
            gg.w = gg.w * c;
        }
        adam_one(pp.x, gg.x, mm.x, vv.x, nullptr, a);
        adam_one(pp.y, gg.y, mm.y, vv.y, nullptr, a);
        adam_one(pp.z, gg.z, mm.z, vv.z, nullptr, a);
        adam_one(pp.w, gg.w, mm.w, vv.w, nullptr, a);
        p4[i] = pp;
        m4[i] = mm;
        v4[i] = vv;
    }
    for (int64_t i = (n4 << 2) + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        adam_one(p[i], sc ? g[i] * c : g[i], m[i], v[i], vmax ? vmax + i : nullptr, a);
}

__global__ void __launch_bounds__(kBlock) k_sgd(float *__restrict__ p, const float *__restrict__ g,
                                                float *__restrict__ buf, int64_t n, float lr, float mu, float keep,
                                                float wd, int nesterov, int first) {
    OM_LDS_POISON();
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float gi = g[i];
        if (wd != 0.0f) gi = gi + wd * p[i];
        if (buf) {
            float b = first ? gi : mu * buf[i] + keep * gi;
            buf[i] = b;
            gi = nesterov ? gi + mu * b : b;
        }
        p[i] = p[i] - lr * gi;
    }
}

}  // namespace

extern "C" {

void om_adam_scalars(float lr, float beta1, float beta2, int64_t t, float *step_size, float *sqrt_bc2) {
    // Adam.IntPow (binary exponentiation in double) and Adam.BeginStep (Optimizers.cs:483-508).
    double b1 = beta1, b2 = beta2, p1 = 1.0, p2 = 1.0;
    for (int64_t n = t; n > 0; n >>= 1) {
        if (n & 1) p1 *= b1;
        b1 *= b1;
    }
    for (int64_t n = t; n > 0; n >>= 1) {
        if (n & 1) p2 *= b2;
        b2 *= b2;
    }
    double bc1 = 1.0 - p1, bc2 = 1.0 - p2;
    if (step_size) *step_size = (float)((double)lr / bc1);
    if (sqrt_bc2) *sqrt_bc2 = (float)std::sqrt(bc2);
}

static om_status adam_launch(om_ctx *ctx, const char *what, float *p, const float *g, float *m, float *v,
                             float *vmax, int64_t n, float lr, float beta1, float beta2, float eps,
                             float weight_decay, int decoupled, float step_size, float sqrt_bc2,
                             const float *grad_scale) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, n >= 0, "%s: negative length", what);
    if (n == 0) return OM_OK;
    OM_REQUIRE(ctx, p && g && m && v, "%s: NULL pointer", what);
    OM_REQUIRE(ctx, ((uintptr_t)p | (uintptr_t)g | (uintptr_t)m | (uintptr_t)v) % 16 == 0,
               "%s: p, g, m, v must be 16-byte aligned", what);
    AdamArgs a;
    a.lr = lr;
    a.b1 = beta1;
    a.b2 = beta2;
    a.omb1 = 1.0f - beta1;
    a.omb2 = 1.0f - beta2;
    a.eps = eps;
    a.wd = weight_decay;
    a.decay = 1.0f - lr * weight_decay;
    a.step_size = step_size;
    a.sqrt_bc2 = sqrt_bc2;
    a.decoupled = decoupled;
    // Enough waves to cover HBM latency on 256 CUs, grid-stride beyond that.
    unsigned grid = om::grid1d((n + 3) / 4, kBlock, (int64_t)ctx->num_cus * 8);
    // Inside a step-graph capture the per-step scalars come from the graph's device block (om_graph_launch).
    const om_step_block *step = ctx->cap ? ctx->cap->dev : nullptr;
    hipLaunchKernelGGL(k_adam, dim3(grid), dim3(kBlock), 0, ctx->stream, p, g, m, v, vmax, n, a, grad_scale, step);
    return OM_LAUNCH_CHECK(ctx, what);
}

om_status om_adam_step(om_ctx *ctx, float *p, const float *g, float *m, float *v, float *vmax, int64_t n, float lr,
                       float beta1, float beta2, float eps, float weight_decay, int decoupled, float step_size,
                       float sqrt_bc2) {
    return adam_launch(ctx, "om_adam_step", p, g, m, v, vmax, n, lr, beta1, beta2, eps, weight_decay, decoupled,
                       step_size, sqrt_bc2, nullptr);
}

om_status om_adam_step_scaled(om_ctx *ctx, float *p, const float *g, float *m, float *v, float *vmax, int64_t n,
                              float lr, float beta1, float beta2, float eps, float weight_decay, int decoupled,
                              float step_size, float sqrt_bc2, const float *grad_scale) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, grad_scale, "om_adam_step_scaled: grad_scale is NULL");
    return adam_launch(ctx, "om_adam_step_scaled", p, g, m, v, vmax, n, lr, beta1, beta2, eps, weight_decay,
                       decoupled, step_size, sqrt_bc2, grad_scale);
}

om_status om_sgd_step(om_ctx *ctx, float *p, const float *g, float *buf, int64_t n, float lr, float momentum,
                      float dampening, float weight_decay, int nesterov, int first) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, n >= 0, "om_sgd_step: negative length");
    if (n == 0) return OM_OK;
    OM_REQUIRE(ctx, p && g, "om_sgd_step: NULL pointer");
    if (om_status st = om::refuse_in_capture(ctx, "om_sgd_step")) return st;
    hipLaunchKernelGGL(k_sgd, dim3(om::grid1d(n, kBlock, (int64_t)ctx->num_cus * 8)), dim3(kBlock), 0, ctx->stream, p,
                       g, buf, n, lr, momentum, 1.0f - dampening, weight_decay, nesterov, first);
    return OM_LAUNCH_CHECK(ctx, "om_sgd_step");
}

}  // extern "C"
