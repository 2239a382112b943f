// Bandwidth-bound element-wise maps and reductions of the training path. Grid-stride loops over float4 where the
// pointers and length allow it; every element sees the same IEEE operations in the same order as the reference's
// lane loops (TrainElementwise.cs), so position and vector width never change a result.
#include "om_internal.hpp"

namespace {

constexpr int kBlock = 256;

inline unsigned ew_grid(int64_t n4) { return om::grid1d(n4, kBlock, 4096); }

inline bool aligned4(const void *p) { return ((uintptr_t)p & 15) == 0; }

// One functor per map; `apply(a, b)` gets the two inputs of an element.
struct ReluF {
    __device__ float operator()(float x, float) const { return x > 0.0f ? x : (x == x ? 0.0f : x); }
};
struct ReluGradF {
    __device__ float operator()(float g, float y) const { return y > 0.0f ? g : 0.0f; }
};
struct GeluF {
    __device__ float operator()(float x, float) const { return omd::gelu(x); }
};
struct GeluGradF {
    __device__ float operator()(float g, float v) const { return omd::gelu_grad(g, v); }
};
struct GeluFastF {
    __device__ float operator()(float x, float) const { return omd::gelu_fast(x); }
};
struct GeluGradFastF {
    __device__ float operator()(float g, float v) const { return omd::gelu_grad_fast(g, v); }
};
struct AddF {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct SubF {
    __device__ float operator()(float a, float b) const { return a - b; }
};
struct MulF {
    __device__ float operator()(float a, float b) const { return a * b; }
};

template <class F, bool ACC>
__global__ void __launch_bounds__(kBlock) k_map2(const float *__restrict__ a, const float *__restrict__ b,
                                                 float *__restrict__ y, int64_t n, F f) {
    OM_LDS_POISON();
    int64_t stride = (int64_t)gridDim.x * kBlock;
    int64_t n4 = n >> 2;
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    const float4 *b4 = reinterpret_cast<const float4 *>(b);
    float4 *y4 = reinterpret_cast<float4 *>(y);
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
        float4 va = a4[i], vb = b ? b4[i] : va, r;
        r.x = f(va.x, vb.x);
        r.y = f(va.y, vb.y);
        r.z = f(va.z, vb.z);
        r.w = f(va.w, vb.w);
        if (ACC) {
            float4 o = y4[i];
            r.x = o.x + r.x; r.y = o.y + r.y; r.z = o.z + r.z; r.w = o.w + r.w;
        }
        y4[i] = r;
    }
    for (int64_t i = (n4 << 2) + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float r = f(a[i], b ? b[i] : a[i]);
        y[i] = ACC ? y[i] + r : r;
    }
}
template <class F, bool ACC>
__global__ void __launch_bounds__(kBlock) k_map2_scalar(const float *__restrict__ a, const float *__restrict__ b,
                                                        float *__restrict__ y, int64_t n, F f) {
    OM_LDS_POISON();
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float r = f(a[i], b ? b[i] : a[i]);
        y[i] = ACC ? y[i] + r : r;
    }
}

template <class F>
om_status map2(om_ctx *ctx, const char *name, const float *a, const float *b, float *y, int64_t n, int acc, F f) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, n >= 0, "%s: negative length", name);
    if (n == 0) return OM_OK;
    OM_REQUIRE(ctx, a && y, "%s: NULL pointer", name);
    bool vec = aligned4(a) && aligned4(y) && (!b || aligned4(b));
    dim3 grid(ew_grid(vec ? (n + 3) / 4 : n)), block(kBlock);
    if (vec) {
        if (acc) hipLaunchKernelGGL((k_map2<F, true>), grid, block, 0, ctx->stream, a, b, y, n, f);
        else hipLaunchKernelGGL((k_map2<F, false>), grid, block, 0, ctx->stream, a, b, y, n, f);
    } else {
        if (acc) hipLaunchKernelGGL((k_map2_scalar<F, true>), grid, block, 0, ctx->stream, a, b, y, n, f);
        else hipLaunchKernelGGL((k_map2_scalar<F, false>), grid, block, 0, ctx->stream, a, b, y, n, f);
    }
    return OM_LAUNCH_CHECK(ctx, name);
}

// Ops.Add with the second operand broadcast over the rows (Ops.cs:15-56), as a Linear's bias add issues it
// (Ops.Layers.cs:715-733): y[r][c] = x[r][c] + b[c], one rounding per element.
__global__ void __launch_bounds__(kBlock) k_add_rows4(const float4 *__restrict__ x, const float4 *__restrict__ b,
                                                      float4 *__restrict__ y, int64_t n4, int cols4) {
    OM_LDS_POISON();
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
        const float4 v = x[i], w = b[i % cols4];
        y[i] = float4{v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w};
    }
}
__global__ void __launch_bounds__(kBlock) k_add_rows(const float *__restrict__ x, const float *__restrict__ b,
                                                     float *__restrict__ y, int64_t n, int cols) {
    OM_LDS_POISON();
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) y[i] = x[i] + b[i % cols];
}

__global__ void __launch_bounds__(kBlock) k_axpy(float alpha, const float *__restrict__ s, float *__restrict__ d,
                                                 int64_t n, int overwrite) {
    OM_LDS_POISON();
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float v = alpha == 1.0f ? s[i] : s[i] * alpha;
        d[i] = overwrite ? v : d[i] + v;
    }
}

// ---------------------------------------------------------------------------------------------- reductions
// Sum of all elements in double: stage 1 gives one partial per block (fixed element->block assignment from n),
// stage 2 adds the partials in block order.
constexpr int kSumBlocks = 1024;
__global__ void __launch_bounds__(kBlock) k_sum_partial(const float *__restrict__ x, int64_t n,
                                                        double *__restrict__ part) {
    OM_LDS_POISON();
    __shared__ double sh[kBlock / 64];
    double acc = 0.0;
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) acc += (double)x[i];
    double t = omd::block_sum<kBlock / 64>(acc, sh);
    if (threadIdx.x == 0) part[blockIdx.x] = t;
}
// Optionally also posts the result to a readback buffer as k_readback does: the value as a system-scope
// write-through store, a wait for its completion, then the sequence number (no L2 write-back).
struct PostTo {
    char *dst;
    uint64_t *seq_at;
    uint64_t seq;
    const uint64_t *seq_dev;  // inside a step graph: the number is read here when the kernel runs
};
__global__ void __launch_bounds__(64) k_sum_final(const double *__restrict__ part, int np, float *__restrict__ out,
                                                  double divisor, PostTo post) {
    OM_LDS_POISON();
    // Lane l adds part[l], part[l + 64], ... in that order; the loads of a round of 16 are all issued before the
    // first add (the partials were just written on every XCD, so each load waits for memory).
    constexpr int R = 16;
    double acc = 0.0;
    for (int base = 0; base < np; base += 64 * R) {
        double v[R];
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int i = base + 64 * u + (int)threadIdx.x;
            v[u] = i < np ? part[i] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < R; u++)
            if (base + 64 * u + (int)threadIdx.x < np) acc += v[u];
    }
    acc = omd::wave_sum(acc);
    if (threadIdx.x == 0) {
        const float v = divisor > 0.0 ? (float)(acc / divisor) : (float)acc;
        out[0] = v;
        if (post.dst) {
            __hip_atomic_store(reinterpret_cast<float *>(post.dst), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __builtin_amdgcn_s_waitcnt(0);
            __hip_atomic_store(post.seq_at, post.seq_dev ? *post.seq_dev : post.seq, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

// Column sums of a [rows, cols] matrix in double. Stage 1: a block covers 64 columns (one per lane, coalesced
// rows) of a chunk of kColChunk rows; its 4 wavefronts take every 4th row and are combined in LDS in wave order,
// giving partial[chunk][col]. Stage 2: a wavefront per column adds its chunk partials (lanes, then a fixed butterfly).
constexpr int kColChunk = 64;
__global__ void __launch_bounds__(kBlock) k_colsum_partial(const float *__restrict__ g, int rows, int cols,
                                                           double *__restrict__ part) {
    OM_LDS_POISON();
    __shared__ double sh[kBlock / 64][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + lane;
    const int r0 = blockIdx.y * kColChunk, r1 = min(rows, r0 + kColChunk);
    // this lane's rows r0 + w, r0 + w + 4, ...: all loads issued before the first add, then added in that order
    constexpr int PER = kColChunk / (kBlock / 64);
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int r = r0 + w + i * (kBlock / 64);
        v[i] = (col < cols && r < r1) ? g[(int64_t)r * cols + col] : 0.0f;
    }
    double acc = 0.0;
#pragma unroll
    for (int i = 0; i < PER; i++)
        if (r0 + w + i * (kBlock / 64) < r1) acc += (double)v[i];
    sh[w][lane] = acc;
    __syncthreads();
    if (w == 0 && col < cols) {
        double t = 0.0;
#pragma unroll
        for (int q = 0; q < kBlock / 64; q++) t += sh[q][lane];
        part[(int64_t)blockIdx.y * cols + col] = t;
    }
}

}  // namespace

// A wavefront per column: lanes add chunk partials c = lane, lane+64, ... then a butterfly; used by every two-stage
// column reduction of the library (bias, LayerNorm and convolution-bias gradients).
__global__ void __launch_bounds__(256) om_k_chunk_final(const double *__restrict__ part, float *__restrict__ out,
                                                        const double *__restrict__ part2, float *__restrict__ out2,
                                                        int chunks, int cols, int acc) {
    OM_LDS_POISON();
    int col = (blockIdx.x * 256 + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (col >= 2 * cols || (col >= cols && !part2)) return;
    const double *src = part;
    float *dst = out;
    if (col >= cols) {
        col -= cols;
        src = part2;
        dst = out2;
    }
    omd::column_sum_wave(src, dst, chunks, cols, col, acc, lane);
}

om_status om::chunk_final(om_ctx *ctx, const double *part, int chunks, int cols, float *out, int acc,
                          const double *part2, float *out2) {
    int waves = part2 ? 2 * cols : cols;
    hipLaunchKernelGGL(om_k_chunk_final, dim3(om::grid1d((int64_t)waves * 64, 256, 1 << 30)), dim3(256), 0,
                       om::cur_stream(ctx), part, out, part2, out2, chunks, cols, acc);
    return OM_LAUNCH_CHECK(ctx, "column reduction");
}

namespace {

// Mean over the middle axis of [outer, n, inner]. inner == 1: one wavefront per output (contiguous row);
// otherwise one thread per output (threads along inner read contiguous memory).
__global__ void __launch_bounds__(kBlock) k_mean_rows(const float *__restrict__ x, float *__restrict__ y, int outer,
                                                      int n) {
    OM_LDS_POISON();
    int wave = (blockIdx.x * kBlock + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (wave >= outer) return;
    const float *xr = x + (int64_t)wave * n;
    double acc = 0.0;
    for (int k = lane; k < n; k += 64) acc += (double)xr[k];
    acc = omd::wave_sum(acc);
    if (lane == 0) y[wave] = (float)(acc / n);
}
// ReLU then the mean of each row (a global average pool over planes): k_mean_rows' sums of the ReLU outputs, in its
// order (lane-strided, loads four strides ahead), so the bits equal om_relu_fwd followed by om_mean_axis.
__global__ void __launch_bounds__(kBlock) k_relu_mean_rows(const float *__restrict__ x, float *__restrict__ y,
                                                           int outer, int n) {
    OM_LDS_POISON();
    int wave = (blockIdx.x * kBlock + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (wave >= outer) return;
    const float *xr = x + (int64_t)wave * n;
    double acc = 0.0;
    int k = lane;
    for (; k + 192 < n; k += 256) {
        const float a = xr[k], b = xr[k + 64], c = xr[k + 128], d = xr[k + 192];
        acc += (double)ReluF{}(a, 0.f);
        acc += (double)ReluF{}(b, 0.f);
        acc += (double)ReluF{}(c, 0.f);
        acc += (double)ReluF{}(d, 0.f);
    }
    for (; k < n; k += 64) acc += (double)ReluF{}(xr[k], 0.f);
    acc = omd::wave_sum(acc);
    if (lane == 0) y[wave] = (float)(acc / n);
}
// Its backward: the mean's backward (g / n broadcast over the row) and ReLU's (kept where x > 0) in one pass.
__global__ void __launch_bounds__(kBlock) k_relu_mean_rows_bwd(const float *__restrict__ g,
                                                               const float *__restrict__ x, float *__restrict__ dx,
                                                               int outer, int n, int acc) {
    OM_LDS_POISON();
    const int64_t total = (int64_t)outer * n, stride = (int64_t)gridDim.x * kBlock;
    const float fn = (float)n;
    for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < total; t += stride) {
        const float v = x[t] > 0.0f ? g[t / n] / fn : 0.0f;
        dx[t] = acc ? dx[t] + v : v;
    }
}
__global__ void __launch_bounds__(kBlock) k_mean_inner(const float *__restrict__ x, float *__restrict__ y, int outer,
                                                       int n, int inner) {
    OM_LDS_POISON();
    int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= (int64_t)outer * inner) return;
    int o = (int)(t / inner), i = (int)(t % inner);
    double acc = 0.0;
    for (int k = 0; k < n; k++) acc += (double)x[((int64_t)o * n + k) * inner + i];
    y[t] = (float)(acc / n);
}
// The CRNN's sequence head: the mean over H of x [B, C, H, W] (k_mean_inner's arithmetic) written as y [W, B, C]
// (Permute(2, 0, 1) of the mean), and its backward: dx[b][c][h][w] (+)= g[w][b][c] / H (k_mean_axis_bwd's).
__global__ void __launch_bounds__(kBlock) k_mean_permute_fwd(const float *__restrict__ x, float *__restrict__ y, int B,
                                                             int Cc, int H, int W) {
    OM_LDS_POISON();
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= (int64_t)B * Cc * W) return;
    const int c = (int)(t % Cc), b = (int)((t / Cc) % B), w = (int)(t / ((int64_t)Cc * B));
    const float *xp = x + ((int64_t)b * Cc + c) * H * W + w;
    double acc = 0.0;
    for (int k = 0; k < H; k++) acc += (double)xp[(int64_t)k * W];
    y[t] = (float)(acc / H);
}
__global__ void __launch_bounds__(kBlock) k_mean_permute_bwd(const float *__restrict__ g, float *__restrict__ dx, int B,
                                                             int Cc, int H, int W, int acc) {
    OM_LDS_POISON();
    const int64_t total = (int64_t)B * Cc * H * W, stride = (int64_t)gridDim.x * kBlock;
    const float fn = (float)H;
    for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < total; t += stride) {
        const int w = (int)(t % W);
        const int64_t bc = t / ((int64_t)H * W);
        const int c = (int)(bc % Cc), b = (int)(bc / Cc);
        const float v = g[((int64_t)w * B + b) * Cc + c] / fn;
        dx[t] = acc ? dx[t] + v : v;
    }
}
__global__ void __launch_bounds__(kBlock) k_mean_axis_bwd(const float *__restrict__ g, float *__restrict__ dx,
                                                          int outer, int n, int inner, int acc) {
    OM_LDS_POISON();
    int64_t total = (int64_t)outer * n * inner, stride = (int64_t)gridDim.x * kBlock;
    float fn = (float)n;
    for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < total; t += stride) {
        int64_t o = t / ((int64_t)n * inner), i = t % inner;
        float v = g[o * inner + i] / fn;
        dx[t] = acc ? dx[t] + v : v;
    }
}
__global__ void __launch_bounds__(kBlock) k_mean_all_bwd(const float *__restrict__ g, float *__restrict__ dx,
                                                         int64_t n, int acc) {
    OM_LDS_POISON();
    float v = g[0] / (float)n;
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < n; t += stride) dx[t] = acc ? dx[t] + v : v;
}

// y[j] = x[perm-order]: y index -> its coordinates -> x offset through the permuted strides.
struct PermDesc {
    int ndim;
    int64_t ydim[6];
    int64_t xstride_for_y[6];
};
__global__ void __launch_bounds__(kBlock) k_permute(const float *__restrict__ x, float *__restrict__ y, int64_t n,
                                                    PermDesc d, int acc) {
    OM_LDS_POISON();
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        int64_t r = i, off = 0;
        for (int a = d.ndim - 1; a >= 0; a--) {
            int64_t c = r % d.ydim[a];
            r /= d.ydim[a];
            off += c * d.xstride_for_y[a];
        }
        float v = x[off];
        y[i] = acc ? y[i] + v : v;
    }
}

// MSE: diff (unless NULL) and per-block double partial sums of fl(diff*diff); a final pass adds the partials in block
// order. With unit != NULL it also writes the gradient for a unit upstream gradient, k_mse_bwd's arithmetic with g = 1.
__global__ void __launch_bounds__(kBlock) k_mse_partial(const float *__restrict__ p, const float *__restrict__ t,
                                                        float *__restrict__ diff, int64_t n,
                                                        double *__restrict__ part, float *__restrict__ unit) {
    OM_LDS_POISON();
    __shared__ double sh[kBlock / 64];
    const float dsq = 1.0f / (float)n;
    double acc = 0.0;
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float d = p[i] - t[i];
        if (diff) diff[i] = d;
        acc += (double)(d * d);
        if (unit) {
            float u = dsq * d;
            unit[i] = u + u;
        }
    }
    double s = omd::block_sum<kBlock / 64>(acc, sh);
    if (threadIdx.x == 0) part[blockIdx.x] = s;
}
__global__ void __launch_bounds__(kBlock) k_mse_bwd(const float *__restrict__ gs, const float *__restrict__ diff,
                                                    float *__restrict__ dp, int64_t n, int acc) {
    OM_LDS_POISON();
    float dsq = gs[0] / (float)n;
    int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float t = dsq * diff[i];
        float v = t + t;
        dp[i] = acc ? dp[i] + v : v;
    }
}

}  // namespace

extern "C" {

om_status om_permute(om_ctx *ctx, const float *x, float *y, int ndim, const int32_t *shape, const int32_t *perm,
                     int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && y && shape && perm && ndim >= 1 && ndim <= 6, "om_permute: bad arguments (rank %d)", ndim);
    int64_t xs[6], n = 1;
    bool seen[6] = {false, false, false, false, false, false};
    for (int a = ndim - 1; a >= 0; a--) {
        OM_REQUIRE(ctx, shape[a] >= 0, "om_permute: negative extent");
        xs[a] = n;
        n *= shape[a];
    }
    PermDesc d;
    d.ndim = ndim;
    for (int a = 0; a < ndim; a++) {
        OM_REQUIRE(ctx, perm[a] >= 0 && perm[a] < ndim && !seen[perm[a]], "om_permute: perm is not a permutation");
        seen[perm[a]] = true;
        d.ydim[a] = shape[perm[a]];
        d.xstride_for_y[a] = xs[perm[a]];
    }
    if (n == 0) return OM_OK;
    hipLaunchKernelGGL(k_permute, dim3(ew_grid(n)), dim3(kBlock), 0, ctx->stream, x, y, n, d, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_permute");
}

static om_status mse_fwd(om_ctx *ctx, const float *pred, const float *target, float *diff, float *loss, float *unit,
                         int64_t n, om_readback *rb) {
    float *scr;
    om_status s = om::scratch(ctx, sizeof(double) * kSumBlocks, &scr);
    if (s) return s;
    double *part = reinterpret_cast<double *>(scr);
    const int nb = (int)om::grid1d(n, kBlock, kSumBlocks);
    PostTo post{nullptr, nullptr, 0, nullptr};
    if (rb) {
        s = om::readback_target(ctx, rb, sizeof(float), &post.dst, &post.seq_at, &post.seq, &post.seq_dev);
        if (s) return s;
    }
    hipLaunchKernelGGL(k_mse_partial, dim3(nb), dim3(kBlock), 0, ctx->stream, pred, target, diff, n, part, unit);
    hipLaunchKernelGGL(k_sum_final, dim3(1), dim3(64), 0, ctx->stream, part, nb, loss, (double)n, post);
    s = OM_LAUNCH_CHECK(ctx, "om_mse_fwd");
    if (s == OM_OK && rb) om::readback_posted(rb, post.seq, sizeof(float));
    return s;
}

om_status om_mse_fwd(om_ctx *ctx, const float *pred, const float *target, float *diff, float *loss, int64_t n) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, pred && target && diff && loss && n > 0, "om_mse_fwd: bad arguments");
    return mse_fwd(ctx, pred, target, diff, loss, nullptr, n, nullptr);
}

om_status om_mse_fwd_unit(om_ctx *ctx, const float *pred, const float *target, float *diff, float *loss,
                          float *dpred_unit, int64_t n) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, pred && target && loss && dpred_unit && n > 0, "om_mse_fwd_unit: bad arguments");
    return mse_fwd(ctx, pred, target, diff, loss, dpred_unit, n, nullptr);
}

om_status om_mse_fwd_post(om_ctx *ctx, const float *pred, const float *target, float *diff, float *loss,
                          float *dpred_unit, int64_t n, om_readback *rb) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, pred && target && loss && n > 0 && rb && (diff || dpred_unit), "om_mse_fwd_post: bad arguments");
    return mse_fwd(ctx, pred, target, diff, loss, dpred_unit, n, rb);
}

om_status om_mean_permute_fwd(om_ctx *ctx, const float *x, float *y, int B, int C, int H, int W) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && y && B > 0 && C > 0 && H > 0 && W > 0, "om_mean_permute_fwd: bad arguments");
    const int64_t n = (int64_t)B * C * W;
    hipLaunchKernelGGL(k_mean_permute_fwd, dim3((unsigned)((n + kBlock - 1) / kBlock)), dim3(kBlock), 0, ctx->stream, x,
                       y, B, C, H, W);
    return OM_LAUNCH_CHECK(ctx, "om_mean_permute_fwd");
}

om_status om_mean_permute_bwd(om_ctx *ctx, const float *g, float *dx, int B, int C, int H, int W, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && dx && B > 0 && C > 0 && H > 0 && W > 0, "om_mean_permute_bwd: bad arguments");
    hipLaunchKernelGGL(k_mean_permute_bwd, dim3(ew_grid((int64_t)B * C * H * W)), dim3(kBlock), 0, ctx->stream, g, dx,
                       B, C, H, W, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_mean_permute_bwd");
}

om_status om_mse_bwd(om_ctx *ctx, const float *g_scalar, const float *diff, float *dpred, int64_t n, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g_scalar && diff && dpred && n > 0, "om_mse_bwd: bad arguments");
    hipLaunchKernelGGL(k_mse_bwd, dim3(ew_grid(n)), dim3(kBlock), 0, ctx->stream, g_scalar, diff, dpred, n,
                       accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_mse_bwd");
}

om_status om_relu_fwd(om_ctx *ctx, const float *x, float *y, int64_t n) {
    return map2(ctx, "om_relu_fwd", x, nullptr, y, n, 0, ReluF{});
}
om_status om_relu_bwd(om_ctx *ctx, const float *g, const float *y, float *dx, int64_t n, int accumulate) {
    OM_REQUIRE(ctx, y || n == 0, "om_relu_bwd: NULL saved output");
    return map2(ctx, "om_relu_bwd", g, y, dx, n, accumulate, ReluGradF{});
}
om_status om_gelu_fwd(om_ctx *ctx, const float *x, float *y, int64_t n) {
    if (ctx && ctx->gelu_mode != OM_GELU_REFERENCE) return map2(ctx, "om_gelu_fwd", x, nullptr, y, n, 0, GeluFastF{});
    return map2(ctx, "om_gelu_fwd", x, nullptr, y, n, 0, GeluF{});
}
om_status om_gelu_bwd(om_ctx *ctx, const float *g, const float *x, float *dx, int64_t n, int accumulate) {
    OM_REQUIRE(ctx, x || n == 0, "om_gelu_bwd: NULL saved input");
    if (ctx && ctx->gelu_mode != OM_GELU_REFERENCE)
        return map2(ctx, "om_gelu_bwd", g, x, dx, n, accumulate, GeluGradFastF{});
    return map2(ctx, "om_gelu_bwd", g, x, dx, n, accumulate, GeluGradF{});
}
om_status om_add(om_ctx *ctx, const float *a, const float *b, float *y, int64_t n) {
    OM_REQUIRE(ctx, b || n == 0, "om_add: NULL operand");
    return map2(ctx, "om_add", a, b, y, n, 0, AddF{});
}
om_status om_sub(om_ctx *ctx, const float *a, const float *b, float *y, int64_t n) {
    OM_REQUIRE(ctx, b || n == 0, "om_sub: NULL operand");
    return map2(ctx, "om_sub", a, b, y, n, 0, SubF{});
}
om_status om_mul(om_ctx *ctx, const float *a, const float *b, float *y, int64_t n) {
    OM_REQUIRE(ctx, b || n == 0, "om_mul: NULL operand");
    return map2(ctx, "om_mul", a, b, y, n, 0, MulF{});
}
om_status om_add_rows(om_ctx *ctx, const float *x, const float *b, float *y, int rows, int cols) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, rows >= 0 && cols > 0, "om_add_rows: bad shape");
    if (rows == 0) return OM_OK;
    OM_REQUIRE(ctx, x && b && y, "om_add_rows: NULL pointer");
    const int64_t n = (int64_t)rows * cols;
    if (cols % 4 == 0 && aligned4(x) && aligned4(b) && aligned4(y))
        hipLaunchKernelGGL(k_add_rows4, dim3(ew_grid(n / 4)), dim3(kBlock), 0, ctx->stream,
                           reinterpret_cast<const float4 *>(x), reinterpret_cast<const float4 *>(b),
                           reinterpret_cast<float4 *>(y), n / 4, cols / 4);
    else
        hipLaunchKernelGGL(k_add_rows, dim3(ew_grid(n)), dim3(kBlock), 0, ctx->stream, x, b, y, n, cols);
    return OM_LAUNCH_CHECK(ctx, "om_add_rows");
}
om_status om_axpy(om_ctx *ctx, float alpha, const float *src, float *dst, int64_t n) {
    OM_CHECK_CTX(ctx);
    if (n <= 0) return OM_OK;
    OM_REQUIRE(ctx, src && dst, "om_axpy: NULL pointer");
    hipLaunchKernelGGL(k_axpy, dim3(ew_grid(n)), dim3(kBlock), 0, ctx->stream, alpha, src, dst, n, 0);
    return OM_LAUNCH_CHECK(ctx, "om_axpy");
}
om_status om_scale(om_ctx *ctx, float alpha, const float *src, float *dst, int64_t n) {
    OM_CHECK_CTX(ctx);
    if (n <= 0) return OM_OK;
    OM_REQUIRE(ctx, src && dst, "om_scale: NULL pointer");
    hipLaunchKernelGGL(k_axpy, dim3(ew_grid(n)), dim3(kBlock), 0, ctx->stream, alpha, src, dst, n, 1);
    return OM_LAUNCH_CHECK(ctx, "om_scale");
}

om_status om_sum_all(om_ctx *ctx, const float *x, float *out, int64_t n, int mean) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && out && n >= 0, "om_sum_all: bad arguments");
    float *scr;
    om_status s = om::scratch(ctx, sizeof(double) * kSumBlocks, &scr);
    if (s) return s;
    double *part = reinterpret_cast<double *>(scr);
    int nb = (int)om::grid1d(n, kBlock, kSumBlocks);
    hipLaunchKernelGGL(k_sum_partial, dim3(nb), dim3(kBlock), 0, ctx->stream, x, n, part);
    hipLaunchKernelGGL(k_sum_final, dim3(1), dim3(64), 0, ctx->stream, part, nb, out, mean ? (double)n : 0.0,
                       PostTo{nullptr, nullptr, 0});
    return OM_LAUNCH_CHECK(ctx, "om_sum_all");
}

om_status om_sum_all_post(om_ctx *ctx, const float *x, float *out, int64_t n, int mean, om_readback *rb) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && out && n >= 0 && rb, "om_sum_all_post: bad arguments");
    float *scr;
    om_status s = om::scratch(ctx, sizeof(double) * kSumBlocks, &scr);
    if (s) return s;
    double *part = reinterpret_cast<double *>(scr);
    PostTo post{nullptr, nullptr, 0, nullptr};
    s = om::readback_target(ctx, rb, sizeof(float), &post.dst, &post.seq_at, &post.seq, &post.seq_dev);
    if (s) return s;
    int nb = (int)om::grid1d(n, kBlock, kSumBlocks);
    hipLaunchKernelGGL(k_sum_partial, dim3(nb), dim3(kBlock), 0, ctx->stream, x, n, part);
    hipLaunchKernelGGL(k_sum_final, dim3(1), dim3(64), 0, ctx->stream, part, nb, out, mean ? (double)n : 0.0, post);
    s = OM_LAUNCH_CHECK(ctx, "om_sum_all_post");
    if (s == OM_OK) om::readback_posted(rb, post.seq, sizeof(float));
    return s;
}

om_status om_colsum(om_ctx *ctx, const float *g, float *db, int rows, int cols, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && db && rows >= 0 && cols > 0, "om_colsum: bad arguments");
    if (rows == 0) return om_fill(ctx, db, 0.0f, accumulate ? 0 : cols);
    int chunks = (rows + kColChunk - 1) / kColChunk;
    float *scr;
    om_status s = om::scratch(ctx, sizeof(double) * (uint64_t)chunks * cols, &scr);
    if (s) return s;
    double *part = reinterpret_cast<double *>(scr);
    dim3 g1((cols + 63) / 64, chunks);
    hipLaunchKernelGGL(k_colsum_partial, g1, dim3(kBlock), 0, om::cur_stream(ctx), g, rows, cols, part);
    s = OM_LAUNCH_CHECK(ctx, "om_colsum");
    if (s) return s;
    return om::chunk_final(ctx, part, chunks, cols, db, accumulate);
}

om_status om_mean_axis(om_ctx *ctx, const float *x, float *y, int outer, int n, int inner) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && y && outer > 0 && n > 0 && inner > 0, "om_mean_axis: bad arguments");
    if (inner == 1)
        hipLaunchKernelGGL(k_mean_rows, dim3(om::grid1d((int64_t)outer * 64, kBlock, 1 << 30)), dim3(kBlock), 0,
                           ctx->stream, x, y, outer, n);
    else
        hipLaunchKernelGGL(k_mean_inner, dim3(om::grid1d((int64_t)outer * inner, kBlock, 1 << 30)), dim3(kBlock), 0,
                           ctx->stream, x, y, outer, n, inner);
    return OM_LAUNCH_CHECK(ctx, "om_mean_axis");
}

om_status om_mean_axis_bwd(om_ctx *ctx, const float *g, float *dx, int outer, int n, int inner, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && dx && outer > 0 && n > 0 && inner > 0, "om_mean_axis_bwd: bad arguments");
    hipLaunchKernelGGL(k_mean_axis_bwd, dim3(ew_grid((int64_t)outer * n * inner)), dim3(kBlock), 0, ctx->stream, g,
                       dx, outer, n, inner, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_mean_axis_bwd");
}

om_status om_relu_mean_rows(om_ctx *ctx, const float *x, float *y, int outer, int n) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && y && outer > 0 && n > 0, "om_relu_mean_rows: bad arguments");
    hipLaunchKernelGGL(k_relu_mean_rows, dim3(om::grid1d((int64_t)outer * 64, kBlock, 1 << 30)), dim3(kBlock), 0,
                       ctx->stream, x, y, outer, n);
    return OM_LAUNCH_CHECK(ctx, "om_relu_mean_rows");
}

om_status om_relu_mean_rows_bwd(om_ctx *ctx, const float *g, const float *x, float *dx, int outer, int n,
                                int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && x && dx && outer > 0 && n > 0, "om_relu_mean_rows_bwd: bad arguments");
    hipLaunchKernelGGL(k_relu_mean_rows_bwd, dim3(ew_grid((int64_t)outer * n)), dim3(kBlock), 0, ctx->stream, g, x, dx,
                       outer, n, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_relu_mean_rows_bwd");
}

om_status om_mean_all_bwd(om_ctx *ctx, const float *g, float *dx, int64_t n, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && dx && n > 0, "om_mean_all_bwd: bad arguments");
    hipLaunchKernelGGL(k_mean_all_bwd, dim3(ew_grid(n)), dim3(kBlock), 0, ctx->stream, g, dx, n, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_mean_all_bwd");
}

}  // extern "C"

om_status om::mse_of(om_ctx *ctx, const float *pred, const float *target, float *unit, float *loss, int64_t n,
                     om_readback *rb) {
    return mse_fwd(ctx, pred, target, nullptr, loss, unit, n, rb);
}

om_status om::mse_final(om_ctx *ctx, const double *part, int np, float *loss, int64_t n, om_readback *rb) {
    PostTo post{nullptr, nullptr, 0, nullptr};
    if (rb) {
        om_status s = om::readback_target(ctx, rb, sizeof(float), &post.dst, &post.seq_at, &post.seq, &post.seq_dev);
        if (s) return s;
    }
    hipLaunchKernelGGL(k_sum_final, dim3(1), dim3(64), 0, ctx->stream, part, np, loss, (double)n, post);
    om_status s = OM_LAUNCH_CHECK(ctx, "om_linear_fwd_resid_mse");
    if (s == OM_OK && rb) om::readback_posted(rb, post.seq, sizeof(float));
    return s;
}
