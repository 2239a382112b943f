// Layers of the reference's training models beyond the dense/attention/conv path: BatchNorm2d, AvgPool2d, Embedding
// and Dropout, forward and backward.
//
//   BatchNorm2d   one workgroup per channel: fp64 sums over the channel's N x plane values in a fixed tree (the
//                 reference sums serially; the fp64 results differ only in their last bits), then the elementwise
//                 pass with the reference's float expression.
//   AvgPool2d     forward: a thread per output, the window summed in (row, column) order from 0; backward: a thread
//                 per input pixel gathering the shares of the windows that cover it in (oy, ox) order, which is the
//                 order the reference's scatter adds them in — bit-exact both ways.
//   Embedding     forward: a row gather; backward (dense): a wavefront per table row collects the positions that
//                 looked it up by ballots over the ids and adds their gradient rows in increasing position order —
//                 the reference's order, so bit-exact, and no atomics.
//   Dropout       the mask is the reference's counter-based SplitMix64 function of (seed, draw, index), recomputed
//                 by the backward instead of stored: y = x * m, dx = g * m, bit-exact.
#include <rocprim/device/device_radix_sort.hpp>

#include "om_internal.hpp"

#include <cmath>
#include <cstdlib>

namespace {

constexpr int kBlock = 256;

// ------------------------------------------------------------------------------------------------ BatchNorm2d
template <class T>
__device__ __forceinline__ T block_sum(T v, T *sh) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) sh[w] = v;
    __syncthreads();
    T t = sh[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; i++) t += sh[i];
    return t;
}

// Ops.BatchNorm2d (Ops.Layers.cs:158-246). Training: batch mean and biased variance in fp64, the saved inverse
// standard deviation 1/sqrtf((float)var + eps), running statistics updated with the unbiased variance in the
// reference's mixed float/double expression. Evaluation: the running statistics. Then y = ((x - mean) * inv) * g + b.
__global__ void __launch_bounds__(kBlock) k_bn_fwd(const float *__restrict__ x, const float *__restrict__ gamma,
                                                   const float *__restrict__ beta, float *__restrict__ rm,
                                                   float *__restrict__ rv, float *__restrict__ y,
                                                   float *__restrict__ mean_out, float *__restrict__ inv_out, int n,
                                                   int c, int plane, int training, float momentum, float eps) {
    OM_LDS_POISON();
    __shared__ double sh[kBlock / 64];
    __shared__ float stat[2];
    const int ch = blockIdx.x;
    const int64_t total = (int64_t)n * plane;
    auto at = [&](int64_t e) { return ((int64_t)(e / plane) * c + ch) * plane + e % plane; };
    if (training) {
        double s = 0.0;
        for (int64_t e = threadIdx.x; e < total; e += kBlock) s += (double)x[at(e)];
        const double m = (double)total;
        const double mu = block_sum(s, sh) / m;
        double ss = 0.0;
        for (int64_t e = threadIdx.x; e < total; e += kBlock) {
            const double d = (double)x[at(e)] - mu;
            ss += d * d;
        }
        const double var = block_sum(ss, sh) / m;
        if (threadIdx.x == 0) {
            const float inv = 1.0f / sqrtf((float)var + eps);
            stat[0] = (float)mu;
            stat[1] = inv;
            mean_out[ch] = (float)mu;
            inv_out[ch] = inv;
            const double unbiased = m > 1 ? var * m / (m - 1) : var;
            const float keep = 1.0f - momentum;
            rm[ch] = (float)((double)(keep * rm[ch]) + (double)momentum * mu);
            rv[ch] = (float)((double)(keep * rv[ch]) + (double)momentum * unbiased);
        }
    } else if (threadIdx.x == 0) {
        const float inv = 1.0f / sqrtf(rv[ch] + eps);
        stat[0] = rm[ch];
        stat[1] = inv;
        mean_out[ch] = rm[ch];
        inv_out[ch] = inv;
    }
    __syncthreads();
    const float mm = stat[0], s = stat[1], gg = gamma[ch], bb = beta[ch];
    for (int64_t e = threadIdx.x; e < total; e += kBlock) {
        const int64_t o = at(e);
        y[o] = (((x[o] - mm) * s) * gg) + bb;
    }
}

// BatchNormBackward (BackwardNn.cs:244-307): sg = sum g * xhat and sb = sum g in fp64 per channel; training
// dx = (gamma * inv) * (g - (float)(sb/m) - xhat * (float)(sg/m)), evaluation dx = (gamma * inv) * g;
// dgamma = (float)sg, dbeta = (float)sb.
__global__ void __launch_bounds__(kBlock) k_bn_bwd(const float *__restrict__ g, const float *__restrict__ x,
                                                   const float *__restrict__ gamma, const float *__restrict__ mean,
                                                   const float *__restrict__ inv, float *__restrict__ dx,
                                                   float *__restrict__ dgamma, float *__restrict__ dbeta, int n,
                                                   int c, int plane, int training, int acc_dx, int acc_params) {
    OM_LDS_POISON();
    __shared__ double sh[kBlock / 64];
    const int ch = blockIdx.x;
    const int64_t total = (int64_t)n * plane;
    auto at = [&](int64_t e) { return ((int64_t)(e / plane) * c + ch) * plane + e % plane; };
    const float mm = mean[ch], s = inv[ch];
    double a = 0.0, b = 0.0;
    for (int64_t e = threadIdx.x; e < total; e += kBlock) {
        const int64_t o = at(e);
        const float gg = g[o];
        a += (double)(gg * ((x[o] - mm) * s));
        b += (double)gg;
    }
    const double sg = block_sum(a, sh);
    const double sb = block_sum(b, sh);
    if (threadIdx.x == 0) {
        if (dgamma) dgamma[ch] = acc_params ? dgamma[ch] + (float)sg : (float)sg;
        if (dbeta) dbeta[ch] = acc_params ? dbeta[ch] + (float)sb : (float)sb;
    }
    if (!dx) return;
    const double m = (double)total;
    const float k = gamma[ch] * s, cb = (float)(sb / m), cg = (float)(sg / m);
    for (int64_t e = threadIdx.x; e < total; e += kBlock) {
        const int64_t o = at(e);
        const float v = training ? k * (g[o] - cb - (((x[o] - mm) * s) * cg)) : k * g[o];
        dx[o] = acc_dx ? dx[o] + v : v;
    }
}

// ------------------------------------------------------------------------------------------------ AvgPool2d
struct PoolGeo {
    int h, w, oh, ow, kh, kw, sh, sw, ph, pw, cip;
};

// PoolWindow (BackwardNn.cs:494-506): the in-bounds window of output (oy, ox) and its divisor.
__device__ __forceinline__ void window(const PoolGeo &q, int oy, int ox, int &y0, int &y1, int &x0, int &x1,
                                       int &count) {
    const int ys = oy * q.sh - q.ph, xs = ox * q.sw - q.pw;
    const int ye = min(ys + q.kh, q.h + q.ph), xe = min(xs + q.kw, q.w + q.pw);
    const int padded = (ye - ys) * (xe - xs);
    y0 = max(ys, 0);
    x0 = max(xs, 0);
    y1 = min(ye, q.h);
    x1 = min(xe, q.w);
    count = q.cip ? padded : max(1, (y1 - y0) * (x1 - x0));
}

__global__ void __launch_bounds__(kBlock) k_avgpool_fwd(const float *__restrict__ x, float *__restrict__ y,
                                                        int64_t planes, PoolGeo q) {
    OM_LDS_POISON();
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= planes * q.oh * q.ow) return;
    const int ox = (int)(t % q.ow), oy = (int)((t / q.ow) % q.oh);
    const int64_t pl = t / ((int64_t)q.oh * q.ow);
    int y0, y1, x0, x1, count;
    window(q, oy, ox, y0, y1, x0, x1, count);
    const float *xp = x + pl * q.h * q.w;
    float sum = 0.0f;
    for (int yy = y0; yy < y1; yy++)
        for (int xx = x0; xx < x1; xx++) sum += xp[(int64_t)yy * q.w + xx];
    y[t] = sum / (float)count;
}

__global__ void __launch_bounds__(kBlock) k_avgpool_bwd(const float *__restrict__ g, float *__restrict__ dx,
                                                        int64_t planes, PoolGeo q, int acc) {
    OM_LDS_POISON();
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= planes * q.h * q.w) return;
    const int xx = (int)(t % q.w), yy = (int)((t / q.w) % q.h);
    const int64_t pl = t / ((int64_t)q.h * q.w);
    // Outputs whose window [o*s - p, o*s - p + k) covers the pixel: o in [ceil((y + p - k + 1) / s), (y + p) / s].
    const int oy_lo = max(0, (yy + q.ph - q.kh + q.sh) / q.sh), oy_hi = min(q.oh - 1, (yy + q.ph) / q.sh);
    const int ox_lo = max(0, (xx + q.pw - q.kw + q.sw) / q.sw), ox_hi = min(q.ow - 1, (xx + q.pw) / q.sw);
    const float *gp = g + pl * q.oh * q.ow;
    float v = 0.0f;
    for (int oy = oy_lo; oy <= oy_hi; oy++)
        for (int ox = ox_lo; ox <= ox_hi; ox++) {
            int y0, y1, x0, x1, count;
            window(q, oy, ox, y0, y1, x0, x1, count);
            if (yy >= y0 && yy < y1 && xx >= x0 && xx < x1) v += gp[(int64_t)oy * q.ow + ox] / (float)count;
        }
    dx[t] = acc ? dx[t] + v : v;
}

// ------------------------------------------------------------------------------------------------ Embedding
__global__ void __launch_bounds__(kBlock) k_embedding_fwd(const float *__restrict__ table,
                                                          const int32_t *__restrict__ ids, float *__restrict__ y,
                                                          int64_t n_ids, int dim, int rows) {
    OM_LDS_POISON();
    const int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (t >= n_ids * dim) return;
    const int64_t i = t / dim;
    const int j = (int)(t % dim);
    const int id = ids[i];
    // The reference rejects an out-of-range id before looking anything up; an id that reaches the device out of
    // range reads nothing and yields NaN.
    y[t] = (id >= 0 && id < rows) ? table[(int64_t)id * dim + j] : __int_as_float(0x7FC00000);
}

// Row r of the dense table gradient: the gradient rows of the positions i with ids[i] == r (r != pad), added to a
// zero row in increasing i (EmbeddingBackward, BackwardNn.cs:521-540). A wavefront per table row; ballots over 64
// ids at a time give the matching positions in order.
__global__ void __launch_bounds__(kBlock) k_embedding_bwd(const float *__restrict__ g, const int32_t *__restrict__ ids,
                                                          float *__restrict__ dtable, int64_t n_ids, int dim,
                                                          int rows, int pad, int acc) {
    OM_LDS_POISON();
    const int r = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;  // whole wavefronts leave together
    float *out = dtable + (int64_t)r * dim;
    for (int j0 = 0; j0 < dim; j0 += 64) {
        const int j = j0 + lane;
        float v = 0.0f;
        if (r != pad) {
            for (int64_t i0 = 0; i0 < n_ids; i0 += 64) {
                const int64_t i = i0 + lane;
                const bool hit = i < n_ids && ids[i] == r;
                uint64_t bits = __ballot(hit);
                while (bits) {
                    const int b = __ffsll((unsigned long long)bits) - 1;
                    bits &= bits - 1;
                    if (j < dim) v += g[(i0 + b) * dim + j];
                }
            }
        }
        if (j < dim) out[j] = acc ? out[j] + v : v;
    }
}

// The same sums for large tables, where a scan of every id per row would cost rows x n_ids: the (id, position)
// pairs are sorted by id first (a stable radix sort, so each id's positions stay in increasing order), and row r's
// wavefront finds its run of positions by binary search in the sorted ids and adds those gradient rows in that order,
// which is k_embedding_bwd's order: the results are the same bits. Positions with the padding id (or an id outside
// the table) carry the key `rows`, which sorts after every row.
__global__ void __launch_bounds__(kBlock) k_embedding_keys(const int32_t *__restrict__ ids, int32_t *__restrict__ key,
                                                           int32_t *__restrict__ pos, int64_t n_ids, int rows,
                                                           int pad) {
    OM_LDS_POISON();
    const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n_ids) return;
    const int id = ids[i];
    key[i] = (id >= 0 && id < rows && id != pad) ? id : rows;
    pos[i] = (int32_t)i;
}
__device__ __forceinline__ int64_t lower_bound_key(const int32_t *__restrict__ key, int64_t n, int v) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (key[mid] < v) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}
__global__ void __launch_bounds__(kBlock) k_embedding_bwd_sorted(const float *__restrict__ g,
                                                                 const int32_t *__restrict__ key,
                                                                 const int32_t *__restrict__ pos,
                                                                 float *__restrict__ dtable, int64_t n_ids, int dim,
                                                                 int rows, int acc) {
    OM_LDS_POISON();
    const int r = blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;  // whole wavefronts leave together
    const int64_t lo = lower_bound_key(key, n_ids, r), hi = lower_bound_key(key, n_ids, r + 1);
    float *out = dtable + (int64_t)r * dim;
    for (int j0 = 0; j0 < dim; j0 += 64) {
        const int j = j0 + lane;
        float v = 0.0f;
        if (j < dim)
            for (int64_t s = lo; s < hi; s++) v += g[(int64_t)pos[s] * dim + j];
        if (j < dim) out[j] = acc ? out[j] + v : v;
    }
}

// ------------------------------------------------------------------------------------------------ Dropout
// Generator.Mix (Generator.cs:41-47), the SplitMix64 output function.
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Dropout.Forward (Layers.cs:341-368): element i keeps iff (Mix(stream + (i + 1) * golden) >> 40) / 2^24 >= p,
// stream = Mix(seed + draw * golden); kept elements are multiplied by 1 / (1 - p). out = in * mask (the forward's
// Ops.Mul, or the backward's g * mask).
__global__ void __launch_bounds__(kBlock) k_dropout(const float *__restrict__ in, float *__restrict__ out, int64_t n,
                                                    float p, float scale, uint64_t stream, int acc) {
    OM_LDS_POISON();
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        const uint64_t bits = mix64(stream + (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull);
        const float u = (float)(bits >> 40) * (1.0f / 16777216.0f);
        const float v = in[i] * (u >= p ? scale : 0.0f);
        out[i] = acc ? out[i] + v : v;
    }
}

om_status dropout_launch(om_ctx *ctx, const char *what, const float *in, float *out, int64_t n, float p,
                         uint64_t seed, int64_t draw, int acc) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, in && out && n >= 0, "%s: bad arguments", what);
    OM_REQUIRE(ctx, p >= 0.0f && p < 1.0f, "%s: the probability must be in [0, 1) (got %g)", what, (double)p);
    OM_REQUIRE(ctx, draw >= 0, "%s: negative draw index", what);
    if (n == 0) return OM_OK;
    const float scale = 1.0f / (1.0f - p);
    const uint64_t stream = mix64(seed + (uint64_t)draw * 0x9E3779B97F4A7C15ull);
    hipLaunchKernelGGL(k_dropout, dim3(om::grid1d(n, kBlock, (int64_t)ctx->num_cus * 16)), dim3(kBlock), 0,
                       ctx->stream, in, out, n, p, scale, stream, acc);
    return OM_LAUNCH_CHECK(ctx, what);
}

}  // namespace

extern "C" {

om_status om_batchnorm2d_fwd(om_ctx *ctx, const float *x, const float *gamma, const float *beta, float *running_mean,
                             float *running_var, float *y, float *mean, float *inv, int n, int c, int plane,
                             int training, float momentum, float eps) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && gamma && beta && running_mean && running_var && y && mean && inv,
               "om_batchnorm2d_fwd: NULL pointer");
    OM_REQUIRE(ctx, n >= 0 && c > 0 && plane >= 0, "om_batchnorm2d_fwd: bad shape");
    OM_REQUIRE(ctx, !training || (int64_t)n * plane >= 1,
               "om_batchnorm2d_fwd: training needs at least one value per channel");
    hipLaunchKernelGGL(k_bn_fwd, dim3(c), dim3(kBlock), 0, ctx->stream, x, gamma, beta, running_mean, running_var, y,
                       mean, inv, n, c, plane, training, momentum, eps);
    return OM_LAUNCH_CHECK(ctx, "om_batchnorm2d_fwd");
}

om_status om_batchnorm2d_bwd(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                             const float *inv, float *dx, float *dgamma, float *dbeta, int n, int c, int plane,
                             int training, int acc_dx, int acc_params) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && x && gamma && mean && inv, "om_batchnorm2d_bwd: NULL input");
    OM_REQUIRE(ctx, n >= 0 && c > 0 && plane >= 0, "om_batchnorm2d_bwd: bad shape");
    if (!dx && !dgamma && !dbeta) return OM_OK;
    hipLaunchKernelGGL(k_bn_bwd, dim3(c), dim3(kBlock), 0, ctx->stream, g, x, gamma, mean, inv, dx, dgamma, dbeta, n,
                       c, plane, training, acc_dx, acc_params);
    return OM_LAUNCH_CHECK(ctx, "om_batchnorm2d_bwd");
}

static om_status pool_geo(om_ctx *ctx, const char *what, int h, int w, int kh, int kw, int sh, int sw, int ph, int pw,
                          int cip, PoolGeo &q) {
    OM_REQUIRE(ctx, h > 0 && w > 0 && kh > 0 && kw > 0 && sh > 0 && sw > 0 && ph >= 0 && pw >= 0,
               "%s: bad window", what);
    OM_REQUIRE(ctx, 2 * ph <= kh && 2 * pw <= kw, "%s: padding must be at most half the window", what);
    q.h = h;
    q.w = w;
    q.kh = kh;
    q.kw = kw;
    q.sh = sh;
    q.sw = sw;
    q.ph = ph;
    q.pw = pw;
    q.cip = cip ? 1 : 0;
    q.oh = (h + 2 * ph - kh) / sh + 1;
    q.ow = (w + 2 * pw - kw) / sw + 1;
    OM_REQUIRE(ctx, q.oh > 0 && q.ow > 0, "%s: the window does not fit the input", what);
    return OM_OK;
}

om_status om_avgpool2d_fwd(om_ctx *ctx, const float *x, float *y, int planes, int h, int w, int kh, int kw, int sh,
                           int sw, int ph, int pw, int count_include_pad) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && y && planes >= 0, "om_avgpool2d_fwd: bad arguments");
    PoolGeo q;
    om_status st = pool_geo(ctx, "om_avgpool2d_fwd", h, w, kh, kw, sh, sw, ph, pw, count_include_pad, q);
    if (st) return st;
    const int64_t total = (int64_t)planes * q.oh * q.ow;
    if (total == 0) return OM_OK;
    hipLaunchKernelGGL(k_avgpool_fwd, dim3(om::grid1d(total, kBlock, 1 << 30)), dim3(kBlock), 0, ctx->stream, x, y,
                       (int64_t)planes, q);
    return OM_LAUNCH_CHECK(ctx, "om_avgpool2d_fwd");
}

om_status om_avgpool2d_bwd(om_ctx *ctx, const float *g, float *dx, int planes, int h, int w, int kh, int kw, int sh,
                           int sw, int ph, int pw, int count_include_pad, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && dx && planes >= 0, "om_avgpool2d_bwd: bad arguments");
    PoolGeo q;
    om_status st = pool_geo(ctx, "om_avgpool2d_bwd", h, w, kh, kw, sh, sw, ph, pw, count_include_pad, q);
    if (st) return st;
    const int64_t total = (int64_t)planes * h * w;
    if (total == 0) return OM_OK;
    hipLaunchKernelGGL(k_avgpool_bwd, dim3(om::grid1d(total, kBlock, 1 << 30)), dim3(kBlock), 0, ctx->stream, g, dx,
                       (int64_t)planes, q, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_avgpool2d_bwd");
}

om_status om_embedding_fwd(om_ctx *ctx, const float *table, const int32_t *ids, float *y, int64_t n_ids, int dim,
                           int rows) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, table && ids && y && n_ids >= 0 && dim > 0 && rows > 0, "om_embedding_fwd: bad arguments");
    if (n_ids == 0) return OM_OK;
    hipLaunchKernelGGL(k_embedding_fwd, dim3(om::grid1d(n_ids * dim, kBlock, 1 << 30)), dim3(kBlock), 0, ctx->stream,
                       table, ids, y, n_ids, dim, rows);
    return OM_LAUNCH_CHECK(ctx, "om_embedding_fwd");
}

om_status om_embedding_bwd(om_ctx *ctx, const float *g, const int32_t *ids, float *dtable, int64_t n_ids, int dim,
                           int rows, int padding_index, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && ids && dtable && n_ids >= 0 && dim > 0 && rows > 0, "om_embedding_bwd: bad arguments");
    const unsigned row_grid = (unsigned)((rows + kBlock / 64 - 1) / (kBlock / 64));
    // Small tables (or few ids): one launch that scans the ids for every row. Beyond about 2^22 id visits the sort
    // costs less than the scan. In a tuning build OM_EMBEDDING_SORT=0 keeps every size on the scan (for comparisons).
    const char *env = om::tuning_env("OM_EMBEDDING_SORT");
    const bool no_sort = env && env[0] == '0';
    if (no_sort || (double)rows * (double)n_ids <= (double)(1 << 22) || n_ids > INT32_MAX) {
        hipLaunchKernelGGL(k_embedding_bwd, dim3(row_grid), dim3(kBlock), 0, ctx->stream, g, ids, dtable, n_ids, dim,
                           rows, padding_index, accumulate);
        return OM_LAUNCH_CHECK(ctx, "om_embedding_bwd");
    }
    // The radix sort's launches may include memory fills a step graph must not hold.
    if (om_status st = om::refuse_in_capture(ctx, "om_embedding_bwd (large table)")) return st;
    int bits = 1;
    while (bits < 31 && (1ll << bits) <= (long long)rows) bits++;  // keys 0 .. rows
    size_t temp_bytes = 0;
    hipError_t e = rocprim::radix_sort_pairs(nullptr, temp_bytes, (int32_t *)nullptr, (int32_t *)nullptr,
                                             (int32_t *)nullptr, (int32_t *)nullptr, (size_t)n_ids, 0, bits,
                                             ctx->stream);
    if (e != hipSuccess) return om::check_hip(ctx, e, "om_embedding_bwd sort size");
    const uint64_t pair = (uint64_t)n_ids * sizeof(int32_t), pad_pair = (pair + 255) / 256 * 256;
    float *scr;
    om_status st = om::scratch(ctx, 4 * pad_pair + temp_bytes, &scr);
    if (st) return st;
    char *base = reinterpret_cast<char *>(scr);
    int32_t *k_in = reinterpret_cast<int32_t *>(base), *p_in = reinterpret_cast<int32_t *>(base + pad_pair);
    int32_t *k_out = reinterpret_cast<int32_t *>(base + 2 * pad_pair), *p_out = reinterpret_cast<int32_t *>(base + 3 * pad_pair);
    hipLaunchKernelGGL(k_embedding_keys, dim3(om::grid1d(n_ids, kBlock)), dim3(kBlock), 0, ctx->stream, ids, k_in,
                       p_in, n_ids, rows, padding_index);
    e = rocprim::radix_sort_pairs(base + 4 * pad_pair, temp_bytes, k_in, k_out, p_in, p_out, (size_t)n_ids, 0, bits,
                                  ctx->stream);
    if (e != hipSuccess) return om::check_hip(ctx, e, "om_embedding_bwd sort");
    hipLaunchKernelGGL(k_embedding_bwd_sorted, dim3(row_grid), dim3(kBlock), 0, ctx->stream, g, k_out, p_out, dtable,
                       n_ids, dim, rows, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_embedding_bwd");
}

om_status om_dropout_fwd(om_ctx *ctx, const float *x, float *y, int64_t n, float p, uint64_t seed, int64_t draw) {
    return dropout_launch(ctx, "om_dropout_fwd", x, y, n, p, seed, draw, 0);
}

om_status om_dropout_bwd(om_ctx *ctx, const float *g, float *dx, int64_t n, float p, uint64_t seed, int64_t draw,
                         int accumulate) {
    return dropout_launch(ctx, "om_dropout_bwd", g, dx, n, p, seed, draw, accumulate);
}

}  // extern "C"
