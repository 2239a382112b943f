// Row kernels: LayerNorm forward/backward, softmax and log-softmax forward/backward, NLL and the fused softmax
// cross-entropy gradient, and the attention score-gradient row pass. All HBM-bound: rows are read with coalesced
// loads, reductions stay in registers and wavefront shuffles, column sums go through LDS and a fixed-order second
// pass.
#include "om_internal.hpp"

#include <mutex>

namespace {

constexpr int kBlock = 256;

using omd::max16;
__device__ __forceinline__ float sum16_combine(float p) { return omd::sum16(p); }

// LayerNorm forward: one row per 16-lane group (4 rows per wavefront). NormKernels.Rows (NormKernels.cs:79-127):
// mean = Sum16(x)/n, ssq = Sum16((x-mean)^2), inv = 1/sqrt(ssq/n + eps), y = (((x-mean)*inv)*gamma)+beta.
__global__ void __launch_bounds__(kBlock) k_ln_fwd(const float *__restrict__ x, const float *__restrict__ gamma,
                                                   const float *__restrict__ beta, float *__restrict__ y,
                                                   float *__restrict__ mean_out, float *__restrict__ rstd_out,
                                                   int rows, int cols, float eps) {
    OM_LDS_POISON();
    int row = (blockIdx.x * kBlock + threadIdx.x) >> 4;
    int t = threadIdx.x & 15;
    if (row >= rows) return;  // whole 16-lane groups leave together
    const float *xr = x + (int64_t)row * cols;
    float *yr = y + (int64_t)row * cols;
    float n = (float)cols;
    float p = 0.0f;
    for (int j = t; j < cols; j += 16) p += xr[j];
    float mean = sum16_combine(p) / n;
    p = 0.0f;
    for (int j = t; j < cols; j += 16) {
        float d = xr[j] - mean;
        p += d * d;
    }
    float ssq = sum16_combine(p);
    float inv = 1.0f / sqrtf(ssq / n + eps);
    if (t == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = inv;
    }
    for (int j = t; j < cols; j += 16) yr[j] = omd::canon(((xr[j] - mean) * inv) * gamma[j] + beta[j]);
}

// The same computation with the block's 16 rows staged through LDS: global traffic is float4-coalesced and the
// 16-lane strided Sum16 walks run on LDS (row stride cols+16 keeps the four rows of a wavefront on distinct banks);
// y goes back out through LDS as well. Requires cols % 4 == 0 and cols <= kLnLdsMaxCols.
constexpr int kLnLdsMaxCols = 960;  // keeps dynamic LDS under 64 KB
template <int NTH>
__global__ void __launch_bounds__(NTH) k_ln_fwd_lds(const float *__restrict__ x, const float *__restrict__ gamma,
                                                    const float *__restrict__ beta, float *__restrict__ y,
                                                    float *__restrict__ mean_out, float *__restrict__ rstd_out,
                                                    int rows, int cols, float eps) {
    OM_LDS_POISON();
    constexpr int NR = NTH / 16;  // rows per block, a 16-lane group each
    extern __shared__ float sh[];  // [NR][cols + 16]
    const int ld = cols + 16, c4 = cols >> 2;
    const int r0 = blockIdx.x * NR;
    const int nr = min(NR, rows - r0);
    const int n4 = nr * c4;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (int64_t)r0 * cols);
    for (int i = threadIdx.x; i < n4; i += NTH) {
        int r = i / c4, q = i - r * c4;
        *reinterpret_cast<float4 *>(sh + r * ld + 4 * q) = x4[i];
    }
    __syncthreads();
    const int lr = threadIdx.x >> 4, t = threadIdx.x & 15;
    if (lr < nr) {
        float *xr = sh + lr * ld;
        const float n = (float)cols;
        float p = 0.0f;
        for (int j = t; j < cols; j += 16) p += xr[j];
        float mean = sum16_combine(p) / n;
        p = 0.0f;
        for (int j = t; j < cols; j += 16) {
            float d = xr[j] - mean;
            p += d * d;
        }
        float ssq = sum16_combine(p);
        float inv = 1.0f / sqrtf(ssq / n + eps);
        if (t == 0) {
            if (mean_out) mean_out[r0 + lr] = mean;
            if (rstd_out) rstd_out[r0 + lr] = inv;
        }
        for (int j = t; j < cols; j += 16) xr[j] = omd::canon(((xr[j] - mean) * inv) * gamma[j] + beta[j]);
    }
    __syncthreads();
    float4 *y4 = reinterpret_cast<float4 *>(y + (int64_t)r0 * cols);
    for (int i = threadIdx.x; i < n4; i += NTH) {
        int r = i / c4, q = i - r * c4;
        y4[i] = *reinterpret_cast<const float4 *>(sh + r * ld + 4 * q);
    }
}

// LayerNorm forward for a compile-time width (a multiple of 16): a 16-lane group per row, lane t holding elements
// t, t+16, ... in registers. All of a row's loads (and gamma/beta, once per wavefront) are issued before any use, and
// the Sum16 chains run on registers; the arithmetic is k_ln_fwd's, bit for bit.
template <int COLS>
__global__ void __launch_bounds__(kBlock) k_ln_fwd_w(const float *__restrict__ x, const float *__restrict__ gamma,
                                                     const float *__restrict__ beta, float *__restrict__ y,
                                                     float *__restrict__ mean_out, float *__restrict__ rstd_out,
                                                     int rows, float eps) {
    OM_LDS_POISON();
    constexpr int PER = COLS / 16;
    const int row = (blockIdx.x * kBlock + threadIdx.x) >> 4, t = threadIdx.x & 15;
    if (row >= rows) return;  // whole 16-lane groups leave together
    const float *xr = x + (int64_t)row * COLS + t;
    float v[PER], gm[PER], bt[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) v[k] = xr[16 * k];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        gm[k] = gamma[t + 16 * k];
        bt[k] = beta[t + 16 * k];
    }
    const float n = (float)COLS;
    float p = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; k++) p += v[k];
    const float mean = sum16_combine(p) / n;
    p = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        float d = v[k] - mean;
        p += d * d;
    }
    const float ssq = sum16_combine(p);
    const float inv = 1.0f / sqrtf(ssq / n + eps);
    if (t == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = inv;
    }
    float *yr = y + (int64_t)row * COLS + t;
#pragma unroll
    for (int k = 0; k < PER; k++) yr[16 * k] = omd::canon(((v[k] - mean) * inv) * gm[k] + bt[k]);
}

// LayerNorm backward (BackwardNn.cs:170-223), cols <= 64*kMaxPer: a wavefront per row, a block per chunk of rows.
// dx is written per row; the dgamma/dbeta column contributions are kept per lane in double and summed over the
// block's waves in LDS (fixed order), giving partial[chunk][col] for the second pass.
constexpr int kMaxPer = 16;
// PER = column slots per lane (cols <= 64 * PER); the row walk is fully unrolled when cols == 64 * PER.
template <int PER>
__global__ void __launch_bounds__(kBlock) k_ln_bwd(const float *__restrict__ g, const float *__restrict__ x,
                                                   const float *__restrict__ gamma, const float *__restrict__ mean,
                                                   const float *__restrict__ rstd, float *dx, const float *dxin,
                                                   double *__restrict__ part_g, double *__restrict__ part_b, int rows,
                                                   int cols, int rows_per_chunk) {
    OM_LDS_POISON();
    __shared__ double lds[kBlock / 64][64 * PER];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r0 = blockIdx.x * rows_per_chunk, r1 = min(rows, r0 + rows_per_chunk);
    const bool full = cols == 64 * PER;
    double pg[PER], pb[PER];
    float gam[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        pg[i] = pb[i] = 0.0;
        int j = lane + 64 * i;
        gam[i] = (full || j < cols) ? gamma[j] : 0.0f;
    }
    for (int r = r0 + w; r < r1; r += kBlock / 64) {
        const float *xr = x + (int64_t)r * cols;
        const float *gr = g + (int64_t)r * cols;
        float m = mean[r], s = rstd[r];
        double sum1 = 0.0, sum2 = 0.0;
        float xh[PER], gv[PER];
#pragma unroll
        for (int i = 0; i < PER; i++) {
            int j = lane + 64 * i;
            const bool in = full || j < cols;
            xh[i] = in ? xr[j] : 0.0f;
            gv[i] = in ? gr[j] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < PER; i++) {
            int j = lane + 64 * i;
            if (full || j < cols) {
                float xhat = (xh[i] - m) * s;
                float gg = gv[i];
                float dxhat = gg * gam[i];
                sum1 += (double)dxhat;
                sum2 += (double)(dxhat * xhat);
                pg[i] += (double)(gg * xhat);
                pb[i] += (double)gg;
                xh[i] = xhat;
            }
        }
        sum1 = omd::wave_sum(sum1);
        sum2 = omd::wave_sum(sum2);
        if (dx) {
            float m1 = (float)(sum1 / cols), m2 = (float)(sum2 / cols);
            float *dr = dx + (int64_t)r * cols;
            const float *di = dxin ? dxin + (int64_t)r * cols : nullptr;
#pragma unroll
            for (int i = 0; i < PER; i++) {
                int j = lane + 64 * i;
                if (full || j < cols) {
                    float v = s * (((gv[i] * gam[i]) - m1) - (xh[i] * m2));
                    dr[j] = di ? di[j] + v : v;
                }
            }
        }
    }
    if (!part_g && !part_b) return;
    for (int pass = 0; pass < 2; pass++) {
        double *part = pass == 0 ? part_g : part_b;
        if (!part) continue;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < PER; i++) lds[w][lane + 64 * i] = pass == 0 ? pg[i] : pb[i];
        __syncthreads();
        for (int j = threadIdx.x; j < cols; j += kBlock) {
            double t = 0.0;
#pragma unroll
            for (int q = 0; q < kBlock / 64; q++) t += lds[q][j];
            part[(int64_t)blockIdx.x * cols + j] = t;
        }
    }
}
// LayerNorm backward for a compile-time width (a multiple of 64): a wavefront per row, lane l holding columns
// l, l+64, ...; each wavefront walks RPW consecutive rows with the next row's loads in flight while the current row
// computes, and the workgroup's fp64 column partials of dgamma / dbeta go out once. Same arithmetic as k_ln_bwd.
template <int COLS, int RPW, int NW>
__global__ void __launch_bounds__(NW * 64) k_ln_bwd_w(const float *__restrict__ g, const float *__restrict__ x,
                                                     const float *__restrict__ gamma, const float *__restrict__ mean,
                                                     const float *__restrict__ rstd, float *dx, const float *dxin,
                                                     double *__restrict__ part_g, double *__restrict__ part_b,
                                                     int rows) {
    OM_LDS_POISON();
    constexpr int PER = COLS / 64;
    __shared__ double lds[NW][COLS];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int rbase = (blockIdx.x * NW + w) * RPW;
    double pg[PER], pb[PER];
    float gam[PER];
#pragma unroll
    for (int c = 0; c < PER; c++) {
        pg[c] = pb[c] = 0.0;
        gam[c] = gamma[lane + 64 * c];
    }
    float xv[2][PER], gv[2][PER], mv[2], sv[2];
    auto load = [&](int slot, int r) {
        if (r < rows) {
            const float *xr = x + (int64_t)r * COLS + lane, *gr = g + (int64_t)r * COLS + lane;
#pragma unroll
            for (int c = 0; c < PER; c++) {
                xv[slot][c] = xr[64 * c];
                gv[slot][c] = gr[64 * c];
            }
            mv[slot] = mean[r];
            sv[slot] = rstd[r];
        }
    };
    load(0, rbase);
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const int cur = i & 1, r = rbase + i;
        if (i + 1 < RPW) load(cur ^ 1, r + 1);
        if (r >= rows) break;
        const float m = mv[cur], s = sv[cur];
        double sum1 = 0.0, sum2 = 0.0;
        float xh[PER];
#pragma unroll
        for (int c = 0; c < PER; c++) {
            const float xhat = (xv[cur][c] - m) * s;
            const float gg = gv[cur][c];
            const float dxhat = gg * gam[c];
            sum1 += (double)dxhat;
            sum2 += (double)(dxhat * xhat);
            pg[c] += (double)(gg * xhat);
            pb[c] += (double)gg;
            xh[c] = xhat;
        }
        sum1 = omd::wave_sum(sum1);
        sum2 = omd::wave_sum(sum2);
        if (dx) {
            const float m1 = (float)(sum1 / COLS), m2 = (float)(sum2 / COLS);
            float *dr = dx + (int64_t)r * COLS + lane;
            const float *di = dxin ? dxin + (int64_t)r * COLS + lane : nullptr;
#pragma unroll
            for (int c = 0; c < PER; c++) {
                const float v = s * (((gv[cur][c] * gam[c]) - m1) - (xh[c] * m2));
                dr[64 * c] = di ? di[64 * c] + v : v;
            }
        }
    }
    if (!part_g && !part_b) return;
    for (int pass = 0; pass < 2; pass++) {
        double *part = pass == 0 ? part_g : part_b;
        if (!part) continue;
        __syncthreads();
#pragma unroll
        for (int c = 0; c < PER; c++) lds[w][lane + 64 * c] = pass == 0 ? pg[c] : pb[c];
        __syncthreads();
        for (int j = threadIdx.x; j < COLS; j += NW * 64) {
            double t = 0.0;
#pragma unroll
            for (int q = 0; q < NW; q++) t += lds[q][j];
            part[(int64_t)blockIdx.x * COLS + j] = t;
        }
    }
}

// Generic (any width) LayerNorm backward for dx only: a wavefront per row, columns strided.
__global__ void __launch_bounds__(kBlock) k_ln_bwd_dx_wide(const float *__restrict__ g, const float *__restrict__ x,
                                                           const float *__restrict__ gamma,
                                                           const float *__restrict__ mean,
                                                           const float *__restrict__ rstd, float *dx,
                                                           const float *dxin, int rows, int cols) {
    OM_LDS_POISON();
    int r = (blockIdx.x * kBlock + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *xr = x + (int64_t)r * cols, *gr = g + (int64_t)r * cols;
    float m = mean[r], s = rstd[r];
    double sum1 = 0.0, sum2 = 0.0;
    for (int j = lane; j < cols; j += 64) {
        float xhat = (xr[j] - m) * s, dxhat = gr[j] * gamma[j];
        sum1 += (double)dxhat;
        sum2 += (double)(dxhat * xhat);
    }
    sum1 = omd::wave_sum(sum1);
    sum2 = omd::wave_sum(sum2);
    float m1 = (float)(sum1 / cols), m2 = (float)(sum2 / cols);
    float *dr = dx + (int64_t)r * cols;
    const float *di = dxin ? dxin + (int64_t)r * cols : nullptr;
    for (int j = lane; j < cols; j += 64) {
        float xhat = (xr[j] - m) * s;
        float v = s * (((gr[j] * gamma[j]) - m1) - (xhat * m2));
        dr[j] = di ? di[j] + v : v;
    }
}
// Generic column partials of g*xhat and g for wide rows: one thread per column per chunk of rows.
__global__ void __launch_bounds__(kBlock) k_ln_param_partial_wide(const float *__restrict__ g,
                                                                  const float *__restrict__ x,
                                                                  const float *__restrict__ mean,
                                                                  const float *__restrict__ rstd,
                                                                  double *__restrict__ part_g,
                                                                  double *__restrict__ part_b, int rows, int cols,
                                                                  int rows_per_chunk) {
    OM_LDS_POISON();
    int col = blockIdx.x * kBlock + threadIdx.x;
    if (col >= cols) return;
    int r0 = blockIdx.y * rows_per_chunk, r1 = min(rows, r0 + rows_per_chunk);
    double a = 0.0, b = 0.0;
    for (int r = r0; r < r1; r++) {
        float gg = g[(int64_t)r * cols + col];
        float xhat = (x[(int64_t)r * cols + col] - mean[r]) * rstd[r];
        a += (double)(gg * xhat);
        b += (double)gg;
    }
    if (part_g) part_g[(int64_t)blockIdx.y * cols + col] = a;
    if (part_b) part_b[(int64_t)blockIdx.y * cols + col] = b;
}

// Softmax rows, exact flavour (Softmax.cs:70-133): max, e = expNonPositive(x - max), l = Sum16(e), y = e / l.
__global__ void __launch_bounds__(kBlock) k_softmax_rows(const float *x, float *y, int rows, int cols) {
    OM_LDS_POISON();
    int row = (blockIdx.x * kBlock + threadIdx.x) >> 4;
    int t = threadIdx.x & 15;
    if (row >= rows) return;
    const float *xr = x + (int64_t)row * cols;
    float *yr = y + (int64_t)row * cols;
    float mx = -__int_as_float(0x7F800000);
    for (int j = t; j < cols; j += 16) {
        float v = xr[j];
        mx = v > mx ? v : mx;
    }
    mx = max16(mx);
    float p = 0.0f;
    for (int j = t; j < cols; j += 16) {
        float e = omd::exp_nonpos(xr[j] - mx);
        yr[j] = e;
        p += e;
    }
    float l = sum16_combine(p);
    for (int j = t; j < cols; j += 16) yr[j] = omd::canon(yr[j] / l);
}

// y * (g - (float)sum(double)(g*y)) per row (BackwardNn.cs:26-52); with `scale` (attention, BackwardNn.cs:674-688)
// the result is multiplied by scale. Wavefront per row; in place on g allowed.
__global__ void __launch_bounds__(kBlock) k_softmax_bwd_rows(const float *g, const float *__restrict__ y, float *dx,
                                                             int rows, int cols, float scale, int use_scale,
                                                             int acc) {
    OM_LDS_POISON();
    int r = (blockIdx.x * kBlock + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *gr = g + (int64_t)r * cols, *yr = y + (int64_t)r * cols;
    float *dr = dx + (int64_t)r * cols;
    double dot = 0.0;
    for (int j = lane; j < cols; j += 64) dot += (double)(gr[j] * yr[j]);
    dot = omd::wave_sum(dot);
    float df = (float)dot;
    for (int j = lane; j < cols; j += 64) {
        float v = yr[j] * (gr[j] - df);
        if (use_scale) v = v * scale;
        dr[j] = acc ? dr[j] + v : v;
    }
}

// LogSoftmax rows (Ops.Layers.cs:47-96): max, double sum of exp(x - max), lse = max + log((float)sum).
__global__ void __launch_bounds__(kBlock) k_logsoftmax_rows(const float *__restrict__ x, float *__restrict__ y,
                                                            int rows, int cols) {
    OM_LDS_POISON();
    int r = (blockIdx.x * kBlock + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *xr = x + (int64_t)r * cols;
    float mx = -__int_as_float(0x7F800000);
    for (int j = lane; j < cols; j += 64) mx = xr[j] > mx ? xr[j] : mx;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float w = __shfl_xor(mx, o, 64);
        mx = w > mx ? w : mx;
    }
    double sum = 0.0;
    for (int j = lane; j < cols; j += 64) sum += (double)expf(xr[j] - mx);
    sum = omd::wave_sum(sum);
    float lse = mx + logf((float)sum);
    for (int j = lane; j < cols; j += 64) y[(int64_t)r * cols + j] = xr[j] - lse;
}
// LogSoftmax backward (BackwardNn.cs:54-80): dx = g - exp(y) * (float)sum(double) g.
__global__ void __launch_bounds__(kBlock) k_logsoftmax_bwd_rows(const float *__restrict__ g,
                                                                const float *__restrict__ y, float *__restrict__ dx,
                                                                int rows, int cols, int acc) {
    OM_LDS_POISON();
    int r = (blockIdx.x * kBlock + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *gr = g + (int64_t)r * cols, *yr = y + (int64_t)r * cols;
    double sum = 0.0;
    for (int j = lane; j < cols; j += 64) sum += (double)gr[j];
    float s = (float)omd::wave_sum(sum);
    for (int j = lane; j < cols; j += 64) {
        float v = gr[j] - expf(yr[j]) * s;
        float *d = dx + (int64_t)r * cols + j;
        *d = acc ? *d + v : v;
    }
}

// A loss value posted to a readback buffer by the launch that computes it: the value as a system-scope write-through
// store, a wait for its completion, then the sequence number (read from seq_dev inside a step graph).
struct LossPost {
    char *dst;
    uint64_t *seq_at;
    uint64_t seq;
    const uint64_t *seq_dev;
};

// NllLoss forward (Ops.Layers.cs:644-699): one block; double sum of -logp[i, t_i] over counted rows; the first
// out-of-range row (smallest index) is reported.
__global__ void __launch_bounds__(kBlock) k_nll_fwd(const float *__restrict__ logp, const int32_t *__restrict__ tg,
                                                    float *__restrict__ loss, int32_t *__restrict__ bad, int rows,
                                                    int cols, int mean, int ignore, LossPost post) {
    OM_LDS_POISON();
    __shared__ double sh[kBlock / 64];
    __shared__ int shbad;
    if (threadIdx.x == 0) shbad = 0x7FFFFFFF;
    __syncthreads();
    double acc = 0.0;
    double cnt = 0.0;
    // Rows i = threadIdx.x + kBlock u in increasing u, eight at a time: the eight targets load together, then the
    // eight gathered log-probabilities, then the sums run in row order.
    constexpr int R = 8;
    for (int base = 0; base < rows; base += kBlock * R) {
        int t[R];
        float lp[R];
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int i = base + kBlock * u + (int)threadIdx.x;
            t[u] = i < rows ? tg[i] : ignore;
        }
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int i = base + kBlock * u + (int)threadIdx.x;
            const bool use = i < rows && t[u] != ignore && (unsigned)t[u] < (unsigned)cols;
            lp[u] = use ? logp[(int64_t)i * cols + t[u]] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int i = base + kBlock * u + (int)threadIdx.x;
            if (i >= rows || t[u] == ignore) continue;
            if ((unsigned)t[u] >= (unsigned)cols) {
                atomicMin(&shbad, i);
                continue;
            }
            acc -= (double)lp[u];
            cnt += 1.0;
        }
    }
    double total = omd::block_sum<kBlock / 64>(acc, sh);
    double count = omd::block_sum<kBlock / 64>(cnt, sh);
    __syncthreads();
    if (threadIdx.x == 0) {
        int b = shbad == 0x7FFFFFFF ? -1 : shbad;
        if (bad) bad[0] = b;
        const float v = b >= 0 ? __int_as_float(0x7FC00000)
                               : (float)(mean ? total / (count > 1.0 ? count : 1.0) : total);
        loss[0] = v;
        if (post.dst) {
            __hip_atomic_store(reinterpret_cast<float *>(post.dst), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __builtin_amdgcn_s_waitcnt(0);
            __hip_atomic_store(post.seq_at, post.seq_dev ? *post.seq_dev : post.seq, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

// One row of the cross-entropy forward with the unit gradient (a wavefront): logp = x - (max + log(double sum of
// exp(x - max))), then k_xent_bwd's arithmetic for g = 1: dx = d - exp(logp) s with d = -scale at the target (when the
// row counts) and s = -scale (0 for an ignored row). lpt, when given, receives logp at the target (0 <= t < cols).
__device__ __forceinline__ void xent_row(const float *__restrict__ x, float *__restrict__ y, float *__restrict__ dx,
                                         int r, int cols, int t, int ignore, float scale, int lane, float *lpt) {
    const float *xr = x + (int64_t)r * cols;
    float *yr = y + (int64_t)r * cols, *dr = dx + (int64_t)r * cols;
    float mx = -__int_as_float(0x7F800000);
    for (int j = lane; j < cols; j += 64) mx = xr[j] > mx ? xr[j] : mx;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float w = __shfl_xor(mx, o, 64);
        mx = w > mx ? w : mx;
    }
    double sum = 0.0;
    for (int j = lane; j < cols; j += 64) sum += (double)expf(xr[j] - mx);
    sum = omd::wave_sum(sum);
    const float lse = mx + logf((float)sum);
    const bool counted = t != ignore;
    const float sr = counted ? -scale : 0.0f;
    for (int j = lane; j < cols; j += 64) {
        const float lp = xr[j] - lse;
        yr[j] = lp;
        if (lpt && j == t) *lpt = lp;
        const float d = (counted && j == t) ? -scale : 0.0f;
        dr[j] = d - expf(lp) * sr;
    }
}

// Cross-entropy forward with the unit gradient: per row (a wavefront each), k_logsoftmax_rows' arithmetic writing
// logp, then k_xent_bwd's for g = 1 and the mean reduction, reading the logp values just computed. The count of
// rows that are not ignored, which the gradient's scale needs, is formed by every block from all targets (an exact
// integer count, so the same in every block).
__global__ void __launch_bounds__(kBlock) k_xent_fwd_rows(const float *__restrict__ x, const int32_t *__restrict__ tg,
                                                          float *__restrict__ y, float *__restrict__ dx, int rows,
                                                          int cols, int ignore) {
    OM_LDS_POISON();
    __shared__ int shc[kBlock / 64];
    int c = 0;
    for (int i = threadIdx.x; i < rows; i += kBlock) c += tg[i] != ignore ? 1 : 0;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
    if ((threadIdx.x & 63) == 0) shc[threadIdx.x >> 6] = c;
    __syncthreads();
    int count = 0;
#pragma unroll
    for (int i = 0; i < kBlock / 64; i++) count += shc[i];
    int r = (blockIdx.x * kBlock + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (r >= rows) return;
    xent_row(x, y, dx, r, cols, tg[r], ignore, 1.0f / (float)(count > 1 ? count : 1), lane, nullptr);
}

// Fused NllBackward + LogSoftmax backward (BackwardNn.cs:54-80, 602-632). scale = g/max(1,count) (or g); the NLL
// gradient d has -scale at the target; its double row sum is s = -scale (0 for an ignored row); dx = d - exp(y)*s.
__global__ void __launch_bounds__(kBlock) k_xent_count(const int32_t *__restrict__ tg, int rows, int ignore,
                                                       int *__restrict__ count) {
    OM_LDS_POISON();
    __shared__ double sh[kBlock / 64];
    double c = 0.0;
    for (int i = threadIdx.x; i < rows; i += kBlock) c += tg[i] != ignore ? 1.0 : 0.0;
    double t = omd::block_sum<kBlock / 64>(c, sh);
    if (threadIdx.x == 0) count[0] = (int)t;
}
__global__ void __launch_bounds__(kBlock) k_xent_bwd(const float *__restrict__ gs, const int *__restrict__ count,
                                                     const float *__restrict__ y, const int32_t *__restrict__ tg,
                                                     float *__restrict__ dx, int rows, int cols, int mean, int ignore,
                                                     int acc) {
    OM_LDS_POISON();
    int r = (blockIdx.x * kBlock + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (r >= rows) return;
    float g = gs[0];
    int c = count[0];
    float scale = mean ? g / (float)(c > 1 ? c : 1) : g;
    int t = tg[r];
    bool counted = t != ignore;
    float s = counted ? -scale : 0.0f;
    for (int j = lane; j < cols; j += 64) {
        float d = (counted && j == t) ? -scale : 0.0f;
        float v = d - expf(y[(int64_t)r * cols + j]) * s;
        float *o = dx + (int64_t)r * cols + j;
        *o = acc ? *o + v : v;
    }
}

// NllBackward (BackwardNn.cs:602-632) alone: scale = g/max(1,count) (or g); dx is -scale at each counted row's target
// and 0 elsewhere (Tensor.Zeros), added into an existing gradient when acc (Engine.AddInto).
__global__ void __launch_bounds__(kBlock) k_nll_bwd(const float *__restrict__ gs, const int *__restrict__ count,
                                                    const int32_t *__restrict__ tg, float *__restrict__ dx, int rows,
                                                    int cols, int mean, int ignore, int acc) {
    OM_LDS_POISON();
    const int64_t n = (int64_t)rows * cols, stride = (int64_t)gridDim.x * kBlock;
    const float g = gs[0];
    const int c = count[0];
    const float scale = mean ? g / (float)(c > 1 ? c : 1) : g;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        const int r = (int)(i / cols), j = (int)(i % cols), t = tg[r];
        const float d = (t != ignore && j == t) ? -scale : 0.0f;
        dx[i] = acc ? dx[i] + d : d;
    }
}

inline unsigned rows_grid(int rows, int lanes_per_row) {
    return om::grid1d((int64_t)rows * lanes_per_row, kBlock, 1 << 30);
}

}  // namespace

extern "C" {

om_status om_layernorm_fwd(om_ctx *ctx, const float *x, const float *gamma, const float *beta, float *y, float *mean,
                           float *rstd, int rows, int cols, float eps) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && gamma && beta && y && rows >= 0 && cols > 0, "om_layernorm_fwd: bad arguments");
    if (rows == 0) return OM_OK;
    const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0);
    if (cols == 384 || cols == 768) {
        if (cols == 384)
            hipLaunchKernelGGL(k_ln_fwd_w<384>, dim3(rows_grid(rows, 16)), dim3(kBlock), 0, ctx->stream, x, gamma,
                               beta, y, mean, rstd, rows, eps);
        else
            hipLaunchKernelGGL(k_ln_fwd_w<768>, dim3(rows_grid(rows, 16)), dim3(kBlock), 0, ctx->stream, x, gamma,
                               beta, y, mean, rstd, rows, eps);
    } else if (cols % 4 == 0 && cols <= kLnLdsMaxCols && aligned) {
        // Four rows per 64-thread block: many small blocks keep several in flight per CU.
        const size_t lds = (size_t)4 * (cols + 16) * sizeof(float);
        hipLaunchKernelGGL(k_ln_fwd_lds<64>, dim3((rows + 3) / 4), dim3(64), lds, ctx->stream, x, gamma, beta, y,
                           mean, rstd, rows, cols, eps);
    } else {
        hipLaunchKernelGGL(k_ln_fwd, dim3(rows_grid(rows, 16)), dim3(kBlock), 0, ctx->stream, x, gamma, beta, y,
                           mean, rstd, rows, cols, eps);
    }
    return OM_LAUNCH_CHECK(ctx, "om_layernorm_fwd");
}

}  // extern "C"

// dx = dxin + v when dxin is given (dxin == dx for accumulation), else dx = v.
// Rows per chunk of the fp64 column partials: 16 for the fixed widths (256 chunks at 4096 rows), else 8.
static int ln_rows_per_chunk(int cols) { return cols == 384 || cols == 768 ? 16 : 8; }

// The backward's main launch(es): dx (dx = dxin + v when dxin is given, dxin == dx to accumulate) and the per-chunk
// partials pg / pb of dgamma / dbeta (either may be NULL).
static om_status ln_bwd_main(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                             const float *rstd, float *dx, const float *dxin, double *pg, double *pb, int rows,
                             int cols) {
    const bool wide_fixed = cols == 384 || cols == 768;
    const int rpc = ln_rows_per_chunk(cols);
    const int chunks = (rows + rpc - 1) / rpc;
    const bool params = pg || pb;
    if (wide_fixed) {
        // 16 wavefronts of one row each per block: every row's loads are in flight at once, and the block's 16
        // rows share one set of fp64 column partials.
        if (cols == 384)
            hipLaunchKernelGGL((k_ln_bwd_w<384, 1, 16>), dim3(chunks), dim3(1024), 0, ctx->stream, g, x, gamma, mean,
                               rstd, dx, dxin, pg, pb, rows);
        else
            hipLaunchKernelGGL((k_ln_bwd_w<768, 1, 16>), dim3(chunks), dim3(1024), 0, ctx->stream, g, x, gamma, mean,
                               rstd, dx, dxin, pg, pb, rows);
    } else if (cols <= 64 * kMaxPer) {
        const int per = (cols + 63) / 64;
#define OM_LNB(P)                                                                                                   \
    hipLaunchKernelGGL(k_ln_bwd<P>, dim3(chunks), dim3(kBlock), 0, ctx->stream, g, x, gamma, mean, rstd, dx, dxin, pg, \
                       pb, rows, cols, rpc)
        if (per <= 2) OM_LNB(2);
        else if (per <= 4) OM_LNB(4);
        else if (per <= 6) OM_LNB(6);
        else if (per <= 8) OM_LNB(8);
        else if (per <= 12) OM_LNB(12);
        else OM_LNB(16);
#undef OM_LNB
    } else {
        if (dx)
            hipLaunchKernelGGL(k_ln_bwd_dx_wide, dim3(rows_grid(rows, 64)), dim3(kBlock), 0, ctx->stream, g, x, gamma,
                               mean, rstd, dx, dxin, rows, cols);
        if (params)
            hipLaunchKernelGGL(k_ln_param_partial_wide, dim3((cols + kBlock - 1) / kBlock, chunks), dim3(kBlock), 0,
                               ctx->stream, g, x, mean, rstd, pg, pb, rows, cols, rpc);
    }
    return OM_LAUNCH_CHECK(ctx, "om_layernorm_bwd");
}

// Fixed device scratch for om_layernorm_bwd_noalloc's fp64 dgamma / dbeta partials (2 * chunks * cols doubles):
// OM_NOALLOC_SLOTS slots of OM_NOALLOC_SCRATCH_BYTES, one copy per GPU for the life of the process. Each live
// context that calls the entry point holds a slot of its own, so calls from contexts on other streams or threads of
// one GPU never share memory. Host code never passes this name to a kernel: it is a host-side stand-in; kernels get
// the device address that noalloc_init looks up per device.
static __device__ __align__(256) unsigned char ln_scratch[(size_t)OM_NOALLOC_SLOTS * OM_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_ln_scratch_mu;
void *g_ln_scratch_at[kMaxDevices];     // per device: ln_scratch's device address, once looked up
unsigned g_ln_slots_held[kMaxDevices];  // per device: bit i set while a live context holds slot i
static_assert(OM_NOALLOC_SLOTS <= 32, "the slot mask is 32 bits");
}  // namespace

om_status om::noalloc_init(om_ctx *ctx) {
    ctx->noalloc_scratch = nullptr;
    ctx->noalloc_slot = -1;
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return om::fail(ctx, OM_E_DEVICE, "allocation-free scratch: device %d is beyond %d", ctx->device, kMaxDevices);
    std::lock_guard<std::mutex> g(g_ln_scratch_mu);
    if (!g_ln_scratch_at[ctx->device]) {
        void *p = nullptr;  // ctx->device is current (om_ctx_create set it)
        om_status s = om::check_hip(ctx, hipGetSymbolAddress(&p, HIP_SYMBOL(ln_scratch)), "hipGetSymbolAddress");
        if (s) return s;
        g_ln_scratch_at[ctx->device] = p;
    }
    ctx->noalloc_scratch = g_ln_scratch_at[ctx->device];
    return OM_OK;
}

om_status om::noalloc_slot(om_ctx *ctx, double **out) {
    if (!ctx->noalloc_scratch)
        return om::fail(ctx, OM_E_STATE, "om_layernorm_bwd_noalloc: the fixed scratch has no device address here");
    if (ctx->noalloc_slot < 0) {
        std::lock_guard<std::mutex> g(g_ln_scratch_mu);
        unsigned &held = g_ln_slots_held[ctx->device];
        for (int i = 0; i < OM_NOALLOC_SLOTS && ctx->noalloc_slot < 0; i++)
            if (!(held & (1u << i))) {
                held |= 1u << i;
                ctx->noalloc_slot = i;
            }
        if (ctx->noalloc_slot < 0)
            return om::fail(ctx, OM_E_STATE,
                            "om_layernorm_bwd_noalloc: all %d slots of the fixed scratch on device %d are held by "
                            "other live contexts",
                            OM_NOALLOC_SLOTS, ctx->device);
    }
    *out = reinterpret_cast<double *>(static_cast<unsigned char *>(ctx->noalloc_scratch) +
                                      (size_t)ctx->noalloc_slot * OM_NOALLOC_SCRATCH_BYTES);
    return OM_OK;
}

void om::noalloc_release(om_ctx *ctx) {
    if (ctx->noalloc_slot < 0 || ctx->device < 0 || ctx->device >= kMaxDevices) return;
    std::lock_guard<std::mutex> g(g_ln_scratch_mu);
    g_ln_slots_held[ctx->device] &= ~(1u << ctx->noalloc_slot);
    ctx->noalloc_slot = -1;
}

// fixed: the partials' device memory when the caller provides it (the allocation-free entry point), else NULL and
// the context's scratch is used.
static om_status ln_bwd(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                        const float *rstd, float *dx, const float *dxin, float *dgamma, float *dbeta, int rows,
                        int cols, int acc_params, double *fixed = nullptr) {
    const int rpc = ln_rows_per_chunk(cols);
    const int chunks = (rows + rpc - 1) / rpc;
    double *pg = nullptr, *pb = nullptr;
    if (dgamma || dbeta) {
        double *base = fixed;
        if (!base) {
            float *scr;
            om_status s = om::scratch(ctx, sizeof(double) * 2ull * chunks * cols, &scr);
            if (s) return s;
            base = reinterpret_cast<double *>(scr);
        }
        pg = dgamma ? base : nullptr;
        pb = dbeta ? base + (size_t)chunks * cols : nullptr;
    }
    om_status s = ln_bwd_main(ctx, g, x, gamma, mean, rstd, dx, dxin, pg, pb, rows, cols);
    if (s) return s;
    if (dgamma && dbeta) return om::chunk_final(ctx, pg, chunks, cols, dgamma, acc_params, pb, dbeta);
    if (dgamma) return om::chunk_final(ctx, pg, chunks, cols, dgamma, acc_params);
    if (dbeta) return om::chunk_final(ctx, pb, chunks, cols, dbeta, acc_params);
    return OM_OK;
}

extern "C" {

om_status om_layernorm_bwd(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                           const float *rstd, float *dx, float *dgamma, float *dbeta, int rows, int cols, int acc_dx,
                           int acc_params) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && x && gamma && mean && rstd && rows > 0 && cols > 0, "om_layernorm_bwd: bad arguments");
    return ln_bwd(ctx, g, x, gamma, mean, rstd, dx, acc_dx && dx ? dx : nullptr, dgamma, dbeta, rows, cols, acc_params);
}

om_status om_layernorm_bwd_noalloc(om_ctx *ctx, const float *g, const float *x, const float *gamma,
                                   const float *mean, const float *rstd, float *dx, float *dgamma, float *dbeta,
                                   int rows, int cols, int acc_dx, int acc_params) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && x && gamma && mean && rstd && rows > 0 && cols > 0,
               "om_layernorm_bwd_noalloc: bad arguments");
    const int rpc = ln_rows_per_chunk(cols);
    const uint64_t chunks = ((uint64_t)rows + rpc - 1) / rpc;
    const uint64_t need = (dgamma || dbeta) ? sizeof(double) * 2ull * chunks * (uint64_t)cols : 0;
    OM_REQUIRE(ctx, need <= (uint64_t)OM_NOALLOC_SCRATCH_BYTES,
               "om_layernorm_bwd_noalloc: %d x %d needs %llu bytes of dgamma/dbeta partials, more than the %llu of "
               "its fixed scratch",
               rows, cols, (unsigned long long)need, (unsigned long long)OM_NOALLOC_SCRATCH_BYTES);
    double *slot = nullptr;
    if (need) {
        om_status s = om::noalloc_slot(ctx, &slot);
        if (s) return s;
    }
    return ln_bwd(ctx, g, x, gamma, mean, rstd, dx, acc_dx && dx ? dx : nullptr, dgamma, dbeta, rows, cols,
                  acc_params, slot);
}

int om_layernorm_bwd_chunks(int rows, int cols) {
    if (rows <= 0 || cols <= 0) return 0;
    const int rpc = ln_rows_per_chunk(cols);
    return (rows + rpc - 1) / rpc;
}

om_status om_layernorm_bwd_partials(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                                    const float *rstd, const float *dx_add, float *dx, int acc_dx, double *part_g,
                                    double *part_b, int rows, int cols) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && x && gamma && mean && rstd && rows > 0 && cols > 0 && (!dx_add || dx),
               "om_layernorm_bwd_partials: bad arguments");
    return ln_bwd_main(ctx, g, x, gamma, mean, rstd, dx, dx_add ? dx_add : (acc_dx && dx ? dx : nullptr), part_g, part_b,
                       rows, cols);
}

om_status om_layernorm_bwd_add(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                               const float *rstd, const float *dx_add, float *dx, float *dgamma, float *dbeta, int rows,
                               int cols, int acc_params) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && x && gamma && mean && rstd && dx_add && dx && rows > 0 && cols > 0,
               "om_layernorm_bwd_add: bad arguments");
    return ln_bwd(ctx, g, x, gamma, mean, rstd, dx, dx_add, dgamma, dbeta, rows, cols, acc_params);
}

om_status om_softmax_fwd(om_ctx *ctx, const float *x, float *y, int rows, int cols) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && y && rows >= 0 && cols > 0, "om_softmax_fwd: bad arguments");
    if (rows == 0) return OM_OK;
    hipLaunchKernelGGL(k_softmax_rows, dim3(rows_grid(rows, 16)), dim3(kBlock), 0, ctx->stream, x, y, rows, cols);
    return OM_LAUNCH_CHECK(ctx, "om_softmax_fwd");
}

om_status om_softmax_bwd(om_ctx *ctx, const float *g, const float *y, float *dx, int rows, int cols, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && y && dx && rows >= 0 && cols > 0, "om_softmax_bwd: bad arguments");
    if (rows == 0) return OM_OK;
    hipLaunchKernelGGL(k_softmax_bwd_rows, dim3(rows_grid(rows, 64)), dim3(kBlock), 0, ctx->stream, g, y, dx, rows,
                       cols, 1.0f, 0, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_softmax_bwd");
}

om_status om_logsoftmax_fwd(om_ctx *ctx, const float *x, float *y, int rows, int cols) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && y && rows >= 0 && cols > 0, "om_logsoftmax_fwd: bad arguments");
    if (rows == 0) return OM_OK;
    hipLaunchKernelGGL(k_logsoftmax_rows, dim3(rows_grid(rows, 64)), dim3(kBlock), 0, ctx->stream, x, y, rows, cols);
    return OM_LAUNCH_CHECK(ctx, "om_logsoftmax_fwd");
}

om_status om_logsoftmax_bwd(om_ctx *ctx, const float *g, const float *y, float *dx, int rows, int cols,
                            int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && y && dx && rows >= 0 && cols > 0, "om_logsoftmax_bwd: bad arguments");
    if (rows == 0) return OM_OK;
    hipLaunchKernelGGL(k_logsoftmax_bwd_rows, dim3(rows_grid(rows, 64)), dim3(kBlock), 0, ctx->stream, g, y, dx, rows,
                       cols, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_logsoftmax_bwd");
}

om_status om_nll_fwd(om_ctx *ctx, const float *logp, const int32_t *target, float *loss, int32_t *bad_row, int rows,
                     int cols, int mean, int ignore_index) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, logp && target && loss && rows >= 0 && cols > 0, "om_nll_fwd: bad arguments");
    hipLaunchKernelGGL(k_nll_fwd, dim3(1), dim3(kBlock), 0, ctx->stream, logp, target, loss, bad_row, rows, cols, mean,
                       ignore_index, LossPost{nullptr, nullptr, 0, nullptr});
    return OM_LAUNCH_CHECK(ctx, "om_nll_fwd");
}

om_status om_xent_fwd_unit(om_ctx *ctx, const float *logits, const int32_t *target, float *logp, float *loss,
                           int32_t *bad_row, float *dlogits_unit, int rows, int cols, int ignore_index,
                           om_readback *rb) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, logits && target && logp && loss && dlogits_unit && rows >= 0 && cols > 0,
               "om_xent_fwd_unit: bad arguments");
    LossPost post{nullptr, nullptr, 0, nullptr};
    if (rb) {
        om_status s = om::readback_target(ctx, rb, sizeof(float), &post.dst, &post.seq_at, &post.seq, &post.seq_dev);
        if (s) return s;
    }
    if (rows > 0)
        hipLaunchKernelGGL(k_xent_fwd_rows, dim3(rows_grid(rows, 64)), dim3(kBlock), 0, ctx->stream, logits, target,
                           logp, dlogits_unit, rows, cols, ignore_index);
    hipLaunchKernelGGL(k_nll_fwd, dim3(1), dim3(kBlock), 0, ctx->stream, logp, target, loss, bad_row, rows, cols, 1,
                       ignore_index, post);
    om_status s = OM_LAUNCH_CHECK(ctx, "om_xent_fwd_unit");
    if (s == OM_OK && rb) om::readback_posted(rb, post.seq, sizeof(float));
    return s;
}

om_status om_nll_bwd(om_ctx *ctx, const float *g_scalar, const int32_t *target, float *dlogp, int rows, int cols,
                     int mean, int ignore_index, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g_scalar && target && dlogp && rows >= 0 && cols > 0, "om_nll_bwd: bad arguments");
    if (rows == 0) return OM_OK;
    float *scr;
    om_status s = om::scratch(ctx, 256, &scr);
    if (s) return s;
    int *count = reinterpret_cast<int *>(scr);
    hipLaunchKernelGGL(k_xent_count, dim3(1), dim3(kBlock), 0, ctx->stream, target, rows, ignore_index, count);
    hipLaunchKernelGGL(k_nll_bwd, dim3(om::grid1d((int64_t)rows * cols, kBlock, 4096)), dim3(kBlock), 0, ctx->stream,
                       g_scalar, count, target, dlogp, rows, cols, mean, ignore_index, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_nll_bwd");
}

om_status om_xent_bwd(om_ctx *ctx, const float *g_scalar, const float *logp, const int32_t *target, float *dlogits,
                      int rows, int cols, int mean, int ignore_index, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g_scalar && logp && target && dlogits && rows >= 0 && cols > 0, "om_xent_bwd: bad arguments");
    if (rows == 0) return OM_OK;
    float *scr;
    om_status s = om::scratch(ctx, 256, &scr);
    if (s) return s;
    int *count = reinterpret_cast<int *>(scr);
    hipLaunchKernelGGL(k_xent_count, dim3(1), dim3(kBlock), 0, ctx->stream, target, rows, ignore_index, count);
    hipLaunchKernelGGL(k_xent_bwd, dim3(rows_grid(rows, 64)), dim3(kBlock), 0, ctx->stream, g_scalar, count, logp,
                       target, dlogits, rows, cols, mean, ignore_index, accumulate);
    return OM_LAUNCH_CHECK(ctx, "om_xent_bwd");
}

}  // extern "C"

// Used by the attention backward (om_attention.hip): ds = (p * (dp - rowsum(dp*p))) * scale, in place on dp.
om_status om_internal_attn_ds(om_ctx *ctx, float *dp, const float *p, int rows, int cols, float scale) {
    hipLaunchKernelGGL(k_softmax_bwd_rows, dim3(rows_grid(rows, 64)), dim3(kBlock), 0, ctx->stream, dp, p, dp, rows,
                       cols, scale, 1, 0);
    return OM_LAUNCH_CHECK(ctx, "attention ds");
}
om_status om_internal_softmax_rows(om_ctx *ctx, float *x, int rows, int cols) {
    hipLaunchKernelGGL(k_softmax_rows, dim3(rows_grid(rows, 16)), dim3(kBlock), 0, ctx->stream, x, x, rows, cols);
    return OM_LAUNCH_CHECK(ctx, "attention softmax");
}
