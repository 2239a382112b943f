/*
 * om_oracle.c — TEST INFRASTRUCTURE ONLY. A plain-C, CPU restatement of the reference's training path
 * (recursive-ai-oss/onemodel-csharp, RecursiveAI.OneModel.Training + the tensor-layer backward rules), used as the
 * parity checker for the HIP library. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it;
 * nothing in the product links, calls or falls back to it.
 *
 * Each function cites the reference file:line it restates. Conventions (all from the reference):
 *   - fp32 row-major contiguous tensors; "fp64 sum" means a double accumulator in increasing element order,
 *     rounded to float once (BackwardOps.cs:196-269, BackwardNn.cs:225-242).
 *   - GEMM in the reference's fast mode: one accumulator per output, increasing k, from +0, fused multiply-add
 *     (docs/kernels-gemm.md:73-85; Gemm.cs:48). Transposed operands read through strides; the reference copies them to
 *     row-major scratch first (Dense.cs:12-49), which does not change the arithmetic.
 *   - Transcendentals the reference fixes in both modes (GELU erf form, exp/expNonPositive/log polynomials) are the
 *     reference's own published polynomials (Transcendental.cs:39-263, docs/exact-transcendentals.md) evaluated with
 *     separate IEEE roundings (no contraction: this file is built with -ffp-contract=off and calls fmaf() only where
 *     the reference's fast mode fuses). MathF.Exp/Log in fast-mode LogSoftmax are libm expf/logf here.
 *   - CTC uses the reference's double exp/ln/logadd (Ctc.cs:515-616, docs/ctc.md:53-74).
 *
 * Parallelism: OpenMP over independent outputs only; every output is computed by one thread with the whole of its
 * reduction in one order, so results do not depend on the thread count (docs/kernels-gemm.md:56-71).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

static inline float bits_f(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }
static inline float canon(float x) { return x == x ? x : bits_f(0x7FC00000u); }

/* ------------------------------------------------------------------------------------------------ generator */
/* SplitMix64 (Steele, Lea, Flood 2014) as Generator.cs:26-47: state += golden gamma, then the Mix scramble. */
EXPORT uint64_t or_splitmix_next(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
/* Generator.NextSingle (Generator.cs:33): 24 random bits times 2^-24. */
EXPORT float or_next_single(uint64_t *state) { return (float)(or_splitmix_next(state) >> 40) * (1.0f / 16777216.0f); }
/* Init.Uniform (Layers.cs:11-21) with Generator.Uniform (Generator.cs:38): low + (high-low)*u, row-major order. */
EXPORT void or_fill_uniform(uint64_t *state, float low, float high, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = low + (high - low) * or_next_single(state);
}
/* Synthetic N(0,1) inputs (the benchmark's own generator, not a reference function): Box-Muller in double on two
 * 53-bit uniforms from the same SplitMix64 stream, cosine branch only, rounded to float. */
EXPORT void or_fill_normal(uint64_t *state, float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        double u1 = ((double)(or_splitmix_next(state) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(or_splitmix_next(state) >> 11) * (1.0 / 9007199254740992.0);
        dst[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
}
/* Uniform integers in [lo, hi) from the same stream: lo + (u64 % span). */
EXPORT void or_fill_int(uint64_t *state, int32_t lo, int32_t hi, int32_t *dst, int64_t n) {
    uint64_t span = (uint64_t)(hi - lo);
    for (int64_t i = 0; i < n; i++) dst[i] = lo + (int32_t)(or_splitmix_next(state) % span);
}

/* ------------------------------------------------------------------------------------------------ fp32 polynomials */
#define ROUND_MAGIC 12582912.0f
/* Transcendental.Exp (Transcendental.cs:39-70): Cody-Waite reduction, degree-4 Q, two-step 2^n scaling. */
EXPORT float or_exp(float x) {
    float t = x * 1.44269502f + ROUND_MAGIC;
    float nf = t - ROUND_MAGIC;
    float r = (x - nf * 0.693145751953125f) - nf * 1.4286068e-6f;
    float q = 0.0013814613f;
    q = 0.00836871f + q * r;
    q = 0.04166839f + q * r;
    q = 0.16666521f + q * r;
    q = 0.49999994f + q * r;
    float p = 1.0f + (r + (r * r) * q);
    int32_t n = (int32_t)f_bits(t) - (int32_t)f_bits(ROUND_MAGIC);
    int32_t a = n >> 1, b = n - a;
    float pa = bits_f((uint32_t)((a + 127) << 23)), pb = bits_f((uint32_t)((b + 127) << 23));
    float res = (p * pa) * pb;
    if (x > 88.72283172607422f) res = INFINITY;
    if (x < -103.97207641601562f) res = 0.0f;
    return canon(x == x ? res : x);
}
/* Transcendental.ExpNonPositive (Transcendental.cs:77-97). */
EXPORT float or_exp_nonpos(float x) {
    float t = x * 1.44269502f + ROUND_MAGIC;
    float nf = t - ROUND_MAGIC;
    float r = (x - nf * 0.693145751953125f) - nf * 1.4286068e-6f;
    float q = 0.0013814613f;
    q = 0.00836871f + q * r;
    q = 0.04166839f + q * r;
    q = 0.16666521f + q * r;
    q = 0.49999994f + q * r;
    float p = 1.0f + (r + (r * r) * q);
    int32_t n = (int32_t)f_bits(t) - (int32_t)f_bits(ROUND_MAGIC);
    float res = p * bits_f((uint32_t)((n + 127) << 23));
    if (x < -87.33654f) res = 0.0f;
    return x == x ? res : bits_f(0x7FC00000u);
}
/* Transcendental.ErfParts (Transcendental.cs:167-233): erf and 1+erf. */
static void erf_parts(float x, float *erf, float *ope) {
    uint32_t sign = f_bits(x) & 0x80000000u;
    float ax = bits_f(f_bits(x) & 0x7FFFFFFFu);
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
    static const float G[17] = {-0.00057763467f, 0.0017893383f, -0.00010074016f, -0.004373198f, 0.0034639547f,
                                0.0015023724f, -0.0009413088f, -0.0018891813f, -0.0002586738f, 0.0052144383f,
                                -0.0103428485f, 0.015788378f, -0.018338649f, 0.008167262f, 0.035529688f,
                                -0.1543716f, 0.42758358f};
    float g = G[0];
    for (int i = 1; i < 17; i++) g = G[i] + g * s;
    float split = ax * 4097.0f;
    float axHi = split - (split - ax);
    float axLo = ax - axHi;
    float zLo = ((axHi * axHi - z) + 2.0f * (axHi * axLo)) + axLo * axLo;
    if (!(ax < 64.0f)) zLo = 0.0f;
    float expNegZ = or_exp(0.0f - z) * (1.0f - zLo);
    float erfc = expNegZ * (t * g);
    int isSmall = ax < 0.5f;
    float erfAbs = isSmall ? small : 1.0f - erfc;
    float erfSigned = bits_f(f_bits(erfAbs) | sign);
    float opeLarge = x < 0.0f ? erfc : 2.0f - erfc;
    float opeSmall = 1.0f + bits_f(f_bits(small) | sign);
    int ok = x == x;
    *erf = canon(ok ? erfSigned : x);
    *ope = canon(ok ? (isSmall ? opeSmall : opeLarge) : x);
}
EXPORT float or_erf(float x) { float e, o; erf_parts(x, &e, &o); return e; }
/* Transcendental.GeluErf (Transcendental.cs:252-263): 0.5*x*(1+erf(x*0.70710677)). */
EXPORT float or_gelu(float x) {
    float e, ope;
    erf_parts(x * 0.70710677f, &e, &ope);
    float res = (0.5f * x) * ope;
    if (x == -INFINITY) res = -0.0f;
    return canon(x == x ? res : x);
}
/* GeluGradBin erf branch (TrainElementwise.cs:59-85): slope = 0.5(1+erf(x/sqrt2)) + x*exp(-0.5x^2)*0.3989423. */
static inline float gelu_slope(float v) {
    float cdf = 0.5f * (1.0f + or_erf(v * 0.70710677f));
    float pdf = or_exp((-0.5f * v) * v) * 0.3989423f;
    return cdf + v * pdf;
}

/* RowReduce.Sum16 (Softmax.cs:139-179): 16 partials, element j into partial j%16, halving combine. */
static float sum16(const float *x, int n) {
    float part[16] = {0};
    for (int j = 0; j < n; j++) part[j & 15] += x[j];
    float a[8], b[4];
    for (int t = 0; t < 8; t++) a[t] = part[t] + part[t + 8];
    for (int t = 0; t < 4; t++) b[t] = a[t] + a[t + 4];
    float c0 = b[0] + b[2], c1 = b[1] + b[3];
    return c0 + c1;
}
/* NormKernels.SumSquaredDeviations (NormKernels.cs:130-156): Sum16 order over (x-mean)^2. */
static float ssd16(const float *x, int n, float mean) {
    float part[16] = {0};
    for (int j = 0; j < n; j++) { float d = x[j] - mean; part[j & 15] += d * d; }
    float a[8], b[4];
    for (int t = 0; t < 8; t++) a[t] = part[t] + part[t + 8];
    for (int t = 0; t < 4; t++) b[t] = a[t] + a[t + 4];
    float c0 = b[0] + b[2], c1 = b[1] + b[3];
    return c0 + c1;
}

/* ------------------------------------------------------------------------------------------------ GEMM */
/* C[m,n] (+)= op(A)[m,k] op(B)[k,n]. Canonical fast-mode order (docs/kernels-gemm.md:73-85): acc from +0, increasing k,
 * fmaf per product. accumulate=1 adds the finished dot product to C in one rounding (how the conv dW loop adds each
 * image's product, BackwardNn.cs:359-366). */
EXPORT void or_gemm(int transA, int transB, int m, int n, int k, const float *A, int lda, const float *B, int ldb,
                    float *C, int ldc, int accumulate) {
    /* A transposed B is copied to row-major scratch first, as Dense.Gemm does (Dense.cs:34-40). */
    float *bt = NULL;
    if (transB && n > 0 && k > 0) {
        bt = (float *)malloc(sizeof(float) * (size_t)k * n);
        for (int j = 0; j < n; j++)
            for (int p = 0; p < k; p++) bt[(int64_t)p * n + j] = B[(int64_t)j * ldb + p];
        B = bt;
        ldb = n;
    }
#pragma omp parallel for schedule(static)
    for (int i = 0; i < m; i++) {
        float *acc = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
        for (int j = 0; j < n; j++) acc[j] = 0.0f;
        for (int p = 0; p < k; p++) {
            float a = transA ? A[(int64_t)p * lda + i] : A[(int64_t)i * lda + p];
            const float *brow = B + (int64_t)p * ldb;
            for (int j = 0; j < n; j++) acc[j] = fmaf(a, brow[j], acc[j]);
        }
        float *crow = C + (int64_t)i * ldc;
        if (accumulate) for (int j = 0; j < n; j++) crow[j] += acc[j];
        else for (int j = 0; j < n; j++) crow[j] = acc[j];
        free(acc);
    }
    free(bt);
}

/* ------------------------------------------------------------------------------------------------ elementwise */
/* Ops.Linear (Ops.Layers.cs:715-733): MatMul(x, W^T) then broadcast Add(bias): y = fl(dot) + b. */
EXPORT void or_linear_fwd(const float *x, const float *w, const float *b, float *y, int rows, int in, int out) {
    or_gemm(0, 1, rows, out, in, x, in, w, in, y, out, 0);
    if (b) {
#pragma omp parallel for schedule(static)
        for (int r = 0; r < rows; r++)
            for (int o = 0; o < out; o++) y[(int64_t)r * out + o] += b[o];
    }
}
/* Linear backward = MatMul backward (BackwardOps.cs:69-82) + Permute backward of W^T (BackwardOps.cs:107-118) + SumTo of
 * the bias (BackwardOps.cs:201-269): dx = g W, dW = g^T x (the same products in the same k order as (x^T g)^T),
 * db = fp64 column sums. Each output is written (not accumulated); the tape adds into existing leaves. */
EXPORT void or_linear_bwd(const float *g, const float *x, const float *w, float *dx, float *dw, float *db, int rows,
                          int in, int out) {
    if (dx) or_gemm(0, 0, rows, in, out, g, out, w, in, dx, in, 0);
    if (dw) or_gemm(1, 0, out, in, rows, g, out, x, in, dw, in, 0);
    if (db) {
        for (int o = 0; o < out; o++) {
            double s = 0.0;
            for (int r = 0; r < rows; r++) s += g[(int64_t)r * out + o];
            db[o] = (float)s;
        }
    }
}
/* ReluUn (TrainElementwise.cs:93-98): x if x>0, NaN kept, else 0. */
EXPORT void or_relu_fwd(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = x[i] > 0.0f ? x[i] : (x[i] == x[i] ? 0.0f : x[i]);
}
/* ReluGradBin (TrainElementwise.cs:41-45): g where y>0 else 0. */
EXPORT void or_relu_bwd(const float *g, const float *y, float *dx, int64_t n) {
    for (int64_t i = 0; i < n; i++) dx[i] = y[i] > 0.0f ? g[i] : 0.0f;
}
/* Ops.Gelu erf form (Ops.Nn.cs:86-112). */
EXPORT void or_gelu_fwd(const float *x, float *y, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) y[i] = or_gelu(x[i]);
}
/* Gelu backward (BackwardNn.cs:12-14, TrainElementwise.cs:59-85): g * slope(x). */
EXPORT void or_gelu_bwd(const float *g, const float *x, float *dx, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) dx[i] = canon(g[i] * gelu_slope(x[i]));
}
/* y = a + b (same shape); Engine.AddInto order (Engine.cs:331-344) is elementwise, so any order is the same. */
EXPORT void or_add(const float *a, const float *b, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = a[i] + b[i];
}

/* ------------------------------------------------------------------------------------------------ reductions */
/* Ops.Sum/Mean over all elements (Ops.Nn.cs:162-231): fp64 sum in element order; mean = (float)(acc/n). */
EXPORT float or_sum_all(const float *x, int64_t n, int mean) {
    double acc = 0.0;
    for (int64_t i = 0; i < n; i++) acc += x[i];
    return mean ? (float)(acc / (double)n) : (float)acc;
}
/* Mean over axis with [outer, n, inner] layout (Ops.Nn.cs:202-216). */
EXPORT void or_mean_axis(const float *x, float *y, int outer, int n, int inner) {
    for (int o = 0; o < outer; o++)
        for (int i = 0; i < inner; i++) {
            double acc = 0.0;
            for (int k = 0; k < n; k++) acc += x[((int64_t)o * n + k) * inner + i];
            y[(int64_t)o * inner + i] = (float)(acc / n);
        }
}
/* ReduceBackward for Mean over an axis (BackwardNn.cs:145-168): broadcast g, then divide by n (float division). */
EXPORT void or_mean_axis_bwd(const float *g, float *dx, int outer, int n, int inner) {
    float fn = (float)n;
    for (int o = 0; o < outer; o++)
        for (int k = 0; k < n; k++)
            for (int i = 0; i < inner; i++) dx[((int64_t)o * n + k) * inner + i] = g[(int64_t)o * inner + i] / fn;
}

/* ------------------------------------------------------------------------------------------------ softmax family */
/* Softmax.Rows exact flavour (Softmax.cs:70-133; docs/kernels-attention.md "Softmax"): max, expNonPositive, Sum16,
 * divide; NaN -> canonical. */
EXPORT void or_softmax_rows(const float *x, float *y, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (int64_t)r * cols;
        float *yr = y + (int64_t)r * cols;
        float mx = -INFINITY;
        for (int j = 0; j < cols; j++) mx = xr[j] > mx ? xr[j] : mx;
        for (int j = 0; j < cols; j++) yr[j] = or_exp_nonpos(xr[j] - mx);
        float l = sum16(yr, cols);
        for (int j = 0; j < cols; j++) yr[j] = canon(yr[j] / l);
    }
}
/* Softmax backward (BackwardNn.cs:26-52): dot in fp64 of fl(g*y); dx = y*(g - (float)dot). */
EXPORT void or_softmax_bwd(const float *g, const float *y, float *dx, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        int64_t o = (int64_t)r * cols;
        double dot = 0.0;
        for (int j = 0; j < cols; j++) dot += (double)(g[o + j] * y[o + j]);
        float df = (float)dot;
        for (int j = 0; j < cols; j++) dx[o + j] = y[o + j] * (g[o + j] - df);
    }
}
/* Ops.LogSoftmax (Ops.Layers.cs:47-96): max; fp64 sum of exp(x-max); lse = max + log((float)sum); y = x - lse. */
EXPORT void or_logsoftmax_fwd(const float *x, float *y, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        const float *s = x + (int64_t)r * cols;
        float *d = y + (int64_t)r * cols;
        float mx = -INFINITY;
        for (int j = 0; j < cols; j++) if (s[j] > mx) mx = s[j];
        double sum = 0.0;
        for (int j = 0; j < cols; j++) sum += expf(s[j] - mx);
        float lse = mx + logf((float)sum);
        for (int j = 0; j < cols; j++) d[j] = s[j] - lse;
    }
}
/* LogSoftmax backward (BackwardNn.cs:54-80): s = (float)fp64 sum of g; dx = g - exp(y)*s. */
EXPORT void or_logsoftmax_bwd(const float *g, const float *y, float *dx, int rows, int cols) {
    for (int r = 0; r < rows; r++) {
        int64_t o = (int64_t)r * cols;
        double sum = 0.0;
        for (int j = 0; j < cols; j++) sum += g[o + j];
        float s = (float)sum;
        for (int j = 0; j < cols; j++) dx[o + j] = g[o + j] - expf(y[o + j]) * s;
    }
}
/* Ops.NllLoss (Ops.Layers.cs:644-699): fp64 sum of -logp[i, t_i] over rows whose target != ignore; mean divides by
 * max(1,count). Returns -1 in *bad_row for a target outside [0, cols). */
EXPORT float or_nll_fwd(const float *logp, const int32_t *target, int rows, int cols, int mean, int ignore,
                        int *bad_row) {
    double sum = 0.0;
    int count = 0;
    *bad_row = -1;
    for (int i = 0; i < rows; i++) {
        int t = target[i];
        if (t == ignore) continue;
        if ((unsigned)t >= (unsigned)cols) { *bad_row = i; return NAN; }
        sum -= logp[(int64_t)i * cols + t];
        count++;
    }
    return (float)(mean ? sum / (count > 1 ? count : 1) : sum);
}
/* NllBackward (BackwardNn.cs:602-632): dx = 0 except dx[i, t_i] = -(g/count or g). */
EXPORT void or_nll_bwd(float g, const int32_t *target, float *dx, int rows, int cols, int mean, int ignore) {
    int count = 0;
    for (int i = 0; i < rows; i++) if (target[i] != ignore) count++;
    float scale = mean ? g / (float)(count > 1 ? count : 1) : g;
    memset(dx, 0, sizeof(float) * (size_t)rows * cols);
    for (int i = 0; i < rows; i++) if (target[i] != ignore) dx[(int64_t)i * cols + target[i]] = -scale;
}

/* ------------------------------------------------------------------------------------------------ normalisation */
/* Ops.LayerNorm -> NormKernels.Rows (NormKernels.cs:79-127): mean = Sum16/n, inv = 1/sqrt(ssd/n + eps),
 * y = (((x-mean)*inv)*gamma)+beta; saves mean and inv per row. */
EXPORT void or_layernorm_fwd(const float *x, const float *gamma, const float *beta, float *y, float *mean_out,
                             float *inv_out, int rows, int cols, float eps) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (int64_t)r * cols;
        float *yr = y + (int64_t)r * cols;
        float n = (float)cols;
        float mean = sum16(xr, cols) / n;
        float ssq = ssd16(xr, cols, mean);
        float inv = 1.0f / sqrtf(ssq / n + eps);
        if (mean_out) mean_out[r] = mean;
        if (inv_out) inv_out[r] = inv;
        for (int j = 0; j < cols; j++) yr[j] = canon(((xr[j] - mean) * inv) * gamma[j] + beta[j]);
    }
}
/* LayerNormBackward (BackwardNn.cs:170-223). dgamma/dbeta are fp64 column sums in row order. */
EXPORT void or_layernorm_bwd(const float *g, const float *x, const float *gamma, const float *mean, const float *inv,
                             float *dx, float *dgamma, float *dbeta, int rows, int cols) {
    double *sg = (double *)calloc((size_t)cols, sizeof(double));
    double *sb = (double *)calloc((size_t)cols, sizeof(double));
    for (int r = 0; r < rows; r++) {
        int64_t o = (int64_t)r * cols;
        float m = mean[r], s = inv[r];
        double sum1 = 0.0, sum2 = 0.0;
        for (int j = 0; j < cols; j++) {
            float xhat = (x[o + j] - m) * s;
            float dxhat = g[o + j] * gamma[j];
            sum1 += dxhat;
            sum2 += (double)(dxhat * xhat);
            sg[j] += (double)(g[o + j] * xhat);
            sb[j] += g[o + j];
        }
        if (dx) {
            float m1 = (float)(sum1 / cols), m2 = (float)(sum2 / cols);
            for (int j = 0; j < cols; j++) {
                float xhat = (x[o + j] - m) * s;
                dx[o + j] = s * ((g[o + j] * gamma[j]) - m1 - (xhat * m2));
            }
        }
    }
    for (int j = 0; j < cols; j++) {
        if (dgamma) dgamma[j] = (float)sg[j];
        if (dbeta) dbeta[j] = (float)sb[j];
    }
    free(sg);
    free(sb);
}
/* Ops.BatchNorm2d training branch (Ops.Layers.cs:185-233): fp64 mean/variance per channel, running-stat update. */
EXPORT void or_batchnorm_fwd(const float *x, const float *gamma, const float *beta, float *rm, float *rv, float *y,
                             float *mean_out, float *inv_out, int n, int c, int plane, float momentum, float eps) {
    double m = (double)n * plane;
    for (int ch = 0; ch < c; ch++) {
        double sum = 0.0;
        for (int i = 0; i < n; i++)
            for (int p = 0; p < plane; p++) sum += x[((int64_t)i * c + ch) * plane + p];
        double mu = sum / m, ss = 0.0;
        for (int i = 0; i < n; i++)
            for (int p = 0; p < plane; p++) { double d = x[((int64_t)i * c + ch) * plane + p] - mu; ss += d * d; }
        double var = ss / m;
        mean_out[ch] = (float)mu;
        inv_out[ch] = 1.0f / sqrtf((float)var + eps);
        double unb = m > 1 ? var * m / (m - 1) : var;
        rm[ch] = (float)((1 - momentum) * rm[ch] + momentum * mu);
        rv[ch] = (float)((1 - momentum) * rv[ch] + momentum * unb);
    }
    for (int i = 0; i < n; i++)
        for (int ch = 0; ch < c; ch++) {
            int64_t o = ((int64_t)i * c + ch) * plane;
            float mm = mean_out[ch], s = inv_out[ch], gg = gamma[ch], bb = beta[ch];
            for (int p = 0; p < plane; p++) y[o + p] = (((x[o + p] - mm) * s) * gg) + bb;
        }
}
/* BatchNormBackward training (BackwardNn.cs:244-307). */
EXPORT void or_batchnorm_bwd(const float *g, const float *x, const float *gamma, const float *mean, const float *inv,
                             float *dx, float *dgamma, float *dbeta, int n, int c, int plane) {
    double m = (double)n * plane;
    double *sg = (double *)calloc((size_t)c, sizeof(double)), *sb = (double *)calloc((size_t)c, sizeof(double));
    for (int i = 0; i < n; i++)
        for (int ch = 0; ch < c; ch++) {
            int64_t o = ((int64_t)i * c + ch) * plane;
            float mm = mean[ch], s = inv[ch];
            double a = 0, b = 0;
            for (int p = 0; p < plane; p++) { float gg = g[o + p]; a += (double)(gg * ((x[o + p] - mm) * s)); b += gg; }
            sg[ch] += a;
            sb[ch] += b;
        }
    if (dx)
        for (int i = 0; i < n; i++)
            for (int ch = 0; ch < c; ch++) {
                int64_t o = ((int64_t)i * c + ch) * plane;
                float mm = mean[ch], s = inv[ch], k = gamma[ch] * s;
                float cb = (float)(sb[ch] / m), cg = (float)(sg[ch] / m);
                for (int p = 0; p < plane; p++) dx[o + p] = k * (g[o + p] - cb - (((x[o + p] - mm) * s) * cg));
            }
    for (int ch = 0; ch < c; ch++) { dgamma[ch] = (float)sg[ch]; dbeta[ch] = (float)sb[ch]; }
    free(sg);
    free(sb);
}

/* ------------------------------------------------------------------------------------------------ attention */
/* Mask row offset for a mask of shape [Lq,Lk] (batch-broadcast) or [B,Lq,Lk] (BackwardNn.cs:715-717). */
static inline const float *mask_row(const float *mask, int mask_batched, int b, int i, int lq, int lk) {
    return mask ? mask + (mask_batched ? (int64_t)b * lq * lk : 0) + (int64_t)i * lk : NULL;
}
/* Ops.Attention forward, the exact definition of docs/kernels-attention.md:10-33 (online softmax over 64-key blocks,
 * separate roundings, expNonPositive, Sum16 block sums, out = acc/l). q [B,H,Lq,D], k/v [B,H,Lk,D]. */
EXPORT void or_attention_fwd(const float *q, const float *k, const float *v, const float *mask, int mask_batched,
                             float *out, int B, int H, int lq, int lk, int d, float scale) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; b++)
        for (int h = 0; h < H; h++) {
            const float *qh = q + ((int64_t)b * H + h) * lq * d;
            const float *kh = k + ((int64_t)b * H + h) * lk * d;
            const float *vh = v + ((int64_t)b * H + h) * lk * d;
            float *oh = out + ((int64_t)b * H + h) * lq * d;
            float *acc = (float *)malloc(sizeof(float) * (size_t)d);
            float s[64], p[64];
            for (int i = 0; i < lq; i++) {
                const float *mr = mask_row(mask, mask_batched, b, i, lq, lk);
                float m = -INFINITY, l = 0.0f;
                for (int x = 0; x < d; x++) acc[x] = 0.0f;
                for (int kb = 0; kb < lk; kb += 64) {
                    int nb = lk - kb < 64 ? lk - kb : 64;
                    float bm = -INFINITY;
                    for (int j = 0; j < nb; j++) {
                        float dot = 0.0f;
                        for (int x = 0; x < d; x++) dot = dot + qh[(int64_t)i * d + x] * kh[(int64_t)(kb + j) * d + x];
                        s[j] = (mr ? mr[kb + j] : 0.0f) + dot * scale;
                        if (s[j] > bm) bm = s[j];
                    }
                    float mNew = m > bm ? m : bm;
                    float shift = mNew == -INFINITY ? 0.0f : mNew;
                    for (int j = 0; j < nb; j++) p[j] = or_exp_nonpos(s[j] - shift);
                    float bs = sum16(p, nb);
                    float alpha = m == -INFINITY ? 0.0f : (m == shift ? 1.0f : or_exp_nonpos(m - shift));
                    l = l * alpha + bs;
                    if (alpha != 1.0f) for (int x = 0; x < d; x++) acc[x] = acc[x] * alpha;
                    m = mNew;
                    for (int j = 0; j < nb; j++)
                        for (int x = 0; x < d; x++) acc[x] = acc[x] + p[j] * vh[(int64_t)(kb + j) * d + x];
                }
                for (int x = 0; x < d; x++) oh[(int64_t)i * d + x] = canon(acc[x] / l);
            }
            free(acc);
        }
}
/* AttentionBackward (BackwardNn.cs:636-701): per (b,h) recompute S = QK^T*scale + mask, P = softmax rows,
 * dV = P^T dO, dP = dO V^T, dS = P(dP - (float)fp64 rowsum(dP*P))*scale, dQ = dS K, dK = dS^T Q. */
EXPORT void or_attention_bwd(const float *q, const float *k, const float *v, const float *mask, int mask_batched,
                             const float *g, float *dq, float *dk, float *dv, int B, int H, int lq, int lk, int d,
                             float scale) {
    float *sv = (float *)malloc(sizeof(float) * (size_t)lq * lk);
    float *pv = (float *)malloc(sizeof(float) * (size_t)lq * lk);
    float *dpv = (float *)malloc(sizeof(float) * (size_t)lq * lk);
    for (int b = 0; b < B; b++)
        for (int h = 0; h < H; h++) {
            int64_t qo = ((int64_t)b * H + h) * lq * d, ko = ((int64_t)b * H + h) * lk * d;
            or_gemm(0, 1, lq, lk, d, q + qo, d, k + ko, d, sv, lk, 0);
            for (int i = 0; i < lq; i++) {
                const float *mr = mask_row(mask, mask_batched, b, i, lq, lk);
                for (int j = 0; j < lk; j++) sv[(int64_t)i * lk + j] = sv[(int64_t)i * lk + j] * scale + (mr ? mr[j] : 0.0f);
            }
            or_softmax_rows(sv, pv, lq, lk);
            or_gemm(1, 0, lk, d, lq, pv, lk, g + qo, d, dv + ko, d, 0);
            or_gemm(0, 1, lq, lk, d, g + qo, d, v + ko, d, dpv, lk, 0);
            for (int i = 0; i < lq; i++) {
                int64_t o = (int64_t)i * lk;
                double dot = 0.0;
                for (int j = 0; j < lk; j++) dot += (double)(dpv[o + j] * pv[o + j]);
                float df = (float)dot;
                for (int j = 0; j < lk; j++) dpv[o + j] = (pv[o + j] * (dpv[o + j] - df)) * scale;
            }
            or_gemm(0, 0, lq, d, lk, dpv, lk, k + ko, d, dq + qo, d, 0);
            or_gemm(1, 0, lk, d, lq, dpv, lk, q + qo, d, dk + ko, d, 0);
        }
    free(sv);
    free(pv);
    free(dpv);
}

/* ------------------------------------------------------------------------------------------------ convolution */
typedef struct { int N, Cin, H, W, Cout, KH, KW, stride, pad, OH, OW; } conv_shape;
static conv_shape mk_conv(int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad) {
    conv_shape s = {N, Cin, H, W, Cout, KH, KW, stride, pad, (H + 2 * pad - KH) / stride + 1, (W + 2 * pad - KW) / stride + 1};
    return s;
}
/* Im2ColPatchMajor (BackwardNn.cs:404-428): cols[p, (c*KH+ky)*KW+kx], zero outside the image. */
static void im2col(const conv_shape *s, const float *x, float *cols) {
    int kk = s->Cin * s->KH * s->KW;
    for (int oy = 0; oy < s->OH; oy++)
        for (int ox = 0; ox < s->OW; ox++) {
            float *row = cols + ((int64_t)oy * s->OW + ox) * kk;
            int kq = 0;
            for (int c = 0; c < s->Cin; c++)
                for (int ky = 0; ky < s->KH; ky++) {
                    int iy = oy * s->stride - s->pad + ky;
                    for (int kx = 0; kx < s->KW; kx++, kq++) {
                        int ix = ox * s->stride - s->pad + kx;
                        row[kq] = ((unsigned)iy < (unsigned)s->H && (unsigned)ix < (unsigned)s->W)
                                      ? x[((int64_t)c * s->H + iy) * s->W + ix] : 0.0f;
                    }
                }
        }
}
/* Col2Im (BackwardNn.cs:430-462): dx[c,iy,ix] += dcols[k, p], taps in increasing (k, p) order. */
static void col2im(const conv_shape *s, const float *dcols, float *dx) {
    int plane = s->OH * s->OW, kq = 0;
    for (int c = 0; c < s->Cin; c++)
        for (int ky = 0; ky < s->KH; ky++)
            for (int kx = 0; kx < s->KW; kx++, kq++) {
                const float *row = dcols + (int64_t)kq * plane;
                for (int oy = 0; oy < s->OH; oy++) {
                    int iy = oy * s->stride - s->pad + ky;
                    if ((unsigned)iy >= (unsigned)s->H) continue;
                    for (int ox = 0; ox < s->OW; ox++) {
                        int ix = ox * s->stride - s->pad + kx;
                        if ((unsigned)ix < (unsigned)s->W) dx[((int64_t)c * s->H + iy) * s->W + ix] += row[oy * s->OW + ox];
                    }
                }
            }
}
/* Ops.Conv2d on the im2col path (docs/kernels-gemm.md "Convolution"; Conv.cs:54): per image
 * out[co, p] = sum_k W[co,k] cols[p,k] (canonical GEMM), then the bias is added (Conv.AddChannelBias, Conv.cs:311). */
EXPORT void or_conv2d_fwd(const float *x, const float *w, const float *bias, float *y, int N, int Cin, int H, int W,
                          int Cout, int KH, int KW, int stride, int pad) {
    conv_shape s = mk_conv(N, Cin, H, W, Cout, KH, KW, stride, pad);
    int kk = Cin * KH * KW, plane = s.OH * s.OW;
    float *cols = (float *)malloc(sizeof(float) * (size_t)plane * kk);
    float *colsT = (float *)malloc(sizeof(float) * (size_t)plane * kk);
    for (int n = 0; n < N; n++) {
        im2col(&s, x + (int64_t)n * Cin * H * W, cols);
        for (int p = 0; p < plane; p++)
            for (int q = 0; q < kk; q++) colsT[(int64_t)q * plane + p] = cols[(int64_t)p * kk + q];
        or_gemm(0, 0, Cout, plane, kk, w, kk, colsT, plane, y + (int64_t)n * Cout * plane, plane, 0);
        if (bias)
            for (int co = 0; co < Cout; co++)
                for (int p = 0; p < plane; p++) y[((int64_t)n * Cout + co) * plane + p] += bias[co];
    }
    free(cols);
    free(colsT);
}
/* ConvBackward (BackwardNn.cs:317-402), groups = 1: dbias fp64 per (n, co) row sums added in image order;
 * dW = sum over images (in order) of fl(g_n cols_n) added with one rounding; dX = col2im(W^T g_n). */
EXPORT void or_conv2d_bwd(const float *g, const float *x, const float *w, float *dx, float *dw, float *db, int N,
                          int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad) {
    conv_shape s = mk_conv(N, Cin, H, W, Cout, KH, KW, stride, pad);
    int kk = Cin * KH * KW, plane = s.OH * s.OW;
    if (db) {
        double *a = (double *)calloc((size_t)Cout, sizeof(double));
        for (int n = 0; n < N; n++)
            for (int co = 0; co < Cout; co++) {
                const float *row = g + ((int64_t)n * Cout + co) * plane;
                double t = 0.0;
                for (int i = 0; i < plane; i++) t += row[i];
                a[co] += t;
            }
        for (int co = 0; co < Cout; co++) db[co] = (float)a[co];
        free(a);
    }
    if (dw) {
        float *cols = (float *)malloc(sizeof(float) * (size_t)plane * kk);
        memset(dw, 0, sizeof(float) * (size_t)Cout * kk);
        for (int n = 0; n < N; n++) {
            im2col(&s, x + (int64_t)n * Cin * H * W, cols);
            or_gemm(0, 0, Cout, kk, plane, g + (int64_t)n * Cout * plane, plane, cols, kk, dw, kk, 1);
        }
        free(cols);
    }
    if (dx) {
        float *dcols = (float *)malloc(sizeof(float) * (size_t)kk * plane);
        memset(dx, 0, sizeof(float) * (size_t)N * Cin * H * W);
        for (int n = 0; n < N; n++) {
            or_gemm(1, 0, kk, plane, Cout, w, kk, g + (int64_t)n * Cout * plane, plane, dcols, plane, 0);
            col2im(&s, dcols, dx + (int64_t)n * Cin * H * W);
        }
        free(dcols);
    }
}

/* ------------------------------------------------------------------------------------------------ pooling */
/* ReferenceKernels.MaxPool2d (TensorKernels.cs:242-296): window in (ky, kx) order; the first candidate, a strictly
 * larger value (when the best is not NaN), or the first NaN wins; index = flat input index (n,c,y,x). */
EXPORT void or_maxpool_fwd(const float *x, float *y, int32_t *idx, int N, int C, int H, int W, int KH, int KW, int SH,
                           int SW, int PH, int PW) {
    int OH = (H + 2 * PH - KH) / SH + 1, OW = (W + 2 * PW - KW) / SW + 1;
    for (int n = 0; n < N; n++)
        for (int c = 0; c < C; c++)
            for (int oy = 0; oy < OH; oy++)
                for (int ox = 0; ox < OW; ox++) {
                    float best = -INFINITY;
                    int bi = -1;
                    for (int ky = 0; ky < KH; ky++) {
                        int yy = oy * SH - PH + ky;
                        if ((unsigned)yy >= (unsigned)H) continue;
                        for (int kx = 0; kx < KW; kx++) {
                            int xx = ox * SW - PW + kx;
                            if ((unsigned)xx >= (unsigned)W) continue;
                            int fi = ((n * C + c) * H + yy) * W + xx;
                            float v = x[fi];
                            int wins = bi < 0 || (v > best && best == best) || (v != v && best == best);
                            if (wins) { best = v; bi = fi; }
                        }
                    }
                    int64_t o = (((int64_t)n * C + c) * OH + oy) * OW + ox;
                    y[o] = best;
                    idx[o] = bi;
                }
}
/* MaxPoolBackward (BackwardOps.cs:285-298): dx = 0; dx[idx[i]] += g[i] in output order. */
EXPORT void or_maxpool_bwd(const float *g, const int32_t *idx, float *dx, int64_t n_out, int64_t n_in) {
    memset(dx, 0, sizeof(float) * (size_t)n_in);
    for (int64_t i = 0; i < n_out; i++) dx[idx[i]] += g[i];
}
/* PoolWindow (BackwardNn.cs:494-506) and Ops.AvgPool2d (Ops.Layers.cs:412-455), countIncludePad. */
static void pool_window(int kh, int kw, int sh, int sw, int ph, int pw, int cip, int h, int w, int oy, int ox, int *y0,
                        int *y1, int *x0, int *x1, int *count) {
    int ys = oy * sh - ph, xs = ox * sw - pw;
    int ye = ys + kh < h + ph ? ys + kh : h + ph, xe = xs + kw < w + pw ? xs + kw : w + pw;
    int padded = (ye - ys) * (xe - xs);
    *y0 = ys > 0 ? ys : 0;
    *x0 = xs > 0 ? xs : 0;
    *y1 = ye < h ? ye : h;
    *x1 = xe < w ? xe : w;
    int real = (*y1 - *y0) * (*x1 - *x0);
    *count = cip ? padded : (real > 1 ? real : 1);
}
EXPORT void or_avgpool_fwd(const float *x, float *y, int planes, int H, int W, int KH, int KW, int SH, int SW, int PH,
                           int PW, int cip) {
    int OH = (H + 2 * PH - KH) / SH + 1, OW = (W + 2 * PW - KW) / SW + 1;
    for (int pl = 0; pl < planes; pl++)
        for (int oy = 0; oy < OH; oy++)
            for (int ox = 0; ox < OW; ox++) {
                int y0, y1, x0, x1, cnt;
                pool_window(KH, KW, SH, SW, PH, PW, cip, H, W, oy, ox, &y0, &y1, &x0, &x1, &cnt);
                float sum = 0.0f;
                for (int yy = y0; yy < y1; yy++)
                    for (int xx = x0; xx < x1; xx++) sum += x[((int64_t)pl * H + yy) * W + xx];
                y[((int64_t)pl * OH + oy) * OW + ox] = sum / (float)cnt;
            }
}
/* AvgPoolBackward (BackwardNn.cs:464-492). */
EXPORT void or_avgpool_bwd(const float *g, float *dx, int planes, int H, int W, int KH, int KW, int SH, int SW, int PH,
                           int PW, int cip) {
    int OH = (H + 2 * PH - KH) / SH + 1, OW = (W + 2 * PW - KW) / SW + 1;
    memset(dx, 0, sizeof(float) * (size_t)planes * H * W);
    for (int pl = 0; pl < planes; pl++)
        for (int oy = 0; oy < OH; oy++)
            for (int ox = 0; ox < OW; ox++) {
                int y0, y1, x0, x1, cnt;
                pool_window(KH, KW, SH, SW, PH, PW, cip, H, W, oy, ox, &y0, &y1, &x0, &x1, &cnt);
                float share = g[((int64_t)pl * OH + oy) * OW + ox] / (float)cnt;
                for (int yy = y0; yy < y1; yy++)
                    for (int xx = x0; xx < x1; xx++) dx[((int64_t)pl * H + yy) * W + xx] += share;
            }
}
/* Embedding forward (row gather) and dense backward (BackwardNn.cs:508-541): rows added in id order. */
EXPORT void or_embedding_fwd(const float *table, const int32_t *ids, float *y, int n_ids, int dim) {
    for (int i = 0; i < n_ids; i++) memcpy(y + (int64_t)i * dim, table + (int64_t)ids[i] * dim, sizeof(float) * (size_t)dim);
}
EXPORT void or_embedding_bwd(const float *g, const int32_t *ids, float *dtable, int n_ids, int dim, int rows, int pad) {
    memset(dtable, 0, sizeof(float) * (size_t)rows * dim);
    for (int i = 0; i < n_ids; i++) {
        if (ids[i] == pad) continue;
        for (int j = 0; j < dim; j++) dtable[(int64_t)ids[i] * dim + j] += g[(int64_t)i * dim + j];
    }
}

/* ------------------------------------------------------------------------------------------------ CTC (double) */
/* CtcMath.Exp / Log / LogAdd (Ctc.cs:515-616; docs/ctc.md:53-63). */
EXPORT double or_ctc_exp(double x) {
    if (!(x > -700.0)) return 0.0;
    if (x > 700.0) x = 700.0;
    double k = floor((x * 1.4426950408889634) + 0.5);
    double r = (x - (k * 6.93147180369123816490e-01)) - (k * 1.90821492927058770002e-10);
    static const double C[14] = {1.0 / 6227020800.0, 1.0 / 479001600.0, 1.0 / 39916800.0, 1.0 / 3628800.0,
                                 1.0 / 362880.0, 1.0 / 40320.0, 1.0 / 5040.0, 1.0 / 720.0, 1.0 / 120.0, 1.0 / 24.0,
                                 1.0 / 6.0, 0.5, 1.0, 1.0};
    double p = C[0];
    for (int i = 1; i < 14; i++) p = (p * r) + C[i];
    int64_t eb = (int64_t)((int)k + 1023) << 52;
    double sc;
    memcpy(&sc, &eb, 8);
    return p * sc;
}
EXPORT double or_ctc_log(double x) {
    if (x == 0.0) return -INFINITY;
    if (!(x > 0.0) || isinf(x)) return x;
    int64_t bits;
    memcpy(&bits, &x, 8);
    int e = (int)((bits >> 52) & 0x7FF);
    if (e == 0) {
        double xs = x * 18014398509481984.0;
        memcpy(&bits, &xs, 8);
        e = (int)((bits >> 52) & 0x7FF) - 54;
    }
    e -= 1023;
    int64_t mb = (bits & 0x000FFFFFFFFFFFFFLL) | 0x3FF0000000000000LL;
    double m;
    memcpy(&m, &mb, 8);
    if (m > 1.4142135623730951) { m *= 0.5; e++; }
    double s = (m - 1.0) / (m + 1.0);
    double z = s * s;
    static const double Q[10] = {1.0 / 19.0, 1.0 / 17.0, 1.0 / 15.0, 1.0 / 13.0, 1.0 / 11.0,
                                 1.0 / 9.0, 1.0 / 7.0, 1.0 / 5.0, 1.0 / 3.0, 1.0};
    double q = Q[0];
    for (int i = 1; i < 10; i++) q = (q * z) + Q[i];
    return (e * 0.6931471805599453) + (2.0 * s * q);
}
EXPORT double or_ctc_logadd(double a, double b) {
    if (a < b) { double t = a; a = b; b = t; }
    if (isinf(b) && b < 0) return a;
    double d = b - a;
    return d < -40.0 ? a : a + or_ctc_log(1.0 + or_ctc_exp(d));
}
static inline int ctc_label(const int32_t *tgt, int blank, int s) { return (s & 1) == 0 ? blank : tgt[s >> 1]; }
static inline int ctc_can_skip(const int32_t *tgt, int s) { return s >= 2 && (s & 1) == 1 && tgt[s >> 1] != tgt[(s >> 1) - 1]; }
/* CtcLossMath.Alpha (CtcLoss.cs:170-213). lp is [T,B,C]; alpha holds len*(2L+1). */
static double ctc_alpha(const float *lp, int batch, int classes, int b, int len, const int32_t *tgt, int L, int blank,
                        double *alpha) {
    int ext = 2 * L + 1;
    if (len == 0) return L == 0 ? 0.0 : INFINITY;
    for (int t = 0; t < len; t++)
        for (int s = 0; s < ext; s++) {
            double a;
            if (t == 0) a = s <= 1 ? 0.0 : -INFINITY;
            else {
                a = alpha[(t - 1) * ext + s];
                if (s >= 1) a = or_ctc_logadd(a, alpha[(t - 1) * ext + s - 1]);
                if (ctc_can_skip(tgt, s)) a = or_ctc_logadd(a, alpha[(t - 1) * ext + s - 2]);
            }
            alpha[t * ext + s] = (isinf(a) && a < 0) ? -INFINITY
                                 : a + (double)lp[((int64_t)t * batch + b) * classes + ctc_label(tgt, blank, s)];
        }
    double p = alpha[(len - 1) * ext + ext - 1];
    if (ext >= 2) p = or_ctc_logadd(p, alpha[(len - 1) * ext + ext - 2]);
    return (isinf(p) && p < 0) ? INFINITY : -p;
}
/* Ops.CtcLoss (CtcLoss.cs:40-153): per-sequence nll, reductions 0=None,1=Mean,2=Sum; zero_inf maps +inf to 0.
 * out has B entries for None, else 1. */
EXPORT void or_ctc_loss(const float *lp, const int32_t *targets, const int32_t *in_len, const int32_t *tgt_len, int T,
                        int B, int C, int blank, int reduction, int zero_inf, float *out) {
    int maxS = 1;
    for (int b = 0; b < B; b++) maxS = 2 * tgt_len[b] + 1 > maxS ? 2 * tgt_len[b] + 1 : maxS;
    double *alpha = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1) * maxS);
    double *per = (double *)malloc(sizeof(double) * (size_t)B);
    int off = 0;
    for (int b = 0; b < B; b++) {
        double nll = ctc_alpha(lp, B, C, b, in_len[b], targets + off, tgt_len[b], blank, alpha);
        off += tgt_len[b];
        per[b] = (isinf(nll) && zero_inf) ? 0.0 : nll;
    }
    if (reduction == 0) for (int b = 0; b < B; b++) out[b] = (float)per[b];
    else {
        double sum = 0.0;
        for (int b = 0; b < B; b++) sum += reduction == 1 ? per[b] / (tgt_len[b] > 1 ? tgt_len[b] : 1) : per[b];
        out[0] = (float)(reduction == 1 ? sum / B : sum);
    }
    free(alpha);
    free(per);
}
/* CtcBackward (BackwardRecurrent.cs:253-296) with CtcLossMath.Gradient (CtcLoss.cs:219-281): dlp = 0, then per
 * sequence grad[t,b,c] += (float)(-scale*exp(logsum_{s:l'(s)=c}(alpha+beta) - lp + nll)). g holds B values for None,
 * else 1. */
EXPORT void or_ctc_grad(const float *lp, const int32_t *targets, const int32_t *in_len, const int32_t *tgt_len,
                        const float *g, int T, int B, int C, int blank, int reduction, float *dlp) {
    int maxS = 1;
    for (int b = 0; b < B; b++) maxS = 2 * tgt_len[b] + 1 > maxS ? 2 * tgt_len[b] + 1 : maxS;
    size_t cap = (size_t)(T > 0 ? T : 1) * maxS;
    double *alpha = (double *)malloc(sizeof(double) * cap), *beta = (double *)malloc(sizeof(double) * cap);
    double *acc = (double *)malloc(sizeof(double) * (size_t)C);
    memset(dlp, 0, sizeof(float) * (size_t)T * B * C);
    int off = 0;
    for (int b = 0; b < B; b++) {
        int len = in_len[b], L = tgt_len[b];
        const int32_t *tgt = targets + off;
        off += L;
        double scale = reduction == 0 ? g[b] : g[0];
        if (reduction == 1) scale = scale / (L > 1 ? L : 1) / B;
        int ext = 2 * L + 1;
        double nll = ctc_alpha(lp, B, C, b, len, tgt, L, blank, alpha);
        if (len == 0 || isinf(nll)) continue;
        for (int t = len - 1; t >= 0; t--) {
            for (int s = ext - 1; s >= 0; s--) {
                double v;
                if (t == len - 1) v = s >= ext - 2 ? 0.0 : -INFINITY;
                else {
                    v = beta[(t + 1) * ext + s];
                    if (s + 1 < ext) v = or_ctc_logadd(v, beta[(t + 1) * ext + s + 1]);
                    if (s + 2 < ext && ctc_can_skip(tgt, s + 2)) v = or_ctc_logadd(v, beta[(t + 1) * ext + s + 2]);
                }
                beta[t * ext + s] = (isinf(v) && v < 0) ? -INFINITY
                                    : v + (double)lp[((int64_t)t * B + b) * C + ctc_label(tgt, blank, s)];
            }
            for (int c = 0; c < C; c++) acc[c] = -INFINITY;
            for (int s = 0; s < ext; s++) {
                double ab = alpha[t * ext + s] + beta[t * ext + s];
                if (!(isinf(ab) && ab < 0) && ab == ab) {
                    int cls = ctc_label(tgt, blank, s);
                    acc[cls] = or_ctc_logadd(acc[cls], ab);
                }
            }
            for (int c = 0; c < C; c++) {
                if (isinf(acc[c]) && acc[c] < 0) continue;
                double l = (double)lp[((int64_t)t * B + b) * C + c];
                dlp[((int64_t)t * B + b) * C + c] += (float)(-scale * or_ctc_exp(acc[c] - l + nll));
            }
        }
    }
    free(alpha);
    free(beta);
    free(acc);
}

/* ------------------------------------------------------------------------------------------------ optimizers */
/* Adam.IntPow (Optimizers.cs:483-498) and Adam.BeginStep (Optimizers.cs:501-508). */
EXPORT void or_adam_scalars(float lr, float beta1, float beta2, int64_t t, float *step_size, float *sqrt_bc2) {
    double b1 = beta1, b2 = beta2, p1 = 1.0, p2 = 1.0;
    for (int64_t n = t; n > 0; n >>= 1) { if (n & 1) p1 *= b1; b1 *= b1; }
    for (int64_t n = t; n > 0; n >>= 1) { if (n & 1) p2 *= b2; b2 *= b2; }
    double bc1 = 1.0 - p1, bc2 = 1.0 - p2;
    *step_size = (float)((double)lr / bc1);
    *sqrt_bc2 = (float)sqrt(bc2);
}
/* Adam.UpdateRange (Optimizers.cs:554-589): IEEE float, no fusion, per element in this order. */
EXPORT void or_adam_update(float *p, const float *grad, float *m, float *v, float *vmax, int64_t n, float lr, float beta1,
                           float beta2, float eps, float wd, int decoupled, float step_size, float sqrt_bc2) {
    float omb1 = 1.0f - beta1, omb2 = 1.0f - beta2, decay = 1.0f - lr * wd;
    for (int64_t i = 0; i < n; i++) {
        float g = grad[i], pi = p[i];
        if (wd != 0.0f) {
            if (decoupled) pi *= decay;
            else g += wd * pi;
        }
        float mi = beta1 * m[i] + omb1 * g;
        float vi = beta2 * v[i] + omb2 * g * g;
        m[i] = mi;
        v[i] = vi;
        float vd = vi;
        if (vmax) { vd = vmax[i] > vi ? vmax[i] : vi; vmax[i] = vd; }
        float denom = sqrtf(vd) / sqrt_bc2 + eps;
        p[i] = pi - step_size * mi / denom;
    }
}
/* Sgd.Update (Optimizers.cs, class Sgd): g += wd*p; buf = first ? g : mu*buf + (1-d)*g; g = nesterov ? g+mu*buf : buf;
 * p -= lr*g. buf may be NULL for plain SGD. */
EXPORT void or_sgd_update(float *p, const float *grad, float *buf, int64_t n, float lr, float momentum, float dampening,
                          float wd, int nesterov, int first) {
    float keep = 1.0f - dampening;
    for (int64_t i = 0; i < n; i++) {
        float g = grad[i];
        if (wd != 0.0f) g += wd * p[i];
        if (buf) {
            float b = first ? g : momentum * buf[i] + keep * g;
            buf[i] = b;
            g = nesterov ? g + momentum * b : b;
        }
        p[i] -= lr * g;
    }
}

/* ------------------------------------------------------------------------------------------------ gradient clipping */
/* GradClip.ClipNorm (Schedules.cs:22-100), serially as the reference runs it: squares (double)g*g summed in one double
 * accumulator in segment then element order (L2), or the running largest |g| where a larger value or a NaN replaces
 * it (infinity); the norm is the square root (L2) or the accumulator; nothing is scaled when it is not finite,
 * otherwise coef = (float)(max_norm / (norm + 1e-6)) and every element becomes g * coef when coef < 1. NULL or empty
 * segments are skipped. Returns the norm as float; *coef_out (may be NULL) gets coef, or 1 for a non-finite norm. */
EXPORT float or_clip_norm(float *const *grads, const int64_t *lens, int count, float max_norm, int inf,
                          float *coef_out) {
    double acc = 0.0;
    for (int i = 0; i < count; i++) {
        if (!grads[i] || lens[i] <= 0) continue;
        const float *s = grads[i];
        for (int64_t j = 0; j < lens[i]; j++) {
            if (inf) {
                double a = fabs((double)s[j]);
                if (a > acc || isnan(a)) acc = a;
            } else {
                acc += (double)s[j] * s[j];
            }
        }
    }
    double norm = inf ? acc : sqrt(acc);
    float total = (float)norm;
    if (!isfinite(norm)) {
        if (coef_out) *coef_out = 1.0f;
        return total;
    }
    float coef = (float)((double)max_norm / (norm + 1e-6));
    if (coef < 1.0f)
        for (int i = 0; i < count; i++) {
            if (!grads[i] || lens[i] <= 0) continue;
            for (int64_t j = 0; j < lens[i]; j++) grads[i][j] *= coef;
        }
    if (coef_out) *coef_out = coef;
    return total;
}
/* GradClip.ClipValue (Schedules.cs:119-149): v > c ? c : v < -c ? -c : v, so NaN stays NaN. */
EXPORT void or_clip_value(float *const *grads, const int64_t *lens, int count, float c) {
    for (int i = 0; i < count; i++) {
        if (!grads[i] || lens[i] <= 0) continue;
        for (int64_t j = 0; j < lens[i]; j++) {
            float v = grads[i][j];
            grads[i][j] = v > c ? c : v < -c ? -c : v;
        }
    }
}

/* ------------------------------------------------------------------------------------------------ dropout */
/* Dropout.Forward in training mode (Layers.cs:341-368): stream = Mix(seed + draw * G); element i keeps iff
 * (Mix(stream + (i + 1) * G) >> 40) * 2^-24 >= p, and out = in * (keep ? 1/(1-p) : 0) (Ops.Mul; the backward's Mul rule
 * is the same product with g). Mix is SplitMix64's output function (Generator.cs:41-47). */
static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
EXPORT void or_dropout(const float *in, float *out, int64_t n, float p, uint64_t seed, int64_t draw) {
    const uint64_t G = 0x9E3779B97F4A7C15ull;
    uint64_t stream = mix64(seed + (uint64_t)draw * G);
    float scale = 1.0f / (1.0f - p);
    for (int64_t i = 0; i < n; i++) {
        uint64_t bits = mix64(stream + (uint64_t)(i + 1) * G);
        float u = (float)(bits >> 40) * (1.0f / 16777216.0f);
        out[i] = in[i] * (u >= p ? scale : 0.0f);
    }
}
