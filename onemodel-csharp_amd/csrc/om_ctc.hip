// CTC loss forward and gradient in double (Ops.CtcLoss, CtcLoss.cs:40-153; CtcLossMath, CtcLoss.cs:155-281;
// CtcBackward, BackwardRecurrent.cs:253-296), with the reference's own fixed exp/ln/logadd (Ctc.cs:515-616).
//
// One workgroup per sequence. The recursions are sequential in t; within a step every extended-label position s is
// independent, so threads own positions and meet at a barrier per step. The alpha (and beta) tables live in LDS when
// they fit (T x (2L + 1) doubles each, up to 32 KB), so a step's reads of the previous one stay on chip; longer
// sequences keep them in device scratch. Each value is computed by exactly the
// operations of the reference in the same order (no contraction: -ffp-contract=off), so the loss, the alignment
// sums and the gradient are bit-identical to the CPU recursions.
#include "om_internal.hpp"

#include <cmath>

namespace {

constexpr int kBlock = 64;
constexpr uint64_t kLdsTable = 32768;  // bytes of one alpha or beta table kept in LDS

__device__ double ctc_exp(double x) {
    if (!(x > -700.0)) return 0.0;
    if (x > 700.0) x = 700.0;
    double k = floor((x * 1.4426950408889634) + 0.5);
    double r = (x - (k * 6.93147180369123816490e-01)) - (k * 1.90821492927058770002e-10);
    double p = 1.0 / 6227020800.0;
    p = (p * r) + (1.0 / 479001600.0);
    p = (p * r) + (1.0 / 39916800.0);
    p = (p * r) + (1.0 / 3628800.0);
    p = (p * r) + (1.0 / 362880.0);
    p = (p * r) + (1.0 / 40320.0);
    p = (p * r) + (1.0 / 5040.0);
    p = (p * r) + (1.0 / 720.0);
    p = (p * r) + (1.0 / 120.0);
    p = (p * r) + (1.0 / 24.0);
    p = (p * r) + (1.0 / 6.0);
    p = (p * r) + 0.5;
    p = (p * r) + 1.0;
    p = (p * r) + 1.0;
    return p * __longlong_as_double((long long)((int)k + 1023) << 52);
}
__device__ double ctc_log(double x) {
    if (x == 0.0) return -__longlong_as_double(0x7FF0000000000000LL);
    if (!(x > 0.0) || isinf(x)) return x;
    long long bits = __double_as_longlong(x);
    int e = (int)((bits >> 52) & 0x7FF);
    if (e == 0) {
        bits = __double_as_longlong(x * 18014398509481984.0);
        e = (int)((bits >> 52) & 0x7FF) - 54;
    }
    e -= 1023;
    double m = __longlong_as_double((bits & 0x000FFFFFFFFFFFFFLL) | 0x3FF0000000000000LL);
    if (m > 1.4142135623730951) {
        m *= 0.5;
        e++;
    }
    double s = (m - 1.0) / (m + 1.0);
    double z = s * s;
    double q = 1.0 / 19.0;
    q = (q * z) + (1.0 / 17.0);
    q = (q * z) + (1.0 / 15.0);
    q = (q * z) + (1.0 / 13.0);
    q = (q * z) + (1.0 / 11.0);
    q = (q * z) + (1.0 / 9.0);
    q = (q * z) + (1.0 / 7.0);
    q = (q * z) + (1.0 / 5.0);
    q = (q * z) + (1.0 / 3.0);
    q = (q * z) + 1.0;
    return (e * 0.6931471805599453) + (2.0 * s * q);
}
__device__ __forceinline__ bool is_neg_inf(double v) { return isinf(v) && v < 0.0; }
__device__ double ctc_logadd(double a, double b) {
    if (a < b) {
        double t = a;
        a = b;
        b = t;
    }
    if (is_neg_inf(b)) return a;
    double d = b - a;
    return d < -40.0 ? a : a + ctc_log(1.0 + ctc_exp(d));
}

__device__ __forceinline__ int label_at(const int32_t *tgt, int blank, int s) { return (s & 1) == 0 ? blank : tgt[s >> 1]; }
__device__ __forceinline__ bool can_skip(const int32_t *tgt, int s) {
    return s >= 2 && (s & 1) == 1 && tgt[s >> 1] != tgt[(s >> 1) - 1];
}

// One lane's extended positions s = lane + 64 k (k < NPL) for a recursion: their labels and skip flags, read from
// the targets once, and the log-probabilities of the current and the next time step (the next one's loads are issued
// before the current step's arithmetic, so their latency hides behind it). BETA selects the backward recursion (the
// skip is the one into s + 2, the steps run down from len - 1).
template <int NPL, bool BETA>
struct RecLane {
    int s[NPL], lab[NPL];
    bool ok[NPL], sk[NPL];
    float cur[NPL], nxt[NPL];
    __device__ __forceinline__ void init(const int32_t *tgt, int blank, int ext, int lane) {
#pragma unroll
        for (int k = 0; k < NPL; k++) {
            s[k] = lane + 64 * k;
            ok[k] = s[k] < ext;
            lab[k] = ok[k] ? label_at(tgt, blank, s[k]) : 0;
            sk[k] = ok[k] && (BETA ? (s[k] + 2 < ext && can_skip(tgt, s[k] + 2)) : can_skip(tgt, s[k]));
        }
    }
    __device__ __forceinline__ void fetch(float (&dst)[NPL], const float *lp, int B, int C, int b, int t) {
#pragma unroll
        for (int k = 0; k < NPL; k++) dst[k] = ok[k] ? lp[((int64_t)t * B + b) * C + lab[k]] : 0.0f;
    }
    // Step t of the recursion into table[t * ext + s] from row `from` (t - 1 for alpha, t + 1 for beta), with the
    // reference's operations in its order.
    __device__ __forceinline__ void step(double *table, int ext, int t, bool first) {
        const double NEG = -__longlong_as_double(0x7FF0000000000000LL);
        const double *prev = table + (BETA ? t + 1 : t - 1) * ext;
#pragma unroll
        for (int k = 0; k < NPL; k++) {
            if (!ok[k]) continue;
            const int p = s[k];
            double a;
            if (first) {
                a = BETA ? (p >= ext - 2 ? 0.0 : NEG) : (p <= 1 ? 0.0 : NEG);
            } else if (BETA) {
                a = prev[p];
                if (p + 1 < ext) a = ctc_logadd(a, prev[p + 1]);
                if (sk[k]) a = ctc_logadd(a, prev[p + 2]);
            } else {
                a = prev[p];
                if (p >= 1) a = ctc_logadd(a, prev[p - 1]);
                if (sk[k]) a = ctc_logadd(a, prev[p - 2]);
            }
            table[t * ext + p] = is_neg_inf(a) ? NEG : a + (double)cur[k];
        }
    }
};

// alpha[t*ext + s] for t < len (CtcLossMath.Alpha) by the 64 threads of the workgroup; returns nll via *nll_out from
// thread 0. NPL positions per lane (ext <= 64 NPL); NPL = 0 walks any ext without the per-lane state.
template <int NPL>
__device__ void alpha_pass(const float *lp, int B, int C, int b, int len, const int32_t *tgt, int L, int blank,
                           double *alpha, double *nll_out) {
    const int ext = 2 * L + 1;
    const double NEG = -__longlong_as_double(0x7FF0000000000000LL);
    if constexpr (NPL > 0) {
        RecLane<NPL, false> rl;
        rl.init(tgt, blank, ext, threadIdx.x);
        if (len > 0) rl.fetch(rl.cur, lp, B, C, b, 0);
        for (int t = 0; t < len; t++) {
            if (t + 1 < len) rl.fetch(rl.nxt, lp, B, C, b, t + 1);
            rl.step(alpha, ext, t, t == 0);
#pragma unroll
            for (int k = 0; k < NPL; k++) rl.cur[k] = rl.nxt[k];
            __syncthreads();
        }
    } else {
        for (int t = 0; t < len; t++) {
            for (int s = threadIdx.x; s < ext; s += blockDim.x) {
                double a;
                if (t == 0) {
                    a = s <= 1 ? 0.0 : NEG;
                } else {
                    a = alpha[(t - 1) * ext + s];
                    if (s >= 1) a = ctc_logadd(a, alpha[(t - 1) * ext + s - 1]);
                    if (can_skip(tgt, s)) a = ctc_logadd(a, alpha[(t - 1) * ext + s - 2]);
                }
                alpha[t * ext + s] =
                    is_neg_inf(a) ? NEG : a + (double)lp[((int64_t)t * B + b) * C + label_at(tgt, blank, s)];
            }
            __syncthreads();
        }
    }
    if (threadIdx.x == 0) {
        double nll;
        if (len == 0) {
            nll = L == 0 ? 0.0 : __longlong_as_double(0x7FF0000000000000LL);
        } else {
            double p = alpha[(len - 1) * ext + ext - 1];
            if (ext >= 2) p = ctc_logadd(p, alpha[(len - 1) * ext + ext - 2]);
            nll = is_neg_inf(p) ? __longlong_as_double(0x7FF0000000000000LL) : -p;
        }
        *nll_out = nll;
    }
    __syncthreads();
}

__global__ void __launch_bounds__(kBlock) k_ctc_fwd(const float *__restrict__ lp, const int32_t *__restrict__ targets,
                                                    const int32_t *__restrict__ in_len,
                                                    const int32_t *__restrict__ tgt_len, int T, int B, int C, int blank,
                                                    int max_ext, double *__restrict__ alpha_ws,
                                                    double *__restrict__ per, int in_lds) {
    OM_LDS_POISON();
    __shared__ double nll;
    extern __shared__ double tables[];
    int b = blockIdx.x;
    int off = 0;
    for (int i = 0; i < b; i++) off += tgt_len[i];
    double *alpha = in_lds ? tables : alpha_ws + (int64_t)b * (T > 0 ? T : 1) * max_ext;
    const int ext = 2 * tgt_len[b] + 1;
    if (ext <= 64) alpha_pass<1>(lp, B, C, b, in_len[b], targets + off, tgt_len[b], blank, alpha, &nll);
    else if (ext <= 128) alpha_pass<2>(lp, B, C, b, in_len[b], targets + off, tgt_len[b], blank, alpha, &nll);
    else if (ext <= 256) alpha_pass<4>(lp, B, C, b, in_len[b], targets + off, tgt_len[b], blank, alpha, &nll);
    else alpha_pass<0>(lp, B, C, b, in_len[b], targets + off, tgt_len[b], blank, alpha, &nll);
    if (threadIdx.x == 0) per[b] = nll;
}
// Reduction in sequence order (CtcLoss.cs:98-125).
__global__ void k_ctc_reduce(const double *__restrict__ per, const int32_t *__restrict__ tgt_len, int B, int reduction,
                             int zero_inf, float *__restrict__ loss) {
    OM_LDS_POISON();
    if (threadIdx.x != 0) return;
    double sum = 0.0;
    for (int b = 0; b < B; b++) {
        double v = per[b];
        if (isinf(v) && v > 0 && zero_inf) v = 0.0;
        if (reduction == 0) loss[b] = (float)v;
        else sum += reduction == 1 ? v / (double)(tgt_len[b] > 1 ? tgt_len[b] : 1) : v;
    }
    if (reduction != 0) loss[0] = (float)(reduction == 1 ? sum / B : sum);
}

// The alpha (wavefront 0, t up) and beta (wavefront 1, t down) recursions of one sequence side by side, one barrier
// per step for the whole workgroup.
template <int NPL>
__device__ void recursions(const float *lp, int B, int C, int b, int len, const int32_t *tgt, int blank, int ext,
                           double *alpha, double *beta, int wave, int lane) {
    RecLane<NPL, false> ra;
    RecLane<NPL, true> rb;
    if (wave == 0) {
        ra.init(tgt, blank, ext, lane);
        if (len > 0) ra.fetch(ra.cur, lp, B, C, b, 0);
    } else if (wave == 1) {
        rb.init(tgt, blank, ext, lane);
        if (len > 0) rb.fetch(rb.cur, lp, B, C, b, len - 1);
    }
    for (int i = 0; i < len; i++) {
        if (wave == 0) {
            if (i + 1 < len) ra.fetch(ra.nxt, lp, B, C, b, i + 1);
            ra.step(alpha, ext, i, i == 0);
#pragma unroll
            for (int k = 0; k < NPL; k++) ra.cur[k] = ra.nxt[k];
        } else if (wave == 1) {
            const int t = len - 1 - i;
            if (t > 0) rb.fetch(rb.nxt, lp, B, C, b, t - 1);
            rb.step(beta, ext, t, i == 0);
#pragma unroll
            for (int k = 0; k < NPL; k++) rb.cur[k] = rb.nxt[k];
        }
        __syncthreads();
    }
}

// Both recursions of one sequence into alpha and beta (any ext): the two-wavefront form above when a lane's positions
// fit NPL <= 4, else wavefront 0 walks alpha up and wavefront 1 beta down over all positions.
__device__ void both_recursions(const float *lp, int B, int C, int b, int len, const int32_t *tgt, int blank, int ext,
                                double *alpha, double *beta, int wave, int lane) {
    const double NEG = -__longlong_as_double(0x7FF0000000000000LL);
    if (ext <= 64) recursions<1>(lp, B, C, b, len, tgt, blank, ext, alpha, beta, wave, lane);
    else if (ext <= 128) recursions<2>(lp, B, C, b, len, tgt, blank, ext, alpha, beta, wave, lane);
    else if (ext <= 256) recursions<4>(lp, B, C, b, len, tgt, blank, ext, alpha, beta, wave, lane);
    else for (int i = 0; i < len; i++) {
        if (wave == 0) {
            const int t = i;
            for (int s = lane; s < ext; s += 64) {
                double a;
                if (t == 0) {
                    a = s <= 1 ? 0.0 : NEG;
                } else {
                    a = alpha[(t - 1) * ext + s];
                    if (s >= 1) a = ctc_logadd(a, alpha[(t - 1) * ext + s - 1]);
                    if (can_skip(tgt, s)) a = ctc_logadd(a, alpha[(t - 1) * ext + s - 2]);
                }
                alpha[t * ext + s] =
                    is_neg_inf(a) ? NEG : a + (double)lp[((int64_t)t * B + b) * C + label_at(tgt, blank, s)];
            }
        } else if (wave == 1) {
            const int t = len - 1 - i;
            for (int s = lane; s < ext; s += 64) {
                double v;
                if (t == len - 1) {
                    v = s >= ext - 2 ? 0.0 : NEG;
                } else {
                    v = beta[(t + 1) * ext + s];
                    if (s + 1 < ext) v = ctc_logadd(v, beta[(t + 1) * ext + s + 1]);
                    if (s + 2 < ext && can_skip(tgt, s + 2)) v = ctc_logadd(v, beta[(t + 1) * ext + s + 2]);
                }
                beta[t * ext + s] =
                    is_neg_inf(v) ? NEG : v + (double)lp[((int64_t)t * B + b) * C + label_at(tgt, blank, s)];
            }
        }
        __syncthreads();
    }
}

// The sequence's negative log-likelihood from its alpha table (CtcLossMath.Alpha's end), as alpha_pass forms it.
__device__ __forceinline__ double nll_from_alpha(const double *alpha, int len, int L, int ext) {
    if (len == 0) return L == 0 ? 0.0 : __longlong_as_double(0x7FF0000000000000LL);
    double p = alpha[(len - 1) * ext + ext - 1];
    if (ext >= 2) p = ctc_logadd(p, alpha[(len - 1) * ext + ext - 2]);
    return is_neg_inf(p) ? __longlong_as_double(0x7FF0000000000000LL) : -p;
}

// The gradient phase: every (t, class) entry of dlp for sequence b is independent; the workgroup's threads take them
// in turn, and each accumulates logadd(alpha + beta) over the class's positions in increasing s, exactly the
// reference's order, so the values are those of the sequential loop bit for bit. Jobs 0 .. T - 1 are the blank
// class's entries (its chain runs over all L + 1 even positions), one per thread of the first wavefronts; the other
// classes' entries (at most a few positions each) follow in (t, c) order, so no wavefront holds more than its share of
// long chains.
__device__ void gradient_phase(const float *lp, const int32_t *tgt, const double *alpha, const double *beta, double nll,
                               const float *g, float *dlp, int T, int B, int C, int b, int len, int L, int ext,
                               int blank, int reduction, int acc) {
    const double NEG = -__longlong_as_double(0x7FF0000000000000LL);
    // +inf (an impossible alignment) and an empty input give a zero gradient (CtcBackward, BackwardRecurrent.cs)
    const bool none = len == 0 || (isinf(nll) && nll > 0);
    double scale = reduction == 0 ? (double)g[b] : (double)g[0];
    if (reduction == 1) scale = scale / (double)(L > 1 ? L : 1) / (double)B;
    const bool blank_ok = blank >= 0 && blank < C;
    for (int job = threadIdx.x; job < T * C; job += blockDim.x) {
        int t, c;
        if (!blank_ok) {
            t = job / C;
            c = job - t * C;
        } else if (job < T) {
            t = job;
            c = blank;
        } else {
            const int k = job - T;
            t = k / (C - 1);
            const int cc = k - t * (C - 1);
            c = cc < blank ? cc : cc + 1;
        }
        float *d = dlp + ((int64_t)t * B + b) * C + c;
        float v = acc ? *d : 0.0f;
        if (!none && t < len) {
            double a = NEG;
            for (int s = 0; s < ext; s++) {
                if (label_at(tgt, blank, s) != c) continue;
                double ab = alpha[t * ext + s] + beta[t * ext + s];
                if (!is_neg_inf(ab) && ab == ab) a = ctc_logadd(a, ab);
            }
            if (!is_neg_inf(a)) {
                double l = (double)lp[((int64_t)t * B + b) * C + c];
                v = v + (float)(-scale * ctc_exp(a - l + nll));
            }
        }
        *d = v;
    }
}

__device__ __forceinline__ const int32_t *seq_targets(const int32_t *targets, const int32_t *tgt_len, int b) {
    int off = 0;
    for (int i = 0; i < b; i++) off += tgt_len[i];
    return targets + off;
}

// CtcLossMath.Gradient (CtcLoss.cs:219-281) per sequence, in two phases: the alpha recursion (recomputed, as the
// reference recomputes it) and the beta recursion side by side on two wavefronts, alpha forward and beta backward in
// t, one barrier per step (each lane owns extended positions s, s + 64, ...); then the gradient phase.
constexpr int kBwdBlock = 256;
__global__ void __launch_bounds__(kBwdBlock) k_ctc_bwd(const float *__restrict__ lp, const int32_t *__restrict__ targets,
                                                       const int32_t *__restrict__ in_len,
                                                       const int32_t *__restrict__ tgt_len, const float *__restrict__ g,
                                                       float *__restrict__ dlp, int T, int B, int C, int blank,
                                                       int reduction, int max_ext, int acc, double *__restrict__ ws,
                                                       int in_lds) {
    OM_LDS_POISON();
    __shared__ double nll_s;
    extern __shared__ double tables[];
    const int b = blockIdx.x;
    const int len = in_len[b], L = tgt_len[b];
    const int32_t *tgt = seq_targets(targets, tgt_len, b);
    const int tt = T > 0 ? T : 1;
    double *alpha = in_lds ? tables : ws + (int64_t)b * 2 * tt * max_ext;
    double *beta = alpha + (int64_t)tt * max_ext;
    const int ext = 2 * L + 1;
    both_recursions(lp, B, C, b, len, tgt, blank, ext, alpha, beta, threadIdx.x >> 6, threadIdx.x & 63);
    if (threadIdx.x == 0) nll_s = nll_from_alpha(alpha, len, L, ext);
    __syncthreads();
    gradient_phase(lp, tgt, alpha, beta, nll_s, g, dlp, T, B, C, b, len, L, ext, blank, reduction, acc);
}

// The forward of the saved-tables pair: k_ctc_bwd's recursions (alpha as k_ctc_fwd forms it, beta beside it on the
// second wavefront) with the sequence's loss term in per[b]; the tables end in `saved` (alpha [tt][max_ext] then beta,
// per sequence), through LDS when they fit there.
__global__ void __launch_bounds__(kBwdBlock) k_ctc_fwd_tables(const float *__restrict__ lp,
                                                              const int32_t *__restrict__ targets,
                                                              const int32_t *__restrict__ in_len,
                                                              const int32_t *__restrict__ tgt_len, int T, int B, int C,
                                                              int blank, int max_ext, double *__restrict__ saved,
                                                              double *__restrict__ per, int in_lds) {
    OM_LDS_POISON();
    extern __shared__ double tables[];
    const int b = blockIdx.x;
    const int len = in_len[b], L = tgt_len[b];
    const int32_t *tgt = seq_targets(targets, tgt_len, b);
    const int tt = T > 0 ? T : 1;
    double *out = saved + (int64_t)b * 2 * tt * max_ext;
    double *alpha = in_lds ? tables : out;
    double *beta = alpha + (int64_t)tt * max_ext;
    const int ext = 2 * L + 1;
    both_recursions(lp, B, C, b, len, tgt, blank, ext, alpha, beta, threadIdx.x >> 6, threadIdx.x & 63);
    if (threadIdx.x == 0) per[b] = nll_from_alpha(alpha, len, L, ext);
    if (in_lds) {
        __syncthreads();
        // the rows the recursions wrote (t < len, s < ext) of both tables; the rest is never read
        for (int e = threadIdx.x; e < 2 * len * ext; e += blockDim.x) {
            const int h = e / (len * ext), r = e - h * len * ext, t = r / ext, s = r - t * ext;
            const int64_t o = (int64_t)h * tt * max_ext + (int64_t)t * ext + s;
            out[o] = tables[o];
        }
    }
}

// The gradient of the saved-tables pair: k_ctc_bwd's gradient phase over the tables k_ctc_fwd_tables left in `saved`
// (staged into LDS when they fit), with the loss term formed again from alpha.
__global__ void __launch_bounds__(kBwdBlock) k_ctc_bwd_tables(const float *__restrict__ lp,
                                                              const int32_t *__restrict__ targets,
                                                              const int32_t *__restrict__ in_len,
                                                              const int32_t *__restrict__ tgt_len,
                                                              const float *__restrict__ g, float *__restrict__ dlp,
                                                              int T, int B, int C, int blank, int reduction,
                                                              int max_ext, int acc, const double *__restrict__ saved,
                                                              int in_lds) {
    OM_LDS_POISON();
    __shared__ double nll_s;
    extern __shared__ double tables[];
    const int b = blockIdx.x;
    const int len = in_len[b], L = tgt_len[b];
    const int32_t *tgt = seq_targets(targets, tgt_len, b);
    const int tt = T > 0 ? T : 1;
    const double *src = saved + (int64_t)b * 2 * tt * max_ext;
    const int ext = 2 * L + 1;
    const double *alpha = src;
    if (in_lds) {
        for (int e = threadIdx.x; e < 2 * len * ext; e += blockDim.x) {
            const int h = e / (len * ext), r = e - h * len * ext, t = r / ext, s = r - t * ext;
            const int64_t o = (int64_t)h * tt * max_ext + (int64_t)t * ext + s;
            tables[o] = src[o];
        }
        __syncthreads();
        alpha = tables;
    }
    const double *beta = alpha + (int64_t)tt * max_ext;
    if (threadIdx.x == 0) nll_s = nll_from_alpha(alpha, len, L, ext);
    __syncthreads();
    gradient_phase(lp, tgt, alpha, beta, nll_s, g, dlp, T, B, C, b, len, L, ext, blank, reduction, acc);
}

// The host-side checks both entry points run on the host copies of the lengths and labels (CtcLoss.cs:40-153 raises
// the same conditions); on success *max_ext is the longest extended label sequence, 2 * max(tgt_len) + 1. The
// kernels index lp, dlp and their scratch with the device copies, which the caller keeps equal to these.
om_status check_args(om_ctx *ctx, const char *who, const int32_t *h_in_len, const int32_t *h_tgt_len,
                     const int32_t *h_targets, int n_targets, int T, int B, int C, int blank, int reduction,
                     int *max_ext) {
    OM_REQUIRE(ctx, h_in_len && h_tgt_len && (h_targets || n_targets == 0) && n_targets >= 0,
               "%s: the host lengths and targets are required", who);
    OM_REQUIRE(ctx, T >= 0 && B > 0 && C > 0, "%s: CtcLoss needs log-probabilities [T,B,C]", who);
    OM_REQUIRE(ctx, (unsigned)blank < (unsigned)C, "%s: The blank index %d is outside [0, %d).", who, blank, C);
    OM_REQUIRE(ctx, reduction >= 0 && reduction <= 2, "%s: bad reduction %d", who, reduction);
    int64_t total = 0;
    int ext = 1;
    for (int b = 0; b < B; b++) {
        OM_REQUIRE(ctx, (unsigned)h_in_len[b] <= (unsigned)T,
                   "%s: Input length %d of sequence %d is outside [0, %d].", who, h_in_len[b], b, T);
        OM_REQUIRE(ctx, h_tgt_len[b] >= 0 && h_tgt_len[b] <= (1 << 20),
                   "%s: Target length %d of sequence %d is negative or too long.", who, h_tgt_len[b], b);
        total += h_tgt_len[b];
        ext = 2 * h_tgt_len[b] + 1 > ext ? 2 * h_tgt_len[b] + 1 : ext;
    }
    OM_REQUIRE(ctx, total == n_targets, "%s: The target lengths sum to %lld but %d labels were given.", who,
               (long long)total, n_targets);
    for (int i = 0; i < n_targets; i++)
        OM_REQUIRE(ctx, (unsigned)h_targets[i] < (unsigned)C && h_targets[i] != blank,
                   "%s: Target label %d must be in [0, %d) and differ from the blank %d.", who, h_targets[i], C, blank);
    *max_ext = ext;
    return OM_OK;
}

}  // namespace

extern "C" {

om_status om_ctc_fwd(om_ctx *ctx, const float *lp, const int32_t *targets, const int32_t *in_len,
                     const int32_t *tgt_len, const int32_t *h_in_len, const int32_t *h_tgt_len,
                     const int32_t *h_targets, int n_targets, int T, int B, int C, int blank, int reduction,
                     int zero_infinity, float *loss) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, lp && targets && in_len && tgt_len && loss, "om_ctc_fwd: NULL pointer");
    int max_ext = 1;
    om_status s = check_args(ctx, "om_ctc_fwd", h_in_len, h_tgt_len, h_targets, n_targets, T, B, C, blank, reduction,
                             &max_ext);
    if (s) return s;
    float *scr;
    const uint64_t table = sizeof(double) * (uint64_t)(T > 0 ? T : 1) * max_ext;
    const bool in_lds = table <= kLdsTable;
    uint64_t need = sizeof(double) * B + (in_lds ? 0 : table * B);
    s = om::scratch(ctx, need, &scr);
    if (s) return s;
    double *per = reinterpret_cast<double *>(scr);
    double *alpha = in_lds ? nullptr : per + B;
    hipLaunchKernelGGL(k_ctc_fwd, dim3(B), dim3(kBlock), in_lds ? table : 0, ctx->stream, lp, targets, in_len, tgt_len,
                       T, B, C, blank, max_ext, alpha, per, in_lds ? 1 : 0);
    hipLaunchKernelGGL(k_ctc_reduce, dim3(1), dim3(64), 0, ctx->stream, per, tgt_len, B, reduction, zero_infinity,
                       loss);
    return OM_LAUNCH_CHECK(ctx, "om_ctc_fwd");
}

om_status om_ctc_bwd(om_ctx *ctx, const float *lp, const int32_t *targets, const int32_t *in_len,
                     const int32_t *tgt_len, const int32_t *h_in_len, const int32_t *h_tgt_len,
                     const int32_t *h_targets, int n_targets, const float *g, float *dlp, int T, int B, int C,
                     int blank, int reduction, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, lp && targets && in_len && tgt_len && g && dlp, "om_ctc_bwd: NULL pointer");
    int max_ext = 1;
    om_status s = check_args(ctx, "om_ctc_bwd", h_in_len, h_tgt_len, h_targets, n_targets, T, B, C, blank, reduction,
                             &max_ext);
    if (s) return s;
    float *scr = nullptr;
    uint64_t tt = T > 0 ? T : 1;
    const uint64_t table = sizeof(double) * tt * max_ext;  // one of the two tables
    const bool in_lds = table <= kLdsTable;
    if (!in_lds) {
        s = om::scratch(ctx, 2 * table * B, &scr);
        if (s) return s;
    }
    hipLaunchKernelGGL(k_ctc_bwd, dim3(B), dim3(kBwdBlock), in_lds ? 2 * table : 0, ctx->stream, lp, targets, in_len,
                       tgt_len, g, dlp, T, B, C, blank, reduction, max_ext, accumulate,
                       reinterpret_cast<double *>(scr), in_lds ? 1 : 0);
    return OM_LAUNCH_CHECK(ctx, "om_ctc_bwd");
}

uint64_t om_ctc_tables_bytes(int T, int B, int max_tgt_len) {
    if (T < 0 || B < 0 || max_tgt_len < 0) return 0;
    return sizeof(double) * 2 * (uint64_t)B * (uint64_t)(T > 0 ? T : 1) * (uint64_t)(2 * (int64_t)max_tgt_len + 1);
}

om_status om_ctc_fwd_tables(om_ctx *ctx, const float *lp, const int32_t *targets, const int32_t *in_len,
                            const int32_t *tgt_len, const int32_t *h_in_len, const int32_t *h_tgt_len,
                            const int32_t *h_targets, int n_targets, int T, int B, int C, int blank, int reduction,
                            int zero_infinity, float *loss, double *tables, uint64_t tables_bytes) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, lp && targets && in_len && tgt_len && loss && tables, "om_ctc_fwd_tables: NULL pointer");
    int max_ext = 1;
    om_status s = check_args(ctx, "om_ctc_fwd_tables", h_in_len, h_tgt_len, h_targets, n_targets, T, B, C, blank,
                             reduction, &max_ext);
    if (s) return s;
    const uint64_t tt = T > 0 ? T : 1, table = sizeof(double) * tt * max_ext;  // one of the two tables
    OM_REQUIRE(ctx, tables_bytes >= 2 * table * B,
               "om_ctc_fwd_tables: the tables need %llu bytes (om_ctc_tables_bytes), %llu given",
               (unsigned long long)(2 * table * B), (unsigned long long)tables_bytes);
    float *scr;
    s = om::scratch(ctx, sizeof(double) * B, &scr);
    if (s) return s;
    double *per = reinterpret_cast<double *>(scr);
    const bool in_lds = table <= kLdsTable;
    hipLaunchKernelGGL(k_ctc_fwd_tables, dim3(B), dim3(kBwdBlock), in_lds ? 2 * table : 0, ctx->stream, lp, targets,
                       in_len, tgt_len, T, B, C, blank, max_ext, tables, per, in_lds ? 1 : 0);
    hipLaunchKernelGGL(k_ctc_reduce, dim3(1), dim3(64), 0, ctx->stream, per, tgt_len, B, reduction, zero_infinity,
                       loss);
    return OM_LAUNCH_CHECK(ctx, "om_ctc_fwd_tables");
}

om_status om_ctc_bwd_tables(om_ctx *ctx, const float *lp, const int32_t *targets, const int32_t *in_len,
                            const int32_t *tgt_len, const int32_t *h_in_len, const int32_t *h_tgt_len,
                            const int32_t *h_targets, int n_targets, const float *g, float *dlp, int T, int B, int C,
                            int blank, int reduction, int accumulate, const double *tables, uint64_t tables_bytes) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, lp && targets && in_len && tgt_len && g && dlp && tables, "om_ctc_bwd_tables: NULL pointer");
    int max_ext = 1;
    om_status s = check_args(ctx, "om_ctc_bwd_tables", h_in_len, h_tgt_len, h_targets, n_targets, T, B, C, blank,
                             reduction, &max_ext);
    if (s) return s;
    const uint64_t tt = T > 0 ? T : 1, table = sizeof(double) * tt * max_ext;
    OM_REQUIRE(ctx, tables_bytes >= 2 * table * B,
               "om_ctc_bwd_tables: the tables need %llu bytes (om_ctc_tables_bytes), %llu given",
               (unsigned long long)(2 * table * B), (unsigned long long)tables_bytes);
    const bool in_lds = table <= kLdsTable;
    hipLaunchKernelGGL(k_ctc_bwd_tables, dim3(B), dim3(kBwdBlock), in_lds ? 2 * table : 0, ctx->stream, lp, targets,
                       in_len, tgt_len, g, dlp, T, B, C, blank, reduction, max_ext, accumulate, tables,
                       in_lds ? 1 : 0);
    return OM_LAUNCH_CHECK(ctx, "om_ctc_bwd_tables");
}

}  // extern "C"
