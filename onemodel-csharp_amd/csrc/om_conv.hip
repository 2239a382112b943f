// 2-D convolution (groups 1) as implicit GEMM on the MFMA engine, and max pooling with Int32 indices.
//
// Forward  (per image n):  y_n[co, p]   = sum_k W[co, k] * col_n[k, p]            M=Cout, N=OH*OW, K=Cin*KH*KW
// dX       (per image n):  dx_n[ci, q]  = sum_{co,ky,kx} Wt[ci, (co,ky,kx)] * g_n[co, oy(q,ky), ox(q,kx)]
//                                                                                 M=Cin,  N=H*W,   K=Cout*KH*KW
// dW       (per image n):  dW_n[co, k]  = sum_p g_n[co, p] * col_n[p, k]           M=Cout, N=Cin*KH*KW, K=OH*OW
//          then dW = sum over n in image order (fixed-order reduce of the per-image partials)
// col_n is the reference's im2col unfolding (BackwardNn.cs:404-428), gathered on the fly by the B loaders and never
// materialised; Wt is W with (ci) and (co) swapped, a small per-call transpose.
#include "om_gemm.hpp"

#include <cstdlib>

// 3x3, stride 1, padding 1 kernels (om_conv3.hip); each returns false when the shape is not one it takes. With
// `pool` (a ReLU stage whose max pool windows tile the output exactly), a forward that sums input-channel splits in
// a pass of its own pools in that pass and sets *pooled.
bool om_conv3_fwd(om_ctx *ctx, const float *x, const float *w, const float *bias, float *y, int N, int Cin, int H,
                  int W, int Cout, int acc, om_status *st, bool flip_weights, bool relu, const Conv3Pool *pool = nullptr,
                  bool *pooled = nullptr);
bool om_conv3_dw(om_ctx *ctx, const float *g, const float *x, float *dw, float *db, int N, int Cin, int H, int W,
                 int Cout, int acc, om_status *st);

namespace {

// The 3x3 / stride 1 / padding 1 geometry the staged kernels take (in a tuning build OM_CONV3=0 keeps every shape on
// k_conv, for comparisons).
bool conv3_geometry(int KH, int KW, int stride, int pad) {
    static const char *s = om::tuning_env("OM_CONV3");
    return KH == 3 && KW == 3 && stride == 1 && pad == 1 && !(s && s[0] == '0');
}

using namespace omg;

// B operand of the forward: B[k][p] = x[ci][oy*s - pad + ky][ox*s - pad + kx]; rows of the LDS tile are p (output
// pixels). Thread t always covers tile row t % ROWS, so its pixel decomposition is computed once per tile.
template <int ROWS>
struct LoadIm2colKP {
    static constexpr bool KLAYOUT = false;
    static constexpr int TOT = ROWS * BK, NE = (TOT + NT - 1) / NT;
    float v[NE];
    int oy, ox;
    bool valid;
    __device__ __forceinline__ void init(const Params &p, int r0) {
        int pix = r0 + (int)(threadIdx.x % ROWS);
        valid = pix < p.oh * p.ow;
        oy = valid ? pix / p.ow : 0;
        ox = valid ? pix % p.ow : 0;
    }
    __device__ __forceinline__ void fetch(const Params &p, const float *x, int kend, int k0) {
        const int khw = p.kh * p.kw;
#pragma unroll
        for (int i = 0; i < NE; i++) {
            int e = threadIdx.x + i * NT;
            float t = 0.0f;
            if (TOT % NT == 0 || e < TOT) {
                int kk = k0 + e / ROWS;
                if (valid && kk < kend) {
                    int ci = kk / khw, r = kk % khw, ky = r / p.kw, kx = r % p.kw;
                    int iy = oy * p.stride - p.pad + ky, ix = ox * p.stride - p.pad + kx;
                    if ((unsigned)iy < (unsigned)p.h && (unsigned)ix < (unsigned)p.w)
                        t = x[((int64_t)ci * p.h + iy) * p.w + ix];
                }
            }
            v[i] = t;
        }
    }
    __device__ __forceinline__ void put(float *T) const {
#pragma unroll
        for (int i = 0; i < NE; i++) {
            int e = threadIdx.x + i * NT;
            if (TOT % NT != 0 && e >= TOT) break;
            T[(e / ROWS) * (ROWS + PAD) + e % ROWS] = v[i];
        }
    }
};

// B operand of dW: B[k = p][n' = kk] = x[ci][oy*s - pad + ky][ox*s - pad + kx]; rows are kk = (ci, ky, kx).
template <int ROWS>
struct LoadIm2colPK {
    static constexpr bool KLAYOUT = false;
    static constexpr int TOT = ROWS * BK, NE = (TOT + NT - 1) / NT;
    float v[NE];
    int ci, ky, kx;
    bool valid;
    __device__ __forceinline__ void init(const Params &p, int r0) {
        int kk = r0 + (int)(threadIdx.x % ROWS);
        int khw = p.kh * p.kw;
        valid = kk < p.n;
        ci = valid ? kk / khw : 0;
        int r = valid ? kk % khw : 0;
        ky = r / p.kw;
        kx = r % p.kw;
    }
    __device__ __forceinline__ void fetch(const Params &p, const float *x, int kend, int k0) {
#pragma unroll
        for (int i = 0; i < NE; i++) {
            int e = threadIdx.x + i * NT;
            float t = 0.0f;
            if (TOT % NT == 0 || e < TOT) {
                int pix = k0 + e / ROWS;
                if (valid && pix < kend) {
                    int oy = pix / p.ow, ox = pix % p.ow;
                    int iy = oy * p.stride - p.pad + ky, ix = ox * p.stride - p.pad + kx;
                    if ((unsigned)iy < (unsigned)p.h && (unsigned)ix < (unsigned)p.w)
                        t = x[((int64_t)ci * p.h + iy) * p.w + ix];
                }
            }
            v[i] = t;
        }
    }
    __device__ __forceinline__ void put(float *T) const {
#pragma unroll
        for (int i = 0; i < NE; i++) {
            int e = threadIdx.x + i * NT;
            if (TOT % NT != 0 && e >= TOT) break;
            T[(e / ROWS) * (ROWS + PAD) + e % ROWS] = v[i];
        }
    }
};

// B operand of dX: B[k = (co, ky, kx)][q = (iy, ix)] = g[co][oy][ox] with oy*s - pad + ky = iy (and likewise x),
// zero where no output pixel maps there; rows are input pixels q.
template <int ROWS>
struct LoadConvDx {
    static constexpr bool KLAYOUT = false;
    static constexpr int TOT = ROWS * BK, NE = (TOT + NT - 1) / NT;
    float v[NE];
    int iy, ix;
    bool valid;
    __device__ __forceinline__ void init(const Params &p, int r0) {
        int q = r0 + (int)(threadIdx.x % ROWS);
        valid = q < p.h * p.w;
        iy = valid ? q / p.w : 0;
        ix = valid ? q % p.w : 0;
    }
    __device__ __forceinline__ void fetch(const Params &p, const float *g, int kend, int k0) {
        const int khw = p.kh * p.kw;
#pragma unroll
        for (int i = 0; i < NE; i++) {
            int e = threadIdx.x + i * NT;
            float t = 0.0f;
            if (TOT % NT == 0 || e < TOT) {
                int kk = k0 + e / ROWS;
                if (valid && kk < kend) {
                    int co = kk / khw, r = kk % khw, ky = r / p.kw, kx = r % p.kw;
                    int ny = iy + p.pad - ky, nx = ix + p.pad - kx;
                    if (ny >= 0 && nx >= 0 && ny % p.stride == 0 && nx % p.stride == 0) {
                        int oy = ny / p.stride, ox = nx / p.stride;
                        if (oy < p.oh && ox < p.ow) t = g[((int64_t)co * p.oh + oy) * p.ow + ox];
                    }
                }
            }
            v[i] = t;
        }
    }
    __device__ __forceinline__ void put(float *T) const {
#pragma unroll
        for (int i = 0; i < NE; i++) {
            int e = threadIdx.x + i * NT;
            if (TOT % NT != 0 && e >= TOT) break;
            T[(e / ROWS) * (ROWS + PAD) + e % ROWS] = v[i];
        }
    }
};

// mode 0: forward (A = W [Cout][K], B = im2col(x_n), C = y_n, bias per row)
// mode 1: dX (A = Wt [Cin][Cout*KK], B = gather(g_n), C = dx_n)
// mode 2: dW partial (A = g_n [Cout][P], B = im2col(x_n)^T, C = ws[n*splits + s] [Cout][Cin*KK], K range split s)
template <int BM, int BN, int MODE, bool VEC>
__global__ void __launch_bounds__(NT) k_conv(Params p) {
    OM_LDS_POISON();
    __shared__ __attribute__((aligned(16))) float As[2 * lds_size<BM, BK, true>()];
    __shared__ __attribute__((aligned(16))) float Bs[2 * lds_size<BN, BK, false>()];
    const int tiles_n = (p.n + BN - 1) / BN, tiles_m = (p.m + BM - 1) / BM;
    int tm, tn, zz;
    tile_coords(p, tiles_n, tiles_m, tm, tn, zz);
    if (zz >= p.batch * p.splits) return;
    const int img = zz / p.splits, split = zz % p.splits;
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = split * p.k_split, kend = min(p.k, kbeg + p.k_split);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int wm0 = (wv >> 1) * (BM / 2), wn0 = (wv & 1) * (BN / 2);
    const float *A = p.a + img * p.sa_outer;  // W (mode 0/1: sa_outer = 0) or g_n (mode 2)
    const float *Bsrc = p.b + img * p.sb_outer;
    LoadKContig<BM, BK, VEC> la;
    Tile<BM, BN, BK, true, false> t;
    const int M = p.m;
    const int64_t lda = p.lda;
    if constexpr (MODE == 0) {
        LoadIm2colKP<BN> lb;
        lb.init(p, n0);
        run_k<BM, BN, BK>(
            t, la, lb, [&](LoadKContig<BM, BK, VEC> &l, int k0) { l.fetch(A, lda, M, kend, m0, k0); },
            [&](LoadIm2colKP<BN> &l, int k0) { l.fetch(p, Bsrc, kend, k0); }, kbeg, kend, As, Bs, wm0, wn0, lane);
        store_tile(p, t, m0, n0, wm0, wn0, lane, p.c + img * p.sc_outer, p.ldc, nullptr, 0);
    } else if constexpr (MODE == 1) {
        LoadConvDx<BN> lb;
        lb.init(p, n0);
        run_k<BM, BN, BK>(
            t, la, lb, [&](LoadKContig<BM, BK, VEC> &l, int k0) { l.fetch(A, lda, M, kend, m0, k0); },
            [&](LoadConvDx<BN> &l, int k0) { l.fetch(p, Bsrc, kend, k0); }, kbeg, kend, As, Bs, wm0, wn0, lane);
        store_tile(p, t, m0, n0, wm0, wn0, lane, p.c + img * p.sc_outer, p.ldc, nullptr, 0);
    } else {
        LoadIm2colPK<BN> lb;
        lb.init(p, n0);
        run_k<BM, BN, BK>(
            t, la, lb, [&](LoadKContig<BM, BK, VEC> &l, int k0) { l.fetch(A, lda, M, kend, m0, k0); },
            [&](LoadIm2colPK<BN> &l, int k0) { l.fetch(p, Bsrc, kend, k0); }, kbeg, kend, As, Bs, wm0, wn0, lane);
        // partial of (image, split) -> ws slot img * splits + split (plain store, reduced in order afterwards)
        Params q = p;
        q.splits = 1;
        q.alpha = 1.0f;
        q.bias = nullptr;
        q.accumulate = 0;
        store_tile(q, t, m0, n0, wm0, wn0, lane, p.ws + (int64_t)zz * p.m * p.n, p.n, nullptr, 0);
    }
}

// dW = the sum over slots (image-major, then K split): a workgroup takes 64 consecutive weights (one per lane) and its
// four wavefronts the four quarters of the slot range, each in slot order, added in order at the end.
__global__ void __launch_bounds__(256) k_conv_dw_reduce(const float *__restrict__ ws, int slots, int64_t total,
                                                        float *__restrict__ dw, int acc) {
    OM_LDS_POISON();
    __shared__ float qs[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t e = (int64_t)blockIdx.x * 64 + lane;
    const int k0 = (int)((int64_t)slots * w / 4), k1 = (int)((int64_t)slots * (w + 1) / 4);
    float v = 0.0f;
    if (e < total) {
#pragma unroll 8
        for (int s = k0; s < k1; s++) v += ws[(int64_t)s * total + e];
    }
    qs[w][lane] = v;
    __syncthreads();
    if (w == 0 && e < total) {
        const float t = ((qs[0][lane] + qs[1][lane]) + qs[2][lane]) + qs[3][lane];
        dw[e] = acc ? dw[e] + t : t;
    }
}
// Wt[ci][co*KK + r] = W[co][ci][r]
__global__ void k_conv_wt(const float *__restrict__ w, float *__restrict__ wt, int cout, int cin, int kk) {
    OM_LDS_POISON();
    int64_t total = (int64_t)cout * cin * kk, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        int r = (int)(e % kk);
        int64_t t = e / kk;
        int ci = (int)(t % cin), co = (int)(t / cin);
        wt[((int64_t)ci * cout + co) * kk + r] = w[e];
    }
}
// dbias: per (n, co) plane a double sum (a wavefront per plane), then per co the planes in image order
// (BackwardNn.cs:325-345).
__global__ void k_conv_db_planes(const float *__restrict__ g, int planes, int plane, double *__restrict__ part) {
    OM_LDS_POISON();
    int wv = (blockIdx.x * blockDim.x + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (wv >= planes) return;
    const float *r = g + (int64_t)wv * plane;
    double acc = 0.0;
    for (int i = lane; i < plane; i += 64) acc += (double)r[i];
    acc = omd::wave_sum(acc);
    if (lane == 0) part[wv] = acc;
}
// A wavefront per output channel: lane l adds the planes of images l, l + 64, ... in order, then the fixed butterfly.
__global__ void k_conv_db_final(const double *__restrict__ part, int n, int cout, float *__restrict__ db, int acc) {
    OM_LDS_POISON();
    const int co = (int)(((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6), lane = threadIdx.x & 63;
    if (co >= cout) return;  // whole wavefronts leave together
    double s = 0.0;
    for (int i = lane; i < n; i += 64) s += part[(int64_t)i * cout + co];
    s = omd::wave_sum(s);
    if (lane == 0) {
        const float v = (float)s;
        db[co] = acc ? db[co] + v : v;
    }
}

template <int MODE>
void launch_conv(const Params &p, int bm, int bn, bool vec, hipStream_t st) {
    int64_t tiles = (int64_t)((p.m + bm - 1) / bm) * ((p.n + bn - 1) / bn) * p.batch * p.splits;
#define OMC(BM_, BN_)                                                                                          \
    if (bm == BM_ && bn == BN_) {                                                                              \
        if (vec) hipLaunchKernelGGL((k_conv<BM_, BN_, MODE, true>), dim3((unsigned)tiles), dim3(NT), 0, st, p); \
        else hipLaunchKernelGGL((k_conv<BM_, BN_, MODE, false>), dim3((unsigned)tiles), dim3(NT), 0, st, p);    \
        return;                                                                                                \
    }
    OMC(128, 128)
    OMC(64, 128)
    OMC(64, 64)
    OMC(32, 128)
#undef OMC
}

// Tile choice for a conv product: M is a channel count (often small), N a pixel or weight count.
void conv_tiles(int m, int n, int64_t batch, int cus, int &bm, int &bn) {
    if (m <= 32) {
        bm = 32;
        bn = 128;
        return;
    }
    if (m <= 64) {
        bm = 64;
        int64_t t128 = (int64_t)((n + 127) / 128) * batch;
        bn = t128 >= cus ? 128 : 64;
        return;
    }
    int64_t t = (int64_t)((m + 127) / 128) * ((n + 127) / 128) * batch;
    if (t >= cus) {
        bm = bn = 128;
    } else {
        bm = 64;
        bn = 128;
        if ((int64_t)((m + 63) / 64) * ((n + 127) / 128) * batch < cus) bn = 64;
    }
}

om_status conv_check(om_ctx *ctx, const char *what, int N, int Cin, int H, int W, int Cout, int KH, int KW,
                     int stride, int pad, int &OH, int &OW) {
    OM_REQUIRE(ctx, N > 0 && Cin > 0 && H > 0 && W > 0 && Cout > 0 && KH > 0 && KW > 0 && stride > 0 && pad >= 0,
               "%s: bad geometry N=%d Cin=%d H=%d W=%d Cout=%d K=%dx%d stride=%d pad=%d", what, N, Cin, H, W, Cout, KH,
               KW, stride, pad);
    OH = (H + 2 * pad - KH) / stride + 1;
    OW = (W + 2 * pad - KW) / stride + 1;
    OM_REQUIRE(ctx, H + 2 * pad >= KH && W + 2 * pad >= KW && OH >= 1 && OW >= 1,
               "%s: invalid convolution geometry for input %dx%d and kernel %dx%d", what, H, W, KH, KW);
    OM_REQUIRE(ctx, (int64_t)Cin * KH * KW < INT32_MAX && (int64_t)Cout * KH * KW < INT32_MAX &&
                        (int64_t)H * W < INT32_MAX, "%s: sizes overflow", what);
    return OM_OK;
}

Params conv_params(int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad, int OH, int OW) {
    Params p{};
    p.batch = N;
    p.batch_div = 1;
    p.alpha = 1.0f;
    p.splits = 1;
    p.cin = Cin;
    p.h = H;
    p.w = W;
    p.cout = Cout;
    p.kh = KH;
    p.kw = KW;
    p.stride = stride;
    p.pad = pad;
    p.oh = OH;
    p.ow = OW;
    p.xcd_remap = 1;
    return p;
}

// MaxPool2d forward (TensorKernels.cs:242-296): one thread per output; window in (ky, kx) order; the first candidate,
// a strictly larger value (unless the best is NaN), or the first NaN wins.
__global__ void k_maxpool_fwd(const float *__restrict__ x, float *__restrict__ y, int32_t *__restrict__ idx, int N,
                              int C, int H, int W, int OH, int OW, int KH, int KW, int SH, int SW, int PH, int PW) {
    OM_LDS_POISON();
    int64_t total = (int64_t)N * C * OH * OW, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += stride) {
        int ox = (int)(o % OW);
        int64_t t = o / OW;
        int oy = (int)(t % OH);
        int64_t nc = t / OH;
        float best = -__int_as_float(0x7F800000);
        int bi = -1;
        for (int ky = 0; ky < KH; ky++) {
            int yy = oy * SH - PH + ky;
            if ((unsigned)yy >= (unsigned)H) continue;
            for (int kx = 0; kx < KW; kx++) {
                int xx = ox * SW - PW + kx;
                if ((unsigned)xx >= (unsigned)W) continue;
                int fi = (int)((nc * H + yy) * W + xx);
                float v = x[fi];
                bool wins = bi < 0 || (v > best && best == best) || (v != v && best == best);
                if (wins) {
                    best = v;
                    bi = fi;
                }
            }
        }
        y[o] = best;
        if (idx) idx[o] = bi;
    }
}
// MaxPoolBackward (BackwardOps.cs:285-298) as a gather: each input element adds the gradients of the outputs whose
// saved index is that element, in increasing output order (the order of the reference's scatter loop). With relu_y
// (the pool's input, a ReLU's output) the ReLU backward follows in the same pass: the sum where relu_y > 0, else 0.
__global__ void k_maxpool_bwd(const float *__restrict__ g, const int32_t *__restrict__ idx, float *__restrict__ dx,
                              int N, int C, int H, int W, int OH, int OW, int KH, int KW, int SH, int SW, int PH,
                              int PW, int acc, const float *__restrict__ relu_y) {
    OM_LDS_POISON();
    int64_t total = (int64_t)N * C * H * W, stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        int ix = (int)(e % W);
        int64_t t = e / W;
        int iy = (int)(t % H);
        int64_t nc = t / H;
        // outputs whose window covers (iy, ix): oy*SH - PH <= iy < oy*SH - PH + KH
        int oy0 = iy + PH - KH + 1, oy1 = iy + PH;
        int ox0 = ix + PW - KW + 1, ox1 = ix + PW;
        oy0 = oy0 <= 0 ? 0 : (oy0 + SH - 1) / SH;
        ox0 = ox0 <= 0 ? 0 : (ox0 + SW - 1) / SW;
        oy1 = oy1 < 0 ? -1 : min(oy1 / SH, OH - 1);
        ox1 = ox1 < 0 ? -1 : min(ox1 / SW, OW - 1);
        float s = 0.0f;
        for (int oy = oy0; oy <= oy1; oy++)
            for (int ox = ox0; ox <= ox1; ox++) {
                int64_t o = (nc * OH + oy) * OW + ox;
                if (idx[o] == (int32_t)e) s += g[o];
            }
        if (relu_y) s = relu_y[e] > 0.0f ? s : 0.0f;
        dx[e] = acc ? dx[e] + s : s;
    }
}
// The same for windows that tile the input exactly (stride = window, no padding, H and W multiples of the window:
// every input element lies in exactly one window): a thread per window writes its KH x KW inputs, the window's
// gradient at the saved index (0 + g, as the gather's sum starting from zero gives) and zero elsewhere.
__global__ void k_maxpool_bwd_tiled(const float *__restrict__ g, const int32_t *__restrict__ idx,
                                    float *__restrict__ dx, int planes, int H, int W, int OH, int OW, int KH, int KW,
                                    int acc, const float *__restrict__ relu_y) {
    OM_LDS_POISON();
    const int total = planes * OH * OW;
    for (int o = blockIdx.x * blockDim.x + threadIdx.x; o < total; o += gridDim.x * blockDim.x) {
        const int ox = o % OW, t = o / OW, oy = t % OH, pl = t / OH;
        const int win = idx[o];
        const float gv = 0.0f + g[o];
        for (int ky = 0; ky < KH; ky++) {
            const int e0 = (pl * H + oy * KH + ky) * W + ox * KW;
            for (int kx = 0; kx < KW; kx++) {
                const int e = e0 + kx;
                float v = e == win ? gv : 0.0f;
                if (relu_y) v = relu_y[e] > 0.0f ? v : 0.0f;
                dx[e] = acc ? dx[e] + v : v;
            }
        }
    }
}
// Launches the tiled form where it applies, else the gather.
void maxpool_bwd_launch(hipStream_t st, const float *g, const int32_t *idx, float *dx, int N, int C, int H, int W,
                        int OH, int OW, int KH, int KW, int SH, int SW, int PH, int PW, int acc, const float *relu_y) {
    if (SH == KH && SW == KW && PH == 0 && PW == 0 && H == OH * KH && W == OW * KW &&
        (int64_t)N * C * H * W <= INT32_MAX) {
        hipLaunchKernelGGL(k_maxpool_bwd_tiled, dim3(om::grid1d((int64_t)N * C * OH * OW, 256, 1 << 20)), dim3(256), 0,
                           st, g, idx, dx, N * C, H, W, OH, OW, KH, KW, acc, relu_y);
        return;
    }
    hipLaunchKernelGGL(k_maxpool_bwd, dim3(om::grid1d((int64_t)N * C * H * W, 256, 1 << 20)), dim3(256), 0, st, g, idx,
                       dx, N, C, H, W, OH, OW, KH, KW, SH, SW, PH, PW, acc, relu_y);
}

}  // namespace

extern "C" {

static om_status conv_fwd(om_ctx *ctx, const char *what, const float *x, const float *w, const float *bias, float *y,
                          int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad, bool relu) {
    OM_CHECK_CTX(ctx);
    int OH, OW;
    om_status s = conv_check(ctx, what, N, Cin, H, W, Cout, KH, KW, stride, pad, OH, OW);
    if (s) return s;
    OM_REQUIRE(ctx, x && w && y, "%s: NULL pointer", what);
    if (conv3_geometry(KH, KW, stride, pad) && om_conv3_fwd(ctx, x, w, bias, y, N, Cin, H, W, Cout, 0, &s, false, relu))
        return s;
    Params p = conv_params(N, Cin, H, W, Cout, KH, KW, stride, pad, OH, OW);
    p.m = Cout;
    p.n = OH * OW;
    p.k = Cin * KH * KW;
    p.k_split = p.k;
    p.a = w;
    p.lda = p.k;
    p.sa_outer = 0;
    p.b = x;
    p.sb_outer = (int64_t)Cin * H * W;
    p.c = y;
    p.ldc = p.n;
    p.sc_outer = (int64_t)Cout * p.n;
    p.bias = bias;
    p.bias_per_row = 1;
    p.epi = relu ? omg::EPI_RELU : omg::EPI_NONE;  // ReLU after the bias, in the store
    bool vec = ((uintptr_t)w % 16 == 0) && p.k % 4 == 0;
    int bm, bn;
    conv_tiles(p.m, p.n, N, ctx->num_cus, bm, bn);
    launch_conv<0>(p, bm, bn, vec, ctx->stream);
    return OM_LAUNCH_CHECK(ctx, what);
}

om_status om_conv2d_fwd(om_ctx *ctx, const float *x, const float *w, const float *bias, float *y, int N, int Cin,
                        int H, int W, int Cout, int KH, int KW, int stride, int pad) {
    return conv_fwd(ctx, "om_conv2d_fwd", x, w, bias, y, N, Cin, H, W, Cout, KH, KW, stride, pad, false);
}

om_status om_conv2d_relu_fwd(om_ctx *ctx, const float *x, const float *w, const float *bias, float *y, int N, int Cin,
                             int H, int W, int Cout, int KH, int KW, int stride, int pad) {
    return conv_fwd(ctx, "om_conv2d_relu_fwd", x, w, bias, y, N, Cin, H, W, Cout, KH, KW, stride, pad, true);
}

om_status om_conv2d_relu_pool_fwd(om_ctx *ctx, const float *x, const float *w, const float *bias, float *a, float *y,
                                  int32_t *idx, int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride,
                                  int pad, int pkh, int pkw, int psh, int psw) {
    OM_CHECK_CTX(ctx);
    int OH, OW;
    om_status s = conv_check(ctx, "om_conv2d_relu_pool_fwd", N, Cin, H, W, Cout, KH, KW, stride, pad, OH, OW);
    if (s) return s;
    OM_REQUIRE(ctx, x && w && a && y, "om_conv2d_relu_pool_fwd: NULL pointer");
    OM_REQUIRE(ctx, pkh > 0 && pkw > 0 && psh > 0 && psw > 0 && pkh <= OH && pkw <= OW,
               "om_conv2d_relu_pool_fwd: bad pooling window %dx%d / %dx%d over %dx%d", pkh, pkw, psh, psw, OH, OW);
    OM_REQUIRE(ctx, (int64_t)N * Cout * OH * OW <= INT32_MAX, "om_conv2d_relu_pool_fwd: Int32 indices cannot address "
                                                              "the convolution's output");
    if (conv3_geometry(KH, KW, stride, pad) && psh == pkh && psw == pkw && OH % pkh == 0 && OW % pkw == 0) {
        const Conv3Pool pool{y, idx, pkh, pkw};
        bool pooled = false;
        if (om_conv3_fwd(ctx, x, w, bias, a, N, Cin, H, W, Cout, 0, &s, false, true, &pool, &pooled)) {
            if (s || pooled) return s;
            return om_maxpool_fwd(ctx, a, y, idx, N, Cout, OH, OW, pkh, pkw, psh, psw, 0, 0);
        }
    }
    s = om_conv2d_relu_fwd(ctx, x, w, bias, a, N, Cin, H, W, Cout, KH, KW, stride, pad);
    return s ? s : om_maxpool_fwd(ctx, a, y, idx, N, Cout, OH, OW, pkh, pkw, psh, psw, 0, 0);
}

om_status om_conv2d_bwd(om_ctx *ctx, const float *g, const float *x, const float *w, float *dx, float *dw, float *db,
                        int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad, int acc_dx,
                        int acc_params) {
    OM_CHECK_CTX(ctx);
    int OH, OW;
    om_status s = conv_check(ctx, "om_conv2d_bwd", N, Cin, H, W, Cout, KH, KW, stride, pad, OH, OW);
    if (s) return s;
    OM_REQUIRE(ctx, g && (!dx || w) && (!dw || x), "om_conv2d_bwd: NULL pointer");
    const int P = OH * OW, KK = KH * KW, Kc = Cin * KK;
    const bool c3 = conv3_geometry(KH, KW, stride, pad);
    // the staged weight-gradient kernels also produce the bias gradient from the g tiles they stage
    if (dw && c3 && om_conv3_dw(ctx, g, x, dw, db, N, Cin, H, W, Cout, acc_params, &s)) {
        if (s) return s;
        dw = nullptr;  // done
        db = nullptr;
    }
    if (db) {
        float *scr;
        s = om::scratch(ctx, sizeof(double) * (uint64_t)N * Cout, &scr);
        if (s) return s;
        double *part = reinterpret_cast<double *>(scr);
        hipLaunchKernelGGL(k_conv_db_planes, dim3(om::grid1d((int64_t)N * Cout * 64, 256, 1 << 30)), dim3(256), 0,
                           ctx->stream, g, N * Cout, P, part);
        hipLaunchKernelGGL(k_conv_db_final, dim3((unsigned)((Cout + 3) / 4)), dim3(256), 0, ctx->stream, part, N, Cout,
                           db, acc_params);
        s = OM_LAUNCH_CHECK(ctx, "om_conv2d_bwd db");
        if (s) return s;
    }
    if (dx && c3 && om_conv3_fwd(ctx, g, w, nullptr, dx, N, Cout, H, W, Cin, acc_dx, &s, true, false)) {
        if (s) return s;
        dx = nullptr;  // done
    }
    if (dw) {
        Params p = conv_params(N, Cin, H, W, Cout, KH, KW, stride, pad, OH, OW);
        p.m = Cout;
        p.n = Kc;
        p.k = P;
        int bm, bn;
        conv_tiles(p.m, p.n, N, ctx->num_cus, bm, bn);
        int64_t tiles = (int64_t)((p.m + bm - 1) / bm) * ((p.n + bn - 1) / bn) * N;
        // split the pixels of an image when images alone leave the chip idle
        int splits = 1;
        if (tiles < 2 * ctx->num_cus && P >= 1024) {
            splits = (int)((2 * ctx->num_cus + tiles - 1) / tiles);
            int maxs = P / 512;
            if (splits > maxs) splits = maxs > 1 ? maxs : 1;
        }
        p.k_split = ((P + splits - 1) / splits + BK - 1) / BK * BK;
        p.splits = (P + p.k_split - 1) / p.k_split;
        p.a = g;
        p.lda = P;
        p.sa_outer = (int64_t)Cout * P;
        p.b = x;
        p.sb_outer = (int64_t)Cin * H * W;
        int slots = N * p.splits;
        float *ws;
        s = om::scratch(ctx, sizeof(float) * (uint64_t)slots * Cout * Kc + 256, &ws);
        if (s) return s;
        p.ws = ws;
        bool vec = ((uintptr_t)g % 16 == 0) && P % 4 == 0;
        launch_conv<2>(p, bm, bn, vec, ctx->stream);
        hipLaunchKernelGGL(k_conv_dw_reduce, dim3((unsigned)(((int64_t)Cout * Kc + 63) / 64)), dim3(256), 0,
                           ctx->stream, ws, slots, (int64_t)Cout * Kc, dw, acc_params);
        s = OM_LAUNCH_CHECK(ctx, "om_conv2d_bwd dw");
        if (s) return s;
    }
    if (dx) {
        // Wt lives in the step region's scratch-free space: allocate from the context scratch after the dW
        // partials are consumed (same stream, so ordering holds).
        float *wt;
        s = om::scratch(ctx, sizeof(float) * (uint64_t)Cout * Kc + 256, &wt);
        if (s) return s;
        hipLaunchKernelGGL(k_conv_wt, dim3(om::grid1d((int64_t)Cout * Kc, 256, 4096)), dim3(256), 0, ctx->stream, w,
                           wt, Cout, Cin, KK);
        Params p = conv_params(N, Cin, H, W, Cout, KH, KW, stride, pad, OH, OW);
        p.m = Cin;
        p.n = H * W;
        p.k = Cout * KK;
        p.k_split = p.k;
        p.a = wt;
        p.lda = p.k;
        p.sa_outer = 0;
        p.b = g;
        p.sb_outer = (int64_t)Cout * P;
        p.c = dx;
        p.ldc = p.n;
        p.sc_outer = (int64_t)Cin * H * W;
        p.accumulate = acc_dx;
        bool vec = p.k % 4 == 0;
        int bm, bn;
        conv_tiles(p.m, p.n, N, ctx->num_cus, bm, bn);
        launch_conv<1>(p, bm, bn, vec, ctx->stream);
        s = OM_LAUNCH_CHECK(ctx, "om_conv2d_bwd dx");
        if (s) return s;
    }
    return OM_OK;
}

om_status om_maxpool_fwd(om_ctx *ctx, const float *x, float *y, int32_t *idx, int N, int C, int H, int W, int KH,
                         int KW, int SH, int SW, int PH, int PW) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && y && N > 0 && C > 0 && H > 0 && W > 0 && KH > 0 && KW > 0 && SH > 0 && SW > 0 && PH >= 0 &&
                        PW >= 0, "om_maxpool_fwd: bad arguments");
    OM_REQUIRE(ctx, (int64_t)N * C * H * W <= INT32_MAX, "om_maxpool_fwd: Int32 indices cannot address the input");
    int OH = (H + 2 * PH - KH) / SH + 1, OW = (W + 2 * PW - KW) / SW + 1;
    OM_REQUIRE(ctx, OH >= 1 && OW >= 1, "om_maxpool_fwd: window larger than the padded input");
    hipLaunchKernelGGL(k_maxpool_fwd, dim3(om::grid1d((int64_t)N * C * OH * OW, 256, 1 << 20)), dim3(256), 0,
                       ctx->stream, x, y, idx, N, C, H, W, OH, OW, KH, KW, SH, SW, PH, PW);
    return OM_LAUNCH_CHECK(ctx, "om_maxpool_fwd");
}

om_status om_maxpool_bwd(om_ctx *ctx, const float *g, const int32_t *idx, float *dx, int N, int C, int H, int W,
                         int OH, int OW, int KH, int KW, int SH, int SW, int PH, int PW, int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && idx && dx && N > 0 && C > 0 && H > 0 && W > 0 && OH > 0 && OW > 0 && SH > 0 && SW > 0,
               "om_maxpool_bwd: bad arguments");
    maxpool_bwd_launch(ctx->stream, g, idx, dx, N, C, H, W, OH, OW, KH, KW, SH, SW, PH, PW, accumulate, nullptr);
    return OM_LAUNCH_CHECK(ctx, "om_maxpool_bwd");
}

om_status om_maxpool_relu_bwd(om_ctx *ctx, const float *g, const int32_t *idx, const float *y, float *dx, int N,
                              int C, int H, int W, int OH, int OW, int KH, int KW, int SH, int SW, int PH, int PW,
                              int accumulate) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && idx && y && dx && N > 0 && C > 0 && H > 0 && W > 0 && OH > 0 && OW > 0 && SH > 0 && SW > 0,
               "om_maxpool_relu_bwd: bad arguments");
    maxpool_bwd_launch(ctx->stream, g, idx, dx, N, C, H, W, OH, OW, KH, KW, SH, SW, PH, PW, accumulate, y);
    return OM_LAUNCH_CHECK(ctx, "om_maxpool_relu_bwd");
}

}  // extern "C"
