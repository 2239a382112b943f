// 3x3 convolutions with stride 1 and padding 1 (every convolution of the benchmark's conv block and CRNN) as
// implicit GEMM on MFMA, the input staged through LDS once per tile (Ops.Conv2d, Ops.Layers.cs:279-336; ConvBackward,
// BackwardNn.cs:317-402).
//
// Forward: y[n][co][p] = bias[co] + sum over taps t = (ky, kx) and channels ci of W[co][ci][t] x[n][ci][p + shift(t)]
// (zero outside the image). A workgroup takes 128 output pixels (flattened, so any width works) of one image and a
// block of 32 or 64 output channels; per chunk of 8 input channels it stages the input rows those pixels touch, halo
// included, into LDS (each input value is then read by all nine taps from there) and the chunk's weights, laid out
// [tap][co][ci]. Each lane keeps the LDS offsets of its two pixels; a tap is a constant shift of them, so the inner
// loop has no index arithmetic. Four wavefronts of 32 pixels x all the block's channels, v_mfma_f32_16x16x4f32.
// dX: for stride 1 and padding 1, dx[n][ci][q] = sum over taps and co of W[co][ci][8 - t] g[n][co][q + shift(t)]:
// the same kernel over g with the weights flipped and transposed ([ci][tap][co]).
// dW: dW[co][ci][t] = sum over images and pixels of g[n][co][p] x[n][ci][p + shift(t)]: a workgroup takes 64 output
// channels x 16 input channels x all nine taps and a slot of (image, 64-pixel chunk) work items, stages each chunk's
// g block and input rows, and accumulates in registers; the slots' partials are summed in slot order afterwards, so
// the result depends only on the shape.
// Sums run in another order than the reference's im2col GEMM; they are fp32 sums of the same products (1e-5 scaled
// error, tested).
#include "om_internal.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kThreads = 256;
constexpr int kFwdCk = 8;    // input channels per staged chunk (forward, dX)
constexpr int kFwdPx = 128;  // output pixels per workgroup (forward, dX)
constexpr int kWLd = kFwdCk + 4;  // row stride of the staged weights [tap][co][ci]
constexpr int kDwCi = 16;    // input channels per workgroup (dW)
constexpr int kDwCo = 64;    // output channels per workgroup (dW)
constexpr int kDwPx = 64;    // pixels per staged chunk (dW)
constexpr int kGLd = kDwPx + 4;

// Workgroup id with consecutive ids on one XCD (the hardware deals workgroups round-robin over the 8 XCDs).
__device__ __forceinline__ int xcd_lin() {
    int lin = blockIdx.x;
    const int total = gridDim.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    return lin;
}

// The input rows a tile touches, staged into LDS as planes [chans][ps] of R rows of rs = W + 8 floats: column
// ix (0 <= ix < W) at 4 + ix, the halo columns ix = -1 and ix = W at 3 and W + 4 (zero, written once per kernel by
// zero_halo), so the interior of a row is 16-byte aligned and moves as float4. Each thread handles up to NS float4
// of the tile, whose LDS offsets and row numbers it works out once; per chunk it loads them into registers (issued
// ahead, while the previous chunk computes) and stores them later. Rows outside the image store zeros.
template <int NS>
struct RowStage {
    int lo[NS];   // LDS offset of the float4 (-1: none)
    int gb[NS];   // its global offset within the channel's plane for a tile starting at row 0: row r - 1, column 4 q
    int rk[NS];   // its staged row r (low 16 bits) and channel (high bits)
    floatx4 v[NS];
    __device__ __forceinline__ void init(int chans, int W, int R, int ps) {
        const int Q = W / 4, rs = W + 8, total = chans * R * Q;
#pragma unroll
        for (int k = 0; k < NS; k++) {
            const int f = threadIdx.x + k * kThreads;
            lo[k] = -1;
            gb[k] = 0;
            rk[k] = 0;
            if (f < total) {
                const int q = f % Q, cr = f / Q, r = cr % R, ci = cr / R;
                lo[k] = ci * ps + r * rs + 4 + 4 * q;
                rk[k] = r;
                gb[k] = (r - 1) * W + 4 * q;  // load adds the channel's plane and the tile's first row
                rk[k] |= ci << 16;            // the channel rides in the high half
            }
        }
    }
    __device__ __forceinline__ void load(const float *src, int H, int W, int oy0) {
#pragma unroll
        for (int k = 0; k < NS; k++) {
            const int r = rk[k] & 0xFFFF, ci = rk[k] >> 16, iy = oy0 - 1 + r;
            v[k] = floatx4{0.f, 0.f, 0.f, 0.f};
            if (lo[k] >= 0 && (unsigned)iy < (unsigned)H)
                v[k] = *reinterpret_cast<const floatx4 *>(src + ((int64_t)ci * H + oy0) * W + gb[k]);
        }
    }
    __device__ __forceinline__ void store(float *dst) const {
#pragma unroll
        for (int k = 0; k < NS; k++)
            if (lo[k] >= 0) *reinterpret_cast<floatx4 *>(dst + lo[k]) = v[k];
    }
};

__device__ __forceinline__ void zero_halo(float *dst, int chans, int W, int R, int ps) {
    const int rs = W + 8;
    for (int f = threadIdx.x; f < chans * R * 2; f += kThreads) {
        const int side = f & 1, cr = f >> 1, r = cr % R, ci = cr / R;
        dst[ci * ps + r * rs + (side ? W + 4 : 3)] = 0.0f;
    }
}

// out[n][co][p] (+)= bias[co] + sum_{tap, ci} wr[co][tap][ci] in[n][ci][p + shift(tap)], BM output channels per
// workgroup. in is [N][cin][H][W], out [N][cout][H][W], wr [cout][9][cin].
template <int BM, int NS>
__global__ void __launch_bounds__(kThreads) k_conv3_fwd(const float *__restrict__ in, const float *__restrict__ wr,
                                                        const float *__restrict__ bias, float *out, int cin, int cout,
                                                        int H, int W, int R, int ps, int ntile, int acc) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    constexpr int MB = BM / 16, NWI = (9 * BM * 2 + kThreads - 1) / kThreads;
    float *Ws = lds;                   // [9][BM][kWLd]
    float *Xs = lds + 9 * BM * kWLd;   // [kFwdCk][ps]
    const int P = H * W, rs = W + 8, ncb = cout / BM;
    const int lin = xcd_lin();
    const int tile = lin % ntile, cb = (lin / ntile) % ncb, n = lin / ntile / ncb;
    const int p0 = tile * kFwdPx, co0 = cb * BM, oy0 = p0 / W;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = lane & 15, kl = lane >> 4;
    int boff[2];
    bool pv[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int p = p0 + 32 * w + 16 * j + t;
        pv[j] = p < P;
        boff[j] = pv[j] ? (p / W - oy0) * rs + p % W + 3 : 0;  // column ix + kx - 1 sits at 4 + ix + kx - 1
    }
    // the weight float4s this thread stages: global offset without the chunk's c0, and LDS offset
    int wgo[NWI], wlo[NWI];
    floatx4 wv4[NWI];
#pragma unroll
    for (int i = 0; i < NWI; i++) {
        const int f = threadIdx.x + i * kThreads, half = f & 1, co = (f >> 1) % BM, tap = (f >> 1) / BM;
        wlo[i] = f < 9 * BM * 2 ? (tap * BM + co) * kWLd + 4 * half : -1;
        wgo[i] = ((co0 + co) * 9 + tap) * cin + 4 * half;
    }
    RowStage<NS> xs;
    xs.init(kFwdCk, W, R, ps);
    zero_halo(Xs, kFwdCk, W, R, ps);
    floatx4 accv[MB][2];
#pragma unroll
    for (int i = 0; i < MB; i++) accv[i][0] = accv[i][1] = floatx4{0.f, 0.f, 0.f, 0.f};
    const float *inn = in + (int64_t)n * cin * P;
    auto load = [&](int c0) {
#pragma unroll
        for (int i = 0; i < NWI; i++)
            if (wlo[i] >= 0) wv4[i] = *reinterpret_cast<const floatx4 *>(wr + wgo[i] + c0);
        xs.load(inn + (int64_t)c0 * P, H, W, oy0);
    };
    load(0);
    for (int c0 = 0; c0 < cin; c0 += kFwdCk) {
        __syncthreads();  // the previous chunk's reads are done
#pragma unroll
        for (int i = 0; i < NWI; i++)
            if (wlo[i] >= 0) *reinterpret_cast<floatx4 *>(Ws + wlo[i]) = wv4[i];
        xs.store(Xs);
        __syncthreads();
        if (c0 + kFwdCk < cin) load(c0 + kFwdCk);  // in flight while this chunk computes
#pragma unroll
        for (int tap = 0; tap < 9; tap++) {
            const int toff = (tap / 3) * rs + tap % 3;
            floatx2 a[MB];
#pragma unroll
            for (int i = 0; i < MB; i++)
                a[i] = *reinterpret_cast<const floatx2 *>(Ws + (tap * BM + 16 * i + t) * kWLd + 2 * kl);
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float *xc = Xs + (2 * kl + u) * ps + toff;
                const float b0 = xc[boff[0]], b1 = xc[boff[1]];
#pragma unroll
                for (int i = 0; i < MB; i++) {
                    accv[i][0] = mfma4(a[i][u], b0, accv[i][0]);
                    accv[i][1] = mfma4(a[i][u], b1, accv[i][1]);
                }
            }
        }
    }
    // lane (t, kl), register r: channel co0 + 16 i + 4 kl + r, pixel p0 + 32 w + 16 j + t
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int co = co0 + 16 * i + 4 * kl + r;
            const float bv = bias ? bias[co] : 0.0f;
            float *orow = out + ((int64_t)n * cout + co) * P;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if (!pv[j]) continue;
                const int p = p0 + 32 * w + 16 * j + t;
                const float v = bias ? accv[i][j][r] + bv : accv[i][j][r];
                orow[p] = acc ? orow[p] + v : v;
            }
        }
}

// wr[co][tap][ci] = W[co][ci][tap] (forward); with flip, wr[ci][tap][co] = W[co][ci][8 - tap] (dX).
__global__ void k_conv3_wt(const float *__restrict__ w, float *__restrict__ wr, int cout, int cin, int flip) {
    const int64_t total = (int64_t)cout * cin * 9;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int tap = (int)(e % 9);
        const int64_t cc = e / 9;
        const int ci = (int)(cc % cin), co = (int)(cc / cin);
        if (flip) wr[((int64_t)ci * 9 + (8 - tap)) * cout + co] = w[e];
        else wr[((int64_t)co * 9 + tap) * cin + ci] = w[e];
    }
}

// part[slot][co][tap][ci] = the slot's items' sums of g[n][co][p] x[n][ci][p + shift(tap)]. The next item's g
// block and input rows are loaded into registers while the current one computes.
template <int NS>
__global__ void __launch_bounds__(kThreads) k_conv3_dw(const float *__restrict__ g, const float *__restrict__ x,
                                                       float *__restrict__ part, int cin, int cout, int H, int W,
                                                       int R, int ps, int nchunks, int items, int per) {
    constexpr int NG = kDwCo * kDwPx / 4 / kThreads;
    __shared__ __attribute__((aligned(16))) float Gs[kDwCo * kGLd];
    __shared__ int boff[kDwPx];
    extern __shared__ __attribute__((aligned(16))) float Xs[];  // [kDwCi][ps]
    const int P = H * W, rs = W + 8, ncob = cout / kDwCo, ncib = cin / kDwCi;
    const int lin = xcd_lin();
    const int cib = lin % ncib, cob = (lin / ncib) % ncob, slot = lin / ncib / ncob;
    const int co0 = cob * kDwCo, ci0 = cib * kDwCi;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = lane & 15, kl = lane >> 4;
    int gco[NG], gpx[NG];  // this thread's float4s of the g block: channel, first pixel
    floatx4 gv[NG];
#pragma unroll
    for (int k = 0; k < NG; k++) {
        const int f = threadIdx.x + k * kThreads;
        gco[k] = f / (kDwPx / 4);
        gpx[k] = (f % (kDwPx / 4)) * 4;
    }
    RowStage<NS> xs;
    xs.init(kDwCi, W, R, ps);
    zero_halo(Xs, kDwCi, W, R, ps);
    floatx4 accv[9];
#pragma unroll
    for (int tap = 0; tap < 9; tap++) accv[tap] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int i0 = slot * per, i1 = min(items, i0 + per);
    auto load = [&](int item) {
        const int n = item / nchunks, p0 = (item - n * nchunks) * kDwPx;
        const float *gn = g + ((int64_t)n * cout + co0) * P;
#pragma unroll
        for (int k = 0; k < NG; k++)
            gv[k] = p0 + gpx[k] < P ? *reinterpret_cast<const floatx4 *>(gn + (int64_t)gco[k] * P + p0 + gpx[k])
                                    : floatx4{0.f, 0.f, 0.f, 0.f};
        xs.load(x + ((int64_t)n * cin + ci0) * P, H, W, p0 / W);
    };
    if (i0 < i1) load(i0);
    for (int item = i0; item < i1; item++) {
        const int n = item / nchunks, p0 = (item - n * nchunks) * kDwPx, oy0 = p0 / W;
        __syncthreads();  // the previous item's reads are done
#pragma unroll
        for (int k = 0; k < NG; k++) *reinterpret_cast<floatx4 *>(Gs + gco[k] * kGLd + gpx[k]) = gv[k];
        xs.store(Xs);
        if (threadIdx.x < kDwPx) {
            const int p = p0 + threadIdx.x;
            boff[threadIdx.x] = p < P ? (p / W - oy0) * rs + p % W + 3 : 0;
        }
        __syncthreads();
        if (item + 1 < i1) load(item + 1);  // in flight while this item computes
#pragma unroll
        for (int ks = 0; ks < kDwPx / 16; ks++) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(Gs + (16 * w + t) * kGLd + 16 * ks + 4 * kl);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float *xc = Xs + t * ps + boff[16 * ks + 4 * kl + u];
#pragma unroll
                for (int tap = 0; tap < 9; tap++) accv[tap] = mfma4(a[u], xc[(tap / 3) * rs + tap % 3], accv[tap]);
            }
        }
    }
    // lane (t, kl), register r: output channel co0 + 16 w + 4 kl + r, input channel ci0 + t
#pragma unroll
    for (int tap = 0; tap < 9; tap++)
#pragma unroll
        for (int r = 0; r < 4; r++)
            part[(((int64_t)slot * cout + co0 + 16 * w + 4 * kl + r) * 9 + tap) * cin + ci0 + t] = accv[tap][r];
}

// dW[co][ci][tap] (+)= sum over slots 0, 1, ... of part[slot][co][tap][ci], in that order.
__global__ void k_conv3_dw_reduce(const float *__restrict__ part, int slots, int cout, int cin, float *dw, int acc) {
    const int64_t total = (int64_t)cout * 9 * cin;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        float s = part[e];
        for (int k = 1; k < slots; k++) s += part[(int64_t)k * total + e];
        const int ci = (int)(e % cin);
        const int64_t ct = e / cin;
        const int tap = (int)(ct % 9), co = (int)(ct / 9);
        float *d = dw + ((int64_t)co * cin + ci) * 9 + tap;
        *d = acc ? *d + s : s;
    }
}

// Rows of the staged input a run of `px` flattened output pixels can touch, halo included, and the LDS plane stride
// (rows of W + 8 floats, padded so that 2 * ps is 16 mod 64 floats: lanes of the four k groups read different banks).
void stage_geometry(int W, int px, int &R, int &ps) {
    R = (W - 1 + px - 1) / W + 3;
    ps = R * (W + 8);
    ps += ((8 - ps % 16) + 16) % 16;
}
// float4s per thread to stage `chans` channels of R rows (0 when more than the kernels carry in registers).
int stage_ns(int chans, int W, int R) {
    const int ns = (chans * R * (W / 4) + kThreads - 1) / kThreads;
    for (int c : {1, 2, 3, 4, 6, 8})
        if (ns <= c) return c;
    return 0;
}

}  // namespace

// The 3x3 / stride 1 / padding 1 paths; each returns false (launching nothing) when the shape is not one it takes.
bool om_conv3_fwd(om_ctx *ctx, const float *x, const float *w, const float *bias, float *y, int N, int Cin, int H,
                  int W, int Cout, int acc, om_status *st, bool flip_weights) {
    *st = OM_OK;
    const int P = H * W;
    if (Cin % kFwdCk || Cout % 32 || W % 4 || (int64_t)N * Cin * P > INT32_MAX || (int64_t)N * Cout * P > INT32_MAX ||
        (int64_t)Cout * 9 * Cin > INT32_MAX)
        return false;
    int R, ps;
    stage_geometry(W, kFwdPx, R, ps);
    const int ns = stage_ns(kFwdCk, W, R);
    if (!ns) return false;
    const int BM = Cout % 64 == 0 ? 64 : 32;
    float *wr;
    *st = om::scratch(ctx, sizeof(float) * (uint64_t)Cout * Cin * 9, &wr);
    if (*st) return true;
    // forward: W [Cout][Cin][9] -> wr [Cout][9][Cin]; dX (flip): the layer's W [Cout_l][Cin_l][9], where this call's
    // Cin is Cout_l and its Cout is Cin_l -> wr [Cin_l][9][Cout_l] with the taps reversed
    const int64_t nw = (int64_t)Cout * Cin * 9;
    if (flip_weights)
        hipLaunchKernelGGL(k_conv3_wt, dim3(om::grid1d(nw, 256, 1024)), dim3(256), 0, ctx->stream, w, wr, Cin, Cout, 1);
    else
        hipLaunchKernelGGL(k_conv3_wt, dim3(om::grid1d(nw, 256, 1024)), dim3(256), 0, ctx->stream, w, wr, Cout, Cin, 0);
    const int ntile = (P + kFwdPx - 1) / kFwdPx;
    const size_t lds = sizeof(float) * (9 * (size_t)BM * kWLd + (size_t)kFwdCk * ps);
    const dim3 grid((unsigned)((int64_t)ntile * (Cout / BM) * N));
#define OMC3(BM_, NS_)                                                                                             \
    if (BM == BM_ && ns == NS_) {                                                                                  \
        hipLaunchKernelGGL((k_conv3_fwd<BM_, NS_>), grid, dim3(kThreads), lds, ctx->stream, x, wr, bias, y, Cin, Cout, \
                           H, W, R, ps, ntile, acc);                                                               \
    }
    OMC3(64, 1) OMC3(64, 2) OMC3(64, 3) OMC3(64, 4) OMC3(64, 6) OMC3(64, 8)
    OMC3(32, 1) OMC3(32, 2) OMC3(32, 3) OMC3(32, 4) OMC3(32, 6) OMC3(32, 8)
#undef OMC3
    *st = OM_LAUNCH_CHECK(ctx, flip_weights ? "om_conv2d_bwd dx" : "om_conv2d_fwd");
    return true;
}

bool om_conv3_dw(om_ctx *ctx, const float *g, const float *x, float *dw, int N, int Cin, int H, int W, int Cout,
                 int acc, om_status *st) {
    *st = OM_OK;
    const int P = H * W;
    if (Cin % kDwCi || Cout % kDwCo || W % 4 || (int64_t)N * Cout * P > INT32_MAX || (int64_t)N * Cin * P > INT32_MAX)
        return false;
    int R, ps;
    stage_geometry(W, kDwPx, R, ps);
    const int ns = stage_ns(kDwCi, W, R);
    if (!ns) return false;
    const int nchunks = (P + kDwPx - 1) / kDwPx, items = N * nchunks;
    const int blocks = (Cout / kDwCo) * (Cin / kDwCi);
    // about three workgroups per CU, at least two items per slot where there are enough
    int slots = (int)((3LL * ctx->num_cus + blocks - 1) / blocks);
    if (slots > items / 2) slots = items / 2 > 0 ? items / 2 : 1;
    const int per = (items + slots - 1) / slots;
    slots = (items + per - 1) / per;
    float *part;
    *st = om::scratch(ctx, sizeof(float) * (uint64_t)slots * Cout * 9 * Cin, &part);
    if (*st) return true;
    const size_t lds = sizeof(float) * (size_t)kDwCi * ps;
    const dim3 grid((unsigned)((int64_t)slots * blocks));
#define OMW3(NS_)                                                                                                 \
    if (ns == NS_)                                                                                                \
        hipLaunchKernelGGL(k_conv3_dw<NS_>, grid, dim3(kThreads), lds, ctx->stream, g, x, part, Cin, Cout, H, W, R, ps, \
                           nchunks, items, per);
    OMW3(1) OMW3(2) OMW3(3) OMW3(4) OMW3(6) OMW3(8)
#undef OMW3
    const int64_t total = (int64_t)Cout * 9 * Cin;
    hipLaunchKernelGGL(k_conv3_dw_reduce, dim3(om::grid1d(total, 256, 2048)), dim3(256), 0, ctx->stream, part, slots,
                       Cout, Cin, dw, acc);
    *st = OM_LAUNCH_CHECK(ctx, "om_conv2d_bwd dw");
    return true;
}
