// 3x3 convolutions with stride 1 and padding 1 (every convolution of the benchmark's conv block and CRNN) as
// implicit GEMM on MFMA, the input staged through LDS once per tile (Ops.Conv2d, Ops.Layers.cs:279-336; ConvBackward,
// BackwardNn.cs:317-402).
//
// Forward: y[n][co][p] = bias[co] + sum over taps t = (ky, kx) and channels ci of W[co][ci][t] x[n][ci][p + shift(t)]
// (zero outside the image), optionally followed by ReLU. A workgroup takes 128 output pixels (flattened, so any width
// works) of one image and a block of 32 or 64 output channels; per chunk of 8 input channels it stages the input rows
// those pixels touch, halo included, into LDS (each input value is then read by all nine taps from there) and the
// chunk's weights, laid out [tap][co][ci]. The weights come straight from the layer's [Cout][Cin][3][3] tensor: a
// chunk is 72 contiguous floats per output channel, loaded as float4 and scattered into that layout by the stores.
// Each lane keeps the LDS offsets of its two pixels; a tap is a constant shift of them, so the inner loop has no index
// arithmetic. Four wavefronts of 32 pixels x all the block's channels, v_mfma_f32_16x16x4f32.
// dX: for stride 1 and padding 1, dx[n][ci][q] = sum over taps and co of W[co][ci][8 - t] g[n][co][q + shift(t)]:
// the same kernel over g (FLIP), whose chunk of 8 of the layer's output channels is 9 x BM contiguous floats of W per
// channel, stored flipped and transposed ([8 - t][ci][co]).
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
// tap stride of the staged weights: BM rows plus 8 floats, so the nine taps of one channel's scattered stores start
// on different banks
template <int BM>
constexpr int w_tap_stride() {
    return BM * kWLd + 8;
}
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

// ReLU forward (ReluUn, TrainElementwise.cs): x where x > 0 or NaN, else +0.
__device__ __forceinline__ float relu1(float v) { return v > 0.0f ? v : (v == v ? 0.0f : v); }

// out[n][co][p] (+)= bias[co] + sum_{tap, ci} W[co][ci][tap] in[n][ci][p + shift(tap)] (then ReLU when relu), BM
// output channels per workgroup. in is [N][cin][H][W], out [N][cout][H][W], wt the layer's weights: [cout][cin][9], or
// with FLIP (the input gradient) [cin][cout][9] read as W[co][ci][8 - tap] with this call's co and ci swapped. With
// nsplit > 1 (few tiles: small images) the input channels are cut into nsplit runs of cps chunks, one per workgroup,
// each writing its partial sums to ws[split] ([N][cout][H][W], no bias); k_conv3_sum adds them in split order.
template <int BM, int NS, bool FLIP>
__global__ void __launch_bounds__(kThreads) k_conv3_fwd(const float *__restrict__ in, const float *__restrict__ wt,
                                                        const float *__restrict__ bias, float *out, int cin, int cout,
                                                        int H, int W, int R, int ps, int ntile, int acc, int N,
                                                        int nsplit, int cps, float *__restrict__ ws, int relu) {
    OM_LDS_POISON();
    extern __shared__ __attribute__((aligned(16))) float lds[];
    constexpr int MB = BM / 16, WF4 = 18 * BM, NWI = (WF4 + kThreads - 1) / kThreads, TS = w_tap_stride<BM>();
    float *Ws = lds;           // [9][BM][kWLd], taps TS apart
    float *Xs = lds + 9 * TS;  // [kFwdCk][ps]
    const int P = H * W, rs = W + 8, ncb = cout / BM;
    const int lin = xcd_lin();
    const int tile = lin % ntile, cb = (lin / ntile) % ncb, n = (lin / ntile / ncb) % N, split = lin / ntile / ncb / N;
    const int c_beg = split * cps * kFwdCk, c_end = min(cin, c_beg + cps * kFwdCk);
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
    // The weight float4s this thread stages: global offset without the chunk's part, and the LDS offsets of the four
    // values. Forward: float4 f is floats 4 q .. 4 q + 3 (q = f % 18) of output channel co = f / 18's 72-float run
    // [ci][tap] of the chunk. FLIP: float4 f is floats 4 q .. (q = f / 8) of the run [ci][tap] of the chunk's input
    // channel f % 8 (one of the layer's output channels), over this block's BM channels; the eight channels vary
    // fastest over the lanes, so a wavefront's scattered stores of one component fall on eight-wide runs of banks.
    int wgo[NWI], wlo[NWI][4];
    floatx4 wv4[NWI];
#pragma unroll
    for (int i = 0; i < NWI; i++) {
        const int f = threadIdx.x + i * kThreads;
        const bool ok = f < WF4;
        const int row = FLIP ? f % kFwdCk : f / 18, q = FLIP ? f / kFwdCk : f % 18;
        wgo[i] = FLIP ? (row * cout + co0) * 9 + 4 * q : (co0 + row) * cin * 9 + 4 * q;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int e = 4 * q + k, c = e / 9, tap = e % 9;
            wlo[i][k] = !ok ? -1 : FLIP ? (8 - tap) * TS + c * kWLd + row : tap * TS + row * kWLd + c;
        }
    }
    const int64_t wstep = FLIP ? (int64_t)cout * 9 : 9;  // global offset of the next input channel's run
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
            if (wlo[i][0] >= 0) wv4[i] = *reinterpret_cast<const floatx4 *>(wt + wgo[i] + c0 * wstep);
        xs.load(inn + (int64_t)c0 * P, H, W, oy0);
    };
    load(c_beg);
    for (int c0 = c_beg; c0 < c_end; c0 += kFwdCk) {
        __syncthreads();  // the previous chunk's reads are done
#pragma unroll
        for (int i = 0; i < NWI; i++)
            if (wlo[i][0] >= 0)
#pragma unroll
                for (int k = 0; k < 4; k++) Ws[wlo[i][k]] = wv4[i][k];
        xs.store(Xs);
        __syncthreads();
        if (c0 + kFwdCk < c_end) load(c0 + kFwdCk);  // in flight while this chunk computes
#pragma unroll
        for (int tap = 0; tap < 9; tap++) {
            const int toff = (tap / 3) * rs + tap % 3;
            floatx2 a[MB];
#pragma unroll
            for (int i = 0; i < MB; i++)
                a[i] = *reinterpret_cast<const floatx2 *>(Ws + tap * TS + (16 * i + t) * kWLd + 2 * kl);
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
    if (nsplit > 1) {
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float *orow = ws + (((int64_t)split * N + n) * cout + co0 + 16 * i + 4 * kl + r) * P;
#pragma unroll
                for (int j = 0; j < 2; j++)
                    if (pv[j]) orow[p0 + 32 * w + 16 * j + t] = accv[i][j][r];
            }
        return;
    }
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
                float v = bias ? accv[i][j][r] + bv : accv[i][j][r];
                if (relu) v = relu1(v);
                orow[p] = acc ? orow[p] + v : v;
            }
        }
}

// out (+)= the sum of the nsplit partials in split order, plus bias[co] (the unsplit kernel's arithmetic order), then
// ReLU when relu.
__global__ void k_conv3_sum(const float *__restrict__ ws, int nsplit, int64_t total, int P, int cout,
                            const float *__restrict__ bias, float *out, int acc, int relu) {
    OM_LDS_POISON();
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        float v = ws[e];
        for (int s = 1; s < nsplit; s++) v += ws[(int64_t)s * total + e];
        if (bias) v = v + bias[(e / P) % cout];
        if (relu) v = relu1(v);
        out[e] = acc ? out[e] + v : v;
    }
}

// k_conv3_sum for a ReLU stage followed by a max pool whose kh x kw windows (stride kh, kw) tile the output exactly:
// a thread per pooled output adds the partials of each window element in split order, adds the bias and applies the
// ReLU (k_conv3_sum's arithmetic), stores the element, and pools the window as k_maxpool_fwd does ((ky, kx) order;
// the first candidate, a strictly larger value unless the best is NaN, or the first NaN wins; idx the element's flat
// index).
__global__ void k_conv3_sum_pool(const float *__restrict__ ws, int nsplit, int64_t total, int H, int W, int cout,
                                 const float *__restrict__ bias, float *__restrict__ out, float *__restrict__ py,
                                 int32_t *__restrict__ pidx, int kh, int kw, int64_t pooled) {
    OM_LDS_POISON();
    const int OH = H / kh, OW = W / kw;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < pooled; o += (int64_t)gridDim.x * blockDim.x) {
        const int ox = (int)(o % OW);
        const int64_t t = o / OW;
        const int oy = (int)(t % OH);
        const int64_t nc = t / OH;
        const float bv = bias ? bias[nc % cout] : 0.0f;
        float best = -__int_as_float(0x7F800000);
        int bi = -1;
        for (int ky = 0; ky < kh; ky++)
            for (int kx = 0; kx < kw; kx++) {
                const int64_t e = (nc * H + oy * kh + ky) * W + ox * kw + kx;
                float v = ws[e];
                for (int sp = 1; sp < nsplit; sp++) v += ws[(int64_t)sp * total + e];
                if (bias) v = v + bv;
                v = relu1(v);
                out[e] = v;
                const bool wins = bi < 0 || (v > best && best == best) || (v != v && best == best);
                if (wins) {
                    best = v;
                    bi = (int)e;
                }
            }
        py[o] = best;
        if (pidx) pidx[o] = bi;
    }
}

// part[slot][co][tap][ci] = the slot's items' sums of g[n][co][p] x[n][ci][p + shift(tap)]. The next item's g
// block and input rows are loaded into registers while the current one computes. With dbp, the workgroups of the
// first input-channel block also sum the staged g block per output channel in double (the bias gradient's partial of
// the slot, dbp[slot][co]): thread (co = tid / 4, quarter = tid % 4) adds pixels 16 quarter .. 16 quarter + 15 of
// every item in order, and the quarters are combined in order at the end.
template <int NS>
__global__ void __launch_bounds__(kThreads) k_conv3_dw(const float *__restrict__ g, const float *__restrict__ x,
                                                       float *__restrict__ part, int cin, int cout, int H, int W,
                                                       int R, int ps, int nchunks, int items, int per,
                                                       double *__restrict__ dbp) {
    OM_LDS_POISON();
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
    const bool do_db = dbp && cib == 0;  // uniform over the workgroup
    const int dco = threadIdx.x >> 2, dq = threadIdx.x & 3;
    double dbs = 0.0;
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
            // a pixel past the image (the last chunk's tail) reads the last pixel's staged, finite neighbours: its g
            // is zero, and zero times a finite value adds nothing (LDS that nothing wrote may hold a NaN)
            const int p = min(p0 + (int)threadIdx.x, P - 1);
            boff[threadIdx.x] = (p / W - oy0) * rs + p % W + 3;
        }
        __syncthreads();
        if (item + 1 < i1) load(item + 1);  // in flight while this item computes
        if (do_db) {
            const float *gr = Gs + dco * kGLd + 16 * dq;
#pragma unroll
            for (int j = 0; j < 16; j++) dbs += (double)gr[j];
        }
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
    if (do_db) {
        const double a1 = __shfl_down(dbs, 1, 64), a2 = __shfl_down(dbs, 2, 64), a3 = __shfl_down(dbs, 3, 64);
        if (dq == 0) dbp[(int64_t)slot * cout + co0 + dco] = ((dbs + a1) + a2) + a3;
    }
}

// dW[co][ci][tap] (+)= the sum over slots of part[slot][co][tap][ci]: a workgroup takes 64 consecutive elements (one
// per lane) and its four wavefronts the four quarters of the slot range, each summed in slot order; the quarters are
// then added in order, so the result depends only on the shape. (Many slots per element: one thread walking them all
// would keep too few loads in flight.)
// The blocks after the weights' (when dbp is given) finish the bias gradient the same way, in double: db[co] (+)=
// (float) of the quarters' sums of dbp[slot][co] over the slots, added in order. NW wavefronts split the slots (16
// where each output has hundreds of them and few blocks run: the chains of loads are then NW times shorter).
template <int NW>
__global__ void __launch_bounds__(64 * NW) k_conv3_dw_reduce(const float *__restrict__ part, int slots, int cout,
                                                             int cin, float *dw, int acc,
                                                             const double *__restrict__ dbp, float *db) {
    OM_LDS_POISON();
    __shared__ float qs[NW][64];
    __shared__ double qd[NW][64];
    const int64_t total = (int64_t)cout * 9 * cin;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int k0 = (int)((int64_t)slots * w / NW), k1 = (int)((int64_t)slots * (w + 1) / NW);
    const int64_t nbw = (total + 63) / 64;
    if ((int64_t)blockIdx.x >= nbw) {  // bias gradient (uniform over the block)
        const int co = (int)(((int64_t)blockIdx.x - nbw) * 64 + lane);
        double sd = 0.0;
        if (co < cout) {
#pragma unroll 8
            for (int k = k0; k < k1; k++) sd += dbp[(int64_t)k * cout + co];
        }
        qd[w][lane] = sd;
        __syncthreads();
        if (w == 0 && co < cout) {
            double t = qd[0][lane];
#pragma unroll
            for (int q = 1; q < NW; q++) t += qd[q][lane];
            const float v = (float)t;
            db[co] = acc ? db[co] + v : v;
        }
        return;
    }
    const int64_t e = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.0f;
    if (e < total) {
#pragma unroll 8
        for (int k = k0; k < k1; k++) s += part[(int64_t)k * total + e];
    }
    qs[w][lane] = s;
    __syncthreads();
    if (w == 0 && e < total) {
        float v = qs[0][lane];
#pragma unroll
        for (int q = 1; q < NW; q++) v += qs[q][lane];
        const int ci = (int)(e % cin);
        const int64_t ct = e / cin;
        const int tap = (int)(ct % 9), co = (int)(ct / 9);
        float *d = dw + ((int64_t)co * cin + ci) * 9 + tap;
        *d = acc ? *d + v : v;
    }
}

// dW of a convolution with one input channel (the first layer of an image model): dW[co][0][tap] = sum over images
// and pixels of g[n][co][p] x[n][0][p + shift(tap)], 9 * cout weights over N * H * W pixels. A workgroup takes one
// image's band of `br` rows: the band's input rows with their halo go to LDS (zeros outside the image), wavefront w
// takes output channels 8 w .. 8 w + 7 and lane j the band's pixels j, j + 64, ..., multiplying each pixel's nine
// staged inputs by its eight g values (72 running sums per lane, in pixel order). The lanes' sums combine through the
// fixed butterfly into part[block][co][tap]; k_conv3_dw_reduce adds the blocks in order.
__global__ void __launch_bounds__(1024) k_conv3_dw_c1(const float *__restrict__ g, const float *__restrict__ x,
                                                      float *__restrict__ part, int cout, int H, int W, int br,
                                                      int nbands, double *__restrict__ dbp) {
    OM_LDS_POISON();
    extern __shared__ float xs[];  // [br + 2][W + 2]
    const int n = blockIdx.x / nbands, y0 = (blockIdx.x % nbands) * br, rows = min(br, H - y0), xw = W + 2;
    for (int f = threadIdx.x; f < (br + 2) * xw; f += blockDim.x) {
        const int r = f / xw, c = f - r * xw, iy = y0 - 1 + r, ix = c - 1;
        xs[f] = (r < rows + 2 && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W)
                    ? x[((int64_t)n * H + iy) * W + ix]
                    : 0.0f;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, co0 = 8 * (threadIdx.x >> 6);
    const int64_t P = (int64_t)H * W;
    const float *gn = g + ((int64_t)n * cout + co0) * P + (int64_t)y0 * W;
    float acc[8][9];
    double dsum[8];  // the bias gradient's partials (when dbp): lane-ordered double sums of g, then the butterfly
#pragma unroll
    for (int k = 0; k < 8; k++) {
        dsum[k] = 0.0;
#pragma unroll
        for (int tap = 0; tap < 9; tap++) acc[k][tap] = 0.0f;
    }
    const int np = rows * W;
    // Pixels q = lane, lane + 64, ... in that order; the g loads of U of them are issued before the first is used
    // (clamped in range; a pixel past the band adds nothing).
    constexpr int U = 4;
    for (int q0 = lane; q0 < np; q0 += 64 * U) {
        float gv[U][8];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int q = min(q0 + 64 * u, np - 1);
#pragma unroll
            for (int k = 0; k < 8; k++) gv[u][k] = gn[k * P + q];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int q = q0 + 64 * u;
            if (q >= np) break;
            const int r = q / W, c = q - r * W;
            float xv[9];
#pragma unroll
            for (int tap = 0; tap < 9; tap++) xv[tap] = xs[(r + tap / 3) * xw + c + tap % 3];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                dsum[k] += (double)gv[u][k];
#pragma unroll
                for (int tap = 0; tap < 9; tap++) acc[k][tap] = acc[k][tap] + gv[u][k] * xv[tap];
            }
        }
    }
    if (dbp) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const double v = omd::wave_sum(dsum[k]);
            if (lane == 0) dbp[(int64_t)blockIdx.x * cout + co0 + k] = v;
        }
    }
    // The 72 sums acc[k][tap] over the wavefront's lanes by halving: at lane bit 5, 4 and 3 in turn a lane keeps the
    // half of its values its bit selects, adds the partner's copy of that half and hands the partner the other half;
    // the last 9 (one channel's taps) are summed over the remaining 8 lanes by a butterfly. Lane 8 j then holds the
    // nine tap sums of channel co0 + j.
    float v1[36], v2[18], v3[9];
    const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
#pragma unroll
    for (int i = 0; i < 36; i++) {
        const float lo = acc[i / 9][i % 9], hi = acc[(36 + i) / 9][(36 + i) % 9];
        v1[i] = (b5 ? hi : lo) + __shfl_xor(b5 ? lo : hi, 32, 64);
    }
#pragma unroll
    for (int i = 0; i < 18; i++) v2[i] = (b4 ? v1[18 + i] : v1[i]) + __shfl_xor(b4 ? v1[i] : v1[18 + i], 16, 64);
#pragma unroll
    for (int i = 0; i < 9; i++) {
        v3[i] = (b3 ? v2[9 + i] : v2[i]) + __shfl_xor(b3 ? v2[i] : v2[9 + i], 8, 64);
#pragma unroll
        for (int o = 4; o > 0; o >>= 1) v3[i] += __shfl_xor(v3[i], o, 64);
    }
    if ((lane & 7) == 0) {
        const int k = lane >> 3;  // 4 b5 + 2 b4 + b3
#pragma unroll
        for (int tap = 0; tap < 9; tap++) part[((int64_t)blockIdx.x * cout + co0 + k) * 9 + tap] = v3[tap];
    }
}

// Forward of a 3x3 / stride 1 / padding 1 convolution with one input channel (a CRNN's first layer over a grayscale
// image): y[n][co][p] = (sum over taps t of w[co][t] x[n][p + shift(t)], an fmaf chain in tap order) + bias[co], then
// the ReLU when asked. A workgroup takes one image's band of br rows: the band's input with its halo and all weights
// and biases are staged in LDS, each thread keeps one pixel's nine neighbours in registers and walks the output
// channels four at a time (broadcast LDS reads of their weights), and consecutive threads store consecutive pixels
// of a channel.
constexpr int kC1MaxCout = 128;
__global__ void __launch_bounds__(256) k_conv3_fwd_c1(const float *__restrict__ x, const float *__restrict__ w,
                                                      const float *__restrict__ bias, float *__restrict__ y, int cout,
                                                      int H, int W, int br, int nbands, int relu) {
    OM_LDS_POISON();
    extern __shared__ float xs[];  // [br + 2][W + 2]
    __shared__ float ws[kC1MaxCout * 9], bs[kC1MaxCout];
    const int n = blockIdx.x / nbands, y0 = (blockIdx.x % nbands) * br, rows = min(br, H - y0), xw = W + 2;
    for (int f = threadIdx.x; f < cout * 9; f += blockDim.x) ws[f] = w[f];
    for (int f = threadIdx.x; f < cout; f += blockDim.x) bs[f] = bias ? bias[f] : 0.0f;
    for (int f = threadIdx.x; f < (br + 2) * xw; f += blockDim.x) {
        const int r = f / xw, c = f - r * xw, iy = y0 - 1 + r, ix = c - 1;
        xs[f] = (r < rows + 2 && (unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W)
                    ? x[((int64_t)n * H + iy) * W + ix]
                    : 0.0f;
    }
    __syncthreads();
    const int64_t P = (int64_t)H * W;
    const int np = rows * W;
    for (int q = threadIdx.x; q < np; q += blockDim.x) {
        const int r = q / W, c = q - r * W;
        float xv[9];
#pragma unroll
        for (int tap = 0; tap < 9; tap++) xv[tap] = xs[(r + tap / 3) * xw + c + tap % 3];
        float *yp = y + (int64_t)n * cout * P + (int64_t)y0 * W + q;
        auto one = [&](int co) {
            float v = 0.0f;
#pragma unroll
            for (int tap = 0; tap < 9; tap++) v = __builtin_fmaf(ws[co * 9 + tap], xv[tap], v);
            if (bias) v = v + bs[co];
            if (relu) v = v > 0.0f ? v : (v == v ? 0.0f : v);
            yp[co * P] = v;
        };
        int co = 0;
        for (; co + 4 <= cout; co += 4) {
#pragma unroll
            for (int u = 0; u < 4; u++) one(co + u);
        }
        for (; co < cout; co++) one(co);
    }
}

// k_conv3_fwd_c1 with the ReLU, followed by a max pool whose KH x KW windows (stride KH, KW) tile the output: a
// workgroup per pooled row of an image (its KH + 2 input rows staged in LDS), a thread per window and every fourth
// channel. Each window element is k_conv3_fwd_c1's chain, bias and ReLU, stored; the window is pooled as
// k_maxpool_fwd does ((ky, kx) order; the first candidate, a strictly larger value unless the best is NaN, or the
// first NaN wins; idx the element's flat index).
template <int KH, int KW>
__global__ void __launch_bounds__(256) k_conv3_fwd_c1_pool(const float *__restrict__ x, const float *__restrict__ w,
                                                           const float *__restrict__ bias, float *__restrict__ a,
                                                           float *__restrict__ py, int32_t *__restrict__ pidx,
                                                           int cout, int H, int W) {
    OM_LDS_POISON();
    extern __shared__ float xs[];  // [KH + 2][W + 2]
    __shared__ float ws[kC1MaxCout * 9], bs[kC1MaxCout];
    const int OH2 = H / KH, OW2 = W / KW, xw = W + 2;
    const int n = blockIdx.x / OH2, oy = blockIdx.x % OH2, y0 = oy * KH;
    for (int f = threadIdx.x; f < cout * 9; f += blockDim.x) ws[f] = w[f];
    for (int f = threadIdx.x; f < cout; f += blockDim.x) bs[f] = bias ? bias[f] : 0.0f;
    for (int f = threadIdx.x; f < (KH + 2) * xw; f += blockDim.x) {
        const int r = f / xw, c = f - r * xw, iy = y0 - 1 + r, ix = c - 1;
        xs[f] = ((unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W) ? x[((int64_t)n * H + iy) * W + ix] : 0.0f;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t P2 = (int64_t)OH2 * OW2;
    for (int ox = lane; ox < OW2; ox += 64) {
        float xv[KH + 2][KW + 2];  // the window's input patch, halo included
#pragma unroll
        for (int r = 0; r < KH + 2; r++)
#pragma unroll
            for (int c = 0; c < KW + 2; c++) xv[r][c] = xs[r * xw + ox * KW + c];
        for (int co = wv; co < cout; co += 4) {
            float best = -__int_as_float(0x7F800000);
            int bi = -1;
#pragma unroll
            for (int ky = 0; ky < KH; ky++)
#pragma unroll
                for (int kx = 0; kx < KW; kx++) {
                    float v = 0.0f;
#pragma unroll
                    for (int tap = 0; tap < 9; tap++) v = __builtin_fmaf(ws[co * 9 + tap], xv[ky + tap / 3][kx + tap % 3], v);
                    if (bias) v = v + bs[co];
                    v = v > 0.0f ? v : (v == v ? 0.0f : v);
                    const int64_t e = (((int64_t)n * cout + co) * H + y0 + ky) * W + ox * KW + kx;
                    a[e] = v;
                    const bool wins = bi < 0 || (v > best && best == best) || (v != v && best == best);
                    if (wins) {
                        best = v;
                        bi = (int)e;
                    }
                }
            const int64_t o = ((int64_t)n * cout + co) * P2 + (int64_t)oy * OW2 + ox;
            py[o] = best;
            if (pidx) pidx[o] = bi;
        }
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
                  int W, int Cout, int acc, om_status *st, bool flip_weights, bool relu, const Conv3Pool *pool,
                  bool *pooled) {
    if (pooled) *pooled = false;
    *st = OM_OK;
    const int P = H * W;
    if (Cin == 1 && !flip_weights && !acc && Cout <= kC1MaxCout && (int64_t)N * Cout * P <= INT32_MAX && pool &&
        relu && pooled && pool->kh == 2 && (pool->kw == 2 || pool->kw == 1) && H % 2 == 0 && W % pool->kw == 0 &&
        (int64_t)(W + 2) * 4 * 4 <= 65536) {  // the stage's convolution, ReLU and max pool in one launch
        const size_t lds = sizeof(float) * 4 * (size_t)(W + 2);
        const dim3 grid((unsigned)(N * (H / 2)));
        if (pool->kw == 2)
            hipLaunchKernelGGL((k_conv3_fwd_c1_pool<2, 2>), grid, dim3(256), lds, ctx->stream, x, w, bias, y, pool->y,
                               pool->idx, Cout, H, W);
        else
            hipLaunchKernelGGL((k_conv3_fwd_c1_pool<2, 1>), grid, dim3(256), lds, ctx->stream, x, w, bias, y, pool->y,
                               pool->idx, Cout, H, W);
        *pooled = true;
        *st = OM_LAUNCH_CHECK(ctx, "om_conv2d_relu_pool_fwd");
        return true;
    }
    if (Cin == 1 && !flip_weights && !acc && Cout <= kC1MaxCout && (int64_t)N * Cout * P <= INT32_MAX &&
        (int64_t)(W + 2) * 4 * 3 <= 65536) {
        // bands of rows, about four workgroups per CU over the images, each band's input under 64 KB of LDS
        const int want = (int)((4LL * ctx->num_cus + N - 1) / N);
        int nb = want < H ? want : H;
        int br = (H + nb - 1) / nb;
        while (br > 1 && (int64_t)(br + 2) * (W + 2) * 4 > 65536) br = (br + 1) / 2;
        nb = (H + br - 1) / br;
        const size_t lds = sizeof(float) * (size_t)(br + 2) * (W + 2);
        hipLaunchKernelGGL(k_conv3_fwd_c1, dim3((unsigned)(N * nb)), dim3(256), lds, ctx->stream, x, w, bias, y, Cout, H,
                           W, br, nb, relu ? 1 : 0);
        *st = OM_LAUNCH_CHECK(ctx, "om_conv2d_fwd");
        return true;
    }
    if (Cin % kFwdCk || Cout % 32 || W % 4 || (int64_t)N * Cin * P > INT32_MAX || (int64_t)N * Cout * P > INT32_MAX ||
        (int64_t)Cout * 9 * Cin > INT32_MAX)
        return false;
    int R, ps;
    stage_geometry(W, kFwdPx, R, ps);
    const int ns = stage_ns(kFwdCk, W, R);
    if (!ns) return false;
    const int BM = Cout % 64 == 0 ? 64 : 32;
    // forward: the layer's W [Cout][Cin][9]; dX (flip): the layer's W [Cout_l][Cin_l][9], where this call's Cin is
    // Cout_l and its Cout is Cin_l (the kernel reads it flipped and transposed)
    const int ntile = (P + kFwdPx - 1) / kFwdPx;
    const size_t lds = sizeof(float) * (9 * (size_t)(BM == 64 ? w_tap_stride<64>() : w_tap_stride<32>()) +
                                        (size_t)kFwdCk * ps);
    const int64_t tiles = (int64_t)ntile * (Cout / BM) * N;
    // Fewer tiles than two per CU (small images): split the input channels, at least two chunks per split.
    const int chunks = Cin / kFwdCk;
    int nsplit = 1, cps = chunks;
    if (tiles < 2 * ctx->num_cus && chunks >= 4) {
        int want = (int)((2 * ctx->num_cus + tiles - 1) / tiles);
        if (want > chunks / 2) want = chunks / 2;
        cps = (chunks + want - 1) / want;
        nsplit = (chunks + cps - 1) / cps;
    }
    float *ws = nullptr;
    const int64_t total = (int64_t)N * Cout * P;
    if (nsplit > 1) {
        *st = om::scratch2(ctx, sizeof(float) * (uint64_t)nsplit * total, &ws);
        if (*st) return true;
    }
    const dim3 grid((unsigned)(tiles * nsplit));
    const int rl = relu && nsplit == 1 ? 1 : 0;  // with splits the sum applies it
#define OMC3(BM_, NS_)                                                                                             \
    if (BM == BM_ && ns == NS_) {                                                                                  \
        if (flip_weights)                                                                                          \
            hipLaunchKernelGGL((k_conv3_fwd<BM_, NS_, true>), grid, dim3(kThreads), lds, ctx->stream, x, w, bias, y, \
                               Cin, Cout, H, W, R, ps, ntile, acc, N, nsplit, cps, ws, rl);                         \
        else                                                                                                       \
            hipLaunchKernelGGL((k_conv3_fwd<BM_, NS_, false>), grid, dim3(kThreads), lds, ctx->stream, x, w, bias, \
                               y, Cin, Cout, H, W, R, ps, ntile, acc, N, nsplit, cps, ws, rl);                      \
    }
    OMC3(64, 1) OMC3(64, 2) OMC3(64, 3) OMC3(64, 4) OMC3(64, 6) OMC3(64, 8)
    OMC3(32, 1) OMC3(32, 2) OMC3(32, 3) OMC3(32, 4) OMC3(32, 6) OMC3(32, 8)
#undef OMC3
    if (nsplit > 1 && pool && relu && !acc && pooled) {  // the sum, the ReLU and the max pool in one pass
        const int64_t npool = (int64_t)N * Cout * (H / pool->kh) * (W / pool->kw);
        hipLaunchKernelGGL(k_conv3_sum_pool, dim3(om::grid1d(npool, 256, 4096)), dim3(256), 0, ctx->stream, ws, nsplit,
                           total, H, W, Cout, bias, y, pool->y, pool->idx, pool->kh, pool->kw, npool);
        *pooled = true;
    } else if (nsplit > 1) {
        hipLaunchKernelGGL(k_conv3_sum, dim3(om::grid1d(total, 256, 4096)), dim3(256), 0, ctx->stream, ws, nsplit,
                           total, P, Cout, bias, y, acc, relu ? 1 : 0);
    }
    *st = OM_LAUNCH_CHECK(ctx, flip_weights ? "om_conv2d_bwd dx" : "om_conv2d_fwd");
    return true;
}

bool om_conv3_dw(om_ctx *ctx, const float *g, const float *x, float *dw, float *db, int N, int Cin, int H, int W,
                 int Cout, int acc, om_status *st) {
    *st = OM_OK;
    const int P = H * W;
    if (Cin == 1 && Cout % 8 == 0 && Cout <= 128 && (int64_t)N * Cout * P <= INT32_MAX && (W + 2) * 4 <= 16384) {
        // bands of rows: about two workgroups per CU over the images, the band's input under 64 KB of LDS
        const int want = (int)((2LL * ctx->num_cus + N - 1) / N);
        int nb = want < H ? want : H;
        int br = (H + nb - 1) / nb;
        while (br > 1 && (int64_t)(br + 2) * (W + 2) * 4 > 65536) br = (br + 1) / 2;
        nb = (H + br - 1) / br;
        const int blocks = N * nb;
        const uint64_t pbytes = (sizeof(float) * (uint64_t)blocks * Cout * 9 + 255) / 256 * 256;
        float *part;
        *st = om::scratch(ctx, pbytes + (db ? sizeof(double) * (uint64_t)blocks * Cout : 0), &part);
        if (*st) return true;
        double *dbp = db ? reinterpret_cast<double *>(reinterpret_cast<char *>(part) + pbytes) : nullptr;
        const size_t lds = sizeof(float) * (size_t)(br + 2) * (W + 2);
        hipLaunchKernelGGL(k_conv3_dw_c1, dim3((unsigned)blocks), dim3(64 * (Cout / 8)), lds, ctx->stream, g, x, part,
                           Cout, H, W, br, nb, dbp);
        const unsigned rb = (unsigned)((Cout * 9 + 63) / 64 + (db ? (Cout + 63) / 64 : 0));
        hipLaunchKernelGGL(k_conv3_dw_reduce<16>, dim3(rb), dim3(1024), 0, ctx->stream, part, blocks, Cout, 1, dw, acc,
                           dbp, db);
        *st = OM_LAUNCH_CHECK(ctx, "om_conv2d_bwd dw");
        return true;
    }
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
    const uint64_t pbytes = (sizeof(float) * (uint64_t)slots * Cout * 9 * Cin + 255) / 256 * 256;
    float *part;
    *st = om::scratch(ctx, pbytes + (db ? sizeof(double) * (uint64_t)slots * Cout : 0), &part);
    if (*st) return true;
    double *dbp = db ? reinterpret_cast<double *>(reinterpret_cast<char *>(part) + pbytes) : nullptr;
    const size_t lds = sizeof(float) * (size_t)kDwCi * ps;
    const dim3 grid((unsigned)((int64_t)slots * blocks));
#define OMW3(NS_)                                                                                                 \
    if (ns == NS_)                                                                                                \
        hipLaunchKernelGGL(k_conv3_dw<NS_>, grid, dim3(kThreads), lds, ctx->stream, g, x, part, Cin, Cout, H, W, R, ps, \
                           nchunks, items, per, dbp);
    OMW3(1) OMW3(2) OMW3(3) OMW3(4) OMW3(6) OMW3(8)
#undef OMW3
    const int64_t total = (int64_t)Cout * 9 * Cin;
    const unsigned rb = (unsigned)((total + 63) / 64 + (db ? (Cout + 63) / 64 : 0));
    if (slots >= 256 && rb < (unsigned)ctx->num_cus)
        hipLaunchKernelGGL(k_conv3_dw_reduce<16>, dim3(rb), dim3(1024), 0, ctx->stream, part, slots, Cout, Cin, dw, acc,
                           dbp, db);
    else
        hipLaunchKernelGGL(k_conv3_dw_reduce<4>, dim3(rb), dim3(256), 0, ctx->stream, part, slots, Cout, Cin, dw, acc,
                           dbp, db);
    *st = OM_LAUNCH_CHECK(ctx, "om_conv2d_bwd dw");
    return true;
}
