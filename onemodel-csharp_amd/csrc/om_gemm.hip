// Dense fp32 MFMA GEMM (om_gemm), the Linear layer forward/backward built on it, and the split-K reduction.
//
// Tile selection is a function of the shape and the CU count only. Well-aligned operands (every pointer 16-byte
// aligned, leading dimensions multiples of 4) run the BK = 32 "fast set" of tiles; anything else runs 64 x 64 tiles
// with element-guarded loads. The chooser prefers tilings whose workgroup count fills whole rounds of the 256 CUs
// (128 x 192 for 4096 x 1536 gives exactly 256 tiles, 64 x 96 for 4096 x 384 likewise), because a last round that
// is half empty costs as much as a full one.
#include <cstdlib>
#include <cstring>
#include <utility>

#include "om_gemm.hpp"
#include "om_gemm_x.hpp"

namespace omg {

template <int BM, int BN, int BKT, bool TA, bool TB, bool VEC>
__global__ void __launch_bounds__(NT) k_gemm(Params p) {
    OM_LDS_POISON();
    using LA = typename std::conditional<TA, LoadRContig<BM, BKT, VEC>, LoadKContig<BM, BKT, VEC>>::type;
    using LB = typename std::conditional<TB, LoadKContig<BN, BKT, VEC>, LoadRContig<BN, BKT, VEC>>::type;
    __shared__ __attribute__((aligned(16))) float As[2 * lds_size<BM, BKT, LA::KLAYOUT>()];
    __shared__ __attribute__((aligned(16))) float Bs[2 * lds_size<BN, BKT, LB::KLAYOUT>()];
    const int tiles_n = (p.n + BN - 1) / BN, tiles_m = (p.m + BM - 1) / BM;
    int tm, tn, zz;
    tile_coords(p, tiles_n, tiles_m, tm, tn, zz);
    if (zz >= p.batch * p.splits) return;
    const int z = zz / p.splits, split = zz % p.splits;
    const int outer = z / p.batch_div, inner = z % p.batch_div;
    const float *A = p.a + outer * p.sa_outer + inner * p.sa_inner;
    const float *B = p.b + outer * p.sb_outer + inner * p.sb_inner;
    float *C = p.c + outer * p.sc_outer + inner * p.sc_inner;
    const float *mask = p.mask ? p.mask + outer * p.mask_outer_stride : nullptr;
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = split * p.k_split, kend = min(p.k, kbeg + p.k_split);
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int wm0 = (wv >> 1) * (BM / 2), wn0 = (wv & 1) * (BN / 2);

    LA la;
    LB lb;
    Tile<BM, BN, BKT, LA::KLAYOUT, LB::KLAYOUT> t;
    const int M = p.m, N = p.n;
    const int64_t lda = p.lda, ldb = p.ldb;
    run_k<BM, BN, BKT>(
        t, la, lb, [&](LA &l, int k0) { l.fetch(A, lda, M, kend, m0, k0); },
        [&](LB &l, int k0) { l.fetch(B, ldb, N, kend, n0, k0); }, kbeg, kend, As, Bs, wm0, wn0, lane);
    store_tile<decltype(t), true>(p, t, m0, n0, wm0, wn0, lane, C, p.ldc, mask, split);
}

// Adds the split-K partials in split order and applies the epilogue; four consecutive columns per thread. A fused
// bias gradient's per-split column sums are finished here too (in split order, in double).
__global__ void k_splitk_reduce(Params p) {
    OM_LDS_POISON();
    const int64_t total = (int64_t)p.m * p.n;
    const int nq = (p.n + 3) / 4;
    const int64_t quads = (int64_t)p.m * nq;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p.colsum_ws)
        for (int64_t i = gid; i < p.m; i += stride) {
            double t = 0.0;
            for (int s = 0; s < p.splits; s++) t += p.colsum_ws[(int64_t)s * p.m + i];
            float v = (float)t;
            p.db[i] = p.db_acc ? p.db[i] + v : v;
        }
    for (int64_t q = gid; q < quads; q += stride) {
        int row = (int)(q / nq), col0 = (int)(q % nq) * 4;
        int64_t e = (int64_t)row * p.n + col0;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        if (col0 + 3 < p.n && (p.n & 3) == 0) {
            for (int s = 0; s < p.splits; s++) {
                float4 t = *reinterpret_cast<const float4 *>(p.ws + (int64_t)s * total + e);
                v[0] += t.x;
                v[1] += t.y;
                v[2] += t.z;
                v[3] += t.w;
            }
        } else {
            for (int s = 0; s < p.splits; s++)
                for (int u = 0; u < 4 && col0 + u < p.n; u++) v[u] += p.ws[(int64_t)s * total + e + u];
        }
        for (int u = 0; u < 4 && col0 + u < p.n; u++) epilogue(p, p.c, p.ldc, nullptr, row, col0 + u, v[u]);
    }
}

// The same reduction for n % 4 == 0 and a split count known at compile time: a thread per float4 of C issues the S
// loads of its partials before adding them in split order (0 + p0 + p1 + ...), so the result is k_splitk_reduce's.
template <int S>
__device__ __forceinline__ void reduce_bias_row(const Params &p, int i) {
    double t = 0.0;
#pragma unroll
    for (int s = 0; s < S; s++) t += p.colsum_ws[(int64_t)s * p.m + i];
    float v = (float)t;
    p.db[i] = p.db_acc ? p.db[i] + v : v;
}
template <int S>
__device__ __forceinline__ void reduce_quad(const Params &p, int64_t q) {
    const int nq = p.n / 4;
    const int row = (int)(q / nq), col0 = (int)(q % nq) * 4;
    const float *src = p.ws + (int64_t)row * p.n + col0;
    const int64_t total = (int64_t)p.m * p.n;
    float4 t[S];
#pragma unroll
    for (int s = 0; s < S; s++) t[s] = *reinterpret_cast<const float4 *>(src + s * total);
    float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < S; s++) {
        v[0] += t[s].x;
        v[1] += t[s].y;
        v[2] += t[s].z;
        v[3] += t[s].w;
    }
    // A plain epilogue (every weight gradient) writes the quad as one float4, with the same arithmetic.
    const bool plain = p.alpha == 1.0f && !p.bias && !p.resid && p.epi == EPI_NONE && p.ldc % 4 == 0 &&
                       ((uintptr_t)p.c & 15) == 0;
    if (plain) {
        float4 *dst = reinterpret_cast<float4 *>(p.c + (int64_t)row * p.ldc + col0);
        float4 o = make_float4(v[0], v[1], v[2], v[3]);
        if (p.accumulate) {
            const float4 c = *dst;
            o = make_float4(c.x + v[0], c.y + v[1], c.z + v[2], c.w + v[3]);
        }
        *dst = o;
        return;
    }
#pragma unroll
    for (int u = 0; u < 4; u++) epilogue(p, p.c, p.ldc, nullptr, row, col0 + u, v[u]);
}
template <int S>
__global__ void k_splitk_reduce_s(Params p) {
    OM_LDS_POISON();
    const int64_t quads = (int64_t)p.m * (p.n / 4);
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p.colsum_ws)
        for (int64_t i = gid; i < p.m; i += stride) reduce_bias_row<S>(p, (int)i);
    for (int64_t q = gid; q < quads; q += stride) reduce_quad<S>(p, q);
}
// The reduce of a grouped weight-gradient launch: the column sums, and the same per-row and per-quad work over every
// product. Each kind of work has blocks of its own, in that order (the column sums, a wavefront per column, are the
// longest chains and are dispatched first), so they run at once instead of one after another in the same threads.
template <int S>
__global__ void k_splitk_reduce_group(GroupParams g, int cblocks, int rblocks) {
    OM_LDS_POISON();
    const int b = blockIdx.x;
    if (b < cblocks) {
        const int64_t w = (int64_t)b * (blockDim.x >> 6) + (threadIdx.x >> 6);
        if (w >= g.cstart[g.ncs]) return;  // uniform over each wavefront
        int i = 0;
#pragma unroll
        for (int j = 1; j < kMaxColSums; j++)
            if (j < g.ncs && w >= g.cstart[j]) i = j;
        const ColSumItem &c = g.cs[i];
        omd::column_sum_wave(c.part, c.out, c.chunks, c.cols, (int)(w - g.cstart[i]), c.acc, threadIdx.x & 63);
        return;
    }
    if (b < cblocks + rblocks) {
        const int64_t r = (int64_t)(b - cblocks) * blockDim.x + threadIdx.x;
        if (r >= g.rstart[g.count]) return;
        int i = 0;
#pragma unroll
        for (int j = 1; j < kMaxGroup; j++)
            if (j < g.count && r >= g.rstart[j]) i = j;
        reduce_bias_row<S>(g.p[i], (int)(r - g.rstart[i]));
        return;
    }
    const int64_t q = (int64_t)(b - cblocks - rblocks) * blockDim.x + threadIdx.x;
    if (q >= g.qstart[g.count]) return;
    int i = 0;
#pragma unroll
    for (int j = 1; j < kMaxGroup; j++)
        if (j < g.count && q >= g.qstart[j]) i = j;
    reduce_quad<S>(g.p[i], q - g.qstart[i]);
}

template <int BM, int BN, int BKT, bool TA, bool TB, bool VEC>
static void launch_t(const Params &p, int batch, hipStream_t st) {
    int64_t tiles = (int64_t)((p.m + BM - 1) / BM) * ((p.n + BN - 1) / BN);
    // One linear grid over (z, m-tile, n-tile), n fastest.
    int64_t total = tiles * batch * p.splits;
    hipLaunchKernelGGL((k_gemm<BM, BN, BKT, TA, TB, VEC>), dim3((unsigned)total), dim3(NT), 0, st, p);
}

// Fast set: aligned operands, BK = 32, the three layouts the training path uses (NN, NT, TN).
template <int BM, int BN>
static bool launch_fast(const Params &p, int batch, bool ta, bool tb, hipStream_t st) {
    if (!ta && !tb) launch_t<BM, BN, 32, false, false, true>(p, batch, st);
    else if (!ta && tb) launch_t<BM, BN, 32, false, true, true>(p, batch, st);
    else if (ta && !tb) launch_t<BM, BN, 32, true, false, true>(p, batch, st);
    else return false;
    return true;
}
// General set: any layout and alignment, BK = 16.
template <int BM, int BN>
static void launch_general(const Params &p, int batch, bool ta, bool tb, bool vec, hipStream_t st) {
#define OMG_CASE(TA, TB, V) \
    if (ta == TA && tb == TB && vec == V) return launch_t<BM, BN, 16, TA, TB, V>(p, batch, st);
    OMG_CASE(false, false, false)
    OMG_CASE(false, false, true)
    OMG_CASE(false, true, false)
    OMG_CASE(false, true, true)
    OMG_CASE(true, false, false)
    OMG_CASE(true, false, true)
    OMG_CASE(true, true, false)
    OMG_CASE(true, true, true)
#undef OMG_CASE
}

// The epilogues only some tile instances carry: GELU and its backward terms. EPI_RELU, like the bias and the
// residual, is applied by every instance. An instance's epilogue family GK is 0 (none of them), 1 (the reference's
// polynomials: EPI_GELU, EPI_GELU_GRAD, EPI_GELU_SLOPE) or 2 (the same with erf and exp of stated error:
// EPI_GELU_F, EPI_GELU_GRAD_F, EPI_GELU_SLOPE_F); both families also carry EPI_MUL_AUX (no transcendental).
static bool gelu_epi(int epi) { return epi != EPI_NONE && epi != EPI_RELU; }
// 1 or 2: the family the epilogue needs; 3: either (EPI_MUL_AUX); 0: none.
static int epi_family(int epi) {
    if (epi == EPI_GELU || epi == EPI_GELU_GRAD || epi == EPI_GELU_SLOPE) return 1;
    if (epi == EPI_GELU_F || epi == EPI_GELU_GRAD_F || epi == EPI_GELU_SLOPE_F) return 2;
    return epi == EPI_MUL_AUX ? 3 : 0;
}
// The family an instance set GM (bit 0: family 1 instantiated, bit 1: family 2) runs epilogue `epi` with, or -1.
static int pick_family(int GM, int epi) {
    const int f = epi_family(epi);
    if (f == 0) return 0;
    if (f == 3) return (GM & 2) ? 2 : (GM & 1) ? 1 : -1;
    return (GM & f) ? f : -1;
}

// In a tuning build (om::tuning_env), OM_GEMM_DMA=0 keeps NT products on k_gemm_x's register-staged loads and
// OM_GEMM_DMA=2 puts every NT product with 32-deep chunks (plain or fast GELU) on k_gemm_xd, whose chunks load
// straight into LDS, however many rounds its tiles take (for comparisons); otherwise launch_x's rule decides.
static bool dma_disabled() {
    static const char *s = om::tuning_env("OM_GEMM_DMA");
    return s && s[0] == '0';
}
static bool dma_forced() {
    static const char *s = om::tuning_env("OM_GEMM_DMA");
    return s && s[0] == '2';
}

// Launches kernel K with the epilogue family gk, instantiating only the families GM holds.
#define OMG_L(K, NTH, TA_, TB_)                                                                                  \
    do {                                                                                                         \
        if constexpr ((GM & 1) != 0)                                                                             \
            if (gk == 1) {                                                                                       \
                hipLaunchKernelGGL((gx::K<BM, BN, BKT, TA_, TB_, 1>), dim3(total), dim3(NTH), 0, st, p);         \
                break;                                                                                           \
            }                                                                                                    \
        if constexpr ((GM & 2) != 0)                                                                             \
            if (gk == 2) {                                                                                       \
                hipLaunchKernelGGL((gx::K<BM, BN, BKT, TA_, TB_, 2>), dim3(total), dim3(NTH), 0, st, p);         \
                break;                                                                                           \
            }                                                                                                    \
        hipLaunchKernelGGL((gx::K<BM, BN, BKT, TA_, TB_, 0>), dim3(total), dim3(NTH), 0, st, p);                 \
    } while (0);

// Tile-exact set (om_gemm_x.hpp): NN, NT, TN; GELU epilogue variants (NN / NT only) of the families GM holds.
template <int BM, int BN, int BKT, int GM>
static bool launch_x(const Params &p, int batch, bool ta, bool tb, hipStream_t st, int cus, int dma) {
    const unsigned total = (unsigned)((int64_t)(p.m / BM) * (p.n / BN) * batch * p.splits);
    const int gk = pick_family(GM, p.epi);
    if (gk < 0 || (gk > 0 && ta)) return false;
    if (!ta && !tb) {
        OMG_L(k_gemm_x, NT, false, false)
    } else if (!ta && tb) {
        // Both operands K-contiguous: chunks load straight into LDS, when the grid fits in one round of the CUs at
        // the occupancy the three LDS stages allow (C3: the 256-tile products gain 7-8 %, the 768-tile q|k|v
        // projection would lose 14 % to a second round), or when the tuned table asks for it (dma): the FFN's first
        // products and C5's q|k|v projection, several rounds, plain or with the fast GELU pair (3-7 % faster). Not
        // for the reference's polynomials, whose element-wise tail hides better behind the register-staged kernel's
        // higher occupancy (75 against 81 us for the C3 FFN product).
        if constexpr (BKT == 32) {
            constexpr int lds = 4 * (64 + 3 * (BM + BN) * BKT);
            const unsigned per_cu = (160u << 10) / lds;
            const bool want = (gk == 0 && total <= per_cu * (unsigned)cus) || ((dma || dma_forced()) && gk != 1);
            if (want && !dma_disabled()) {
                if constexpr ((GM & 2) != 0)
                    if (gk == 2) {
                        hipLaunchKernelGGL((gx::k_gemm_xd<BM, BN, BKT, 2>), dim3(total), dim3(NT), 0, st, p);
                        return true;
                    }
                if (gk == 0) {
                    hipLaunchKernelGGL((gx::k_gemm_xd<BM, BN, BKT, 0>), dim3(total), dim3(NT), 0, st, p);
                    return true;
                }
            }
        }
        OMG_L(k_gemm_x, NT, false, true)
    } else if (ta && !tb) {
        hipLaunchKernelGGL((gx::k_gemm_x<BM, BN, BKT, true, false, 0>), dim3(total), dim3(NT), 0, st, p);
    } else {
        return false;
    }
    return true;
}
// Eight-wavefront variant (om_gemm_x.hpp, k_gemm_x2).
template <int BM, int BN, int BKT, int GM>
static bool launch_x2(const Params &p, int batch, bool ta, bool tb, hipStream_t st) {
    const unsigned total = (unsigned)((int64_t)(p.m / BM) * (p.n / BN) * batch * p.splits);
    const int gk = pick_family(GM, p.epi);
    if (gk < 0 || (gk > 0 && ta)) return false;
    if (!ta && !tb) {
        OMG_L(k_gemm_x2, 2 * NT, false, false)
    } else if (!ta && tb) {
        OMG_L(k_gemm_x2, 2 * NT, false, true)
    } else if (ta && !tb) {
        hipLaunchKernelGGL((gx::k_gemm_x2<BM, BN, BKT, true, false, 0>), dim3(total), dim3(2 * NT), 0, st, p);
    } else {
        return false;
    }
    return true;
}
#undef OMG_L

struct XTile {
    int bm, bn, bkt;
    int dma = 0;  // Choice::dma
};
// Launches tile t; false when t (or its variant for the product's epilogue) is not instantiated.
static bool dispatch_x(const XTile &t, const Params &p, int batch, bool ta, bool tb, hipStream_t st, int cus) {
    // bkt 33 / 65 select the eight-wavefront variant of the 32 / 64 chunk. The last template argument lists the
    // GELU epilogue families the tile instantiates (bit 0: the reference's polynomials, bit 1: the fast pair).
    if (t.bkt == 33 && t.bm == 64 && t.bn == 96) return launch_x2<64, 96, 32, 3>(p, batch, ta, tb, st);
    if (t.bkt == 33 && t.bm == 64 && t.bn == 64) return launch_x2<64, 64, 32, 1>(p, batch, ta, tb, st);
    if (t.bkt == 65 && t.bm == 64 && t.bn == 96) return launch_x2<64, 96, 64, 0>(p, batch, ta, tb, st);
    if (t.bkt == 33 && t.bm == 128 && t.bn == 128) return launch_x2<128, 128, 32, 2>(p, batch, ta, tb, st);
    if (t.bkt == 33 && t.bm == 128 && t.bn == 96) return launch_x2<128, 96, 32, 3>(p, batch, ta, tb, st);
#define OMG_X(BM, BN, BKT, GM) \
    if (t.bm == BM && t.bn == BN && t.bkt == BKT) return launch_x<BM, BN, BKT, GM>(p, batch, ta, tb, st, cus, t.dma);
    OMG_X(64, 64, 32, 3)
    OMG_X(64, 96, 32, 3)
    OMG_X(96, 64, 32, 0)
    OMG_X(64, 128, 32, 2)
    OMG_X(128, 64, 32, 2)
    OMG_X(128, 96, 32, 3)
    OMG_X(128, 128, 32, 2)
    OMG_X(64, 64, 64, 1)
    OMG_X(64, 96, 64, 0)
    OMG_X(128, 128, 64, 0)
#undef OMG_X
    return false;
}

// Whether tile t covers the product exactly (full tiles, whole chunks per split, 32-bit in-tile offsets).
static bool x_fits(const XTile &t, const Params &p, int splits, int k_split) {
    const int ck = t.bkt & ~1;  // chunk depth (an odd bkt selects the eight-wavefront variant)
    if (p.m % t.bm || p.n % t.bn || p.k % ck || k_split % ck) return false;
    if (splits > 1 && (int64_t)(splits - 1) * k_split >= p.k) return false;
    const int64_t ld = p.lda > p.ldb ? p.lda : p.ldb;
    const int rows = t.bm > t.bn ? t.bm : t.bn;
    return ld * (rows > ck ? rows : ck) < (int64_t)1 << 31;
}

namespace {
// Tuned choices for the products of the training path's configurations (MI355X, random operands, one sweep of
// the tile-exact kernels over tiles x chunk depths x split counts; C5's 768-wide rows re-swept with the 128 x 96
// tile, which makes 4096 x 768 exactly one tile per CU: 8 % faster for the FFN's second product and the attention
// output, 2-3 % for the q|k|v projection and two input gradients): exact shape -> tile and split count.
struct Tuned {
    int m, n, k;
    bool ta, tb;
    int bm, bn, bkt, splits;
    int dma = 0;  // Choice::dma
};
const Tuned kTuned[] = {
    // Linear forward y = x W^T (NT)
    {4096, 384, 384, false, true, 64, 96, 32, 1},     {4096, 1536, 384, false, true, 64, 96, 32, 1, 1},
    {4096, 384, 1536, false, true, 64, 96, 32, 1},    {4096, 1152, 384, false, true, 64, 96, 32, 1},
    {4096, 768, 768, false, true, 128, 96, 32, 1},    {4096, 3072, 768, false, true, 128, 128, 32, 1, 1},
    {4096, 768, 3072, false, true, 128, 96, 32, 1},   {4096, 2304, 768, false, true, 64, 96, 32, 1, 1},
    // input gradient dx = g W (NN); bkt 33 = the eight-wavefront kernel with 32-deep chunks
    {4096, 384, 384, false, false, 64, 96, 33, 1},    {4096, 384, 1536, false, false, 64, 96, 33, 1},
    {4096, 1536, 384, false, false, 64, 64, 33, 1},   {4096, 384, 1152, false, false, 64, 96, 33, 1},
    {4096, 768, 768, false, false, 64, 64, 32, 1},    {4096, 768, 3072, false, false, 128, 96, 33, 1},
    {4096, 3072, 768, false, false, 128, 128, 33, 1}, {4096, 768, 2304, false, false, 128, 96, 33, 1},
    // weight gradient dW = g^T x (TN), K = tokens
    {384, 384, 4096, true, false, 64, 96, 33, 8},     {1536, 384, 4096, true, false, 64, 96, 32, 8},
    {384, 1536, 4096, true, false, 64, 96, 32, 8},    {1152, 384, 4096, true, false, 64, 64, 32, 4},
    {768, 768, 4096, true, false, 64, 96, 32, 8},     {3072, 768, 4096, true, false, 64, 96, 32, 2},
    {768, 3072, 4096, true, false, 64, 96, 32, 2},    {2304, 768, 4096, true, false, 64, 96, 32, 2},
};
// The same for products with a GELU epilogue (GELU and its slope in the forward, the slope product in the input
// gradient), whose element-wise tail shifts the best tile: the reference's polynomials (family 1) and the slope
// product beside them ...
const Tuned kTunedEpi[] = {
    {4096, 1536, 384, false, true, 64, 64, 32, 1},
    {4096, 1536, 384, false, false, 64, 96, 33, 1},
};
// ... and the fast pair (family 2) with its slope product, whose shorter tail lets the wide tiles of the plain
// products through. The forward products run on the direct-to-LDS kernel; their tiles were picked by the step time
// (C3 0.5304 ms at 64 x 64 against 0.5310 at 64 x 96 and 0.5333 for the register-staged 128 x 96; C5 7.166 ms at
// 64 x 96 against 7.199 at 128 x 128 and 7.185 register-staged), which ranks them differently from the products
// timed alone on warm operands.
const Tuned kTunedGeluFast[] = {
    {4096, 1536, 384, false, true, 64, 64, 32, 1, 1}, {4096, 3072, 768, false, true, 64, 96, 32, 1, 1},
    {4096, 1536, 384, false, false, 64, 96, 33, 1},   {4096, 3072, 768, false, false, 64, 64, 32, 1},
};

// K length of one split: k / splits rounded up to whole chunks.
int split_len(int k, int splits, int bkt) { return ((k + splits - 1) / splits + bkt - 1) / bkt * bkt; }

Choice with_splits(int bm, int bn, int bkt, int k, int splits) {
    Choice c{bm, bn, 1, k, bkt};
    if (splits > 1) {
        c.k_split = split_len(k, splits, bkt & ~1);
        c.splits = (k + c.k_split - 1) / c.k_split;
        if (c.splits <= 1) c.k_split = k;
    }
    return c;
}

// Tuning builds (om::tuning_env): OM_GEMM_X="bm,bn,bkt[,splits]" forces a tile-exact configuration where it fits (read
// at every call, so one process can compare configurations).
bool env_override(Choice &c, int k) {
    const char *s = om::tuning_env("OM_GEMM_X");
    if (!s || !*s || !strcmp(s, "off")) return false;
    int bm = 0, bn = 0, bk = 32, sp = 1;
    if (sscanf(s, "%d,%d,%d,%d", &bm, &bn, &bk, &sp) < 3) return false;
    c = with_splits(bm, bn, bk, k, sp);
    return true;
}
// Tile order of the grouped weight gradients: bands of 8 tile rows walked column by column when the group runs
// unsplit (C5's layers: 1728 tiles, 517 -> ~490 us per launch, the step 7.37 -> 7.26 ms), row-major when it splits K
// (C3's four products: banding cut the fetch but slowed the step). Tuning builds read OM_GROUP_BAND (0: row-major).
int group_band(int splits) {
    static const int b = [] {
        const char *s = om::tuning_env("OM_GROUP_BAND");
        return s && *s ? atoi(s) : -1;
    }();
    return b >= 0 ? b : (splits == 1 ? 8 : 0);
}
bool x_disabled() {
    const char *s = om::tuning_env("OM_GEMM_X");
    return s && !strcmp(s, "off");
}
// Tuning builds: OM_GEMM_T="m,n,k,ta,tb,family:bm,bn,bkt,splits,dma;..." replaces the tuned choice of the products of
// exactly that shape and epilogue family (for step-level comparisons of one product's tile).
struct ShapeOverride {
    int m, n, k, ta, tb, fam, bm, bn, bkt, splits, dma;
};
const std::vector<ShapeOverride> &shape_overrides() {
    static const std::vector<ShapeOverride> v = [] {
        std::vector<ShapeOverride> out;
        const char *s = om::tuning_env("OM_GEMM_T");
        while (s && *s) {
            ShapeOverride o{};
            if (sscanf(s, "%d,%d,%d,%d,%d,%d:%d,%d,%d,%d,%d", &o.m, &o.n, &o.k, &o.ta, &o.tb, &o.fam, &o.bm, &o.bn,
                       &o.bkt, &o.splits, &o.dma) == 11)
                out.push_back(o);
            s = strchr(s, ';');
            if (s) s++;
        }
        return out;
    }();
    return v;
}
}  // namespace

// Aligned operands: the tuned table for the training path's products, else the rule it was distilled into
// (MI355X measurements, random operands):
//   - long-K products with few 64 x 64 tiles (weight gradients, K = tokens) split K into a power-of-two number of
//     slices of at least 256 k, with tiles x splits near three workgroups per CU (64 x 96 tiles when N allows);
//   - otherwise 64 x 96 when N is a multiple of 96 and its tiles fit in one round of the CUs (4096 x 384 becomes
//     exactly 256 tiles: one per CU), else 64 x 64 (occupancy 4, best once there are several tiles per CU).
Choice choose_fast(int m, int n, int k, int batch, bool ta, bool tb, int cus, int family) {
    Choice best{64, 64, 1, k, 32};
    if (env_override(best, k)) return best;
    for (const ShapeOverride &o : shape_overrides())
        if (o.m == m && o.n == n && o.k == k && o.ta == (int)ta && o.tb == (int)tb && o.fam == family && batch == 1) {
            Choice c = with_splits(o.bm, o.bn, o.bkt, k, o.splits);
            c.dma = o.dma;
            return c;
        }
    if (batch == 1 && family == 2)
        for (const Tuned &t : kTunedGeluFast)
            if (t.m == m && t.n == n && t.k == k && t.ta == ta && t.tb == tb) {
                Choice c = with_splits(t.bm, t.bn, t.bkt, k, t.splits);
                c.dma = t.dma;
                return c;
            }
    if (batch == 1 && family == 1)
        for (const Tuned &t : kTunedEpi)
            if (t.m == m && t.n == n && t.k == k && t.ta == ta && t.tb == tb)
                return with_splits(t.bm, t.bn, t.bkt, k, t.splits);
    if (batch == 1)
        for (const Tuned &t : kTuned)
            if (t.m == m && t.n == n && t.k == k && t.ta == ta && t.tb == tb) {
                Choice c = with_splits(t.bm, t.bn, t.bkt, k, t.splits);
                c.dma = t.dma;
                return c;
            }
    const bool n96 = n % 96 == 0 && m >= 64;
    int64_t tiles = (int64_t)((m + 63) / 64) * (n96 ? n / 96 : (n + 63) / 64) * batch;
    // A handful of tiles over a long-enough K (an MLP's first layer: 4 tiles over K = 784) leaves most CUs idle, and
    // each workgroup's chunks then follow one another at memory latency: split K into slices of at least 64 k until
    // there are about as many workgroups as CUs / 2.
    if (batch == 1 && 8 * tiles <= cus && k >= 256) {
        int s = 1;
        while (s < 16 && k / (2 * s) >= 64 && tiles * 2 * s <= cus / 2) s *= 2;
        if (s > 1) return with_splits(64, 64, 32, k, s);
    }
    if (batch == 1 && tiles < 2 * cus && k >= 1024) {
        double want = 3.0 * cus / (double)tiles;
        int s = 1;
        while (s < 16 && k / (2 * s) >= 256 && 2.0 * s <= want * 1.41421356) s *= 2;
        if (s > 1) return with_splits(64, n96 ? 96 : 64, 32, k, s);
    }
    int64_t tiles96 = (int64_t)((m + 63) / 64) * ((n + 95) / 96) * batch;
    if (n96 && tiles96 <= cus) best.bn = 96;
    return best;
}

// Thin products (one side at most 32: a classifier head's weight gradient, 9 x 768 over K = 4096 tokens) take the
// 128 x 32 / 32 x 128 tiles. Products with fewer tiles than CUs (the classifier heads, small batches) split K into
// slices of at least 32 k, up to about one workgroup per CU: their time is the chain of chunk loads each workgroup
// waits for, not arithmetic.
Choice choose(int m, int n, int k, int batch, int cus) {
    Choice c{64, 64, 1, k, 16};
    if (n <= 32) c = Choice{128, 32, 1, k, 16};
    else if (m <= 32) c = Choice{32, 128, 1, k, 16};
    int64_t tiles = (int64_t)((m + c.bm - 1) / c.bm) * ((n + c.bn - 1) / c.bn) * batch;
    if (batch == 1 && tiles < cus && k >= 64) {
        int want = (int)((cus + tiles - 1) / tiles);
        int maxs = k / 32;
        int s = want < maxs ? want : maxs;
        if (s > 1) {
            int ks = ((k + s - 1) / s + 15) / 16 * 16;
            c.splits = (k + ks - 1) / ks;
            c.k_split = ks;
        }
    }
    return c;
}

om_status launch_dense(om_ctx *ctx, Params p, bool ta, bool tb, int batch, const char *what, bool *colsum_fused,
                       int *mse_slots) {
    if (colsum_fused) *colsum_fused = false;
    if (mse_slots) *mse_slots = 0;
    if (p.m <= 0 || p.n <= 0 || batch <= 0) return OM_OK;
    p.batch = batch;
    bool vec = ((uintptr_t)p.a % 16 == 0) && ((uintptr_t)p.b % 16 == 0) && p.lda % 4 == 0 && p.ldb % 4 == 0 &&
               p.sa_outer % 4 == 0 && p.sa_inner % 4 == 0 && p.sb_outer % 4 == 0 && p.sb_inner % 4 == 0;
    bool fast = vec && !(ta && tb) && p.k > 0 && p.m > 32 && p.n > 32 && p.m % 4 == 0 && p.n % 4 == 0 &&
                p.k % 4 == 0;
    // The slope product (EPI_MUL_AUX) takes the tiles of the GELU products of the context's mode, so that in either
    // mode om_linear_bwd_dx_slope of the forward's slope and om_linear_bwd_dx_gelu give the same bits.
    int fam = epi_family(p.epi);
    if (fam == 3) fam = ctx->gelu_mode == OM_GELU_REFERENCE ? 1 : 2;
    Choice c = p.k <= 0 ? Choice{64, 64, 1, 1, 16}
                        : (fast ? choose_fast(p.m, p.n, p.k, batch, ta, tb, ctx->num_cus, fam)
                                : choose(p.m, p.n, p.k, batch, ctx->num_cus));
    if (fast && fam == 1) {  // only some tiles carry the reference's GELU polynomials
        const bool ok = ((c.bkt == 32 || c.bkt == 33) && c.bm == 64 && (c.bn == 64 || c.bn == 96)) ||
                        (c.bkt == 64 && c.bm == 64 && c.bn == 64);
        if (!ok) c = with_splits(64, 64, 32, p.k, c.splits);
    } else if (fast && fam == 2) {  // the fast pair and the slope product: the tiles of dispatch_x's list
        const bool ok = (c.bkt == 32 && ((c.bm == 64 && (c.bn == 64 || c.bn == 96 || c.bn == 128)) ||
                                         (c.bm == 128 && (c.bn == 64 || c.bn == 96 || c.bn == 128)))) ||
                        (c.bkt == 33 && ((c.bm == 64 && c.bn == 96) || (c.bm == 128 && (c.bn == 96 || c.bn == 128))));
        if (!ok) c = with_splits(64, 64, 32, p.k, c.splits);
    }
    bool use_x = fast && !x_disabled() && x_fits(XTile{c.bm, c.bn, c.bkt}, p, c.splits, c.k_split);
    if (fast && !use_x && c.bkt != 32) c = with_splits(c.bm, c.bn, 32, p.k, c.splits);  // guarded set: BK = 32
    c.bkt = use_x ? c.bkt : 32;
    p.splits = c.splits;
    p.k_split = c.splits > 1 ? c.k_split : (p.k > 0 ? p.k : 1);
    p.ws = nullptr;
    p.xcd_remap = 1;
    // A fused bias gradient needs a tile-exact TN launch whose row groups divide the workgroup.
    const bool cs = p.db && use_x && ta && !tb && batch == 1 && ((c.bkt & 1) ? 2 * NT : NT) % c.bm == 0;
    if (!cs) {
        p.db = nullptr;
        p.colsum_ws = nullptr;
    }
    if (p.splits > 1) {
        float *ws;
        const uint64_t cbytes = cs ? (sizeof(double) * (uint64_t)p.splits * p.m + 255) / 256 * 256 : 0;
        om_status s = om::scratch(ctx, cbytes + sizeof(float) * (uint64_t)p.splits * p.m * p.n, &ws);
        if (s) return s;
        p.colsum_ws = cs ? reinterpret_cast<double *>(ws) : nullptr;
        p.ws = reinterpret_cast<float *>(reinterpret_cast<char *>(ws) + cbytes);
    }
    if (colsum_fused) *colsum_fused = cs;
    // The fused MSE needs the tile-exact epilogue over one split (one workgroup per tile, four wavefronts each).
    const bool mse = p.mse_t && use_x && p.splits == 1 && batch == 1;
    if (!mse) {
        p.mse_t = nullptr;
        p.mse_unit = nullptr;
        p.mse_part = nullptr;
    }
    hipStream_t st = om::cur_stream(ctx);
    bool launched = use_x && dispatch_x(XTile{c.bm, c.bn, c.bkt, c.dma}, p, batch, ta, tb, st, ctx->num_cus);
    if (mse && launched && mse_slots) *mse_slots = (p.m / c.bm) * (p.n / c.bn) * 4;
    if (launched) {
    } else if (fast) {
        if (c.bm == 128 && c.bn == 192) launch_fast<128, 192>(p, batch, ta, tb, st);
        else if (c.bm == 192 && c.bn == 128) launch_fast<192, 128>(p, batch, ta, tb, st);
        else if (c.bm == 128 && c.bn == 128) launch_fast<128, 128>(p, batch, ta, tb, st);
        else if (c.bm == 128 && c.bn == 64) launch_fast<128, 64>(p, batch, ta, tb, st);
        else if (c.bm == 64 && c.bn == 128) launch_fast<64, 128>(p, batch, ta, tb, st);
        else if (c.bm == 64 && c.bn == 96) launch_fast<64, 96>(p, batch, ta, tb, st);
        else if (c.bm == 96 && c.bn == 64) launch_fast<96, 64>(p, batch, ta, tb, st);
        else launch_fast<64, 64>(p, batch, ta, tb, st);
    } else {
        if (c.bm == 128 && c.bn == 32) launch_general<128, 32>(p, batch, ta, tb, vec, st);
        else if (c.bm == 32 && c.bn == 128) launch_general<32, 128>(p, batch, ta, tb, vec, st);
        else launch_general<64, 64>(p, batch, ta, tb, vec, st);
    }
    om_status s = OM_LAUNCH_CHECK(ctx, what);
    if (s || p.splits <= 1) return s;
    if (p.n % 4 == 0 && (p.splits == 2 || p.splits == 4 || p.splits == 8 || p.splits == 16)) {
        const int64_t quads = (int64_t)p.m * (p.n / 4);
        const dim3 grid(om::grid1d(quads > p.m ? quads : p.m, 256, 4096));
        if (p.splits == 2) hipLaunchKernelGGL(k_splitk_reduce_s<2>, grid, dim3(256), 0, st, p);
        else if (p.splits == 4) hipLaunchKernelGGL(k_splitk_reduce_s<4>, grid, dim3(256), 0, st, p);
        else if (p.splits == 8) hipLaunchKernelGGL(k_splitk_reduce_s<8>, grid, dim3(256), 0, st, p);
        else hipLaunchKernelGGL(k_splitk_reduce_s<16>, grid, dim3(256), 0, st, p);
    } else {
        hipLaunchKernelGGL(k_splitk_reduce, dim3(om::grid1d((int64_t)p.m * p.n, 256, 4096)), dim3(256), 0, st,
                           p);
    }
    return OM_LAUNCH_CHECK(ctx, what);
}

// Weight gradients dw_i (+)= g_i^T x_i of 2..kMaxGroup products sharing K = rows, with fused bias gradients, in one
// tile-exact launch (and one split-K reduce). Returns false, launching nothing, when the products do not fit it:
// then the caller runs them one by one. Each product's arithmetic is that of k_gemm_x at the group's tile and split.
// Fills the column-sum items of g (prefix counts in wavefronts, one per column).
static void set_column_sums(GroupParams &g, int ncs, const om_column_sum *cs) {
    g.ncs = ncs;
    g.cstart[0] = 0;
    for (int j = 0; j < ncs; j++) {
        g.cs[j] = ColSumItem{cs[j].part, cs[j].out, cs[j].chunks, cs[j].cols, cs[j].acc};
        g.cstart[j + 1] = g.cstart[j] + cs[j].cols;
    }
    for (int j = ncs; j < kMaxColSums; j++) g.cstart[j + 1] = g.cstart[ncs];
}

// The grouped reduce: split-K partials (S splits) of g's products, their fused bias sums and g's column sums.
static om_status launch_group_reduce(om_ctx *ctx, const GroupParams &g, int splits, hipStream_t stream) {
    const int64_t qb = (g.qstart[g.count] + 255) / 256, rb = (g.rstart[g.count] + 255) / 256;
    const int64_t cb = ((int64_t)g.cstart[g.ncs] + 3) / 4;
    if (qb + rb + cb == 0) return OM_OK;
    OM_REQUIRE(ctx, qb + rb + cb < ((int64_t)1 << 31), "grouped reduce: %lld blocks", (long long)(qb + rb + cb));
    const dim3 grid((unsigned)(qb + rb + cb));
    const int c = (int)cb, r = (int)rb;
    if (splits <= 1) hipLaunchKernelGGL(k_splitk_reduce_group<1>, grid, dim3(256), 0, stream, g, c, r);
    else if (splits == 2) hipLaunchKernelGGL(k_splitk_reduce_group<2>, grid, dim3(256), 0, stream, g, c, r);
    else if (splits == 4) hipLaunchKernelGGL(k_splitk_reduce_group<4>, grid, dim3(256), 0, stream, g, c, r);
    else if (splits == 8) hipLaunchKernelGGL(k_splitk_reduce_group<8>, grid, dim3(256), 0, stream, g, c, r);
    else hipLaunchKernelGGL(k_splitk_reduce_group<16>, grid, dim3(256), 0, stream, g, c, r);
    return OM_LAUNCH_CHECK(ctx, "grouped reduce");
}

// A weight gradient the grouped launch can take: whole 64 x 64 tiles over 16-byte aligned operands.
static bool dw_groupable(const om_linear_dw &d) {
    auto al = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
    return d.dw && d.out % 64 == 0 && d.in % 64 == 0 && al(d.g) && al(d.x) && al(d.dw);
}
static bool launch_dw_group(om_ctx *ctx, int count, const om_linear_dw *it, int rows, int ncs, const om_column_sum *cs,
                            om_status *st) {
    *st = OM_OK;
    if (count < 2 || count > kMaxGroup || rows <= 0 || x_disabled()) return false;
    bool n96 = true;
    for (int i = 0; i < count; i++) {
        const om_linear_dw &d = it[i];
        if (!dw_groupable(d)) return false;
        if (d.in % 96) n96 = false;
    }
    // 64 x 64 tiles, split until there are about six workgroups per CU (measured on the four C3 weight gradients:
    // 148 us at 64 x 64 with 4 splits against 152 us for the best 64 x 96 choice, 8 splits).
    int bn = 64;
    int64_t tiles = 0;
    for (int i = 0; i < count; i++) tiles += (int64_t)(it[i].out / 64) * (it[i].in / bn);
    int splits = 1;
    while (splits < 16 && tiles * splits < 6 * (int64_t)ctx->num_cus && rows % (2 * splits * 32) == 0 &&
           rows / (2 * splits) >= 256)
        splits *= 2;
    if (const char *gx = om::tuning_env("OM_GROUP_X")) {  // tuning builds: OM_GROUP_X="bn,splits" for this launch only
        int fbn = 0, fsp = 0;
        if (sscanf(gx, "%d,%d", &fbn, &fsp) == 2 && (fbn == 64 || (fbn == 96 && n96))) {
            bn = fbn;
            splits = fsp;
        }
    }
    Choice forced{};
    if (env_override(forced, rows)) {  // OM_GEMM_X="64,bn,32,splits" for measurements
        if (forced.bm != 64 || forced.bkt != 32 || (forced.bn != 64 && forced.bn != 96) || (forced.bn == 96 && !n96))
            return false;
        bn = forced.bn;
        splits = forced.splits;
    }
    if (splits < 1 || (splits & (splits - 1)) || splits > 16 || rows % (splits * 32)) return false;
    const int k_split = rows / splits;
    GroupParams g{};
    g.count = count;
    g.band = group_band(splits);
    uint64_t ws_floats = 0, cs_doubles = 0;
    for (int i = 0; i < count; i++) {
        const om_linear_dw &d = it[i];
        Params p = dense_params(d.out, d.in, rows, d.g, d.out, d.x, d.in, d.dw, d.in);
        p.accumulate = d.acc_dw;
        p.db = d.db;
        p.db_acc = d.acc_db;
        p.batch = 1;
        p.splits = splits;
        p.k_split = k_split;
        if (!x_fits(XTile{64, bn, 32}, p, splits, k_split)) return false;
        ws_floats += splits > 1 ? (uint64_t)splits * d.out * d.in : 0;
        cs_doubles += splits > 1 && d.db ? (uint64_t)splits * d.out : 0;
        g.p[i] = p;
    }
    if (splits > 1) {
        const uint64_t cbytes = (sizeof(double) * cs_doubles + 255) / 256 * 256;
        float *ws;
        *st = om::scratch(ctx, cbytes + sizeof(float) * ws_floats, &ws);
        if (*st) return true;
        double *cs = reinterpret_cast<double *>(ws);
        float *w = reinterpret_cast<float *>(reinterpret_cast<char *>(ws) + cbytes);
        for (int i = 0; i < count; i++) {
            Params &p = g.p[i];
            p.ws = w;
            w += (uint64_t)splits * p.m * p.n;
            if (p.db) {
                p.colsum_ws = cs;
                cs += (uint64_t)splits * p.m;
            }
        }
    }
    g.start[0] = 0;
    g.qstart[0] = 0;
    g.rstart[0] = 0;
    for (int i = 0; i < count; i++) {
        const Params &p = g.p[i];
        g.start[i + 1] = g.start[i] + (p.m / 64) * (p.n / bn) * splits;
        g.qstart[i + 1] = g.qstart[i] + (int64_t)p.m * (p.n / 4);
        g.rstart[i + 1] = g.rstart[i] + (splits > 1 && p.db ? p.m : 0);
    }
    for (int i = count; i < kMaxGroup; i++) {
        g.start[i + 1] = g.start[count];
        g.qstart[i + 1] = g.qstart[count];
        g.rstart[i + 1] = g.rstart[count];
    }
    hipStream_t stream = om::cur_stream(ctx);
    if (bn == 96) hipLaunchKernelGGL((gx::k_gemm_x_tn_group<64, 96, 32>), dim3(g.start[count]), dim3(NT), 0, stream, g);
    else hipLaunchKernelGGL((gx::k_gemm_x_tn_group<64, 64, 32>), dim3(g.start[count]), dim3(NT), 0, stream, g);
    *st = OM_LAUNCH_CHECK(ctx, "om_param_grads_group");
    if (*st) return true;
    if (splits == 1) {  // the products are complete: only the column sums are left
        g.count = 0;
        for (int i = 0; i <= kMaxGroup; i++) g.qstart[i] = g.rstart[i] = 0;
    }
    set_column_sums(g, ncs, cs);
    *st = launch_group_reduce(ctx, g, splits, stream);
    return true;
}

Params dense_params(int m, int n, int k, const float *a, int64_t lda, const float *b, int64_t ldb, float *c,
                    int64_t ldc) {
    Params p{};
    p.m = m;
    p.n = n;
    p.k = k;
    p.batch_div = 1;
    p.a = a;
    p.lda = lda;
    p.b = b;
    p.ldb = ldb;
    p.c = c;
    p.ldc = ldc;
    p.alpha = 1.0f;
    p.splits = 1;
    return p;
}

}  // namespace omg

// ------------------------------------------------------------------------------------------------------------------
// Linear layers too small for the MFMA engine to pay (rows <= 256, out <= 32, rows * in * out <= 2^21: a classifier
// head over a small batch). Their time is launch latency, so the forward is one launch and the whole backward (dx,
// dW, db) another. Each output is one fmaf chain over k in increasing order, as the reference's fast-mode Dense.Gemm
// accumulates, then the bias add; the bias gradient is a double sum over rows in increasing order.
namespace {
using omg::floatx4;
constexpr int kSmallRows = 256, kSmallOut = 32, kNarrowOut = 64, kNarrowIn = 8192;
bool linear_small(int rows, int in, int out) {
    return rows >= 1 && rows <= kSmallRows && out >= 1 && out <= kSmallOut && in >= 1 &&
           (int64_t)rows * in * out <= ((int64_t)1 << 21);
}
// y[r][o] = (sum over i of x[r][i] w[o][i]) + b[o] (+ resid[r][o]: the Linear then the residual Add, as the
// engine's epilogue orders them): a thread per output, each an fmaf chain over i in increasing order. A workgroup
// takes small_rt(out) consecutive rows with all their outputs; its x rows and all of w pass through LDS in chunks of
// kSmallKC columns, loaded by the whole workgroup (a few loads per thread, all in flight together), the next chunk's
// loads issued before the chains over the current one run. VEC: in % 4 == 0 and 16-byte aligned x and w.
constexpr int kSmallKC = 128, kSmallLd = kSmallKC + 4, kSmallRtMax = 64;
__host__ __device__ constexpr int small_rt(int out) { return 256 / out < kSmallRtMax ? 256 / out : kSmallRtMax; }
constexpr int small_stage_rows() {
    int m = 0;
    for (int o = 1; o <= kNarrowOut; o++) m = small_rt(o) + o > m ? small_rt(o) + o : m;
    return m;
}
constexpr int kSmallStage = small_stage_rows();  // x rows plus w rows of a workgroup, at most
template <bool VEC>
__global__ void __launch_bounds__(256) k_linear_small_fwd(const float *__restrict__ x, const float *__restrict__ w,
                                                          const float *__restrict__ b, const float *__restrict__ resid,
                                                          float *__restrict__ y, int rows, int in, int out) {
    OM_LDS_POISON();
    constexpr int Q = VEC ? kSmallKC / 4 : kSmallKC;  // load items per staged row and chunk
    constexpr int PER = (kSmallStage * Q + 255) / 256;
    __shared__ __attribute__((aligned(16))) float st[kSmallStage * kSmallLd];
    const int r0 = blockIdx.x * small_rt(out), nr = min(small_rt(out), rows - r0), srows = nr + out;
    const int tid = threadIdx.x, rl = tid / out, o = tid - rl * out;
    const bool live = rl < nr;
    // staged row s: x row r0 + s for s < nr, then w row s - nr
    auto src = [&](int s) { return s < nr ? x + (int64_t)(r0 + s) * in : w + (int64_t)(s - nr) * in; };
    // two register sets: the loads of chunk c + 2 are in flight while chunk c is multiplied
    floatx4 rv[2][VEC ? PER : 1];
    float rs[2][VEC ? 1 : PER];
    auto load = [&](int set, int c) {
        const int k0 = c * kSmallKC, kn = min(kSmallKC, in - k0);
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int f = tid + 256 * u, s = f / Q, q = f - s * Q;
            if (VEC) {
                if (s < srows && 4 * q < kn) rv[set][u] = *reinterpret_cast<const floatx4 *>(src(s) + k0 + 4 * q);
            } else {
                if (s < srows && q < kn) rs[set][u] = src(s)[k0 + q];
            }
        }
    };
    auto stage = [&](int set, int kn) {
#pragma unroll
        for (int u = 0; u < PER; u++) {
            const int f = tid + 256 * u, s = f / Q, q = f - s * Q;
            if (VEC) {
                if (s < srows && 4 * q < kn) *reinterpret_cast<floatx4 *>(&st[s * kSmallLd + 4 * q]) = rv[set][u];
            } else {
                if (s < srows && q < kn) st[s * kSmallLd + q] = rs[set][u];
            }
        }
    };
    const int nchunk = (in + kSmallKC - 1) / kSmallKC;
    load(0, 0);
    if (nchunk > 1) load(1, 1);
    float acc = 0.0f;
    const float *xs = st + rl * kSmallLd, *ws = st + (nr + o) * kSmallLd;
    for (int c = 0; c < nchunk; c++) {
        const int kn = min(kSmallKC, in - c * kSmallKC);
        // the set index is static in each branch, so the register sets stay registers
        if ((c & 1) == 0) {
            stage(0, kn);
            __syncthreads();
            if (c + 2 < nchunk) load(0, c + 2);
        } else {
            stage(1, kn);
            __syncthreads();
            if (c + 2 < nchunk) load(1, c + 2);
        }
        if (live) {
            if (kn == kSmallKC) {
                // a whole chunk: 32 values of each row read ahead of the 32 fmafs that use them
                floatx4 xa[8], wa[8], xb[8], wb[8];
                auto rd = [&](floatx4(&xd)[8], floatx4(&wd)[8], int k0) {
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        xd[u] = *reinterpret_cast<const floatx4 *>(xs + k0 + 4 * u);
                        wd[u] = *reinterpret_cast<const floatx4 *>(ws + k0 + 4 * u);
                    }
                };
                auto mac = [&](const floatx4(&xd)[8], const floatx4(&wd)[8]) {
#pragma unroll
                    for (int u = 0; u < 8; u++)
#pragma unroll
                        for (int e = 0; e < 4; e++) acc = __builtin_fmaf(xd[u][e], wd[u][e], acc);
                };
                static_assert(kSmallKC == 128, "four groups of 32 per chunk");
                rd(xa, wa, 0);
                rd(xb, wb, 32);
                mac(xa, wa);
                rd(xa, wa, 64);
                mac(xb, wb);
                rd(xb, wb, 96);
                mac(xa, wa);
                mac(xb, wb);
            } else {
                int k = 0;
#pragma unroll 8
                for (; k + 4 <= kn; k += 4) {
                    const floatx4 a = *reinterpret_cast<const floatx4 *>(xs + k);
                    const floatx4 bb = *reinterpret_cast<const floatx4 *>(ws + k);
#pragma unroll
                    for (int e = 0; e < 4; e++) acc = __builtin_fmaf(a[e], bb[e], acc);
                }
                for (; k < kn; k++) acc = __builtin_fmaf(xs[k], ws[k], acc);
            }
        }
        __syncthreads();
    }
    if (!live) return;
    const int t = (r0 + rl) * out + o;
    float v = b ? acc + b[o] : acc;
    if (resid) v = v + resid[t];
    y[t] = v;
}
void launch_small_fwd(hipStream_t st, const float *x, const float *w, const float *b, const float *resid, float *y,
                      int rows, int in, int out) {
    const dim3 grid((unsigned)((rows + small_rt(out) - 1) / small_rt(out)));
    auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    if (in % 4 == 0 && al(x) && al(w))
        hipLaunchKernelGGL(k_linear_small_fwd<true>, grid, dim3(256), 0, st, x, w, b, resid, y, rows, in, out);
    else
        hipLaunchKernelGGL(k_linear_small_fwd<false>, grid, dim3(256), 0, st, x, w, b, resid, y, rows, in, out);
}
// The backward over a grid of (input columns / 256, 1 + row blocks): workgroups with blockIdx.y = 0 form
// dw[o][i] (+)= sum over r of g[r][o] x[r][i] (a thread per input column i, an fmaf chain per o over r in increasing
// order, x's column loads running kSmallRc rows ahead) and db[o] (+)= (float) double sum over r of g[r][o]; the others
// form dx[r][i] (+)= sum over o of g[r][o] w[o][i] for kSmallDxRows rows each (an fmaf chain over o in increasing
// order). Every lane of a workgroup reads the same g[r][o] at the same time: uniform addresses of read-only memory,
// which the compiler turns into scalar loads (no LDS staging, no barrier). OUT is the layer's output count, a
// compile-time constant so the loops over it unroll.
constexpr int kSmallDxRows = 8, kSmallRc = 32;
// dx[r][i] (+)= sum over o of g[r][o] w[o][i] for rows r0 .. r0 + kSmallDxRows - 1, column i: an fmaf chain over o in
// increasing order per row (OUT = the layer's output count).
template <int OUT>
__device__ __forceinline__ void dx_rows(const float *__restrict__ g, const float *__restrict__ w, float *__restrict__ dx,
                                        int rows, int in, int ax, int r0, int i) {
    const int nr = min(kSmallDxRows, rows - r0);
    if (i >= in) return;
    float wv[OUT];
#pragma unroll
    for (int o = 0; o < OUT; o++) wv[o] = w[(int64_t)o * in + i];
#pragma unroll 4
    for (int r = 0; r < nr; r++) {
        const float *gr = g + (int64_t)(r0 + r) * OUT;
        float acc = 0.0f;
#pragma unroll
        for (int o = 0; o < OUT; o++) acc = __builtin_fmaf(gr[o], wv[o], acc);
        float *d = dx + (int64_t)(r0 + r) * in + i;
        *d = ax ? *d + acc : acc;
    }
}
template <int OUT>
__global__ void __launch_bounds__(256) k_linear_small_bwd(const float *__restrict__ g, const float *__restrict__ x,
                                                          const float *__restrict__ w, float *__restrict__ dx,
                                                          float *__restrict__ dw, float *__restrict__ db, int rows,
                                                          int in, int ax, int aw, int ab) {
    OM_LDS_POISON();
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (blockIdx.y > 0) {
        dx_rows<OUT>(g, w, dx, rows, in, ax, (blockIdx.y - 1) * kSmallDxRows, i);
        return;
    }
    if (blockIdx.x == 0 && db && (int)threadIdx.x < OUT) {
        // rows in increasing order, the loads of sixteen issued before their adds
        const int o = threadIdx.x;
        double s = 0.0;
        for (int r0 = 0; r0 < rows; r0 += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = g[(int64_t)min(r0 + u, rows - 1) * OUT + o];
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (r0 + u < rows) s += v[u];
        }
        const float v = (float)s;
        db[o] = ab ? db[o] + v : v;
    }
    if (!dw || i >= in) return;
    // rows past the end load the last row again (never used), so every load is unconditional
    float xa[kSmallRc], xb[kSmallRc];
    auto ld = [&](float(&d)[kSmallRc], int rb) {
#pragma unroll
        for (int u = 0; u < kSmallRc; u++) d[u] = x[(int64_t)min(rb + u, rows - 1) * in + i];
    };
    float acc[OUT];
#pragma unroll
    for (int o = 0; o < OUT; o++) acc[o] = 0.0f;
    auto use = [&](const float(&d)[kSmallRc], int rb) {
        const float *gr = g + (int64_t)rb * OUT;
        if (rb + kSmallRc <= rows) {
#pragma unroll
            for (int u = 0; u < kSmallRc; u++)
#pragma unroll
                for (int o = 0; o < OUT; o++) acc[o] = __builtin_fmaf(gr[u * OUT + o], d[u], acc[o]);
        } else {
#pragma unroll
            for (int u = 0; u < kSmallRc; u++) {
                if (rb + u >= rows) break;
#pragma unroll
                for (int o = 0; o < OUT; o++) acc[o] = __builtin_fmaf(gr[u * OUT + o], d[u], acc[o]);
            }
        }
    };
    ld(xa, 0);
    for (int rb = 0; rb < rows; rb += 2 * kSmallRc) {
        if (rb + kSmallRc < rows) ld(xb, rb + kSmallRc);
        use(xa, rb);
        if (rb + 2 * kSmallRc < rows) ld(xa, rb + 2 * kSmallRc);
        if (rb + kSmallRc < rows) use(xb, rb + kSmallRc);
    }
#pragma unroll
    for (int o = 0; o < OUT; o++) {
        float *d = dw + (int64_t)o * in + i;
        *d = aw ? *d + acc[o] : acc[o];
    }
}
template <int OUT>
void launch_small_bwd(hipStream_t st, const float *g, const float *x, const float *w, float *dx, float *dw, float *db,
                      int rows, int in, int ax, int aw, int ab) {
    const dim3 grid((unsigned)((in + 255) / 256), 1u + (dx ? (unsigned)((rows + kSmallDxRows - 1) / kSmallDxRows) : 0u));
    hipLaunchKernelGGL(k_linear_small_bwd<OUT>, grid, dim3(256), 0, st, g, x, w, dx, dw, db, rows, in, ax, aw, ab);
}
template <int... OS>
void small_bwd_dispatch(std::integer_sequence<int, OS...>, int out, hipStream_t st, const float *g, const float *x,
                        const float *w, float *dx, float *dw, float *db, int rows, int in, int ax, int aw, int ab) {
    ((out == OS + 1 ? (launch_small_bwd<OS + 1>(st, g, x, w, dx, dw, db, rows, in, ax, aw, ab), 0) : 0), ...);
}

// ------------------------------------------------------------------------------------------------------------------
// Narrow Linear layers: out <= 64 with more rows than the one-launch path takes (a classifier head over a sequence or
// a batch of tokens), where 64-wide MFMA tiles would be mostly padding. The forward is k_linear_small_fwd (any row
// count; one fmaf chain per output as the reference accumulates); dx runs dx_rows over row blocks; dW and db sum
// row chunks (narrow_chunk) into partials, which a second launch adds in chunk order.
constexpr int kNarrowMaxChunks = 64;
bool linear_narrow(int rows, int in, int out) {
    return rows >= 1 && rows <= (1 << 20) && out >= 1 && out <= kNarrowOut && in >= 1 && in <= kNarrowIn &&
           !linear_small(rows, in, out);
}
// Rows per chunk: about 1024 workgroups over the column blocks and chunks (short chunks put all of a lane's x loads
// in flight at once), at most kNarrowMaxChunks chunks, whole groups of four rows.
int narrow_chunk(int rows, int in) {
    const int ncb = (in + 63) / 64;
    int nch = (1024 + ncb - 1) / ncb;
    if (nch > kNarrowMaxChunks) nch = kNarrowMaxChunks;
    if (nch < 1) nch = 1;
    const int c = (rows + nch - 1) / nch;
    return (c + 3) / 4 * 4;
}
template <int OUT>
__global__ void __launch_bounds__(256) k_linear_narrow_dx(const float *__restrict__ g, const float *__restrict__ w,
                                                          float *__restrict__ dx, int rows, int in, int ax) {
    OM_LDS_POISON();
    dx_rows<OUT>(g, w, dx, rows, in, ax, blockIdx.y * kSmallDxRows, blockIdx.x * 256 + threadIdx.x);
}
// part[c][o][i] = sum over the rows of chunk c of g[r][o] x[r][i]: lane l of every wavefront takes column
// 64 blockIdx.x + l, wavefront q the chunk's rows q, q + 4, ... (an fmaf chain per o in increasing row order, x's loads
// sixteen rows ahead); g passes through LDS in blocks of kNarrowSub rows (every lane reads the same g[r][o]: broadcast
// reads). The four wavefronts' sums are then added in wavefront order. The chunk's bias partial dbp[c][o] = double sum
// of its rows in increasing order, read from the same LDS blocks (the workgroups of the first column block).
constexpr int kNarrowSub = 256;
template <int OUT>
__global__ void __launch_bounds__(256) k_linear_narrow_dw(const float *__restrict__ g, const float *__restrict__ x,
                                                          float *__restrict__ part, double *__restrict__ dbp, int rows,
                                                          int in, int chunk) {
    OM_LDS_POISON();
    constexpr int OP = (OUT + 3) / 4 * 4;  // LDS row stride of g: 16-byte rows
    static_assert(kNarrowSub * OP >= 3 * OUT * 64, "the wavefront sums reuse the g block");
    __shared__ __attribute__((aligned(16))) float gs[kNarrowSub * OP];
    const int lane = threadIdx.x & 63, q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = blockIdx.x * 64 + lane, ic = min(i, in - 1);  // columns past the end read column in - 1, unused
    const int r0 = blockIdx.y * chunk, r1 = min(rows, r0 + chunk);
    float acc[OUT];
#pragma unroll
    for (int o = 0; o < OUT; o++) acc[o] = 0.0f;
    double dbacc = 0.0;
    constexpr int G = 16;
    for (int rb = r0; rb < r1; rb += kNarrowSub) {
        const int nb = min(kNarrowSub, r1 - rb);
        // this wavefront's rows of the block: rb + q + 4 j, j < nmine (rows past the end load the block's last row
        // again, unused)
        const int nmine = nb > q ? (nb - q + 3) / 4 : 0;
        auto ld = [&](float(&d)[G], int j0) {
#pragma unroll
            for (int u = 0; u < G; u++) d[u] = x[(int64_t)min(rb + q + 4 * (j0 + u), rb + nb - 1) * in + ic];
        };
        auto use = [&](const float(&d)[G], int j0) {
#pragma unroll
            for (int u = 0; u < G; u++) {
                if (j0 + u >= nmine) break;
                const float *gr = gs + (q + 4 * (j0 + u)) * OP;
#pragma unroll
                for (int o = 0; o < OUT; o++) acc[o] = __builtin_fmaf(gr[o], d[u], acc[o]);
            }
        };
        float xa[G], xb[G];
        if (nmine > 0) ld(xa, 0);
        __syncthreads();  // the previous block's reads are done
        const float *gb = g + (int64_t)rb * OUT;
        for (int e0 = 0; e0 < nb * OUT; e0 += 256 * 8) {  // eight loads per thread in flight together
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int e = e0 + 256 * u + (int)threadIdx.x;
                v[u] = e < nb * OUT ? gb[e] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int e = e0 + 256 * u + (int)threadIdx.x;
                if (e < nb * OUT) {
                    const int rr = e / OUT, o = e - rr * OUT;
                    gs[rr * OP + o] = v[u];
                }
            }
        }
        __syncthreads();
        if (dbp && blockIdx.x == 0 && (int)threadIdx.x < OUT) {
            // the bias partial from the block in LDS, rows in increasing order, sixteen reads ahead of their adds
            const int o = threadIdx.x;
            for (int r = 0; r < nb; r += 16) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = gs[min(r + u, nb - 1) * OP + o];
#pragma unroll
                for (int u = 0; u < 16; u++)
                    if (r + u < nb) dbacc += v[u];
            }
        }
        for (int j = 0; j < nmine; j += 2 * G) {
            if (j + G < nmine) ld(xb, j + G);
            use(xa, j);
            if (j + 2 * G < nmine) ld(xa, j + 2 * G);
            if (j + G < nmine) use(xb, j + G);
        }
    }
    __syncthreads();
    float *sh = gs;  // [3][OUT][64]
    if (q > 0) {
#pragma unroll
        for (int o = 0; o < OUT; o++) sh[((q - 1) * OUT + o) * 64 + lane] = acc[o];
    }
    __syncthreads();
    if (q == 0 && i < in) {
#pragma unroll
        for (int o = 0; o < OUT; o++) {
            float v = acc[o] + sh[o * 64 + lane];
            v = v + sh[(OUT + o) * 64 + lane];
            v = v + sh[(2 * OUT + o) * 64 + lane];
            part[((int64_t)blockIdx.y * OUT + o) * in + i] = v;
        }
    }
    if (dbp && blockIdx.x == 0 && (int)threadIdx.x < OUT) dbp[(int64_t)blockIdx.y * OUT + threadIdx.x] = dbacc;
}
// dw[o][i] (+)= part[0][o][i] + part[1][o][i] + ... (chunk order); db[o] (+)= (float) of dbp[0][o] + dbp[1][o] + ...
__global__ void __launch_bounds__(256) k_linear_narrow_reduce(const float *__restrict__ part,
                                                              const double *__restrict__ dbp, float *__restrict__ dw,
                                                              float *__restrict__ db, int nchunk, int in, int out,
                                                              int aw, int ab) {
    OM_LDS_POISON();
    static_assert(kNarrowMaxChunks == 64, "the partials of one output load in one round");
    const int64_t n = (int64_t)out * in, t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t < n) {
        float pv[kNarrowMaxChunks];  // every partial's load issued before the first add
#pragma unroll
        for (int c = 0; c < kNarrowMaxChunks; c++) pv[c] = part[(int64_t)min(c, nchunk - 1) * n + t];
        float v = pv[0];
#pragma unroll
        for (int c = 1; c < kNarrowMaxChunks; c++)
            if (c < nchunk) v = v + pv[c];
        dw[t] = aw ? dw[t] + v : v;
    }
    if (db && t < out) {
        double s = 0.0;
        for (int c0 = 0; c0 < nchunk; c0 += 16) {
            double pv[16];
#pragma unroll
            for (int u = 0; u < 16; u++) pv[u] = dbp[(int64_t)min(c0 + u, nchunk - 1) * out + t];
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (c0 + u < nchunk) s = c0 + u == 0 ? pv[u] : s + pv[u];
        }
        const float v = (float)s;
        db[t] = ab ? db[t] + v : v;
    }
}
template <int OUT>
void launch_narrow(hipStream_t st, const float *g, const float *x, const float *w, float *dx, float *part, double *dbp,
                   int rows, int in, int ax, int chunk) {
    if (dx)
        hipLaunchKernelGGL(k_linear_narrow_dx<OUT>,
                           dim3((unsigned)((in + 255) / 256), (unsigned)((rows + kSmallDxRows - 1) / kSmallDxRows)),
                           dim3(256), 0, st, g, w, dx, rows, in, ax);
    if (part)
        hipLaunchKernelGGL(k_linear_narrow_dw<OUT>,
                           dim3((unsigned)((in + 63) / 64), (unsigned)((rows + chunk - 1) / chunk)), dim3(256), 0, st,
                           g, x, part, dbp, rows, in, chunk);
}
template <int... OS>
void narrow_dispatch(std::integer_sequence<int, OS...>, hipStream_t st, const float *g, const float *x, const float *w,
                     float *dx, float *part, double *dbp, int rows, int in, int out, int ax, int chunk) {
    ((out == OS + 1 ? (launch_narrow<OS + 1>(st, g, x, w, dx, part, dbp, rows, in, ax, chunk), 0) : 0), ...);
}
// The whole backward of a narrow layer: dx (when asked), and dW with db in two launches (db alone: om_colsum).
om_status narrow_bwd(om_ctx *ctx, const float *g, const float *x, const float *w, float *dx, float *dw, float *db,
                     int rows, int in, int out, int ax, int aw, int ab) {
    const hipStream_t st = om::cur_stream(ctx);
    float *part = nullptr;
    double *dbp = nullptr;
    const int chunk = narrow_chunk(rows, in), nchunk = (rows + chunk - 1) / chunk;
    if (dw) {
        const uint64_t pbytes = ((uint64_t)nchunk * out * in * sizeof(float) + 255) / 256 * 256;
        float *ws;
        om_status s = om::scratch(ctx, pbytes + (uint64_t)nchunk * out * sizeof(double), &ws);
        if (s) return s;
        part = ws;
        if (db) dbp = reinterpret_cast<double *>(reinterpret_cast<char *>(ws) + pbytes);
    }
    if (dx || dw)
        narrow_dispatch(std::make_integer_sequence<int, kNarrowOut>{}, st, g, x, w, dx, part, dbp, rows, in, out, ax,
                        chunk);
    if (dw) {
        const int64_t n = (int64_t)out * in;
        hipLaunchKernelGGL(k_linear_narrow_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, dbp, dw,
                           db, nchunk, in, out, aw, ab);
    }
    om_status s = OM_LAUNCH_CHECK(ctx, "om_linear_bwd (narrow)");
    if (!s && db && !dw) s = om_colsum(ctx, g, db, rows, out, ab);
    return s;
}
}  // namespace

// ------------------------------------------------------------------------------------------------------------------
// Linear layers over a small batch whose product is too large for the VALU paths above but only a few dozen 16 x 16
// MFMA blocks (C1's first layer: 64 rows, 784 -> 256). The engine runs these as a split-K product, its reduce and,
// for dW, two column-sum launches for the bias gradient; here the forward and the weight gradient (with the bias
// gradient) are one launch each, whose time is a short MFMA chain.
namespace {
constexpr int kMidW = 8;  // wavefronts per forward workgroup, each taking every eighth K block of 16
bool linear_mid(int rows, int in, int out) {
    return !linear_small(rows, in, out) && !linear_narrow(rows, in, out) && rows >= 16 && rows <= 256 &&
           rows % 16 == 0 && in % 16 == 0 && out % 16 == 0 && in <= 8192 &&
           (int64_t)(rows / 16) * (out / 16) <= 256;
}
bool al16p(const void *p) { return ((uintptr_t)p & 15) == 0; }

// y[r][o] = (sum over i of x[r][i] w[o][i]) + b[o] (+ resid[r][o]): a workgroup per 16 x 16 block of y. MFMA step s
// of K block kb takes k = 16 kb + 4 kl + s (lane l16 + 16 kl: x row r0 + l16 as A, w row o0 + l16 as B), so a lane
// loads one float4 of each per block, straight from global memory. Wavefront v takes blocks v, v + 8, ..., four
// blocks' loads in flight at a time; wavefront 0 then adds the others' partial sums in wavefront order and applies
// the bias, the residual and the ReLU (the engine's epilogue order).
__global__ void __launch_bounds__(64 * kMidW) k_linear_mid_fwd(const float *__restrict__ x, const float *__restrict__ w,
                                                               const float *__restrict__ b,
                                                               const float *__restrict__ resid, float *__restrict__ y,
                                                               int in, int out, int relu) {
    OM_LDS_POISON();
    __shared__ floatx4 part[kMidW - 1][64];
    const int tb = out / 16, r0 = (blockIdx.x / tb) * 16, o0 = (blockIdx.x % tb) * 16;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, l16 = lane & 15, kl = lane >> 4;
    const float *xa = x + (int64_t)(r0 + l16) * in + 4 * kl, *wb = w + (int64_t)(o0 + l16) * in + 4 * kl;
    const int nkb = in / 16;
    constexpr int R = 4;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int kb0 = wv; kb0 < nkb; kb0 += kMidW * R) {
        floatx4 av[R], bv[R];
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int kb = min(kb0 + kMidW * u, nkb - 1);  // clamped: such a block's loads are not used
            av[u] = *reinterpret_cast<const floatx4 *>(xa + 16 * kb);
            bv[u] = *reinterpret_cast<const floatx4 *>(wb + 16 * kb);
        }
#pragma unroll
        for (int u = 0; u < R; u++)
            if (kb0 + kMidW * u < nkb)  // uniform over the wavefront
#pragma unroll
                for (int s = 0; s < 4; s++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][s], bv[u][s], acc, 0, 0, 0);
    }
    if (wv > 0) part[wv - 1][lane] = acc;
    __syncthreads();
    if (wv > 0) return;
#pragma unroll
    for (int v = 0; v < kMidW - 1; v++) acc += part[v][lane];
    const int col = o0 + l16;
    const float bc = b ? b[col] : 0.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int64_t at = (int64_t)(r0 + 4 * kl + r) * out + col;
        float v = acc[r];
        if (b) v = v + bc;
        if (resid) v = v + resid[at];
        if (relu) v = v > 0.0f ? v : (v == v ? 0.0f : v);
        y[at] = v;
    }
}

// dw[o][i] (+)= sum over r of g[r][o] x[r][i]: a wavefront per 16 x 16 block of dw, K = rows in blocks of 16 (MFMA
// step s of block kb takes r = 16 kb + 4 kl + s: g[r][o0 + l16] as A, x[r][i0 + l16] as B), four blocks' loads in
// flight at a time. The workgroups after the dw blocks' own give each thread a column o of g for db[o] (+)= the sum
// over r of g[r][o] in double, in increasing r. RELU: g[r][o] stands for the ReLU rule's y[r][o] > 0 ? g[r][o] : 0
// (om_relu_bwd's arithmetic, y the ReLU's output [rows, out]) throughout; both loads are issued unconditionally and
// the rule is a select, so no load waits on another.
template <bool RELU>
__global__ void __launch_bounds__(256) k_linear_mid_dw(const float *__restrict__ g, const float *__restrict__ y,
                                                       const float *__restrict__ x, float *__restrict__ dw,
                                                       float *__restrict__ db, int rows, int in, int out, int nblk,
                                                       int acc_dw, int acc_db) {
    OM_LDS_POISON();
    auto gv = [&](int64_t at) {
        const float gg = g[at];
        if constexpr (RELU) {
            const float yy = y[at];
            return yy > 0.0f ? gg : 0.0f;
        }
        return gg;
    };
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, l16 = lane & 15, kl = lane >> 4;
    const int dw_groups = (nblk + 3) / 4;
    if ((int)blockIdx.x >= dw_groups) {
        const int o = ((int)blockIdx.x - dw_groups) * 256 + (int)threadIdx.x;
        if (o >= out) return;
        double s = 0.0;
#pragma unroll 8
        for (int r = 0; r < rows; r++) s += (double)gv((int64_t)r * out + o);
        const float v = (float)s;
        db[o] = acc_db ? db[o] + v : v;
        return;
    }
    const int blk = (int)blockIdx.x * 4 + wv;
    if (blk >= nblk) return;
    const int ti = in / 16, o0 = (blk / ti) * 16, i0 = (blk % ti) * 16;
    const int64_t ga = (int64_t)4 * kl * out + o0 + l16;
    const float *xb = x + (int64_t)4 * kl * in + i0 + l16;
    constexpr int R = 4;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    const int nkb = rows / 16;
    for (int kb0 = 0; kb0 < nkb; kb0 += R) {
        float av[R][4], bv[R][4];
#pragma unroll
        for (int u = 0; u < R; u++) {
            const int kb = min(kb0 + u, nkb - 1);  // clamped: such a block's loads are not used
#pragma unroll
            for (int s = 0; s < 4; s++) {
                av[u][s] = gv(ga + (int64_t)(16 * kb + s) * out);
                bv[u][s] = xb[(int64_t)(16 * kb + s) * in];
            }
        }
#pragma unroll
        for (int u = 0; u < R; u++)
            if (kb0 + u < nkb)
#pragma unroll
                for (int s = 0; s < 4; s++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][s], bv[u][s], acc, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float *p = dw + (int64_t)(o0 + 4 * kl + r) * in + i0 + l16;
        *p = acc_dw ? *p + acc[r] : acc[r];
    }
}

bool launch_mid_fwd(om_ctx *ctx, const float *x, const float *w, const float *b, const float *resid, float *y,
                    int rows, int in, int out, bool relu = false) {
    if (!linear_mid(rows, in, out) || !al16p(x) || !al16p(w)) return false;
    hipLaunchKernelGGL(k_linear_mid_fwd, dim3((unsigned)((rows / 16) * (out / 16))), dim3(64 * kMidW), 0,
                       om::cur_stream(ctx), x, w, b, resid, y, in, out, relu ? 1 : 0);
    return true;
}
}  // namespace

static om_status param_grads(om_ctx *ctx, int n_dw, const om_linear_dw *dw, int rows, int n_cs,
                             const om_column_sum *cs) {
    // The products the grouped launch can take go there together (with the column sums); the others, and all of
    // them when fewer than two fit, run one by one. Outputs do not overlap, so the order between the two sets does
    // not change any result.
    om_status s = OM_OK;
    om_linear_dw fit[omg::kMaxGroup];
    int nfit = 0;
    for (int i = 0; i < n_dw; i++)
        if (omg::dw_groupable(dw[i]) && nfit < omg::kMaxGroup) fit[nfit++] = dw[i];
    const bool grouped = nfit >= 2 && omg::launch_dw_group(ctx, nfit, fit, rows, n_cs, cs, &s);
    if (s) return s;
    int taken = 0;
    for (int i = 0; i < n_dw && !s; i++) {
        const om_linear_dw &d = dw[i];
        if (grouped && taken < nfit && omg::dw_groupable(d)) {
            taken++;
            continue;
        }
        if (d.dw || d.db)
            s = om_linear_bwd(ctx, d.g, d.x, nullptr, nullptr, d.dw, d.db, rows, d.in, d.out, 0, d.acc_dw, d.acc_db);
    }
    if (!s && !grouped && n_cs) {
        omg::GroupParams g{};
        omg::set_column_sums(g, n_cs, cs);
        s = omg::launch_group_reduce(ctx, g, 1, om::cur_stream(ctx));
    }
    return s;
}


extern "C" {

om_status om_gemm(om_ctx *ctx, int trans_a, int trans_b, int m, int n, int k, const float *a, int lda,
                  const float *b, int ldb, float *c, int ldc, const float *bias, int accumulate,
                  const om_batch *batch) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, m >= 0 && n >= 0 && k >= 0, "om_gemm: negative size %d x %d x %d", m, n, k);
    if (m == 0 || n == 0) return OM_OK;
    OM_REQUIRE(ctx, c && (k == 0 || (a && b)), "om_gemm: NULL operand");
    OM_REQUIRE(ctx, lda >= (trans_a ? m : k) && ldb >= (trans_b ? k : n) && ldc >= n,
               "om_gemm: leading dimensions %d/%d/%d too small for %s%s %dx%dx%d", lda, ldb, ldc, trans_a ? "T" : "N",
               trans_b ? "T" : "N", m, n, k);
    omg::Params p = omg::dense_params(m, n, k, a, lda, b, ldb, c, ldc);
    p.bias = bias;
    p.accumulate = accumulate;
    int nb = 1;
    if (batch) {
        OM_REQUIRE(ctx, batch->batch >= 1 && batch->batch_div >= 1, "om_gemm: bad batch %d / %d", batch->batch,
                   batch->batch_div);
        nb = batch->batch;
        p.batch_div = batch->batch_div;
        p.sa_outer = batch->sa_outer;
        p.sa_inner = batch->sa_inner;
        p.sb_outer = batch->sb_outer;
        p.sb_inner = batch->sb_inner;
        p.sc_outer = batch->sc_outer;
        p.sc_inner = batch->sc_inner;
    }
    return omg::launch_dense(ctx, p, trans_a != 0, trans_b != 0, nb, "om_gemm");
}

int om_linear_small(int rows, int in, int out) { return linear_small(rows, in, out) ? 1 : 0; }

om_status om_linear_fwd(om_ctx *ctx, const float *x, const float *w, const float *b, float *y, int rows, int in,
                        int out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && w && y && rows >= 0 && in > 0 && out > 0, "om_linear_fwd: bad arguments");
    if (linear_small(rows, in, out) || linear_narrow(rows, in, out)) {
        launch_small_fwd(om::cur_stream(ctx), x, w, b, nullptr, y, rows, in, out);
        return OM_LAUNCH_CHECK(ctx, "om_linear_fwd");
    }
    if (launch_mid_fwd(ctx, x, w, b, nullptr, y, rows, in, out)) return OM_LAUNCH_CHECK(ctx, "om_linear_fwd");
    omg::Params p = omg::dense_params(rows, out, in, x, in, w, in, y, out);
    p.bias = b;
    return omg::launch_dense(ctx, p, false, true, 1, "om_linear_fwd");
}

om_status om_linear_relu_fwd(om_ctx *ctx, const float *x, const float *w, const float *b, float *y, int rows, int in,
                             int out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && w && y && rows >= 0 && in > 0 && out > 0, "om_linear_relu_fwd: bad arguments");
    if (linear_small(rows, in, out) || linear_narrow(rows, in, out)) {  // the one-launch chains, then the ReLU
        launch_small_fwd(om::cur_stream(ctx), x, w, b, nullptr, y, rows, in, out);
        om_status s = OM_LAUNCH_CHECK(ctx, "om_linear_relu_fwd");
        return s ? s : om_relu_fwd(ctx, y, y, (int64_t)rows * out);
    }
    if (launch_mid_fwd(ctx, x, w, b, nullptr, y, rows, in, out, true)) return OM_LAUNCH_CHECK(ctx, "om_linear_relu_fwd");
    omg::Params p = omg::dense_params(rows, out, in, x, in, w, in, y, out);
    p.bias = b;
    p.epi = omg::EPI_RELU;
    return omg::launch_dense(ctx, p, false, true, 1, "om_linear_relu_fwd");
}

om_status om_linear_bwd(om_ctx *ctx, const float *g, const float *x, const float *w, float *dx, float *dw, float *db,
                        int rows, int in, int out, int acc_dx, int acc_dw, int acc_db) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && rows >= 0 && in > 0 && out > 0, "om_linear_bwd: bad arguments");
    OM_REQUIRE(ctx, (!dx || w) && (!dw || x), "om_linear_bwd: a needed saved tensor is NULL");
    if (linear_small(rows, in, out)) {
        if (!dx && !dw && !db) return OM_OK;
        small_bwd_dispatch(std::make_integer_sequence<int, kSmallOut>{}, out, om::cur_stream(ctx), g, x, w, dx, dw, db,
                           rows, in, acc_dx, acc_dw, acc_db);
        return OM_LAUNCH_CHECK(ctx, "om_linear_bwd");
    }
    if (linear_narrow(rows, in, out)) {
        if (!dx && !dw && !db) return OM_OK;
        return narrow_bwd(ctx, g, x, w, dx, dw, db, rows, in, out, acc_dx, acc_dw, acc_db);
    }
    om_status s = OM_OK;
    if (dx) {
        omg::Params p = omg::dense_params(rows, in, out, g, out, w, in, dx, in);
        p.accumulate = acc_dx;
        s = omg::launch_dense(ctx, p, false, false, 1, "om_linear_bwd dx");
        if (s) return s;
    }
    if (dw && linear_mid(rows, in, out)) {  // dW and db in one launch
        const int nblk = (out / 16) * (in / 16);
        const unsigned grid = (unsigned)((nblk + 3) / 4 + (db ? (out + 255) / 256 : 0));
        hipLaunchKernelGGL(k_linear_mid_dw<false>, dim3(grid), dim3(256), 0, om::cur_stream(ctx), g, nullptr, x, dw, db,
                           rows, in, out, nblk, acc_dw, acc_db);
        return OM_LAUNCH_CHECK(ctx, "om_linear_bwd dw");
    }
    bool db_done = false;
    if (dw) {
        omg::Params p = omg::dense_params(out, in, rows, g, out, x, in, dw, in);
        p.accumulate = acc_dw;
        p.db = db;  // the bias gradient rides along with dW when the kernel can sum g's columns
        p.db_acc = acc_db;
        s = omg::launch_dense(ctx, p, true, false, 1, "om_linear_bwd dw", &db_done);
    }
    if (!s && db && !db_done) s = om_colsum(ctx, g, db, rows, out, acc_db);
    return s;
}

om_status om_linear_relu_bwd(om_ctx *ctx, const float *g, const float *y, const float *x, const float *w, float *dx,
                             float *dw, float *db, int rows, int in, int out, int acc_dx, int acc_dw, int acc_db) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && y && rows >= 0 && in > 0 && out > 0, "om_linear_relu_bwd: bad arguments");
    OM_REQUIRE(ctx, (!dx || w) && (!dw || x), "om_linear_relu_bwd: a needed saved tensor is NULL");
    if (!dx && !dw && !db) return OM_OK;
    if (!dx && dw && linear_mid(rows, in, out)) {  // the ReLU rule inside the dW and db launch
        const int nblk = (out / 16) * (in / 16);
        const unsigned grid = (unsigned)((nblk + 3) / 4 + (db ? (out + 255) / 256 : 0));
        hipLaunchKernelGGL(k_linear_mid_dw<true>, dim3(grid), dim3(256), 0, om::cur_stream(ctx), g, y, x, dw, db, rows,
                           in, out, nblk, acc_dw, acc_db);
        return OM_LAUNCH_CHECK(ctx, "om_linear_relu_bwd");
    }
    // the ReLU rule into the second scratch slot (the products below may use the first), then Linear's backward
    float *gp;
    om_status s = om::scratch2(ctx, sizeof(float) * (uint64_t)rows * out, &gp);
    if (s) return s;
    s = om_relu_bwd(ctx, g, y, gp, (int64_t)rows * out, 0);
    return s ? s : om_linear_bwd(ctx, gp, x, w, dx, dw, db, rows, in, out, acc_dx, acc_dw, acc_db);
}

om_status om_linear_fwd_resid(om_ctx *ctx, const float *x, const float *w, const float *b, const float *resid,
                              float *y, int rows, int in, int out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && w && y && resid && rows >= 0 && in > 0 && out > 0, "om_linear_fwd_resid: bad arguments");
    if (linear_small(rows, in, out) || linear_narrow(rows, in, out)) {  // om_linear_fwd's products for this shape
        launch_small_fwd(om::cur_stream(ctx), x, w, b, resid, y, rows, in, out);
        return OM_LAUNCH_CHECK(ctx, "om_linear_fwd_resid");
    }
    if (launch_mid_fwd(ctx, x, w, b, resid, y, rows, in, out)) return OM_LAUNCH_CHECK(ctx, "om_linear_fwd_resid");
    omg::Params p = omg::dense_params(rows, out, in, x, in, w, in, y, out);
    p.bias = b;
    p.resid = resid;
    p.ldr = out;
    return omg::launch_dense(ctx, p, false, true, 1, "om_linear_fwd_resid");
}

om_status om_linear_fwd_resid_mse(om_ctx *ctx, const float *x, const float *w, const float *b, const float *resid,
                                  const float *target, float *y, float *dpred_unit, float *loss, int rows, int in,
                                  int out, om_readback *rb) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && w && y && resid && target && dpred_unit && loss && rows > 0 && in > 0 && out > 0,
               "om_linear_fwd_resid_mse: bad arguments");
    const int64_t n = (int64_t)rows * out;
    if (linear_small(rows, in, out) || linear_narrow(rows, in, out)) {  // om_linear_fwd_resid's products
        launch_small_fwd(om::cur_stream(ctx), x, w, b, resid, y, rows, in, out);
        om_status s = OM_LAUNCH_CHECK(ctx, "om_linear_fwd_resid_mse");
        return s ? s : om::mse_of(ctx, y, target, dpred_unit, loss, n, rb);
    }
    if (launch_mid_fwd(ctx, x, w, b, resid, y, rows, in, out)) {
        om_status s = OM_LAUNCH_CHECK(ctx, "om_linear_fwd_resid_mse");
        return s ? s : om::mse_of(ctx, y, target, dpred_unit, loss, n, rb);
    }
    // one partial per wavefront of every tile; no tile is smaller than 64 x 64
    float *scr;
    om_status s = om::scratch2(ctx, sizeof(double) * 4 * (uint64_t)((rows + 63) / 64) * ((out + 63) / 64), &scr);
    if (s) return s;
    omg::Params p = omg::dense_params(rows, out, in, x, in, w, in, y, out);
    p.bias = b;
    p.resid = resid;
    p.ldr = out;
    p.mse_t = target;
    p.mse_unit = dpred_unit;
    p.mse_part = reinterpret_cast<double *>(scr);
    p.mse_dsq = 1.0f / (float)n;
    int slots = 0;
    s = omg::launch_dense(ctx, p, false, true, 1, "om_linear_fwd_resid_mse", nullptr, &slots);
    if (s) return s;
    if (slots > 0) return om::mse_final(ctx, reinterpret_cast<const double *>(scr), slots, loss, n, rb);
    return om::mse_of(ctx, y, target, dpred_unit, loss, n, rb);  // the kernel it took has no such epilogue
}

om_status om_linear_gelu_fwd(om_ctx *ctx, const float *x, const float *w, const float *b, float *h, float *a, int rows,
                             int in, int out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && w && h && a && rows >= 0 && in > 0 && out > 0, "om_linear_gelu_fwd: bad arguments");
    omg::Params p = omg::dense_params(rows, out, in, x, in, w, in, h, out);
    p.bias = b;
    p.epi = ctx->gelu_mode == OM_GELU_REFERENCE ? omg::EPI_GELU : omg::EPI_GELU_F;
    p.out2 = a;
    p.ld2 = out;
    return omg::launch_dense(ctx, p, false, true, 1, "om_linear_gelu_fwd");
}

om_status om_linear_gelu_fwd_slope(om_ctx *ctx, const float *x, const float *w, const float *b, float *a, float *s,
                                   int rows, int in, int out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, x && w && a && s && a != s && rows >= 0 && in > 0 && out > 0,
               "om_linear_gelu_fwd_slope: bad arguments");
    omg::Params p = omg::dense_params(rows, out, in, x, in, w, in, a, out);
    p.bias = b;
    p.epi = ctx->gelu_mode == OM_GELU_REFERENCE ? omg::EPI_GELU_SLOPE : omg::EPI_GELU_SLOPE_F;
    p.out2 = s;
    p.ld2 = out;
    return omg::launch_dense(ctx, p, false, true, 1, "om_linear_gelu_fwd_slope");
}

om_status om_param_grads_group(om_ctx *ctx, int n_dw, const om_linear_dw *dw, int rows, int n_cs,
                               const om_column_sum *cs) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, n_dw >= 0 && (n_dw == 0 || dw) && rows >= 0 && n_cs >= 0 && n_cs <= omg::kMaxColSums &&
                        (n_cs == 0 || cs),
               "om_param_grads_group: bad arguments (at most %d column sums)", omg::kMaxColSums);
    for (int i = 0; i < n_dw; i++)
        OM_REQUIRE(ctx, dw[i].g && dw[i].x && dw[i].in > 0 && dw[i].out > 0,
                   "om_param_grads_group: weight item %d has a NULL input or a non-positive size", i);
    for (int j = 0; j < n_cs; j++)
        OM_REQUIRE(ctx, cs[j].part && cs[j].out && cs[j].chunks > 0 && cs[j].cols > 0,
                   "om_param_grads_group: column-sum item %d has a NULL pointer or a non-positive size", j);
    const int probe = om::probe_begin(ctx);
    const om_status s = param_grads(ctx, n_dw, dw, rows, n_cs, cs);
    om::probe_end(ctx, probe);
    return s;
}

om_status om_linear_bwd_dw_group(om_ctx *ctx, int count, const om_linear_dw *items, int rows) {
    return om_param_grads_group(ctx, count, items, rows, 0, nullptr);
}

om_status om_linear_bwd_dx_resid(om_ctx *ctx, const float *g, const float *w, const float *r, float *dx, int rows,
                                 int in, int out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && w && r && dx && rows >= 0 && in > 0 && out > 0, "om_linear_bwd_dx_resid: bad arguments");
    if (linear_small(rows, in, out) || linear_narrow(rows, in, out)) {  // their own dx kernels, then the add
        om_status s = om_linear_bwd(ctx, g, nullptr, w, dx, nullptr, nullptr, rows, in, out, 0, 0, 0);
        return s ? s : om_axpy(ctx, 1.0f, r, dx, (int64_t)rows * in);
    }
    omg::Params p = omg::dense_params(rows, in, out, g, out, w, in, dx, in);
    p.resid = r;  // the engine's epilogue: fl(fl(g w) + r), the bits of the product stored and then added
    p.ldr = in;
    return omg::launch_dense(ctx, p, false, false, 1, "om_linear_bwd_dx_resid");
}

om_status om_linear_bwd_dx_slope(om_ctx *ctx, const float *g, const float *w, const float *s, float *dh, int rows,
                                 int in, int out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && w && s && dh && rows >= 0 && in > 0 && out > 0, "om_linear_bwd_dx_slope: bad arguments");
    omg::Params p = omg::dense_params(rows, in, out, g, out, w, in, dh, in);
    p.epi = omg::EPI_MUL_AUX;
    p.aux = s;
    p.ldaux = in;
    return omg::launch_dense(ctx, p, false, false, 1, "om_linear_bwd_dx_slope");
}

om_status om_linear_bwd_dx_gelu(om_ctx *ctx, const float *g, const float *w, const float *h, float *dh, int rows,
                                int in, int out) {
    OM_CHECK_CTX(ctx);
    OM_REQUIRE(ctx, g && w && h && dh && rows >= 0 && in > 0 && out > 0, "om_linear_bwd_dx_gelu: bad arguments");
    omg::Params p = omg::dense_params(rows, in, out, g, out, w, in, dh, in);
    p.epi = ctx->gelu_mode == OM_GELU_REFERENCE ? omg::EPI_GELU_GRAD : omg::EPI_GELU_GRAD_F;
    p.aux = h;
    p.ldaux = in;
    return omg::launch_dense(ctx, p, false, false, 1, "om_linear_bwd_dx_gelu");
}

}  // extern "C"
