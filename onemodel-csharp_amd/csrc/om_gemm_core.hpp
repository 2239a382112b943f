// fp32 MFMA GEMM engine for gfx950, shared by the dense products (om_gemm.hip), attention (om_attention.hip) and
// the implicit-GEMM convolutions (om_conv.hip).
//
// Structure: a workgroup of 256 threads (4 wavefronts, 2 x 2) computes a BM x BN tile of C; each wavefront owns a
// (BM/2) x (BN/2) sub-tile made of 16 x 16 blocks accumulated by v_mfma_f32_16x16x4_f32 (A fragment: lane l holds
// A[l%16][k(l/16)]; B fragment: lane l holds B[k(l/16)][l%16]; result: lane l holds C[4*(l/16)+r][l%16]).
//
// K advances in chunks of BKT staged through LDS, double-buffered: while the MFMAs consume chunk t from one LDS
// buffer, the global loads of chunk t+1 are in flight in registers and land in the other buffer.
//
// Each operand keeps the LDS layout its global layout gives for free:
//   - "K layout" [ROWS][BKT+4] for operands whose rows are contiguous along k (A not transposed, B transposed): the
//     global float4 along k is stored as it is, and a lane reads the four k of its fragment for four MFMA steps with
//     one ds_read_b128. The +4 pad spreads the 8 lanes of a b128 phase over all 32 banks.
//   - "R layout" [BKT][ROWS+4] for operands contiguous along their rows (A transposed, B not transposed, and the
//     gathered convolution operands): float4 stores along the row, one ds_read_b32 per fragment and step.
// The MFMA k order inside each block of 16 is permuted so that both layouts agree: lane group kl (= l/16) at step s
// (0..3) holds k = 16*blk + 4*kl + s. The product sums the same terms; only the order of the fp32 additions differs.
#pragma once

#include "om_internal.hpp"

namespace omg {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BK = 16;  // chunk depth of the convolution kernels
constexpr int NT = 256;
constexpr int PAD = 4;  // row pad (floats) of both LDS layouts

// Everything a kernel instance needs; plain data so it can be passed by value.
struct Params {
    int m, n, k;
    int batch;  // independent products (grid covers batch * splits * tiles)
    // batch item z: outer = z / batch_div, inner = z % batch_div
    int batch_div;
    // dense operands
    const float *a;
    int64_t lda, sa_outer, sa_inner;
    const float *b;
    int64_t ldb, sb_outer, sb_inner;
    float *c;
    int64_t ldc, sc_outer, sc_inner;
    // epilogue: v = acc * alpha (+ mask) (+ bias) ; C = accumulate ? C + v : v
    float alpha;
    const float *bias;
    int bias_per_row;
    const float *mask;  // additive [Lq, Lk] per batch outer index (attention scores)
    int64_t mask_outer_stride;
    int accumulate;
    // split-K: grid covers batch * splits; split s covers k in [s*k_split, (s+1)*k_split) and writes its partial
    // sum to ws + s*m*n (row-major m x n) instead of C; a reduce pass then applies the epilogue.
    int splits;
    int k_split;
    float *ws;
    // convolution geometry (gather loaders)
    int cin, h, w, cout, kh, kw, stride, pad, oh, ow;
    int xcd_remap;
    // fused epilogue terms, applied after alpha, mask and bias (dense products only):
    //   resid: v += resid[row * ldr + col] (a residual Add after the Linear);
    //   epi EPI_GELU: C gets v (the pre-activation, which GELU's backward reads) and out2 gets gelu(v);
    //   epi EPI_GELU_GRAD: C gets gelu_grad(v, aux[row * ldaux + col]) (GELU's backward of the product).
    //   epi EPI_GELU_SLOPE: C gets gelu(v) and out2 gets GELU's slope at v (all GELU's backward needs);
    //   epi EPI_MUL_AUX: C gets v * aux[row * ldaux + col] (GELU's backward of the product, given that slope);
    //   epi EPI_RELU: C gets ReluUn(v) (v > 0 ? v : 0, NaN kept), om_relu_fwd's arithmetic (a convolution stage).
    const float *resid;
    int64_t ldr;
    int epi;
    float *out2;
    int64_t ld2;
    const float *aux;
    int64_t ldaux;
    // fused bias gradient of a weight-gradient product (A transposed, stored [k][m]): db[m] (+)= sum over k of A in
    // double. The tile-exact kernels' first column of tiles sums its A chunks from LDS; with split K the per-split
    // sums go to colsum_ws[split * m + row] and the split-K reduce finishes them.
    double *colsum_ws;
    float *db;
    int db_acc;
    // The MSE loss of the stored values against mse_t (laid out as C), after every other epilogue step (tile-exact
    // kernels, one split): mse_unit gets the gradient for a unit upstream gradient (k_mse_partial's arithmetic with
    // mse_dsq = 1 / numel) and mse_part[4 * blockIdx.x + wavefront] the wavefront's fp64 sum of the squared
    // differences (its elements in epilogue order, then a butterfly).
    const float *mse_t;
    float *mse_unit;
    double *mse_part;
    float mse_dsq;
};

enum {
    EPI_NONE = 0, EPI_GELU = 1, EPI_GELU_GRAD = 2, EPI_GELU_SLOPE = 3, EPI_MUL_AUX = 4, EPI_RELU = 5,
    // EPI_GELU, EPI_GELU_GRAD and EPI_GELU_SLOPE with erf and exp of stated error (omd::gelu_and_slope_fast)
    EPI_GELU_F = 6, EPI_GELU_GRAD_F = 7, EPI_GELU_SLOPE_F = 8
};

// Several products launched together (the grouped weight-gradient kernel and its reduce): product i owns workgroups
// [start[i], start[i+1]) of the GEMM launch, float4 quads [qstart[i], qstart[i+1]) and bias rows
// [rstart[i], rstart[i+1]) of the reduce.
// The reduce also finishes up to kMaxColSums two-stage column sums (LayerNorm's dgamma/dbeta partials): item j owns
// the wavefronts [cstart[j], cstart[j+1]) of the reduce grid, one per column.
constexpr int kMaxGroup = 4;
constexpr int kMaxColSums = 8;
struct ColSumItem {
    const double *part;
    float *out;
    int chunks, cols, acc;
};
struct GroupParams {
    Params p[kMaxGroup];
    int start[kMaxGroup + 1];
    int64_t qstart[kMaxGroup + 1];
    int rstart[kMaxGroup + 1];
    int count;
    ColSumItem cs[kMaxColSums];
    int cstart[kMaxColSums + 1];
    int ncs;
    int band;  // tile order inside a (product, split): bands of `band` tile rows walked column by column; 0: row-major
};

// The epilogue of one finished dot product v at (row, col): alpha, mask, bias, residual, GELU terms, then C. The
// GELU polynomials are compiled only into the instantiations that can be asked for them (GELU = true): inlined
// into every large-tile kernel they would raise register pressure enough to spill.
template <bool GELU = true>
__device__ __forceinline__ void epilogue(const Params &p, float *cbase, int64_t ldc, const float *mask, int row, int col,
                                         float v) {
    if (p.alpha != 1.0f) v = v * p.alpha;
    if (mask) v = v + mask[(int64_t)row * p.n + col];
    if (p.bias) v = v + p.bias[p.bias_per_row ? row : col];
    if (p.resid) v = v + p.resid[(int64_t)row * p.ldr + col];
    if (p.epi == EPI_RELU) v = v > 0.0f ? v : (v == v ? 0.0f : v);
    if constexpr (GELU) {
        if (p.epi == EPI_GELU) {
            p.out2[(int64_t)row * p.ld2 + col] = omd::gelu(v);
        } else if (p.epi == EPI_GELU_GRAD) {
            v = omd::gelu_grad(v, p.aux[(int64_t)row * p.ldaux + col]);
        } else if (p.epi == EPI_GELU_SLOPE) {
            float a, s;
            omd::gelu_and_slope(v, a, s);
            p.out2[(int64_t)row * p.ld2 + col] = s;
            v = a;
        } else if (p.epi == EPI_MUL_AUX) {
            v = omd::canon(v * p.aux[(int64_t)row * p.ldaux + col]);
        } else if (p.epi == EPI_GELU_F) {
            p.out2[(int64_t)row * p.ld2 + col] = omd::gelu_fast(v);
        } else if (p.epi == EPI_GELU_GRAD_F) {
            v = omd::gelu_grad_fast(v, p.aux[(int64_t)row * p.ldaux + col]);
        } else if (p.epi == EPI_GELU_SLOPE_F) {
            float a, s;
            omd::gelu_and_slope_fast(v, a, s);
            p.out2[(int64_t)row * p.ld2 + col] = s;
            v = a;
        }
    }
    float *dst = cbase + (int64_t)row * ldc + col;
    *dst = p.accumulate ? *dst + v : v;
}

// ------------------------------------------------------------------------------------------------ loaders
// A loader fills one LDS buffer for k in [k0, k0 + BKT) and rows in [r0, r0 + ROWS) of its logical operand (A: rows
// are m; B: rows are n). `fetch` issues the global loads into registers, `put` writes them to LDS. Out-of-range
// elements are zero. KLAYOUT says which of the two LDS layouts `put` writes.

// Dense operand whose rows are contiguous along k ("A not transposed" [m][k], or "B transposed" [n][k]).
template <int ROWS, int BKT, bool VEC>
struct LoadKContig {
    static constexpr bool KLAYOUT = true;
    static constexpr int TOT = ROWS * BKT / 4;       // float4 per chunk
    static constexpr int NV = (TOT + NT - 1) / NT;   // float4 per thread
    float4 v[NV];
    __device__ __forceinline__ void fetch(const float *base, int64_t ld, int rows, int kend, int r0, int k0) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            int f = threadIdx.x + i * NT;
            if (TOT % NT != 0 && f >= TOT) break;
            int r = f / (BKT / 4), kq = (f % (BKT / 4)) * 4;
            int gr = r0 + r, gk = k0 + kq;
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
            if (gr < rows) {
                const float *p = base + (int64_t)gr * ld + gk;
                if (VEC && gk + 3 < kend) {
                    t = *reinterpret_cast<const float4 *>(p);
                } else {
                    if (gk + 0 < kend) t.x = p[0];
                    if (gk + 1 < kend) t.y = p[1];
                    if (gk + 2 < kend) t.z = p[2];
                    if (gk + 3 < kend) t.w = p[3];
                }
            }
            v[i] = t;
        }
    }
    __device__ __forceinline__ void put(float *T) const {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            int f = threadIdx.x + i * NT;
            if (TOT % NT != 0 && f >= TOT) break;
            int r = f / (BKT / 4), kq = (f % (BKT / 4)) * 4;
            *reinterpret_cast<float4 *>(&T[r * (BKT + PAD) + kq]) = v[i];
        }
    }
};

// Dense operand contiguous along its rows ("A transposed" stored [k][m], or "B not transposed" stored [k][n]).
template <int ROWS, int BKT, bool VEC>
struct LoadRContig {
    static constexpr bool KLAYOUT = false;
    static constexpr int TOT = ROWS * BKT / 4;
    static constexpr int NV = (TOT + NT - 1) / NT;
    float4 v[NV];
    __device__ __forceinline__ void fetch(const float *base, int64_t ld, int rows, int kend, int r0, int k0) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            int f = threadIdx.x + i * NT;
            if (TOT % NT != 0 && f >= TOT) break;
            int kk = f / (ROWS / 4), rq = (f % (ROWS / 4)) * 4;
            int gk = k0 + kk, gr = r0 + rq;
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
            if (gk < kend) {
                const float *p = base + (int64_t)gk * ld + gr;
                if (VEC && gr + 3 < rows) {
                    t = *reinterpret_cast<const float4 *>(p);
                } else {
                    if (gr + 0 < rows) t.x = p[0];
                    if (gr + 1 < rows) t.y = p[1];
                    if (gr + 2 < rows) t.z = p[2];
                    if (gr + 3 < rows) t.w = p[3];
                }
            }
            v[i] = t;
        }
    }
    __device__ __forceinline__ void put(float *T) const {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            int f = threadIdx.x + i * NT;
            if (TOT % NT != 0 && f >= TOT) break;
            int kk = f / (ROWS / 4), rq = (f % (ROWS / 4)) * 4;
            *reinterpret_cast<float4 *>(&T[kk * (ROWS + PAD) + rq]) = v[i];
        }
    }
};

// LDS floats of one buffer of an operand tile.
template <int ROWS, int BKT, bool KLAYOUT>
constexpr int lds_size() {
    return KLAYOUT ? ROWS * (BKT + PAD) : BKT * (ROWS + PAD);
}

// ------------------------------------------------------------------------------------------------ engine
template <int BM, int BN, int BKT, bool AK, bool BKL>
struct Tile {
    static_assert(BKT % 16 == 0, "chunk depth must be a multiple of 16");
    static constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 16, TN = WN / 16;
    floatx4 acc[TM][TN];

    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    // Four MFMA k-values of one operand fragment for the 16-k block `blk`: k = 16*blk + 4*kl + s, s = 0..3.
    template <int ROWS, bool KL>
    __device__ __forceinline__ static floatx4 frag(const float *T, int blk, int row, int kl) {
        if constexpr (KL) {
            return *reinterpret_cast<const floatx4 *>(&T[row * (BKT + PAD) + blk * 16 + kl * 4]);
        } else {
            const float *p = &T[(blk * 16 + kl * 4) * (ROWS + PAD) + row];
            return floatx4{p[0], p[ROWS + PAD], p[2 * (ROWS + PAD)], p[3 * (ROWS + PAD)]};
        }
    }
    // One chunk from LDS.
    __device__ __forceinline__ void mma(const float *As, const float *Bs, int wm0, int wn0, int lane) {
        const int ml = lane & 15, kl = lane >> 4;
#pragma unroll
        for (int blk = 0; blk < BKT / 16; blk++) {
            floatx4 a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) a[i] = frag<BM, AK>(As, blk, wm0 + i * 16 + ml, kl);
#pragma unroll
            for (int j = 0; j < TN; j++) b[j] = frag<BN, BKL>(Bs, blk, wn0 + j * 16 + ml, kl);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
        }
    }
};

// Maps the linear workgroup id so that consecutive tiles of the (z, m, n) walk land on one XCD: the hardware deals
// workgroups round-robin over the 8 XCDs, each with its own L2, and neighbouring tiles share operand panels.
__device__ __forceinline__ void tile_coords(const Params &p, int tiles_n, int tiles_m, int &tm, int &tn, int &z) {
    int total = gridDim.x;
    int lin = blockIdx.x;
    if (p.xcd_remap && (total & 7) == 0) {
        int per = total >> 3;
        lin = (lin & 7) * per + (lin >> 3);
    }
    tn = lin % tiles_n;
    int rest = lin / tiles_n;
    tm = rest % tiles_m;
    z = rest / tiles_m;
}

// Epilogue for one accumulator tile: writes C (or the split-K partial).
template <class TL, bool GELU = false>
__device__ __forceinline__ void store_tile(const Params &p, TL &t, int m0, int n0, int wm0, int wn0, int lane,
                                           float *cbase, int64_t ldc, const float *mask, int split) {
    const int col_l = lane & 15, row_l = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < TL::TM; i++)
#pragma unroll
        for (int j = 0; j < TL::TN; j++) {
            int col = n0 + wn0 + j * 16 + col_l;
            if (col >= p.n) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int row = m0 + wm0 + i * 16 + row_l + r;
                if (row >= p.m) continue;
                float v = t.acc[i][j][r];
                if (p.splits > 1) {
                    p.ws[((int64_t)split * p.m + row) * p.n + col] = v;
                    continue;
                }
                epilogue<GELU>(p, cbase, ldc, mask, row, col, v);
            }
        }
}

// The main loop, generic over the two loaders. `fa(la, k0)` / `fb(lb, k0)` issue the global loads of a chunk.
template <int BM, int BN, int BKT, class LA, class LB, class FA, class FB>
__device__ __forceinline__ void run_k(Tile<BM, BN, BKT, LA::KLAYOUT, LB::KLAYOUT> &t, LA &la, LB &lb, FA fa, FB fb,
                                      int kbeg, int kend, float *As0, float *Bs0, int wm0, int wn0, int lane) {
    constexpr int ASZ = lds_size<BM, BKT, LA::KLAYOUT>(), BSZ = lds_size<BN, BKT, LB::KLAYOUT>();
    t.zero();
    if (kbeg >= kend) return;
    int nk = (kend - kbeg + BKT - 1) / BKT;
    fa(la, kbeg);
    fb(lb, kbeg);
    la.put(As0);
    lb.put(Bs0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        int cur = kt & 1;
        bool more = kt + 1 < nk;
        if (more) {
            fa(la, kbeg + (kt + 1) * BKT);
            fb(lb, kbeg + (kt + 1) * BKT);
        }
        t.mma(As0 + cur * ASZ, Bs0 + cur * BSZ, wm0, wn0, lane);
        if (more) {
            la.put(As0 + (cur ^ 1) * ASZ);
            lb.put(Bs0 + (cur ^ 1) * BSZ);
        }
        __syncthreads();
    }
}

}  // namespace omg
