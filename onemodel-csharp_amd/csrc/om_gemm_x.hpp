// Tile-exact fp32 MFMA GEMM for gfx950: the kernel the training path's dense products run on.
//
// Preconditions, checked on the host: every tile is full (m % BM == 0, n % BN == 0), every split's K range is a
// multiple of BKT, operands are 16-byte aligned with leading dimensions (and batch strides) multiples of 4. With
// those, the main loop carries no bounds logic at all: each thread issues a fixed list of float4 global loads and
// LDS stores per chunk.
//
// Pipeline (one workgroup of 4 wavefronts, 2 x 2, each a (BM/2) x (BN/2) sub-tile):
//   - global loads run two chunks ahead, into two register sets used alternately (the loop is unrolled by two so
//     the sets are static); the loads of chunk t+2 are in flight while chunk t is multiplied and chunk t+1 is being
//     written to LDS, which gives each load about two chunks of MFMA time to land;
//   - LDS is double-buffered, one barrier per chunk;
//   - inside a chunk, the fragments of 16-k block b+1 are read from LDS while the MFMAs of block b issue.
// Operand layouts in LDS: K layout [rows][BKT] with XOR-swizzled float4 chunks (kaddr), R layout [BKT][rows+4]. For an
// R-layout operand the wavefront's 16-row (or 16-column) MFMA blocks are interleaved: block i of a wavefront's TX
// blocks covers rows {TX*c + i}, so the TX fragments a lane needs for one k sit side by side and arrive in one wide
// LDS read (b64 / b96 / b128) instead of TX separate ones; the epilogue maps rows and columns back accordingly, and
// for an interleaved B a lane's TX output columns are adjacent, so C is written with wide stores.
#pragma once

#include "om_gemm_core.hpp"

namespace omg {
namespace gx {

// K layout in LDS: row r keeps its BKT values with stride BKT (no pad), its float4 chunks permuted by an XOR with
// kswz(r). A 16-lane phase of the b128 stores (two rows of 8 chunks at BKT 32, one row of 16 chunks at BKT 64) and
// of the fragment reads (16 rows, one chunk each) then covers 16 distinct 4-bank groups of the 64 LDS banks; the
// padded layout [rows][BKT + 4] let the two rows of a store phase overlap on four banks.
template <int BKT>
__device__ __forceinline__ int kswz(int r) {
    static_assert(BKT == 32 || BKT == 64, "K-layout swizzle is defined for 32- and 64-wide chunks");
    return BKT == 32 ? ((r >> 1) & 7) : (r & 15);
}
template <int BKT>
__device__ __forceinline__ int kaddr(int r, int chunk) {
    return r * BKT + 4 * (chunk ^ kswz<BKT>(r));
}

// Exact loader of one operand chunk: ROWS x BKT values (KCONTIG: rows contiguous along k; else along the rows),
// spread over NTH threads (a chunk that does not split evenly leaves whole wavefronts idle on the last load).
template <int ROWS, int BKT, bool KCONTIG, int NTH = NT>
struct Ld {
    static constexpr int TOT = ROWS * BKT / 4;
    static_assert(TOT % 64 == 0, "a chunk must split into whole wavefronts");
    static constexpr int NV = (TOT + NTH - 1) / NTH;
    static constexpr bool RAGGED = TOT % NTH != 0;
    static constexpr int LDSZ = KCONTIG ? ROWS * BKT : BKT * (ROWS + PAD);
    const float *base;  // operand origin of this tile (row r0, k 0)
    int64_t ld;
    int goff[NV];  // per-load element offset from (r0, k0)
    int soff[NV];  // per-load LDS offset

    __device__ __forceinline__ Ld(const float *b, int64_t ld_, int r0) : ld(ld_) {
#pragma unroll
        for (int i = 0; i < NV; i++) {
            int f = threadIdx.x + i * NTH;
            if (RAGGED && f >= TOT) f = TOT - 1;  // unused: the load and store below are skipped for it
            if constexpr (KCONTIG) {
                int r = f / (BKT / 4), kq = (f % (BKT / 4)) * 4;
                goff[i] = (int)(r * ld) + kq;
                soff[i] = kaddr<BKT>(r, kq >> 2);
            } else {
                int kk = f / (ROWS / 4), rq = (f % (ROWS / 4)) * 4;
                goff[i] = (int)(kk * ld) + rq;
                soff[i] = kk * (ROWS + PAD) + rq;
            }
        }
        base = b + (KCONTIG ? (int64_t)r0 * ld : (int64_t)r0);
    }
    __device__ __forceinline__ void fetch(floatx4 (&v)[NV], int k0) const {
        const float *p = base + (KCONTIG ? (int64_t)k0 : (int64_t)k0 * ld);
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (!RAGGED || i + 1 < NV || (int)threadIdx.x + i * NTH < TOT)
                v[i] = *reinterpret_cast<const floatx4 *>(p + goff[i]);
    }
    __device__ __forceinline__ void put(const floatx4 (&v)[NV], float *T) const {
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (!RAGGED || i + 1 < NV || (int)threadIdx.x + i * NTH < TOT)
                *reinterpret_cast<floatx4 *>(T + soff[i]) = v[i];
    }
};

// Fragments of one 16-k block for TX MFMA blocks of one operand: f[s][x] is the value lane (l%16, kl = l/16) feeds
// to the MFMA of block x at step s (k = 16*blk + 4*kl + s).
template <int ROWS, int BKT, int TX, bool KL>
__device__ __forceinline__ void read_frag(float (&f)[4][TX], const float *T, int blk, int w0, int l16, int kl) {
    if constexpr (KL) {
#pragma unroll
        for (int x = 0; x < TX; x++) {
            floatx4 v = *reinterpret_cast<const floatx4 *>(&T[kaddr<BKT>(w0 + x * 16 + l16, blk * 4 + kl)]);
#pragma unroll
            for (int s = 0; s < 4; s++) f[s][x] = v[s];
        }
    } else {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const float *p = &T[(blk * 16 + kl * 4 + s) * (ROWS + PAD) + w0 + TX * l16];
            if constexpr (TX % 4 == 0) {
#pragma unroll
                for (int x = 0; x < TX; x += 4) {
                    floatx4 v = *reinterpret_cast<const floatx4 *>(p + x);
                    f[s][x] = v[0];
                    f[s][x + 1] = v[1];
                    f[s][x + 2] = v[2];
                    f[s][x + 3] = v[3];
                }
            } else if constexpr (TX % 2 == 0) {
#pragma unroll
                for (int x = 0; x < TX; x += 2) {
                    float2 v = *reinterpret_cast<const float2 *>(p + x);
                    f[s][x] = v.x;
                    f[s][x + 1] = v.y;
                }
            } else {
#pragma unroll
                for (int x = 0; x < TX; x++) f[s][x] = p[x];
            }
        }
    }
}

// Fused bias gradient of a weight-gradient product: column sums of A (transposed, staged [BKT][BM+4] in LDS) over
// the k rows of each chunk, in double. Thread x of NTH sums column x % BM over rows x / BM, x / BM + NTH / BM, ...;
// colsum_finish combines the NTH / BM row groups in order and writes the tile's BM sums.
template <int BM, int BKT, int NTH>
struct ColSum {
    static constexpr int RG = NTH / BM;
    static_assert(NTH % BM == 0 && BKT % RG == 0, "column sums need whole row groups");
    double s = 0.0;
    __device__ __forceinline__ void add(const float *Ab) {
        const int c = threadIdx.x % BM, rg = threadIdx.x / BM;
#pragma unroll
        for (int kk = rg; kk < BKT; kk += RG) s += (double)Ab[kk * (BM + PAD) + c];
    }
    // Uses `sh` (RG * BM doubles of LDS, free when called) and ends with a barrier.
    __device__ __forceinline__ void finish(const Params &p, double *sh, int m0, int split) {
        sh[threadIdx.x] = s;
        __syncthreads();
        if ((int)threadIdx.x < BM) {
            double t = sh[threadIdx.x];
#pragma unroll
            for (int g = 1; g < RG; g++) t += sh[g * BM + threadIdx.x];
            const int row = m0 + threadIdx.x;
            if (p.splits > 1) {
                p.colsum_ws[(int64_t)split * p.m + row] = t;
            } else {
                float v = (float)t;
                p.db[row] = p.db_acc ? p.db[row] + v : v;
            }
        }
        __syncthreads();
    }
};

// Epilogue of a wavefront's TM x TN MFMA blocks: output register r of block (i, j) on this lane is row rho = 4*kl + r
// and column l16 of the block, mapped back through the interleaving of R-layout operands. Every operand the epilogue
// reads (bias, residual, GELU input, mask, the old C) is gathered into registers first, in runs of independent loads,
// and the arithmetic follows in the reference's order: alpha, mask, bias, residual, GELU, then accumulate.
template <int TM, int TN, bool AK, bool BKL, int GK>
__device__ __forceinline__ void tile_epilogue(const Params &p, const floatx4 (&acc)[TM][TN], float *C,
                                              const float *mask, int m0, int n0, int wm0, int wn0, int l16, int kl,
                                              int split) {
    int colv[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) colv[j] = n0 + wn0 + (BKL ? j * 16 + l16 : TN * l16 + j);
    float bcol[TN];
    if (p.splits == 1 && p.bias && !p.bias_per_row) {
#pragma unroll
        for (int j = 0; j < TN; j++) bcol[j] = p.bias[colv[j]];
    }
    double mse_acc = 0.0;
    // One MFMA row block (i) at a time keeps the gathered operands to 4 x TN registers each.
#pragma unroll
    for (int i = 0; i < TM; i++) {
        int rowv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) rowv[r] = m0 + wm0 + (AK ? i * 16 + 4 * kl + r : TM * (4 * kl + r) + i);
        if (p.splits > 1) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < TN; j++) p.ws[((int64_t)split * p.m + rowv[r]) * p.n + colv[j]] = acc[i][j][r];
            continue;
        }
        float v[4][TN], t[4][TN];
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int j = 0; j < TN; j++) v[r][j] = acc[i][j][r];
        auto gather = [&](const float *base, int64_t ld) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < TN; j++) t[r][j] = base[(int64_t)rowv[r] * ld + colv[j]];
        };
        if (p.alpha != 1.0f) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < TN; j++) v[r][j] = v[r][j] * p.alpha;
        }
        if (mask) {
            gather(mask, p.n);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < TN; j++) v[r][j] = v[r][j] + t[r][j];
        }
        if (p.bias) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float br = p.bias_per_row ? p.bias[rowv[r]] : 0.0f;
#pragma unroll
                for (int j = 0; j < TN; j++) v[r][j] = v[r][j] + (p.bias_per_row ? br : bcol[j]);
            }
        }
        if (p.resid) {
            gather(p.resid, p.ldr);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < TN; j++) v[r][j] = v[r][j] + t[r][j];
        }
        if (p.epi == EPI_RELU) {
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < TN; j++) v[r][j] = v[r][j] > 0.0f ? v[r][j] : (v[r][j] == v[r][j] ? 0.0f : v[r][j]);
        }
        if constexpr (GK == 1) {  // the reference's polynomials
            if (p.epi == EPI_GELU) {
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int j = 0; j < TN; j++) p.out2[(int64_t)rowv[r] * p.ld2 + colv[j]] = omd::gelu(v[r][j]);
            } else if (p.epi == EPI_GELU_GRAD) {
                gather(p.aux, p.ldaux);
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int j = 0; j < TN; j++) v[r][j] = omd::gelu_grad(v[r][j], t[r][j]);
            } else if (p.epi == EPI_GELU_SLOPE) {
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int j = 0; j < TN; j++) {
                        float a, s;
                        omd::gelu_and_slope(v[r][j], a, s);
                        p.out2[(int64_t)rowv[r] * p.ld2 + colv[j]] = s;
                        v[r][j] = a;
                    }
            }
        } else if constexpr (GK == 2) {  // erf and exp of stated error (omd::gelu_and_slope_fast)
            if (p.epi == EPI_GELU_F) {
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int j = 0; j < TN; j++) p.out2[(int64_t)rowv[r] * p.ld2 + colv[j]] = omd::gelu_fast(v[r][j]);
            } else if (p.epi == EPI_GELU_GRAD_F) {
                gather(p.aux, p.ldaux);
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int j = 0; j < TN; j++) v[r][j] = omd::gelu_grad_fast(v[r][j], t[r][j]);
            } else if (p.epi == EPI_GELU_SLOPE_F) {
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int j = 0; j < TN; j++) {
                        float a, s;
                        omd::gelu_and_slope_fast(v[r][j], a, s);
                        p.out2[(int64_t)rowv[r] * p.ld2 + colv[j]] = s;
                        v[r][j] = a;
                    }
            }
        }
        if constexpr (GK != 0) {
            if (p.epi == EPI_MUL_AUX) {
                gather(p.aux, p.ldaux);
#pragma unroll
                for (int r = 0; r < 4; r++)
#pragma unroll
                    for (int j = 0; j < TN; j++) v[r][j] = omd::canon(v[r][j] * t[r][j]);
            }
        }
        if (p.accumulate) {
            gather(C, p.ldc);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < TN; j++) v[r][j] = t[r][j] + v[r][j];
        }
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int j = 0; j < TN; j++) C[(int64_t)rowv[r] * p.ldc + colv[j]] = v[r][j];
        if (p.mse_t) {  // d = stored value - target; the unit gradient 2 (d / n) as (d dsq) + (d dsq); sum of fl(d d)
            gather(p.mse_t, p.ldc);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const float d = v[r][j] - t[r][j];
                    const float u = p.mse_dsq * d;
                    p.mse_unit[(int64_t)rowv[r] * p.ldc + colv[j]] = u + u;
                    mse_acc += (double)(d * d);
                }
        }
    }
    if (p.mse_t) {  // uniform over the launch; every lane of the wavefront is here
        mse_acc = omd::wave_sum(mse_acc);
        if ((threadIdx.x & 63) == 0) p.mse_part[4 * blockIdx.x + (threadIdx.x >> 6)] = mse_acc;
    }
}

// One tile (tm, tn) of batch-and-split index zz, by one workgroup of NT threads: the body of k_gemm_x and of the
// grouped weight-gradient kernel.
template <int BM, int BN, int BKT, bool TA, bool TB, int GK>
__device__ __forceinline__ void gemm_x_tile(const Params &p, int tm, int tn, int zz) {
    constexpr bool AK = !TA, BKL = TB;  // operands in K layout
    constexpr int TM = BM / 32, TN = BN / 32, NB = BKT / 16;
    using LA = Ld<BM, BKT, AK>;
    using LB = Ld<BN, BKT, BKL>;
    __shared__ __attribute__((aligned(16))) float As[2 * LA::LDSZ];
    __shared__ __attribute__((aligned(16))) float Bs[2 * LB::LDSZ];

    if (zz >= p.batch * p.splits) return;
    const int z = zz / p.splits, split = zz % p.splits;
    const int outer = z / p.batch_div, inner = z % p.batch_div;
    const float *A = p.a + outer * p.sa_outer + inner * p.sa_inner;
    const float *B = p.b + outer * p.sb_outer + inner * p.sb_inner;
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = split * p.k_split;
    const int nk = (min(p.k, kbeg + p.k_split) - kbeg) / BKT;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, l16 = lane & 15, kl = lane >> 4;
    const int wm0 = (wv >> 1) * (BM / 2), wn0 = (wv & 1) * (BN / 2);

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const LA la(A, p.lda, m0);
    const LB lb(B, p.ldb, n0);
    // Fragment sets for even and odd 16-k blocks.
    float fa0[4][TM], fb0[4][TN], fa1[4][TM], fb1[4][TN];
    auto rd = [&](float(&fa)[4][TM], float(&fb)[4][TN], const float *Ab, const float *Bb, int blk) {
        read_frag<BM, BKT, TM, AK>(fa, Ab, blk, wm0, l16, kl);
        read_frag<BN, BKT, TN, BKL>(fb, Bb, blk, wn0, l16, kl);
    };
    auto mm = [&](const float(&fa)[4][TM], const float(&fb)[4][TN]) {
#pragma unroll
        for (int s = 0; s < 4; s++)
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[s][i], fb[s][j], acc[i][j], 0, 0, 0);
    };
    // Bias gradient: the first column of tiles of a TN product sums its A chunks (A is [k][m] in LDS).
    constexpr bool CS_OK = TA && (NT % BM == 0) && (BKT % (NT / BM) == 0);
    ColSum<CS_OK ? BM : 64, BKT, NT> cs;
    const bool do_cs = CS_OK && p.db && tn == 0;
    // Blocks 0 .. NB-2 of the chunk in (Ab, Bb): the fragments of block b+1 are read while block b multiplies.
    auto body = [&](const float *Ab, const float *Bb) {
        if constexpr (CS_OK)
            if (do_cs) cs.add(Ab);
#pragma unroll
        for (int blk = 0; blk + 1 < NB; blk++) {
            if (blk & 1) rd(fa0, fb0, Ab, Bb, blk + 1);
            else rd(fa1, fb1, Ab, Bb, blk + 1);
            __builtin_amdgcn_sched_barrier(0);
            if (blk & 1) mm(fa1, fb1);
            else mm(fa0, fb0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    static_assert(NB % 2 == 0, "chunks hold an even number of 16-k blocks");

    if (nk > 0) {
        floatx4 ra0[LA::NV], rb0[LB::NV], ra1[LA::NV], rb1[LB::NV];
        const int klast = kbeg + (nk - 1) * BKT;
        float *A0 = As, *A1 = As + LA::LDSZ, *B0 = Bs, *B1 = Bs + LB::LDSZ;
        la.fetch(ra0, kbeg);
        lb.fetch(rb0, kbeg);
        la.fetch(ra1, min(kbeg + BKT, klast));
        lb.fetch(rb1, min(kbeg + BKT, klast));
        la.put(ra0, A0);
        lb.put(rb0, B0);
        __syncthreads();
        rd(fa0, fb0, A0, B0, 0);
        // One chunk that has a successor: issue the loads of chunk t+2 into the free register set, multiply blocks
        // 0 .. NB-2, write chunk t+1 (landed meanwhile) into the other LDS buffer, barrier, read block 0 of chunk
        // t+1 while the last block of chunk t multiplies. Chunk t sits in buffer t & 1, register set t & 1 is free.
#define OMG_X_HALF(RA, RB, RAN, RBN, AC, BC, AN, BN_, KF)   \
    la.fetch(RA, min(KF, klast));                          \
    lb.fetch(RB, min(KF, klast));                          \
    __builtin_amdgcn_sched_barrier(0);                     \
    body(AC, BC);                                          \
    la.put(RAN, AN);                                       \
    lb.put(RBN, BN_);                                      \
    __syncthreads();                                       \
    rd(fa0, fb0, AN, BN_, 0);                              \
    __builtin_amdgcn_sched_barrier(0);                     \
    mm(fa1, fb1);                                          \
    __builtin_amdgcn_sched_barrier(0);
        int t = 0;
        // Both halves of the loop body always run (loads past the last chunk are clamped to it), so the body has
        // no branch: a branchy body lets the compiler merge the halves and index the register sets dynamically.
        for (; t + 2 < nk; t += 2) {
            OMG_X_HALF(ra0, rb0, ra1, rb1, A0, B0, A1, B1, kbeg + (t + 2) * BKT)
            OMG_X_HALF(ra1, rb1, ra0, rb0, A1, B1, A0, B0, kbeg + (t + 3) * BKT)
        }
        const float *Al = A0, *Bl = B0;
        if (nk - t == 2) {
            OMG_X_HALF(ra0, rb0, ra1, rb1, A0, B0, A1, B1, klast)
            Al = A1;
            Bl = B1;
        }
#undef OMG_X_HALF
        // The last chunk (block 0's fragments are in set 0).
        body(Al, Bl);
        mm(fa1, fb1);
    }
    if constexpr (CS_OK)
        if (p.db && tn == 0) {  // uniform over the workgroup
            __syncthreads();
            cs.finish(p, reinterpret_cast<double *>(As), m0, split);
        }

    float *C = p.c + outer * p.sc_outer + inner * p.sc_inner;
    const float *mask = p.mask ? p.mask + outer * p.mask_outer_stride : nullptr;
    tile_epilogue<TM, TN, AK, BKL, GK>(p, acc, C, mask, m0, n0, wm0, wn0, l16, kl, split);
}

template <int BM, int BN, int BKT, bool TA, bool TB, int GK = 0>
__global__ void __launch_bounds__(NT) k_gemm_x(Params p) {
    OM_LDS_POISON();
    int tm, tn, zz;
    tile_coords(p, p.n / BN, p.m / BM, tm, tn, zz);
    gemm_x_tile<BM, BN, BKT, TA, TB, GK>(p, tm, tn, zz);
}

// ------------------------------------------------------------------------------------------------------------------
// Tile-exact product with both operands K-contiguous (A [m][k], B [n][k]: every Linear forward) whose chunks travel
// from global memory straight into LDS: `global_load_lds_dwordx4` writes each lane's 16 bytes at M0 + 16 * lane, so a
// wavefront instruction fills 64 consecutive float4 slots of the swizzled K layout, and each lane loads the global
// float4 that belongs in its slot. Three LDS stages form a ring: chunk t sits in stage t % 3, and the loads of chunk
// t + 2 are issued right after the barrier that opens chunk t, so every chunk has two chunks of MFMA time to land,
// with no staging registers and no LDS writes of our own. The loads are inline assembly with explicit waits: the
// compiler tracks such loads only as a whole and would otherwise wait for all of them (vmcnt(0)) before the first
// LDS read of every chunk. Before the barrier opening chunk t each wavefront waits until only chunk t+1's loads may
// still be in flight (vmcnt counts in issue order) and until its own LDS reads are done (lgkmcnt(0)); the barrier
// then also tells every wavefront that all others have finished reading the stage the new loads will overwrite
// (chunk t-1's). No load is in flight at the end.
// Arithmetic, order and epilogue are k_gemm_x's, so the results are bit for bit those of k_gemm_x at the same tile.
// One operand's part of a chunk: wavefront w issues instructions q = 4 j + w, each filling slots [64 q, 64 q + 64)
// of the stage. `src` is this lane's row pointer for j = 0 (row r0 = (64 w + lane) / CH); each further j moves 4 * 64
// slots = 256 / CH rows down. `lds` is the stage's LDS byte address plus this wavefront's first instruction, a
// wavefront-uniform value.
template <int ROWS, int BKT>
__device__ __forceinline__ void dma_chunk(const float *src, int64_t ld, unsigned lds) {
    constexpr int INSTR = ROWS * (BKT / 4) / 64;  // wavefront instructions per stage and operand
    static_assert(INSTR % 4 == 0, "each of the four wavefronts issues whole instructions");
    constexpr int CH = BKT / 4;  // float4 chunks per row
    // m0 is a reserved register: the compiler warns that it does not keep a value of its own in m0 across this
    // statement. That is safe here because nothing else in these kernels reads m0 (no LDS-direct or
    // relative-indexing instructions in their assembly), so each load's m0 is the one set just before it.
#pragma unroll
    for (int j = 0; j < INSTR / 4; j++) {
        const float *g = src + (int64_t)j * (256 / CH) * ld;
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds + j * 4096u)
                     : "memory", "m0");
    }
}

template <int BM, int BN, int BKT, int GK>
__device__ __forceinline__ void gemm_xd_tile(const Params &p, int tm, int tn, int zz) {
    constexpr int TM = BM / 32, TN = BN / 32, NB = BKT / 16;
    constexpr int SA = BM * BKT, SB = BN * BKT, STAGE = SA + SB;
    constexpr int PER = (BM + BN) * (BKT / 4) / 64 / 4;  // loads per wavefront and chunk
    static_assert(PER <= 63, "vmcnt holds at most 63");
    // 64 floats of pad ahead of the stages: no stage starts at LDS address 0
    __shared__ __attribute__((aligned(16))) float S[64 + 3 * STAGE];

    if (zz >= p.batch * p.splits) return;
    const int z = zz / p.splits, split = zz % p.splits;
    const int outer = z / p.batch_div, inner = z % p.batch_div;
    const int m0 = tm * BM, n0 = tn * BN;
    const float *A = p.a + outer * p.sa_outer + inner * p.sa_inner + (int64_t)m0 * p.lda;
    const float *B = p.b + outer * p.sb_outer + inner * p.sb_inner + (int64_t)n0 * p.ldb;
    const int kbeg = split * p.k_split;
    const int nk = (min(p.k, kbeg + p.k_split) - kbeg) / BKT;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, l16 = lane & 15, kl = lane >> 4;
    const int wm0 = (wv >> 1) * (BM / 2), wn0 = (wv & 1) * (BN / 2);

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // This lane's source rows for the first instruction (slot 64 w + lane of the stage), with the swizzle that puts
    // the float4 chunk of column group c into slot column c ^ kswz(r); rows 256 / CH apart share the swizzle.
    constexpr int CH = BKT / 4;
    static_assert((256 / CH) % 16 == 0, "the swizzle repeats every 16 rows");
    const int slot0 = wv * 64 + lane, r0 = slot0 / CH, c0 = (slot0 % CH) ^ kswz<BKT>(r0);
    const float *srcA = A + (int64_t)r0 * p.lda + kbeg + 4 * c0;
    const float *srcB = B + (int64_t)r0 * p.ldb + kbeg + 4 * c0;
    const unsigned wave = __builtin_amdgcn_readfirstlane(wv);
    const unsigned lds0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) void *)(S + 64) + wave * 1024u;
    auto issue = [&](int t, int st) {
        const unsigned base = lds0 + (unsigned)(st * STAGE) * 4u;
        dma_chunk<BM, BKT>(srcA + t * BKT, p.lda, base);
        dma_chunk<BN, BKT>(srcB + t * BKT, p.ldb, base + SA * 4u);
    };
    auto compute = [&](int st) {
        const float *Ab = S + 64 + st * STAGE, *Bb = Ab + SA;
#pragma unroll
        for (int blk = 0; blk < NB; blk++) {
            floatx4 fa[TM], fb[TN];
#pragma unroll
            for (int x = 0; x < TM; x++)
                fa[x] = *reinterpret_cast<const floatx4 *>(&Ab[kaddr<BKT>(wm0 + x * 16 + l16, blk * 4 + kl)]);
#pragma unroll
            for (int x = 0; x < TN; x++)
                fb[x] = *reinterpret_cast<const floatx4 *>(&Bb[kaddr<BKT>(wn0 + x * 16 + l16, blk * 4 + kl)]);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][s], fb[j][s], acc[i][j], 0, 0, 0);
        }
    };
    // lgkmcnt(0) too: this wavefront's LDS reads of the previous chunk must be complete before the barrier, since
    // after it other wavefronts load into that stage (the compiler may leave reads in flight past the barrier asm).
    auto step = [&](int t, int st) {
        if (t + 1 < nk) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(PER) : "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        asm volatile("s_barrier" ::: "memory");
        if (t + 2 < nk) issue(t + 2, st == 0 ? 2 : st - 1);
        compute(st);
    };
    if (nk > 0) issue(0, 0);
    if (nk > 1) issue(1, 1);
    int t = 0;
    for (; t + 3 <= nk; t += 3) {  // unrolled by three so every stage index is a constant
        step(t, 0);
        step(t + 1, 1);
        step(t + 2, 2);
    }
    if (t < nk) step(t, 0);
    if (t + 1 < nk) step(t + 1, 1);

    float *C = p.c + outer * p.sc_outer + inner * p.sc_inner;
    const float *mask = p.mask ? p.mask + outer * p.mask_outer_stride : nullptr;
    tile_epilogue<TM, TN, true, true, GK>(p, acc, C, mask, m0, n0, wm0, wn0, l16, kl, split);
}

template <int BM, int BN, int BKT, int GK = 0>
__global__ void __launch_bounds__(NT) k_gemm_xd(Params p) {
    OM_LDS_POISON();
    int tm, tn, zz;
    tile_coords(p, p.n / BN, p.m / BM, tm, tn, zz);
    gemm_xd_tile<BM, BN, BKT, GK>(p, tm, tn, zz);
}

// Weight gradients of several products in one launch (om_linear_bwd_dw_group): product i owns the workgroups
// [start[i], start[i+1]) of the XCD-remapped grid, each a (tile, split) of its own Params, run by the same tile body.
template <int BM, int BN, int BKT>
__global__ void __launch_bounds__(NT) k_gemm_x_tn_group(GroupParams g) {
    OM_LDS_POISON();
    int lin = blockIdx.x;
    const int total = gridDim.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    int i = 0;
#pragma unroll
    for (int j = 1; j < kMaxGroup; j++)
        if (j < g.count && lin >= g.start[j]) i = j;
    const Params &p = g.p[i];
    const int local = lin - g.start[i], tiles_n = p.n / BN, tiles_m = p.m / BM;
    if (g.band > 0) {
        // Within a split: bands of `band` tile rows (the last band may be shorter), each walked one tile column at a
        // time with the band's rows fastest, so the workgroups that run together on one XCD share few operand slabs.
        const int per = tiles_m * tiles_n, split = local / per, idx = local % per;
        const int bh = g.band < tiles_m ? g.band : tiles_m;
        const int band = idx / (bh * tiles_n), r0 = band * bh, rows = min(bh, tiles_m - r0);
        const int within = idx - r0 * tiles_n;
        gemm_x_tile<BM, BN, BKT, true, false, false>(p, r0 + within % rows, within / rows, split);
        return;
    }
    const int rest = local / tiles_n;
    gemm_x_tile<BM, BN, BKT, true, false, false>(p, rest % tiles_m, local % tiles_n, rest / tiles_m);
}

// The same tile with eight wavefronts: two groups of four (2 x 2 over the tile, as above) split each chunk's 16-k
// blocks between them (group g takes blocks g, g+2, ...), so every SIMD runs two wavefronts of the tile and one's LDS
// and barrier waits hide behind the other's MFMAs. At the end group 1 hands its partial sums to group 0 through LDS
// and group 0 adds them (in that fixed order) and runs the epilogue. For products with about one tile per CU.
template <int BM, int BN, int BKT, bool TA, bool TB, int GK = 0>
__global__ void __launch_bounds__(2 * NT) k_gemm_x2(Params p) {
    OM_LDS_POISON();
    constexpr int NTH = 2 * NT;
    constexpr bool AK = !TA, BKL = TB;
    constexpr int TM = BM / 32, TN = BN / 32, NB = BKT / 16;
    static_assert(NB % 2 == 0, "each group needs whole 16-k blocks");
    using LA = Ld<BM, BKT, AK, NTH>;
    using LB = Ld<BN, BKT, BKL, NTH>;
    __shared__ __attribute__((aligned(16))) float Sh[2 * LA::LDSZ + 2 * LB::LDSZ];
    static_assert(2 * (LA::LDSZ + LB::LDSZ) >= BM * BN, "the partial-sum exchange reuses the operand buffers");
    float *As = Sh, *Bs = Sh + 2 * LA::LDSZ;

    const int tiles_n = p.n / BN, tiles_m = p.m / BM;
    int tm, tn, zz;
    tile_coords(p, tiles_n, tiles_m, tm, tn, zz);
    if (zz >= p.batch * p.splits) return;
    const int z = zz / p.splits, split = zz % p.splits;
    const int outer = z / p.batch_div, inner = z % p.batch_div;
    const float *A = p.a + outer * p.sa_outer + inner * p.sa_inner;
    const float *B = p.b + outer * p.sb_outer + inner * p.sb_inner;
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = split * p.k_split;
    const int nk = (min(p.k, kbeg + p.k_split) - kbeg) / BKT;
    const int lane = threadIdx.x & 63, wv = (threadIdx.x >> 6) & 3, kg = threadIdx.x >> 8;
    const int l16 = lane & 15, kl = lane >> 4;
    const int wm0 = (wv >> 1) * (BM / 2), wn0 = (wv & 1) * (BN / 2);

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    const LA la(A, p.lda, m0);
    const LB lb(B, p.ldb, n0);
    constexpr bool CS_OK = TA && (NTH % BM == 0) && (BKT % (NTH / BM) == 0);
    ColSum<CS_OK ? BM : 64, BKT, NTH> cs;
    const bool do_cs = CS_OK && p.db && tn == 0;
    auto chunk = [&](const float *Ab, const float *Bb) {
        if constexpr (CS_OK)
            if (do_cs) cs.add(Ab);
#pragma unroll
        for (int blk = 0; blk < NB; blk += 2) {
            float fa[4][TM], fb[4][TN];
            read_frag<BM, BKT, TM, AK>(fa, Ab, blk + kg, wm0, l16, kl);
            read_frag<BN, BKT, TN, BKL>(fb, Bb, blk + kg, wn0, l16, kl);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[s][i], fb[s][j], acc[i][j], 0, 0, 0);
        }
    };
    if (nk > 0) {
        floatx4 ra0[LA::NV], rb0[LB::NV], ra1[LA::NV], rb1[LB::NV];
        const int klast = kbeg + (nk - 1) * BKT;
        float *A0 = As, *A1 = As + LA::LDSZ, *B0 = Bs, *B1 = Bs + LB::LDSZ;
        la.fetch(ra0, kbeg);
        lb.fetch(rb0, kbeg);
        la.fetch(ra1, min(kbeg + BKT, klast));
        lb.fetch(rb1, min(kbeg + BKT, klast));
        la.put(ra0, A0);
        lb.put(rb0, B0);
        __syncthreads();
        int t = 0;
        for (; t + 2 < nk; t += 2) {  // both halves always run (clamped loads), see k_gemm_x
            la.fetch(ra0, min(kbeg + (t + 2) * BKT, klast));
            lb.fetch(rb0, min(kbeg + (t + 2) * BKT, klast));
            __builtin_amdgcn_sched_barrier(0);
            chunk(A0, B0);
            la.put(ra1, A1);
            lb.put(rb1, B1);
            __syncthreads();
            la.fetch(ra1, min(kbeg + (t + 3) * BKT, klast));
            lb.fetch(rb1, min(kbeg + (t + 3) * BKT, klast));
            __builtin_amdgcn_sched_barrier(0);
            chunk(A1, B1);
            la.put(ra0, A0);
            lb.put(rb0, B0);
            __syncthreads();
        }
        const float *Al = A0, *Bl = B0;
        if (nk - t == 2) {
            chunk(A0, B0);
            la.put(ra1, A1);
            lb.put(rb1, B1);
            __syncthreads();
            Al = A1;
            Bl = B1;
        }
        chunk(Al, Bl);
    }
    if constexpr (CS_OK)
        if (p.db && tn == 0) {
            __syncthreads();
            cs.finish(p, reinterpret_cast<double *>(Sh), m0, split);
        }
    // Group 1's partial sums -> LDS (the operand buffers, after everyone is done with them) -> group 0.
    __syncthreads();
    float *X = Sh;  // [4 waves][TM*TN*4][64 lanes]
    constexpr int PER = TM * TN * 4;
    if (kg == 1) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) X[(wv * PER + (i * TN + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (kg == 1) return;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = acc[i][j][r] + X[(wv * PER + (i * TN + j) * 4 + r) * 64 + lane];

    float *C = p.c + outer * p.sc_outer + inner * p.sc_inner;
    const float *mask = p.mask ? p.mask + outer * p.mask_outer_stride : nullptr;
    tile_epilogue<TM, TN, AK, BKL, GK>(p, acc, C, mask, m0, n0, wm0, wn0, l16, kl, split);
}

}  // namespace gx
}  // namespace omg
