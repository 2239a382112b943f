// Fused scaled dot-product attention for short sequences (Ops.Attention, Ops.Layers.cs:746-807; AttentionBackward,
// BackwardNn.cs:636-701; definition docs/kernels-attention.md:10-33).
//
// The unfused path (om_attention.hip) runs five GEMM launches and two row passes over a [B, H, L, L] score tensor
// in HBM. For L <= 128 a workgroup holds whole score rows on chip, so forward and backward are one kernel each and
// the scores never reach HBM:
//   forward  (one workgroup per batch item, head and 64 queries; a wavefront per 16 queries):
//            S = scale * Q K^T + mask on MFMA, P = Softmax.Rows(S) in registers, O = P V on MFMA;
//   backward (one workgroup per batch item and head; a wavefront per 16 queries), recomputing P as the reference
//            does: S, P, dP = dO V^T, dS = P (dP - rowsum(dP P)) scale with the row sum in double, then
//            dV = P^T dO, dK = dS^T Q, dQ = dS K, with P^T and dS^T staged through LDS.
// The softmax is the reference's exact row kernel: in the 16x16 MFMA result layout, lane t of a 16-lane group holds
// the row's columns t, t+16, ..., which are exactly the elements of Sum16's partial t, so the partials are summed in
// increasing column order per lane and combined with the halving shuffles, as in Softmax.Rows (Softmax.cs:27-133).
// Q, K, V (and O, dO, dQ, dK, dV) are [B, L, H*D] row blocks of stride ld (packed q|k|v projections welcome).
#include "om_gemm.hpp"

om_status om_internal_softmax_rows(om_ctx *ctx, float *x, int rows, int cols);
extern "C" om_status om_attention_bwd_ld(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                         const float *p, const float *g, int ld_g, float *dq, float *dk, float *dv,
                                         int ld_d, float *ds, int B, int H, int lq, int lk, int d, float scale,
                                         int acc);
extern "C" om_status om_attention_fwd_ld(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                         const float *mask, int mask_batched, float *o, int ld_o, float *p, int B,
                                         int H, int lq, int lk, int d, float scale);

namespace {

using omg::floatx4;

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Staging of ROWS rows of D floats (global stride ld) into LDS rows of stride D + 4, in two steps: load() issues all
// of this thread's global loads into registers, store() writes them to LDS. Callers issue the loads of every operand
// before the first store, so the loads' latencies overlap instead of following one another.
template <int D, int NTH, int ROWS>
struct Stage {
    static constexpr int Q4 = D / 4, TOT = ROWS * Q4, PER = (TOT + NTH - 1) / NTH;
    floatx4 v[PER];
    __device__ __forceinline__ void load(const float *src, int64_t ld) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int f = (int)threadIdx.x + i * NTH;
            if (TOT % NTH == 0 || f < TOT)
                v[i] = *reinterpret_cast<const floatx4 *>(src + (int64_t)(f / Q4) * ld + (f % Q4) * 4);
        }
    }
    __device__ __forceinline__ void store(float *dst) const {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int f = (int)threadIdx.x + i * NTH;
            if (TOT % NTH == 0 || f < TOT) *reinterpret_cast<floatx4 *>(&dst[(f / Q4) * (D + 4) + (f % Q4) * 4]) = v[i];
        }
    }
};

// S = scale * X Y^T (+ mask) for the 16 rows x0.. of X against all L rows of Y (both staged [rows][D+4]):
// s[j] holds columns 16j.. in the MFMA result layout (lane t, group kl, register r = row 4kl+r, column 16j+t).
template <int D, int L>
__device__ __forceinline__ void scores(floatx4 (&s)[L / 16], const float *Xs, const float *Ys, int x0, int t, int kl) {
    constexpr int LDX = D + 4;
#pragma unroll
    for (int j = 0; j < L / 16; j++) s[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int blk = 0; blk < D / 16; blk++) {
        floatx4 a = *reinterpret_cast<const floatx4 *>(&Xs[(x0 + t) * LDX + 16 * blk + 4 * kl]);
#pragma unroll
        for (int j = 0; j < L / 16; j++) {
            floatx4 b = *reinterpret_cast<const floatx4 *>(&Ys[(16 * j + t) * LDX + 16 * blk + 4 * kl]);
#pragma unroll
            for (int u = 0; u < 4; u++) s[j] = mfma4(a[u], b[u], s[j]);
        }
    }
}

// This lane's mask values for its four rows (row stride L), loaded early so their latency hides behind the staging.
template <int L>
__device__ __forceinline__ void load_mask(float (&mv)[4][L / 16], const float *mrow, int t) {
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int j = 0; j < L / 16; j++) mv[r][j] = mrow ? mrow[r * L + 16 * j + t] : 0.0f;
}

// Scale, additive mask and the exact row softmax, in place: s becomes P.
template <int L>
__device__ __forceinline__ void softmax_rows(floatx4 (&s)[L / 16], const float (&mv)[4][L / 16], bool masked,
                                             float scale) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float mx = -__int_as_float(0x7F800000);
#pragma unroll
        for (int j = 0; j < L / 16; j++) {
            float x = s[j][r] * scale;
            if (masked) x = x + mv[r][j];
            s[j][r] = x;
            mx = x > mx ? x : mx;
        }
        mx = omd::max16(mx);
        float p = 0.0f;
#pragma unroll
        for (int j = 0; j < L / 16; j++) {
            float e = omd::exp_nonpos(s[j][r] - mx);
            s[j][r] = e;
            p += e;
        }
        const float l = omd::sum16(p);
#pragma unroll
        for (int j = 0; j < L / 16; j++) s[j][r] = omd::canon(s[j][r] / l);
    }
}

// acc[jn] += A (16 rows, K = L) x B[L][D] where A comes from LDS in K layout (row stride LDA, rows a0 + t, k from 0)
// and B is staged [L][D+4]; B's D/16 column blocks are interleaved (block jn holds columns DB*c + jn), so one lane
// reads its DB values of a row at once.
template <int D, int L, int LDA>
__device__ __forceinline__ void mm_kA(floatx4 (&acc)[D / 16], const float *As, int a0, const float *Bs, int t,
                                      int kl) {
    constexpr int DB = D / 16, LDB = D + 4;
#pragma unroll
    for (int blk = 0; blk < L / 16; blk++) {
        floatx4 a = *reinterpret_cast<const floatx4 *>(&As[(a0 + t) * LDA + 16 * blk + 4 * kl]);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float *brow = &Bs[(16 * blk + 4 * kl + u) * LDB + DB * t];
            float bv[DB];
            if constexpr (DB % 4 == 0) {
#pragma unroll
                for (int x = 0; x < DB; x += 4) {
                    floatx4 w = *reinterpret_cast<const floatx4 *>(brow + x);
                    bv[x] = w[0];
                    bv[x + 1] = w[1];
                    bv[x + 2] = w[2];
                    bv[x + 3] = w[3];
                }
            } else {
#pragma unroll
                for (int x = 0; x < DB; x += 2) {
                    float2 w = *reinterpret_cast<const float2 *>(brow + x);
                    bv[x] = w.x;
                    bv[x + 1] = w.y;
                }
            }
#pragma unroll
            for (int jn = 0; jn < DB; jn++) acc[jn] = mfma4(a[u], bv[jn], acc[jn]);
        }
    }
}

// Writes a 16-row result block (rows row0 + 4kl + r) with interleaved columns DB*t + jn, optionally accumulating.
template <int D>
__device__ __forceinline__ void store_rows(float *dst, int64_t ld, int row0, const floatx4 (&acc)[D / 16], int t,
                                           int kl, int accumulate) {
    constexpr int DB = D / 16;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float *p = dst + (int64_t)(row0 + 4 * kl + r) * ld + DB * t;
#pragma unroll
        for (int jn = 0; jn < DB; jn++) p[jn] = accumulate ? p[jn] + acc[jn][r] : acc[jn][r];
    }
}

// Forward in the transposed form: S^T = K Q^T, so the MFMA result puts keys on (lane group kl, register r) and a
// wavefront's 16 queries on the lane index t. Then
//   - the row softmax of query t runs over this lane's 4 x L/16 values and the four lane groups; Sum16's partial
//     p[key % 16] is this lane's register-r sum over the key blocks (key % 16 = 4 kl + r), so the halving combine
//     p[i] + p[i+8], +4, +2, +1 is two cross-group shuffles (lanes +32, +16) and two in-register adds;
//   - P^T in registers is exactly the B operand of O^T = V^T P^T (no LDS round trip), with V^T staged in LDS;
//   - the mask of query t over keys 4 kl + r is four consecutive floats (one 16-byte load per key block).
// One workgroup per batch item, head and 64 queries (four wavefronts of 16 queries).
template <int D, int L>
__global__ void __launch_bounds__(256) k_attn_fwd(const float *__restrict__ q, const float *__restrict__ k,
                                                  const float *__restrict__ v, int ld, const float *__restrict__ mask,
                                                  int64_t mask_bstride, float *__restrict__ o, int ldo, float scale) {
    OM_LDS_POISON();
    constexpr int LDK = D + 4, LDV = L + 4, NB = L / 16, DB = D / 16;
    __shared__ __attribute__((aligned(16))) float Ks[L * LDK];  // [key][d]
    __shared__ __attribute__((aligned(16))) float Vt[D * LDV];  // [d][key]
    const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int64_t row0 = (int64_t)b * L;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = lane & 15, kl = lane >> 4;
    const int qrow = qb * 64 + 16 * w + t;  // this lane's query
    // Early loads: this lane's query fragment (B operand of S^T) and mask values.
    floatx4 qf[DB];
    const float *qg = q + (row0 + qrow) * ld + h * D;
#pragma unroll
    for (int blk = 0; blk < DB; blk++) qf[blk] = *reinterpret_cast<const floatx4 *>(qg + 16 * blk + 4 * kl);
    floatx4 mv[NB];
    if (mask) {
        const float *mr = mask + b * mask_bstride + (int64_t)qrow * L + 4 * kl;
#pragma unroll
        for (int j = 0; j < NB; j++) mv[j] = *reinterpret_cast<const floatx4 *>(mr + 16 * j);
    }
    // K rows and V^T, all loads first. V^T: thread f takes key f % L and four d from f / L, so each store row is
    // contiguous across the lanes.
    Stage<D, 256, L> ks;
    ks.load(k + row0 * ld + h * D, ld);
    constexpr int VPER = L * (D / 4) / 256;
    static_assert(L * (D / 4) % 256 == 0, "V^T staging covers whole rounds of the workgroup");
    floatx4 vx[VPER];
    const float *vg = v + row0 * ld + h * D;
#pragma unroll
    for (int i = 0; i < VPER; i++) {
        const int f = (int)threadIdx.x + i * 256, key = f % L, c = (f / L) * 4;
        vx[i] = *reinterpret_cast<const floatx4 *>(vg + (int64_t)key * ld + c);
    }
    ks.store(Ks);
#pragma unroll
    for (int i = 0; i < VPER; i++) {
        const int f = (int)threadIdx.x + i * 256, key = f % L, c = (f / L) * 4;
#pragma unroll
        for (int e = 0; e < 4; e++) Vt[(c + e) * LDV + key] = vx[i][e];
    }
    __syncthreads();
    floatx4 s[NB];
#pragma unroll
    for (int j = 0; j < NB; j++) s[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int blk = 0; blk < DB; blk++)
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(&Ks[(16 * j + t) * LDK + 16 * blk + 4 * kl]);
#pragma unroll
            for (int u = 0; u < 4; u++) s[j] = mfma4(a[u], qf[blk][u], s[j]);
        }
    // Softmax over keys for query t.
    float mx = -__int_as_float(0x7F800000);
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float x = s[j][r] * scale;
            if (mask) x = x + mv[j][r];
            s[j][r] = x;
            mx = x > mx ? x : mx;
        }
    {
        float w2 = __shfl_xor(mx, 16, 64);
        mx = w2 > mx ? w2 : mx;
        w2 = __shfl_xor(mx, 32, 64);
        mx = w2 > mx ? w2 : mx;
    }
    float pr[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float e = omd::exp_nonpos(s[j][r] - mx);
            s[j][r] = e;
            pr[r] += e;
        }
#pragma unroll
    for (int r = 0; r < 4; r++) pr[r] = pr[r] + __shfl_down(pr[r], 32, 64);  // p[i] + p[i+8]  (kl + 2)
#pragma unroll
    for (int r = 0; r < 4; r++) pr[r] = pr[r] + __shfl_down(pr[r], 16, 64);  // p[i] + p[i+4]  (kl + 1)
    pr[0] = pr[0] + pr[2];                                                   // p[i] + p[i+2]
    pr[1] = pr[1] + pr[3];
    pr[0] = pr[0] + pr[1];                                                   // p[0] + p[1]
    const float l = __shfl(pr[0], t, 64);  // the total sits on lane t of group 0
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) s[j][r] = omd::canon(s[j][r] / l);
    // O^T = V^T P^T
    floatx4 oa[DB];
#pragma unroll
    for (int db = 0; db < DB; db++) {
        oa[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(&Vt[(16 * db + t) * LDV + 16 * j + 4 * kl]);
#pragma unroll
            for (int u = 0; u < 4; u++) oa[db] = mfma4(a[u], s[j][u], oa[db]);
        }
    }
    float *og = o + (row0 + qrow) * ldo + h * D;
#pragma unroll
    for (int db = 0; db < DB; db++) *reinterpret_cast<floatx4 *>(og + 16 * db + 4 * kl) = oa[db];
}

template <int D, int L>
__global__ void __launch_bounds__(L * 4) k_attn_bwd(const float *__restrict__ q, const float *__restrict__ k,
                                                    const float *__restrict__ v, int ld, const float *__restrict__ mask,
                                                    int64_t mask_bstride, const float *__restrict__ g, int ldg,
                                                    float *dq, float *dk, float *dv, int ldd, float scale, int acc) {
    OM_LDS_POISON();
    constexpr int NTH = L * 4, LDX = D + 4, LDT = L + 4, NB = L / 16;
    __shared__ __attribute__((aligned(16))) float Qs[L * LDX];
    __shared__ __attribute__((aligned(16))) float Ks[L * LDX];
    __shared__ __attribute__((aligned(16))) float Vs[L * LDX];
    __shared__ __attribute__((aligned(16))) float Gs[L * LDX];
    __shared__ __attribute__((aligned(16))) float T[L * LDT];  // P^T, then dS^T: [key][query]
    const int h = blockIdx.x, b = blockIdx.y;
    const int64_t row0 = (int64_t)b * L;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = lane & 15, kl = lane >> 4;
    const int q0 = 16 * w;  // this wavefront's queries; also its block of 16 keys for dK and dV
    float mv[4][L / 16];
    load_mask<L>(mv, mask ? mask + b * mask_bstride + (int64_t)(q0 + 4 * kl) * L : nullptr, t);
    {  // all four operands' loads in flight before the first LDS store
        Stage<D, NTH, L> sq, sk, sv, sg;
        sq.load(q + row0 * ld + h * D, ld);
        sk.load(k + row0 * ld + h * D, ld);
        sv.load(v + row0 * ld + h * D, ld);
        sg.load(g + row0 * ldg + h * D, ldg);
        sq.store(Qs);
        sk.store(Ks);
        sv.store(Vs);
        sg.store(Gs);
    }
    __syncthreads();
    floatx4 s[NB];
    scores<D, L>(s, Qs, Ks, q0, t, kl);
    softmax_rows<L>(s, mv, mask != nullptr, scale);
    floatx4 dp[NB];
    scores<D, L>(dp, Gs, Vs, q0, t, kl);  // dP = dO V^T
    // dS = P (dP - sum_k dP P) scale, the row sum in double (BackwardNn.cs:26-52 via AttentionBackward)
#pragma unroll
    for (int r = 0; r < 4; r++) {
        double dot = 0.0;
#pragma unroll
        for (int j = 0; j < NB; j++) dot += (double)(dp[j][r] * s[j][r]);
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 16);
        const float df = (float)dot;
#pragma unroll
        for (int j = 0; j < NB; j++) dp[j][r] = (s[j][r] * (dp[j][r] - df)) * scale;
    }
    // P^T -> T (four consecutive queries per store)
#pragma unroll
    for (int j = 0; j < NB; j++) *reinterpret_cast<floatx4 *>(&T[(16 * j + t) * LDT + q0 + 4 * kl]) = s[j];
    __syncthreads();
    floatx4 dva[D / 16];
#pragma unroll
    for (int jn = 0; jn < D / 16; jn++) dva[jn] = floatx4{0.f, 0.f, 0.f, 0.f};
    mm_kA<D, L, LDT>(dva, T, q0, Gs, t, kl);  // dV = P^T dO for keys q0..q0+15
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NB; j++) *reinterpret_cast<floatx4 *>(&T[(16 * j + t) * LDT + q0 + 4 * kl]) = dp[j];
    __syncthreads();
    floatx4 dka[D / 16];
#pragma unroll
    for (int jn = 0; jn < D / 16; jn++) dka[jn] = floatx4{0.f, 0.f, 0.f, 0.f};
    mm_kA<D, L, LDT>(dka, T, q0, Qs, t, kl);  // dK = dS^T Q for keys q0..q0+15
    // dQ = dS K for queries q0..q0+15: A = dS[q][key] read column-wise from T = dS^T.
    floatx4 dqa[D / 16];
#pragma unroll
    for (int jn = 0; jn < D / 16; jn++) dqa[jn] = floatx4{0.f, 0.f, 0.f, 0.f};
    {
        constexpr int DB = D / 16;
#pragma unroll
        for (int blk = 0; blk < NB; blk++)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int key = 16 * blk + 4 * kl + u;
                const float a = T[key * LDT + q0 + t];
                const float *brow = &Ks[key * LDX + DB * t];
                float bv[DB];
#pragma unroll
                for (int x = 0; x < DB; x++) bv[x] = brow[x];
#pragma unroll
                for (int jn = 0; jn < DB; jn++) dqa[jn] = mfma4(a, bv[jn], dqa[jn]);
            }
    }
    if (dv) store_rows<D>(dv + row0 * ldd + h * D, ldd, q0, dva, t, kl, acc);
    if (dk) store_rows<D>(dk + row0 * ldd + h * D, ldd, q0, dka, t, kl, acc);
    if (dq) store_rows<D>(dq + row0 * ldd + h * D, ldd, q0, dqa, t, kl, acc);
}

// Backward with P^T and dS^T staged a quarter at a time (32 queries by all keys) in the LDS that V held, so a
// workgroup needs only Q, K, V and dO in LDS (74 KB at L = 128: two workgroups per CU, one round for C3's 384).
// The row phase is k_attn_bwd's (each wavefront: S, P, dP and dS for its 16 queries, in registers). Then, per
// quarter r of the queries (those of wavefronts 2r and 2r+1): those two wavefronts write their P^T columns, every
// wavefront adds the quarter's terms to dV for its 16 keys; the same with dS^T for dK, while four wavefronts each
// take one 16 x 16 block of the quarter's dQ over all keys. Every sum runs over the same index sequence as in
// k_attn_bwd (queries, or keys, in increasing order, one MFMA chain), so the results are bit for bit its results.
// Each workgroup's own path is longer (eight barrier rounds): the launcher takes this kernel only when the
// (head, batch) pairs outnumber the CUs.
template <int D, int L>
__global__ void __launch_bounds__(L * 4, 2) k_attn_bwd_q(const float *__restrict__ q, const float *__restrict__ k,
                                                         const float *__restrict__ v, int ld,
                                                         const float *__restrict__ mask, int64_t mask_bstride,
                                                         const float *__restrict__ g, int ldg, float *dq, float *dk,
                                                         float *dv, int ldd, float scale, int acc) {
    OM_LDS_POISON();
    constexpr int NTH = L * 4, LDX = D + 4, NB = L / 16, NW = L / 16, QT = 32, LDT = QT + 4, DB = D / 16;
    static_assert(D == 32, "the quarter's dQ is four 16 x 16 blocks");
    static_assert(QT * LDT <= L * LDX / 1 && L * LDT <= L * LDX, "a quarter of P^T fits where V was");
    __shared__ __attribute__((aligned(16))) float Qs[L * LDX];
    __shared__ __attribute__((aligned(16))) float Ks[L * LDX];
    __shared__ __attribute__((aligned(16))) float Vs[L * LDX];  // V, then a quarter of P^T or dS^T: [key][32 queries]
    __shared__ __attribute__((aligned(16))) float Gs[L * LDX];
    float *T = Vs;
    const int h = blockIdx.x, b = blockIdx.y;
    const int64_t row0 = (int64_t)b * L;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = lane & 15, kl = lane >> 4;
    const int q0 = 16 * w;  // this wavefront's queries; also its block of 16 keys for dK and dV
    {
        float mv[4][L / 16];
        load_mask<L>(mv, mask ? mask + b * mask_bstride + (int64_t)(q0 + 4 * kl) * L : nullptr, t);
        {
            Stage<D, NTH, L> sq, sk, sv, sg;
            sq.load(q + row0 * ld + h * D, ld);
            sk.load(k + row0 * ld + h * D, ld);
            sv.load(v + row0 * ld + h * D, ld);
            sg.load(g + row0 * ldg + h * D, ldg);
            sq.store(Qs);
            sk.store(Ks);
            sv.store(Vs);
            sg.store(Gs);
        }
        __syncthreads();
        floatx4 s[NB];
        scores<D, L>(s, Qs, Ks, q0, t, kl);
        softmax_rows<L>(s, mv, mask != nullptr, scale);
        floatx4 dp[NB];
        scores<D, L>(dp, Gs, Vs, q0, t, kl);  // dP = dO V^T
#pragma unroll
        for (int r = 0; r < 4; r++) {
            double dot = 0.0;
#pragma unroll
            for (int j = 0; j < NB; j++) dot += (double)(dp[j][r] * s[j][r]);
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) dot += __shfl_xor(dot, o, 16);
            const float df = (float)dot;
#pragma unroll
            for (int j = 0; j < NB; j++) dp[j][r] = (s[j][r] * (dp[j][r] - df)) * scale;
        }
        __syncthreads();  // V is read; its LDS now takes the quarters

        // acc[jn] += A (16 keys a0.., k = the quarter's 32 queries from T) x B (rows qb0.. of Bs, interleaved d)
        auto quarter_mm = [&](floatx4(&accv)[DB], const float *Bs, int qb0) {
#pragma unroll
            for (int blk = 0; blk < QT / 16; blk++) {
                floatx4 a = *reinterpret_cast<const floatx4 *>(&T[(q0 + t) * LDT + 16 * blk + 4 * kl]);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float *brow = &Bs[(qb0 + 16 * blk + 4 * kl + u) * LDX + DB * t];
                    float2 w2 = *reinterpret_cast<const float2 *>(brow);
                    accv[0] = mfma4(a[u], w2.x, accv[0]);
                    accv[1] = mfma4(a[u], w2.y, accv[1]);
                }
            }
        };
        floatx4 dva[DB], dka[DB];
#pragma unroll
        for (int jn = 0; jn < DB; jn++) dva[jn] = dka[jn] = floatx4{0.f, 0.f, 0.f, 0.f};
        // dV = P^T dO, a quarter of the queries at a time
#pragma unroll
        for (int r = 0; r < NW / 2; r++) {
            if ((w >> 1) == r) {
#pragma unroll
                for (int j = 0; j < NB; j++)
                    *reinterpret_cast<floatx4 *>(&T[(16 * j + t) * LDT + 16 * (w & 1) + 4 * kl]) = s[j];
            }
            __syncthreads();
            quarter_mm(dva, Gs, QT * r);
            __syncthreads();
        }
        // dK = dS^T Q and dQ = dS K, the same way
#pragma unroll
        for (int r = 0; r < NW / 2; r++) {
            if ((w >> 1) == r) {
#pragma unroll
                for (int j = 0; j < NB; j++)
                    *reinterpret_cast<floatx4 *>(&T[(16 * j + t) * LDT + 16 * (w & 1) + 4 * kl]) = dp[j];
            }
            __syncthreads();
            quarter_mm(dka, Qs, QT * r);
            // the quarter's dQ: block (qb, db) of four, over all keys in increasing order
            const bool mine = NW == 4 || (w >> 2) == (r & 1);
            if (dq && mine) {
                const int blkq = w & 3, qb = blkq >> 1, db = blkq & 1;
                floatx4 qa = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int blk = 0; blk < NB; blk++)
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int key = 16 * blk + 4 * kl + u;
                        qa = mfma4(T[key * LDT + 16 * qb + t], Ks[key * LDX + 16 * db + t], qa);
                    }
                float *dst = dq + (row0 + QT * r + 16 * qb + 4 * kl) * ldd + h * D + 16 * db + t;
#pragma unroll
                for (int e = 0; e < 4; e++) dst[e * ldd] = acc ? dst[e * ldd] + qa[e] : qa[e];
            }
            __syncthreads();
        }
        if (dv) store_rows<D>(dv + row0 * ldd + h * D, ldd, q0, dva, t, kl, acc);
        if (dk) store_rows<D>(dk + row0 * ldd + h * D, ldd, q0, dka, t, kl, acc);
    }
}

bool fused_ok(const float *q, const float *k, const float *v, int ld, int ldo, int lq, int lk, int d) {
    auto al = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
    return d == 32 && lq == lk && (lq == 64 || lq == 128) && ld % 4 == 0 && ldo % 4 == 0 && al(q) && al(k) && al(v);
}

om_status check(om_ctx *ctx, const char *what, const void *q, const void *k, const void *v, int B, int H, int L,
                int d, int ld, int ldo) {
    OM_REQUIRE(ctx, q && k && v, "%s: NULL q/k/v", what);
    OM_REQUIRE(ctx, B > 0 && H > 0 && L > 0 && d > 0 && d % 2 == 0,
               "%s: needs [B,L,H*D] tensors with positive sizes and even D, got B=%d H=%d L=%d D=%d", what, B, H, L,
               d);
    OM_REQUIRE(ctx, ld >= H * d && ldo >= H * d, "%s: row strides %d / %d below H*D = %d", what, ld, ldo, H * d);
    OM_REQUIRE(ctx, (int64_t)B * H * L <= INT32_MAX, "%s: too many rows", what);
    return OM_OK;
}

}  // namespace

extern "C" {

om_status om_attention_fwd_fused(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                 const float *mask, int mask_batched, float *o, int ld_o, int B, int H, int L, int d,
                                 float scale) {
    OM_CHECK_CTX(ctx);
    om_status s = check(ctx, "om_attention_fwd_fused", q, k, v, B, H, L, d, ld_qkv, ld_o);
    if (s) return s;
    OM_REQUIRE(ctx, o, "om_attention_fwd_fused: NULL output");
    if (scale == 0.0f || scale != scale) scale = 1.0f / sqrtf((float)d);
    const int64_t mstride = (mask && mask_batched) ? (int64_t)L * L : 0;
    if (fused_ok(q, k, v, ld_qkv, ld_o, L, L, d) && ((uintptr_t)o & 15) == 0 && ((uintptr_t)mask & 15) == 0) {
        dim3 grid(L / 64, H, B);
        if (L == 128)
            hipLaunchKernelGGL((k_attn_fwd<32, 128>), grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, o,
                               ld_o, scale);
        else
            hipLaunchKernelGGL((k_attn_fwd<32, 64>), grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, o,
                               ld_o, scale);
        return OM_LAUNCH_CHECK(ctx, "om_attention_fwd_fused");
    }
    float *p;
    s = om::scratch2(ctx, sizeof(float) * (uint64_t)B * H * L * L, &p);
    if (s) return s;
    return om_attention_fwd_ld(ctx, q, k, v, ld_qkv, mask, mask_batched, o, ld_o, p, B, H, L, L, d, scale);
}

om_status om_attention_bwd_fused(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                 const float *mask, int mask_batched, const float *g, int ld_g, float *dq, float *dk,
                                 float *dv, int ld_d, int B, int H, int L, int d, float scale, int acc) {
    OM_CHECK_CTX(ctx);
    om_status s = check(ctx, "om_attention_bwd_fused", q, k, v, B, H, L, d, ld_qkv, ld_d);
    if (s) return s;
    OM_REQUIRE(ctx, g && ld_g >= H * d, "om_attention_bwd_fused: NULL gradient or short stride");
    if (!dq && !dk && !dv) return OM_OK;
    if (scale == 0.0f || scale != scale) scale = 1.0f / sqrtf((float)d);
    const int64_t mstride = (mask && mask_batched) ? (int64_t)L * L : 0;
    if (fused_ok(q, k, v, ld_qkv, ld_d, L, L, d) && ld_g % 4 == 0 && ((uintptr_t)g & 15) == 0) {
        dim3 grid(H, B);
        // More (head, batch) pairs than CUs: the quarter-staged kernel fits two per CU, one round instead of two
        // (C3: 46 against 48 us); fewer: one round either way, and k_attn_bwd's shorter path per workgroup wins.
        // The results are the same bits.
        if ((int64_t)B * H > ctx->num_cus) {
            if (L == 128)
                hipLaunchKernelGGL((k_attn_bwd_q<32, 128>), grid, dim3(512), 0, ctx->stream, q, k, v, ld_qkv, mask,
                                   mstride, g, ld_g, dq, dk, dv, ld_d, scale, acc);
            else
                hipLaunchKernelGGL((k_attn_bwd_q<32, 64>), grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask,
                                   mstride, g, ld_g, dq, dk, dv, ld_d, scale, acc);
            return OM_LAUNCH_CHECK(ctx, "om_attention_bwd_fused");
        }
        if (L == 128)
            hipLaunchKernelGGL((k_attn_bwd<32, 128>), grid, dim3(512), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride,
                               g, ld_g, dq, dk, dv, ld_d, scale, acc);
        else
            hipLaunchKernelGGL((k_attn_bwd<32, 64>), grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride,
                               g, ld_g, dq, dk, dv, ld_d, scale, acc);
        return OM_LAUNCH_CHECK(ctx, "om_attention_bwd_fused");
    }
    // Recompute P (as the reference does) with the GEMM path, then the unfused backward.
    const uint64_t n = (uint64_t)B * H * L * L;
    float *p;
    s = om::scratch2(ctx, sizeof(float) * 2 * n, &p);
    if (s) return s;
    // S and P only (the forward entry point would also run O = P V).
    {
        omg::Params ps = omg::dense_params(L, L, d, nullptr, 0, nullptr, 0, p, L);
        ps.batch_div = H;
        ps.a = q;
        ps.lda = ld_qkv;
        ps.sa_outer = (int64_t)L * ld_qkv;
        ps.sa_inner = d;
        ps.b = k;
        ps.ldb = ld_qkv;
        ps.sb_outer = (int64_t)L * ld_qkv;
        ps.sb_inner = d;
        ps.sc_outer = (int64_t)H * L * L;
        ps.sc_inner = (int64_t)L * L;
        ps.alpha = scale;
        ps.mask = mask;
        ps.mask_outer_stride = mstride;
        s = omg::launch_dense(ctx, ps, false, true, B * H, "attention scores (recompute)");
        if (s) return s;
        s = om_internal_softmax_rows(ctx, p, B * H * L, L);
        if (s) return s;
    }
    return om_attention_bwd_ld(ctx, q, k, v, ld_qkv, p, g, ld_g, dq, dk, dv, ld_d, p + n, B, H, L, L, d, scale, acc);
}

}  // extern "C"
