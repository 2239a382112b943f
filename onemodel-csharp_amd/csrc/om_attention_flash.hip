// Streaming fused attention for sequences longer than a workgroup can hold whole (Ops.Attention,
// Ops.Layers.cs:746-807; AttentionBackward, BackwardNn.cs:636-701; definition docs/kernels-attention.md:10-33).
//
// Forward, one workgroup per batch item, head and 64 queries (a wavefront per 16 queries), walking the keys in chunks
// of 64 staged through LDS: S^T = K Q^T on MFMA, logits x = S * scale * log2(e) + mask * log2(e), a running row
// maximum m and row sum l (the online softmax: earlier terms rescale by 2^(m_old - m_new) when the maximum grows),
// O^T += V^T E^T with E = 2^(x - m) straight from the registers holding it. At the end O = O^T / l, and the row
// statistics m and 1/l (8 bytes per query) are saved, so no [B, H, L, L] tensor is written anywhere.
//
// Backward, one workgroup per batch item, head and 64 keys (a wavefront per 16 keys), walking the queries in chunks
// of 64: S = Q K^T and dP = dO V^T on MFMA, P = 2^(x - m) / l from the saved statistics (one exponential and one
// multiply per score), dS = P (dP - delta) scale with delta = rowsum(dO * O) (equal to the reference's rowsum(dP P),
// since dP P summed over keys is dO . (P V)), and
//   dV^T += dO^T P and dK^T += Q^T dS, accumulated in registers over the query chunks;
//   dQ = dS K for the chunk's queries over this workgroup's 64 keys, a partial per key block in scratch.
// A last launch sums each query's dQ partials over the key blocks in increasing block order, so every result is
// deterministic (the same bits on every run). The softmax exponentials use the hardware exp2; results agree with
// the reference's exact row kernel within the fp32 rounding of the sums (1e-5 scaled error, tested).
//
// Layouts: q, k, v, o, dO and the gradients are [B, L, H*D] row blocks of stride ld (packed q|k|v welcome); mask is
// [L, L] or [B, L, L] additive; stats holds m (log2 units) for all B*H*L queries, then 1/l.
#include "om_internal.hpp"

#include <cmath>
#include <cstdlib>

extern "C" om_status om_attention_fwd_fused(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                            const float *mask, int mask_batched, float *o, int ld_o, int B, int H,
                                            int L, int d, float scale);
extern "C" om_status om_attention_bwd_fused(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                            const float *mask, int mask_batched, const float *g, int ld_g, float *dq,
                                            float *dk, float *dv, int ld_d, int B, int H, int L, int d, float scale,
                                            int acc);

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kChunk = 64;  // queries per forward workgroup, keys per backward workgroup, and the streamed chunk
constexpr int LDSC = kChunk + 4;  // row stride of a [64][64] score block in LDS

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup id -> (block, head, batch) with consecutive ids on one XCD (the hardware deals workgroups round-robin
// over the 8 XCDs, each with its own L2): the blocks of one head then share its K and V (or Q and dO) in one L2.
__device__ __forceinline__ void block_coords(int nb, int H, int &blk, int &h, int &b) {
    int lin = blockIdx.x;
    const int total = gridDim.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    blk = lin % nb;
    const int bh = lin / nb;
    h = bh % H;
    b = bh / H;
}

template <int D, bool MASK>
__global__ void __launch_bounds__(256) k_flash_fwd(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, int ld, const float *__restrict__ mask,
                                                   int64_t mask_bstride, float *__restrict__ o, int ldo,
                                                   float *__restrict__ stat_m, float *__restrict__ stat_r, int H,
                                                   int L, float c) {
    OM_LDS_POISON();
    constexpr int DB = D / 16, LDK = D + 4, Q4 = D / 4, PER = kChunk * Q4 / 256;
    static_assert(kChunk * Q4 % 256 == 0, "a chunk is whole rounds of the workgroup");
    __shared__ __attribute__((aligned(16))) float Ks[kChunk * LDK];  // [key][d]
    __shared__ __attribute__((aligned(16))) float Vt[D * LDSC];      // [d][key]
    const int nb = L / kChunk;
    int qb, h, b;
    block_coords(nb, H, qb, h, b);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = lane & 15, kl = lane >> 4;
    const int qrow = qb * kChunk + 16 * w + t;  // this lane's query
    const int64_t row0 = (int64_t)b * L;
    floatx4 qf[DB];  // B operand of S^T = K Q^T: Q[qrow][16 blk + 4 kl + u]
    const float *qg = q + (row0 + qrow) * ld + h * D;
#pragma unroll
    for (int blk = 0; blk < DB; blk++) qf[blk] = *reinterpret_cast<const floatx4 *>(qg + 16 * blk + 4 * kl);
    const float *mrow = mask ? mask + b * mask_bstride + (int64_t)qrow * L + 4 * kl : nullptr;
    const float *kg = k + row0 * ld + h * D, *vg = v + row0 * ld + h * D;
    // K rows: thread f takes row f / Q4, four d from (f % Q4) * 4; V^T: key f % 64, four d from (f / 64) * 4, so each
    // LDS store row of V^T is contiguous across the lanes.
    floatx4 kx[PER], vx[PER];
    auto load = [&](int kc) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int f = (int)threadIdx.x + 256 * i;
            kx[i] = *reinterpret_cast<const floatx4 *>(kg + (int64_t)(kc * kChunk + f / Q4) * ld + (f % Q4) * 4);
            vx[i] = *reinterpret_cast<const floatx4 *>(vg + (int64_t)(kc * kChunk + f % kChunk) * ld +
                                                       (f / kChunk) * 4);
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int f = (int)threadIdx.x + 256 * i;
            *reinterpret_cast<floatx4 *>(&Ks[(f / Q4) * LDK + (f % Q4) * 4]) = kx[i];
            const int key = f % kChunk, d0 = (f / kChunk) * 4;
#pragma unroll
            for (int e = 0; e < 4; e++) Vt[(d0 + e) * LDSC + key] = vx[i][e];
        }
    };
    float m = -__int_as_float(0x7F800000), l = 0.0f;  // running maximum (log2 units) and sum for query t
    floatx4 oa[DB];                                   // O^T[16 db + 4 kl + r][query t], unnormalised
#pragma unroll
    for (int db = 0; db < DB; db++) oa[db] = floatx4{0.f, 0.f, 0.f, 0.f};
    load(0);
    for (int kc = 0; kc < nb; kc++) {
        __syncthreads();  // the previous chunk's reads of Ks / Vt are done
        store();
        __syncthreads();
        if (kc + 1 < nb) load(kc + 1);  // in flight during this chunk's products
        floatx4 s[4];                   // S^T[key 16 j + 4 kl + r][query t]
#pragma unroll
        for (int j = 0; j < 4; j++) s[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int blk = 0; blk < DB; blk++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const floatx4 a = *reinterpret_cast<const floatx4 *>(&Ks[(16 * j + t) * LDK + 16 * blk + 4 * kl]);
#pragma unroll
                for (int u = 0; u < 4; u++) s[j] = mfma4(a[u], qf[blk][u], s[j]);
            }
        float cm = -__int_as_float(0x7F800000);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            floatx4 mk = floatx4{0.f, 0.f, 0.f, 0.f};
            if constexpr (MASK) mk = *reinterpret_cast<const floatx4 *>(mrow + kc * kChunk + 16 * j);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float x = __builtin_fmaf(s[j][r], c, mk[r] * kLog2e);
                s[j][r] = x;
                cm = x > cm ? x : cm;
            }
        }
        {
            float o2 = __shfl_xor(cm, 16, 64);
            cm = o2 > cm ? o2 : cm;
            o2 = __shfl_xor(cm, 32, 64);
            cm = o2 > cm ? o2 : cm;
        }
        const float mn = cm > m ? cm : m;
        const float mu = mn == -__int_as_float(0x7F800000) ? 0.0f : mn;  // a row masked so far adds nothing
        const float alpha = exp2_hw(m - mu);
        float ps = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float e = exp2_hw(s[j][r] - mu);
                s[j][r] = e;
                ps += e;
            }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        l = l * alpha + ps;
#pragma unroll
        for (int db = 0; db < DB; db++) {
            oa[db] *= alpha;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const floatx4 a = *reinterpret_cast<const floatx4 *>(&Vt[(16 * db + t) * LDSC + 16 * j + 4 * kl]);
#pragma unroll
                for (int u = 0; u < 4; u++) oa[db] = mfma4(a[u], s[j][u], oa[db]);
            }
        }
        m = mn;
    }
    const float rl = 1.0f / l;
    float *og = o + (row0 + qrow) * ldo + h * D;
#pragma unroll
    for (int db = 0; db < DB; db++) *reinterpret_cast<floatx4 *>(og + 16 * db + 4 * kl) = oa[db] * rl;
    if (kl == 0) {
        const int64_t sr = ((int64_t)b * H + h) * L + qrow;
        stat_m[sr] = m;
        stat_r[sr] = rl;
    }
}

// Forward for rows that fit a workgroup whole (L = 64 or 128): the streaming forward's arithmetic in one pass over
// all L keys, so there is no running rescale. One workgroup per batch item, head and 64 queries (a wavefront per 16
// queries); K and V^T of the (batch, head) staged in LDS, S^T = K Q^T with this lane's query on the lane index t,
// E = 2^(x - max) in the registers that hold S^T, which are the B operand of O^T = V^T E^T, and O = O^T / l. The
// statistics are the streaming forward's (m in log2 units, 1/l), so either backward can follow either forward.
template <int D, int L, bool MASK>
__global__ void __launch_bounds__(256) k_rows_fwd(const float *__restrict__ q, const float *__restrict__ k,
                                                  const float *__restrict__ v, int ld, const float *__restrict__ mask,
                                                  int64_t mask_bstride, float *__restrict__ o, int ldo,
                                                  float *__restrict__ stat_m, float *__restrict__ stat_r, int H,
                                                  float c) {
    OM_LDS_POISON();
    constexpr int DB = D / 16, NB = L / 16, LDK = D + 4, LDV = L + 4, Q4 = D / 4, PER = L * Q4 / 256;
    static_assert(L * Q4 % 256 == 0, "K and V are whole rounds of the workgroup");
    __shared__ __attribute__((aligned(16))) float Ks[L * LDK];  // [key][d]
    __shared__ __attribute__((aligned(16))) float Vt[D * LDV];  // [d][key]
    int qb, h, b;
    block_coords(L / 64, H, qb, h, b);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = lane & 15, kl = lane >> 4;
    const int qrow = qb * 64 + 16 * w + t;  // this lane's query
    const int64_t row0 = (int64_t)b * L;
    // Loads in the order the work needs them: K (the first product's A operand, via LDS), Q, then the mask (the
    // largest, needed only after S^T), so the first MFMAs can start while the mask is still arriving.
    // K rows: thread f takes row f / Q4, four d from (f % Q4) * 4. V^T: key f % L, four d from (f / L) * 4, so each
    // LDS store row of V^T is contiguous across the lanes; V's loads are issued once K is in LDS and arrive while
    // S^T and the softmax run.
    const float *kg = k + row0 * ld + h * D, *vg = v + row0 * ld + h * D;
    floatx4 kx[PER], vx[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int f = (int)threadIdx.x + 256 * i;
        kx[i] = *reinterpret_cast<const floatx4 *>(kg + (int64_t)(f / Q4) * ld + (f % Q4) * 4);
    }
    floatx4 qf[DB];  // B operand of S^T = K Q^T: Q[qrow][16 blk + 4 kl + u]
    const float *qg = q + (row0 + qrow) * ld + h * D;
#pragma unroll
    for (int blk = 0; blk < DB; blk++) qf[blk] = *reinterpret_cast<const floatx4 *>(qg + 16 * blk + 4 * kl);
    // mask of query t over keys 16 j + 4 kl + r (scaled to log2 units below); MASK is a template parameter so that no
    // branch joins the paths before the waits for K (a join makes the compiler wait for every load of either path)
    floatx4 mv[NB];
    if constexpr (MASK) {
        const float *mr = mask + b * mask_bstride + (int64_t)qrow * L + 4 * kl;
#pragma unroll
        for (int j = 0; j < NB; j++) mv[j] = *reinterpret_cast<const floatx4 *>(mr + 16 * j);
    } else {
#pragma unroll
        for (int j = 0; j < NB; j++) mv[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int f = (int)threadIdx.x + 256 * i;
        *reinterpret_cast<floatx4 *>(&Ks[(f / Q4) * LDK + (f % Q4) * 4]) = kx[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int f = (int)threadIdx.x + 256 * i;
        vx[i] = *reinterpret_cast<const floatx4 *>(vg + (int64_t)(f % L) * ld + (f / L) * 4);
    }
    floatx4 s[NB];  // S^T[key 16 j + 4 kl + r][query t]
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
    // Nothing that reads the mask may be scheduled among the MFMAs above: it would make them wait for the mask's
    // loads, which are issued last so that this product can run while they arrive.
    __builtin_amdgcn_sched_barrier(0);
    float mx = -__int_as_float(0x7F800000);
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float x = __builtin_fmaf(s[j][r], c, mv[j][r] * kLog2e);
            s[j][r] = x;
            mx = fmaxf(mx, x);  // NaN scores are skipped, as by x > mx ? x : mx
        }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mu = mx == -__int_as_float(0x7F800000) ? 0.0f : mx;  // a fully masked row: l = 0, O = NaN
    float ps = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float e = exp2_hw(s[j][r] - mu);
            s[j][r] = e;
            ps += e;
        }
    ps += __shfl_xor(ps, 16, 64);
    ps += __shfl_xor(ps, 32, 64);
    __builtin_amdgcn_sched_barrier(0);  // the softmax above runs while V's loads are in flight, not after them
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int f = (int)threadIdx.x + 256 * i;
        const int key = f % L, d0 = (f / L) * 4;
#pragma unroll
        for (int e = 0; e < 4; e++) Vt[(d0 + e) * LDV + key] = vx[i][e];
    }
    __syncthreads();
    floatx4 oa[DB];  // O^T[16 db + 4 kl + r][query t], unnormalised
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
    const float rl = 1.0f / ps;
    float *og = o + (row0 + qrow) * ldo + h * D;
#pragma unroll
    for (int db = 0; db < DB; db++) *reinterpret_cast<floatx4 *>(og + 16 * db + 4 * kl) = oa[db] * rl;
    if (kl == 0) {
        const int64_t sr = ((int64_t)b * H + h) * L + qrow;
        stat_m[sr] = mx;
        stat_r[sr] = rl;
    }
}

// delta[(b H + h) L + l] = (float) sum over d, in double, of dO * O for every query row (16 lanes per row).
template <int D>
__global__ void __launch_bounds__(256) k_flash_delta(const float *__restrict__ g, int ldg, const float *__restrict__ o,
                                                     int ldo, float *__restrict__ delta, int H, int L, int64_t rows) {
    OM_LDS_POISON();
    const int64_t row = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;
    const int sub = threadIdx.x & 15;
    double acc = 0.0;
    if (row < rows) {
        const int64_t bh = row / L, l = row % L, b = bh / H, h = bh % H;
        const float *gr = g + (b * L + l) * ldg + h * D, *orow = o + (b * L + l) * ldo + h * D;
        for (int d = 4 * sub; d < D; d += 64) {
            const floatx4 x = *reinterpret_cast<const floatx4 *>(gr + d), y = *reinterpret_cast<const floatx4 *>(orow + d);
#pragma unroll
            for (int e = 0; e < 4; e++) acc += (double)(x[e] * y[e]);
        }
    }
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 16);
    if (row < rows && sub == 0) delta[row] = (float)acc;
}

template <int D, bool MASK>
__global__ void __launch_bounds__(256, 2) k_flash_bwd(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, int ld, const float *__restrict__ mask,
                                                   int64_t mask_bstride, const float *__restrict__ g, int ldg,
                                                   const float *__restrict__ stat_m, const float *__restrict__ stat_r,
                                                   const float *__restrict__ delta, float *dk, float *dv, int ldd,
                                                   float *__restrict__ dq_part, int H, int L, float c, float scale,
                                                   int acc) {
    OM_LDS_POISON();
    constexpr int DB = D / 16, LDX = D + 4, Q4 = D / 4, PER = kChunk * Q4 / 256;
    constexpr int QSZ = kChunk * LDX > kChunk * LDSC ? kChunk * LDX : kChunk * LDSC;
    __shared__ __attribute__((aligned(16))) float QS[QSZ];            // the chunk's Q [q][d], then dS [q][key]
    __shared__ __attribute__((aligned(16))) float Gs[kChunk * LDX];   // the chunk's dO [q][d]
    __shared__ __attribute__((aligned(16))) float Ks[kChunk * LDX];   // this block's K [key][d]
    __shared__ float St[3][kChunk];                                   // m, 1/l, delta of the chunk's queries
    const int nb = L / kChunk;
    int kb, h, b;
    block_coords(nb, H, kb, h, b);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = lane & 15, kl = lane >> 4;
    const int64_t row0 = (int64_t)b * L, bh = (int64_t)b * H + h;
    const int key0 = kb * kChunk, mykey = key0 + 16 * w + t;  // this lane's key in S = Q K^T
    // B operands of S = Q K^T and dP = dO V^T for this wavefront's 16 keys
    floatx4 kf[DB], vf[DB];
    {
        const float *kr = k + (row0 + mykey) * ld + h * D, *vr = v + (row0 + mykey) * ld + h * D;
#pragma unroll
        for (int blk = 0; blk < DB; blk++) {
            kf[blk] = *reinterpret_cast<const floatx4 *>(kr + 16 * blk + 4 * kl);
            vf[blk] = *reinterpret_cast<const floatx4 *>(vr + 16 * blk + 4 * kl);
        }
    }
    const float *qg = q + row0 * ld + h * D, *gg = g + row0 * ldg + h * D;
    floatx4 qx[PER], gx[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {  // this block's K rows, through the Q registers
        const int f = (int)threadIdx.x + 256 * i;
        qx[i] = *reinterpret_cast<const floatx4 *>(k + (row0 + key0 + f / Q4) * ld + h * D + (f % Q4) * 4);
        *reinterpret_cast<floatx4 *>(&Ks[(f / Q4) * LDX + (f % Q4) * 4]) = qx[i];
    }
    auto load = [&](int qc) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int f = (int)threadIdx.x + 256 * i;
            const int64_t r = (int64_t)(qc * kChunk + f / Q4);
            qx[i] = *reinterpret_cast<const floatx4 *>(qg + r * ld + (f % Q4) * 4);
            gx[i] = *reinterpret_cast<const floatx4 *>(gg + r * ldg + (f % Q4) * 4);
        }
    };
    floatx4 dvt[DB], dkt[DB];  // dV^T, dK^T [16 db + 4 kl + r][key 16 w + t]
#pragma unroll
    for (int db = 0; db < DB; db++) dvt[db] = dkt[db] = floatx4{0.f, 0.f, 0.f, 0.f};
    const float *mbase = mask ? mask + b * mask_bstride + mykey : nullptr;
    for (int qc = 0; qc < nb; qc++) {
        // (A) stage the chunk: Q and dO rows, the queries' statistics (other workgroups on the CU cover the loads'
        // latency; holding the next chunk in registers would halve the waves per SIMD)
        load(qc);
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int f = (int)threadIdx.x + 256 * i;
            *reinterpret_cast<floatx4 *>(&QS[(f / Q4) * LDX + (f % Q4) * 4]) = qx[i];
            *reinterpret_cast<floatx4 *>(&Gs[(f / Q4) * LDX + (f % Q4) * 4]) = gx[i];
        }
        if (threadIdx.x < 3 * kChunk) {
            const int which = threadIdx.x / kChunk, qq = threadIdx.x % kChunk;
            const float *src = which == 0 ? stat_m : which == 1 ? stat_r : delta;
            St[which][qq] = src[bh * L + qc * kChunk + qq];
        }
        __syncthreads();
        // (B) S and dP: rows are the chunk's queries 16 i + 4 kl + r, columns this wavefront's keys
        floatx4 s[4], dp[4];
#pragma unroll
        for (int i = 0; i < 4; i++) s[i] = dp[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int blk = 0; blk < DB; blk++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const floatx4 a = *reinterpret_cast<const floatx4 *>(&QS[(16 * i + t) * LDX + 16 * blk + 4 * kl]);
                const floatx4 ga = *reinterpret_cast<const floatx4 *>(&Gs[(16 * i + t) * LDX + 16 * blk + 4 * kl]);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    s[i] = mfma4(a[u], kf[blk][u], s[i]);
                    dp[i] = mfma4(ga[u], vf[blk][u], dp[i]);
                }
            }
        // (C) P from the saved statistics, dS = P (dP - delta) scale (the reference's rounding order)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int qq = 16 * i + 4 * kl + r;
                const float mk = MASK ? mbase[(int64_t)(qc * kChunk + qq) * L] * kLog2e : 0.0f;
                const float x = __builtin_fmaf(s[i][r], c, mk);
                const float p = exp2_hw(x - St[0][qq]) * St[1][qq];
                s[i][r] = p;
                dp[i][r] = (p * (dp[i][r] - St[2][qq])) * scale;
            }
        // (D) dV^T += dO^T P and dK^T += Q^T dS over the chunk's queries
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int qq = 16 * i + 4 * kl + u;
#pragma unroll
                for (int db = 0; db < DB; db++) {
                    dvt[db] = mfma4(Gs[qq * LDX + 16 * db + t], s[i][u], dvt[db]);
                    dkt[db] = mfma4(QS[qq * LDX + 16 * db + t], dp[i][u], dkt[db]);
                }
            }
        __syncthreads();  // every wavefront is done with the chunk's Q and dO
        if (dq_part) {
            // (E) dS into the Q slot as [query][key], then dQ = dS K for this wavefront's 16 queries
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 4; r++) QS[(16 * i + 4 * kl + r) * LDSC + 16 * w + t] = dp[i][r];
            __syncthreads();
            floatx4 dqa[DB];
#pragma unroll
            for (int db = 0; db < DB; db++) dqa[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb2 = 0; kb2 < 4; kb2++) {
                const floatx4 a = *reinterpret_cast<const floatx4 *>(&QS[(16 * w + t) * LDSC + 16 * kb2 + 4 * kl]);
#pragma unroll
                for (int u = 0; u < 4; u++)
#pragma unroll
                    for (int db = 0; db < DB; db++)
                        dqa[db] = mfma4(a[u], Ks[(16 * kb2 + 4 * kl + u) * LDX + 16 * db + t], dqa[db]);
            }
            // partial for key block kb: rows (b H + h) L + query, D columns
            float *pr = dq_part + ((int64_t)kb * gridDim.x / nb * L + bh * L + qc * kChunk + 16 * w + 4 * kl) * D + t;
#pragma unroll
            for (int db = 0; db < DB; db++)
#pragma unroll
                for (int r = 0; r < 4; r++) pr[(int64_t)r * D + 16 * db] = dqa[db][r];
            __syncthreads();  // the dS block is read before the next chunk is staged over it
        }
    }
    const int64_t orow = (row0 + key0 + 16 * w + t) * ldd + h * D + 4 * kl;
#pragma unroll
    for (int db = 0; db < DB; db++) {
        if (dv) {
            floatx4 *p = reinterpret_cast<floatx4 *>(dv + orow + 16 * db);
            *p = acc ? *p + dvt[db] : dvt[db];
        }
        if (dk) {
            floatx4 *p = reinterpret_cast<floatx4 *>(dk + orow + 16 * db);
            *p = acc ? *p + dkt[db] : dkt[db];
        }
    }
}

// Backward for rows that fit a workgroup whole (D = 32, L = 64 or 128): the streaming backward's arithmetic with
// all L queries in one pass. One workgroup per batch item, head and 64 keys (a wavefront per 16 keys), so a
// (batch, head) pair is L / 64 workgroups and the 384 pairs of a C3 step fill the chip evenly (three workgroups per
// CU). In order:
//   1. this block's K rows, the queries' m and 1/l and the first 64 queries' Q and dO rows into LDS; this lane's K and
//      V row fragments into registers (the B operands of S = Q K^T and dP = dO V^T);
//   2. per phase of 64 queries (the next phase's Q, dO and O rows load meanwhile): delta = rowsum(dO * O) of its
//      queries, a product per element summed in double over d, then
//   3. per block of 16 queries: S and dP on MFMA, P = 2^(x - m) / l, dS = P (dP - delta) scale, and at once
//      dV^T += dO^T P and dK^T += Q^T dS, whose B operands are the P and dS registers just computed (the A operands
//      read dO and Q two d at a time: row t of dV^T's A is d = 2t + db, so a lane's outputs are eight consecutive d);
//      dS stays in registers;
//   4. dS into LDS over Q and dO ([query][key]), then dQ = dS K over this block's 64 keys for two blocks of 16
//      queries per wavefront: the final dQ when L = 64, else a partial summed by k_flash_dq_reduce.
template <int L, bool MASK>
__global__ void __launch_bounds__(256, 3) k_rows_bwd(const float *__restrict__ q, const float *__restrict__ k,
                                                     const float *__restrict__ v, int ld, const float *__restrict__ mask,
                                                     int64_t mask_bstride, const float *__restrict__ g, int ldg,
                                                     const float *__restrict__ o, int ldo,
                                                     const float *__restrict__ stat_m, const float *__restrict__ stat_r,
                                                     float *dk, float *dv, float *dq, int ldd,
                                                     float *__restrict__ dq_part, int H, float c, float scale,
                                                     int acc) {
    OM_LDS_POISON();
    constexpr int D = 32, LDX = D + 4, NQB = L / 16, Q4 = D / 4, PERK = kChunk * Q4 / 256;
    constexpr int RP = 64, NPH = L / RP, PERP = RP * Q4 / 256;  // queries per phase, phases, float4 per thread
    constexpr int TPQ = 256 / RP, DPT = D / TPQ;  // threads per query and d per thread for delta
    static_assert(L == 64 || L == 128, "whole rows of 64 or 128 queries");
    static_assert(L * LDSC <= 2 * L * LDX, "dS [L][68] fits where Q and dO were");
    __shared__ __attribute__((aligned(16))) float QG[2 * L * LDX];  // Q [q][d] and dO [q][d]; later dS [q][key]
    __shared__ __attribute__((aligned(16))) float Ks[kChunk * LDX];  // this block's K [key][d]
    __shared__ __attribute__((aligned(16))) float St[3][L];          // m, 1/l, delta of every query
    float *Qs = QG, *Gs = QG + L * LDX;
    int kb, h, b;
    block_coords(L / kChunk, H, kb, h, b);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, t = lane & 15, kl = lane >> 4;
    const int64_t row0 = (int64_t)b * L, bh = (int64_t)b * H + h;
    const int key0 = kb * kChunk, mykey = key0 + 16 * w + t;  // this lane's key in S = Q K^T
    floatx4 kf[2], vf[2];
    {
        const float *kr = k + (row0 + mykey) * ld + h * D, *vr = v + (row0 + mykey) * ld + h * D;
#pragma unroll
        for (int blk = 0; blk < 2; blk++) {
            kf[blk] = *reinterpret_cast<const floatx4 *>(kr + 16 * blk + 4 * kl);
            vf[blk] = *reinterpret_cast<const floatx4 *>(vr + 16 * blk + 4 * kl);
        }
    }
    // 1. This block's K rows, the statistics and the first phase's rows (queries 0 .. 63: Q, dO, and O for delta)
    // into LDS; each later phase's rows load while the previous phase computes.
    const int tid = threadIdx.x;
    floatx4 qx[PERP], gx[PERP], kx[PERK], ox[DPT / 4];
    const float *qg = q + row0 * ld + h * D, *gg = g + row0 * ldg + h * D;
    const int dq_q = tid / TPQ, dq_d0 = (tid % TPQ) * DPT;  // delta: this thread's query in a phase, first d
    auto load_rows = [&](int ph) {
#pragma unroll
        for (int i = 0; i < PERP; i++) {
            const int f = tid + 256 * i, row = ph * RP + f / Q4;
            qx[i] = *reinterpret_cast<const floatx4 *>(qg + (int64_t)row * ld + (f % Q4) * 4);
            gx[i] = *reinterpret_cast<const floatx4 *>(gg + (int64_t)row * ldg + (f % Q4) * 4);
        }
        const float *orow = o + (row0 + ph * RP + dq_q) * ldo + h * D + dq_d0;
#pragma unroll
        for (int e = 0; e < DPT / 4; e++) ox[e] = *reinterpret_cast<const floatx4 *>(orow + 4 * e);
    };
    auto store_rows = [&](int ph) {
#pragma unroll
        for (int i = 0; i < PERP; i++) {
            const int f = tid + 256 * i, row = ph * RP + f / Q4;
            *reinterpret_cast<floatx4 *>(&Qs[row * LDX + (f % Q4) * 4]) = qx[i];
            *reinterpret_cast<floatx4 *>(&Gs[row * LDX + (f % Q4) * 4]) = gx[i];
        }
    };
    // delta = rowsum(dO * O) of the phase's queries, each a product per element summed in double over d
    auto delta = [&](int ph) {
        const int qq = ph * RP + dq_q;
        double dot = 0.0;
#pragma unroll
        for (int e = 0; e < DPT / 4; e++) {
            const floatx4 gv = *reinterpret_cast<const floatx4 *>(&Gs[qq * LDX + dq_d0 + 4 * e]);
#pragma unroll
            for (int x = 0; x < 4; x++) dot += (double)(gv[x] * ox[e][x]);
        }
#pragma unroll
        for (int off = 1; off < TPQ; off <<= 1) dot += __shfl_xor(dot, off, 64);
        if (tid % TPQ == 0) St[2][qq] = (float)dot;
    };
    load_rows(0);
#pragma unroll
    for (int i = 0; i < PERK; i++) {
        const int f = tid + 256 * i;
        kx[i] = *reinterpret_cast<const floatx4 *>(k + (row0 + key0 + f / Q4) * ld + h * D + (f % Q4) * 4);
    }
    float stv = 0.0f;
    if (tid < 2 * L) stv = (tid < L ? stat_m : stat_r)[bh * L + tid % L];
    store_rows(0);
#pragma unroll
    for (int i = 0; i < PERK; i++) {
        const int f = tid + 256 * i;
        *reinterpret_cast<floatx4 *>(&Ks[(f / Q4) * LDX + (f % Q4) * 4]) = kx[i];
    }
    if (tid < 2 * L) St[tid / L][tid % L] = stv;
    __syncthreads();
    // 2, 3. Per phase: delta of its queries; then per block of 16 queries S, dP, P, dS, with dV^T and dK^T accumulating
    // over all L queries. The mask values of block i + 1 (this lane's key at queries 16 (i + 1) + 4 kl + r) load while
    // block i runs.
    const float *mbase = MASK ? mask + b * mask_bstride + mykey : nullptr;
    float mkc[4], mkn[4];
    auto mask_load = [&](float(&dst)[4], int i) {
#pragma unroll
        for (int r = 0; r < 4; r++) dst[r] = MASK ? mbase[(int64_t)(16 * i + 4 * kl + r) * L] : 0.0f;
    };
    mask_load(mkc, 0);
    floatx4 dsv[NQB];
    floatx4 dvt[2], dkt[2];  // [d = 2 (4 kl + r) + db][key t]
#pragma unroll
    for (int db = 0; db < 2; db++) dvt[db] = dkt[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ph = 0; ph < NPH; ph++) {
        delta(ph);
        __syncthreads();
        if (ph + 1 < NPH) load_rows(ph + 1);  // in flight during this phase's blocks
#pragma unroll
        for (int ii = 0; ii < RP / 16; ii++) {
            const int i = ph * (RP / 16) + ii;
            if (i + 1 < NQB) mask_load(mkn, i + 1);
            floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f}, dp = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int blk = 0; blk < 2; blk++) {
                const floatx4 a = *reinterpret_cast<const floatx4 *>(&Qs[(16 * i + t) * LDX + 16 * blk + 4 * kl]);
                const floatx4 ga = *reinterpret_cast<const floatx4 *>(&Gs[(16 * i + t) * LDX + 16 * blk + 4 * kl]);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    s = mfma4(a[u], kf[blk][u], s);
                    dp = mfma4(ga[u], vf[blk][u], dp);
                }
            }
            const floatx4 mq = *reinterpret_cast<const floatx4 *>(&St[0][16 * i + 4 * kl]);
            const floatx4 rq = *reinterpret_cast<const floatx4 *>(&St[1][16 * i + 4 * kl]);
            const floatx4 dl = *reinterpret_cast<const floatx4 *>(&St[2][16 * i + 4 * kl]);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = exp2_hw(__builtin_fmaf(s[r], c, mkc[r] * kLog2e) - mq[r]) * rq[r];
                s[r] = p;
                dp[r] = (p * (dp[r] - dl[r])) * scale;
                mkc[r] = mkn[r];
            }
            dsv[i] = dp;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int qq = 16 * i + 4 * kl + u;
                const float2 gv = *reinterpret_cast<const float2 *>(&Gs[qq * LDX + 2 * t]);
                const float2 qv = *reinterpret_cast<const float2 *>(&Qs[qq * LDX + 2 * t]);
                dvt[0] = mfma4(gv.x, s[u], dvt[0]);
                dvt[1] = mfma4(gv.y, s[u], dvt[1]);
                dkt[0] = mfma4(qv.x, dp[u], dkt[0]);
                dkt[1] = mfma4(qv.y, dp[u], dkt[1]);
            }
        }
        if (ph + 1 < NPH) {
            store_rows(ph + 1);  // rows no block of this phase reads
            __syncthreads();
        }
    }
    __syncthreads();  // every wavefront is done with Q and dO
    // 4. dS [query][key of this block] over Q and dO, then dQ for query blocks w, w + 4, ...
    float *dS = QG;
#pragma unroll
    for (int i = 0; i < NQB; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) dS[(16 * i + 4 * kl + r) * LDSC + 16 * w + t] = dsv[i][r];
    __syncthreads();
    if (dq) {
#pragma unroll
        for (int i = w; i < NQB; i += 4) {
            floatx4 qa[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int kb2 = 0; kb2 < 4; kb2++) {
                const floatx4 a = *reinterpret_cast<const floatx4 *>(&dS[(16 * i + t) * LDSC + 16 * kb2 + 4 * kl]);
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float2 kv = *reinterpret_cast<const float2 *>(&Ks[(16 * kb2 + 4 * kl + u) * LDX + 2 * t]);
                    qa[0] = mfma4(a[u], kv.x, qa[0]);
                    qa[1] = mfma4(a[u], kv.y, qa[1]);
                }
            }
            // rows 16 i + 4 kl + r, d = 2 t and 2 t + 1
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int qq = 16 * i + 4 * kl + r;
                const float2 val = make_float2(qa[0][r], qa[1][r]);
                if (dq_part) {
                    *reinterpret_cast<float2 *>(dq_part + ((int64_t)kb * gridDim.x / (L / kChunk) * L + bh * L + qq) *
                                                              D + 2 * t) = val;
                } else {
                    float2 *p = reinterpret_cast<float2 *>(dq + (row0 + qq) * ldd + h * D + 2 * t);
                    *p = acc ? make_float2(p->x + val.x, p->y + val.y) : val;
                }
            }
        }
    }
    // dV and dK rows of this lane's key: d = 8 kl + 2 r + db
    const int64_t orow = (row0 + mykey) * ldd + h * D + 8 * kl;
    floatx4 lo, hi;
    if (dv) {
        lo = floatx4{dvt[0][0], dvt[1][0], dvt[0][1], dvt[1][1]};
        hi = floatx4{dvt[0][2], dvt[1][2], dvt[0][3], dvt[1][3]};
        floatx4 *p = reinterpret_cast<floatx4 *>(dv + orow);
        p[0] = acc ? p[0] + lo : lo;
        p[1] = acc ? p[1] + hi : hi;
    }
    if (dk) {
        lo = floatx4{dkt[0][0], dkt[1][0], dkt[0][1], dkt[1][1]};
        hi = floatx4{dkt[0][2], dkt[1][2], dkt[0][3], dkt[1][3]};
        floatx4 *p = reinterpret_cast<floatx4 *>(dk + orow);
        p[0] = acc ? p[0] + lo : lo;
        p[1] = acc ? p[1] + hi : hi;
    }
}

// dq[b, l, h, :] (+)= the sum over key blocks 0, 1, ... of the partials, in that order: a thread per four floats.
template <int D>
__global__ void __launch_bounds__(256) k_flash_dq_reduce(const float *__restrict__ part, int nkb, int64_t rows,
                                                         float *dq, int ldd, int H, int L, int acc) {
    OM_LDS_POISON();
    constexpr int Q4 = D / 4;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * Q4) return;
    const int64_t row = idx / Q4;
    const int d = (int)(idx % Q4) * 4;
    floatx4 s = *reinterpret_cast<const floatx4 *>(part + row * D + d);
    for (int kb = 1; kb < nkb; kb++) s += *reinterpret_cast<const floatx4 *>(part + ((int64_t)kb * rows + row) * D + d);
    const int64_t bh = row / L, l = row % L, b = bh / H, h = bh % H;
    floatx4 *p = reinterpret_cast<floatx4 *>(dq + (b * L + l) * ldd + h * D + d);
    *p = acc ? *p + s : s;
}

bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Kernels for D = 32 and L = 64 or 128, where a workgroup holds whole rows. By default the whole-row forward with
// statistics (k_rows_fwd) and the streaming backward. Comparison runs (tuning builds, om::tuning_env):
// OM_ATTN_PATH=exact runs the pair of om_attention_fused.hip instead (the reference's exact softmax recompute, no
// statistics), OM_ATTN_PATH=stream the streaming forward too.
enum ShortPath { kRows, kExact, kStream };
ShortPath short_path() {
    static const ShortPath p = [] {
        const char *s = om::tuning_env("OM_ATTN_PATH");
        if (s && s[0] == 'e') return kExact;
        if (s && s[0] == 's') return kStream;
        return kRows;
    }();
    return p;
}
bool short_rows(int L, int d) { return d == 32 && (L == 64 || L == 128); }

// Shapes the statistics kernels take: D of 32 or 64, L a positive multiple of 64, 16-byte aligned rows.
bool flash_fwd_ok(const float *q, const float *k, const float *v, int ld, const float *mask, const float *o, int ldo,
                  int L, int d) {
    if (short_rows(L, d) && short_path() == kExact) return false;
    return (d == 32 || d == 64) && L >= kChunk && L % kChunk == 0 && ld % 4 == 0 && ldo % 4 == 0 && al16(q) &&
           al16(k) && al16(v) && al16(o) && al16(mask);
}

om_status check(om_ctx *ctx, const char *what, const void *q, const void *k, const void *v, const void *o,
                const void *stats, int B, int H, int L, int d, int ld, int ldo) {
    OM_REQUIRE(ctx, q && k && v && o && stats, "%s: NULL q/k/v/o/stats", what);
    OM_REQUIRE(ctx, B > 0 && H > 0 && L > 0 && d > 0 && d % 2 == 0,
               "%s: needs [B,L,H*D] tensors with positive sizes and even D, got B=%d H=%d L=%d D=%d", what, B, H, L,
               d);
    OM_REQUIRE(ctx, ld >= H * d && ldo >= H * d, "%s: row strides %d / %d below H*D = %d", what, ld, ldo, H * d);
    OM_REQUIRE(ctx, (int64_t)B * H * L <= INT32_MAX, "%s: too many rows", what);
    return OM_OK;
}

}  // namespace

extern "C" {

om_status om_attention_fwd_flash(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                 const float *mask, int mask_batched, float *o, int ld_o, float *stats, int B, int H,
                                 int L, int d, float scale) {
    OM_CHECK_CTX(ctx);
    om_status s = check(ctx, "om_attention_fwd_flash", q, k, v, o, stats, B, H, L, d, ld_qkv, ld_o);
    if (s) return s;
    if (!flash_fwd_ok(q, k, v, ld_qkv, mask, o, ld_o, L, d))
        return om_attention_fwd_fused(ctx, q, k, v, ld_qkv, mask, mask_batched, o, ld_o, B, H, L, d, scale);
    if (scale == 0.0f || scale != scale) scale = 1.0f / sqrtf((float)d);
    const int64_t mstride = (mask && mask_batched) ? (int64_t)L * L : 0;
    const int64_t n = (int64_t)B * H * L;
    const dim3 grid((unsigned)((int64_t)B * H * (L / kChunk)));
    const float c = scale * kLog2e;
    if (short_rows(L, d) && short_path() == kRows) {
        auto launch = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, o, ld_o, stats,
                               stats + n, H, c);
        };
        if (L == 128) mask ? launch(k_rows_fwd<32, 128, true>) : launch(k_rows_fwd<32, 128, false>);
        else mask ? launch(k_rows_fwd<32, 64, true>) : launch(k_rows_fwd<32, 64, false>);
    } else {
        auto launch = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, o, ld_o, stats,
                               stats + n, H, L, c);
        };
        if (d == 64) mask ? launch(k_flash_fwd<64, true>) : launch(k_flash_fwd<64, false>);
        else mask ? launch(k_flash_fwd<32, true>) : launch(k_flash_fwd<32, false>);
    }
    return OM_LAUNCH_CHECK(ctx, "om_attention_fwd_flash");
}

om_status om_attention_bwd_flash(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                 const float *mask, int mask_batched, const float *o, int ld_o, const float *stats,
                                 const float *g, int ld_g, float *dq, float *dk, float *dv, int ld_d, int B, int H,
                                 int L, int d, float scale, int acc) {
    OM_CHECK_CTX(ctx);
    om_status s = check(ctx, "om_attention_bwd_flash", q, k, v, o, stats, B, H, L, d, ld_qkv, ld_o);
    if (s) return s;
    OM_REQUIRE(ctx, g && ld_g >= H * d && ld_d >= H * d, "om_attention_bwd_flash: NULL gradient or short stride");
    if (!dq && !dk && !dv) return OM_OK;
    const bool ok = flash_fwd_ok(q, k, v, ld_qkv, mask, o, ld_o, L, d) && ld_g % 4 == 0 && ld_d % 4 == 0 && al16(g) &&
                    al16(dq) && al16(dk) && al16(dv);
    if (!ok)  // the forward took the same fallback (its conditions are part of these): recompute instead
        return om_attention_bwd_fused(ctx, q, k, v, ld_qkv, mask, mask_batched, g, ld_g, dq, dk, dv, ld_d, B, H, L,
                                      d, scale, acc);
    if (scale == 0.0f || scale != scale) scale = 1.0f / sqrtf((float)d);
    const int64_t mstride = (mask && mask_batched) ? (int64_t)L * L : 0;
    const int64_t n = (int64_t)B * H * L;
    const int nb = L / kChunk;
    const float c = scale * kLog2e;
    const dim3 grid((unsigned)((int64_t)B * H * nb));
    float *scr;
    if (short_rows(L, d) && short_path() == kRows) {
        float *part = nullptr;
        if (dq && nb > 1) {
            s = om::scratch2(ctx, sizeof(float) * (uint64_t)nb * n * d, &part);
            if (s) return s;
        }
        auto launch_bwd = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, g, ld_g, o, ld_o,
                               stats, stats + n, dk, dv, dq, ld_d, part, H, c, scale, acc);
        };
        if (L == 128)
            mask ? launch_bwd(k_rows_bwd<128, true>) : launch_bwd(k_rows_bwd<128, false>);
        else
            mask ? launch_bwd(k_rows_bwd<64, true>) : launch_bwd(k_rows_bwd<64, false>);
        if (part)
            hipLaunchKernelGGL(k_flash_dq_reduce<32>, dim3((unsigned)((n * 8 + 255) / 256)), dim3(256), 0,
                               ctx->stream, part, nb, n, dq, ld_d, H, L, acc);
        return OM_LAUNCH_CHECK(ctx, "om_attention_bwd_flash");
    }
    const uint64_t part_floats = dq ? (uint64_t)nb * n * d : 0;
    s = om::scratch2(ctx, sizeof(float) * ((uint64_t)n + 64 + part_floats), &scr);
    if (s) return s;
    float *delta = scr, *part = dq ? scr + ((n + 63) / 64) * 64 : nullptr;
    const unsigned rows_grid = (unsigned)((n * 16 + 255) / 256);
    auto launch_flash_bwd = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, g, ld_g, stats,
                           stats + n, delta, dk, dv, ld_d, part, H, L, c, scale, acc);
    };
    if (d == 64) {
        hipLaunchKernelGGL(k_flash_delta<64>, dim3(rows_grid), dim3(256), 0, ctx->stream, g, ld_g, o, ld_o, delta, H,
                           L, n);
        mask ? launch_flash_bwd(k_flash_bwd<64, true>) : launch_flash_bwd(k_flash_bwd<64, false>);
        if (dq)
            hipLaunchKernelGGL(k_flash_dq_reduce<64>, dim3((unsigned)((n * 16 + 255) / 256)), dim3(256), 0,
                               ctx->stream, part, nb, n, dq, ld_d, H, L, acc);
    } else {
        hipLaunchKernelGGL(k_flash_delta<32>, dim3(rows_grid), dim3(256), 0, ctx->stream, g, ld_g, o, ld_o, delta, H,
                           L, n);
        mask ? launch_flash_bwd(k_flash_bwd<32, true>) : launch_flash_bwd(k_flash_bwd<32, false>);
        if (dq)
            hipLaunchKernelGGL(k_flash_dq_reduce<32>, dim3((unsigned)((n * 8 + 255) / 256)), dim3(256), 0,
                               ctx->stream, part, nb, n, dq, ld_d, H, L, acc);
    }
    return OM_LAUNCH_CHECK(ctx, "om_attention_bwd_flash");
}

}  // extern "C"
