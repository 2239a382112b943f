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

template <int D>
__global__ void __launch_bounds__(256) k_flash_fwd(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, int ld, const float *__restrict__ mask,
                                                   int64_t mask_bstride, float *__restrict__ o, int ldo,
                                                   float *__restrict__ stat_m, float *__restrict__ stat_r, int H,
                                                   int L, float c) {
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
            if (mrow) mk = *reinterpret_cast<const floatx4 *>(mrow + kc * kChunk + 16 * j);
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

// delta[(b H + h) L + l] = (float) sum over d, in double, of dO * O for every query row (16 lanes per row).
template <int D>
__global__ void __launch_bounds__(256) k_flash_delta(const float *__restrict__ g, int ldg, const float *__restrict__ o,
                                                     int ldo, float *__restrict__ delta, int H, int L, int64_t rows) {
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

template <int D>
__global__ void __launch_bounds__(256, 2) k_flash_bwd(const float *__restrict__ q, const float *__restrict__ k,
                                                   const float *__restrict__ v, int ld, const float *__restrict__ mask,
                                                   int64_t mask_bstride, const float *__restrict__ g, int ldg,
                                                   const float *__restrict__ stat_m, const float *__restrict__ stat_r,
                                                   const float *__restrict__ delta, float *dk, float *dv, int ldd,
                                                   float *__restrict__ dq_part, int H, int L, float c, float scale,
                                                   int acc) {
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
                const float mk = mbase ? mbase[(int64_t)(qc * kChunk + qq) * L] * kLog2e : 0.0f;
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

// dq[b, l, h, :] (+)= the sum over key blocks 0, 1, ... of the partials, in that order: a thread per four floats.
template <int D>
__global__ void __launch_bounds__(256) k_flash_dq_reduce(const float *__restrict__ part, int nkb, int64_t rows,
                                                         float *dq, int ldd, int H, int L, int acc) {
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

// Comparison runs: OM_ATTN_FLASH=1 sends the shapes the whole-row kernels of om_attention_fused.hip take (D = 32,
// L <= 128) through the streaming kernels too.
bool force_flash() {
    static const char *s = std::getenv("OM_ATTN_FLASH");
    return s && s[0] == '1';
}

// Shapes the streaming kernels take: D of 32 or 64, L a positive multiple of 64, 16-byte aligned rows; D = 32 with
// L <= 128 goes to the whole-row kernels.
bool flash_fwd_ok(const float *q, const float *k, const float *v, int ld, const float *mask, const float *o, int ldo,
                  int L, int d) {
    if (d == 32 && L <= 128 && !force_flash()) return false;
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
    if (d == 64)
        hipLaunchKernelGGL(k_flash_fwd<64>, grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, o, ld_o,
                           stats, stats + n, H, L, c);
    else
        hipLaunchKernelGGL(k_flash_fwd<32>, grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, o, ld_o,
                           stats, stats + n, H, L, c);
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
    float *scr;
    const uint64_t part_floats = dq ? (uint64_t)nb * n * d : 0;
    s = om::scratch2(ctx, sizeof(float) * ((uint64_t)n + 64 + part_floats), &scr);
    if (s) return s;
    float *delta = scr, *part = dq ? scr + ((n + 63) / 64) * 64 : nullptr;
    const unsigned rows_grid = (unsigned)((n * 16 + 255) / 256);
    const dim3 grid((unsigned)((int64_t)B * H * nb));
    const float c = scale * kLog2e;
    if (d == 64) {
        hipLaunchKernelGGL(k_flash_delta<64>, dim3(rows_grid), dim3(256), 0, ctx->stream, g, ld_g, o, ld_o, delta, H,
                           L, n);
        hipLaunchKernelGGL(k_flash_bwd<64>, grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, g, ld_g,
                           stats, stats + n, delta, dk, dv, ld_d, part, H, L, c, scale, acc);
        if (dq)
            hipLaunchKernelGGL(k_flash_dq_reduce<64>, dim3((unsigned)((n * 16 + 255) / 256)), dim3(256), 0,
                               ctx->stream, part, nb, n, dq, ld_d, H, L, acc);
    } else {
        hipLaunchKernelGGL(k_flash_delta<32>, dim3(rows_grid), dim3(256), 0, ctx->stream, g, ld_g, o, ld_o, delta, H,
                           L, n);
        hipLaunchKernelGGL(k_flash_bwd<32>, grid, dim3(256), 0, ctx->stream, q, k, v, ld_qkv, mask, mstride, g, ld_g,
                           stats, stats + n, delta, dk, dv, ld_d, part, H, L, c, scale, acc);
        if (dq)
            hipLaunchKernelGGL(k_flash_dq_reduce<32>, dim3((unsigned)((n * 8 + 255) / 256)), dim3(256), 0,
                               ctx->stream, part, nb, n, dq, ld_d, H, L, acc);
    }
    return OM_LAUNCH_CHECK(ctx, "om_attention_bwd_flash");
}

}  // extern "C"
