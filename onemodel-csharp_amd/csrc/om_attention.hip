// Scaled dot-product attention forward and backward on the MFMA GEMM engine (Ops.Attention, Ops.Layers.cs:746-807;
// AttentionBackward, BackwardNn.cs:636-701).
//
// q/o are [B, Lq, H, D] and k/v [B, Lk, H, D]: the Linear outputs with heads interleaved. The reference splits heads
// with Reshape + Permute views and copies them contiguous before its kernel; here the per-head matrices are addressed
// in place (row stride H*D, head offset h*D), so neither direction needs a permute copy. Batch item z = b*H + h.
//
// Forward: S = scale * Q K^T + mask (GEMM epilogue) -> P = softmax rows in place (exact flavour) -> O = P V.
// P [B, H, Lq, Lk] is kept for the backward (the reference recomputes it; 288 GB of HBM makes keeping it cheap).
// Backward: dV = P^T dO, dP = dO V^T, dS = P (dP - rowsum(dP P)) scale, dQ = dS K, dK = dS^T Q.
#include "om_gemm.hpp"

om_status om_internal_attn_ds(om_ctx *ctx, float *dp, const float *p, int rows, int cols, float scale);
om_status om_internal_softmax_rows(om_ctx *ctx, float *x, int rows, int cols);

namespace {

// Per-head view of a [B, L, (H, D)] tensor whose rows are `ld` floats apart (ld = H*D for a plain Linear output,
// 3*H*D for a packed q|k|v projection) as batch item z = b*H + h.
void head_view(omg::Params &p, int which, const float *base, int L, int D, int64_t ld) {
    int64_t outer = (int64_t)L * ld, inner = D;
    if (which == 0) {
        p.a = base;
        p.lda = ld;
        p.sa_outer = outer;
        p.sa_inner = inner;
    } else {
        p.b = base;
        p.ldb = ld;
        p.sb_outer = outer;
        p.sb_inner = inner;
    }
}
// Per-head view of a [B, H, Lq, Lk] score tensor.
void score_view(omg::Params &p, int which, const float *base, int H, int lq, int lk) {
    int64_t outer = (int64_t)H * lq * lk, inner = (int64_t)lq * lk;
    if (which == 0) {
        p.a = base;
        p.lda = lk;
        p.sa_outer = outer;
        p.sa_inner = inner;
    } else {
        p.b = base;
        p.ldb = lk;
        p.sb_outer = outer;
        p.sb_inner = inner;
    }
}

om_status check(om_ctx *ctx, const char *what, const void *q, const void *k, const void *v, int B, int H, int lq,
                int lk, int d) {
    OM_REQUIRE(ctx, q && k && v, "%s: NULL q/k/v", what);
    OM_REQUIRE(ctx, B > 0 && H > 0 && lq > 0 && lk > 0 && d > 0 && d % 2 == 0,
               "%s: needs [B,L,H,D] tensors with positive sizes and even D, got B=%d H=%d Lq=%d Lk=%d D=%d", what, B,
               H, lq, lk, d);
    OM_REQUIRE(ctx, (int64_t)B * H * lq <= INT32_MAX && (int64_t)B * H <= INT32_MAX, "%s: too many rows", what);
    return OM_OK;
}

}  // namespace

extern "C" {

om_status om_attention_fwd_ld(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                              const float *mask, int mask_batched, float *o, int ld_o, float *p, int B, int H, int lq,
                              int lk, int d, float scale) {
    OM_CHECK_CTX(ctx);
    om_status s = check(ctx, "om_attention_fwd", q, k, v, B, H, lq, lk, d);
    if (s) return s;
    OM_REQUIRE(ctx, o && p, "om_attention_fwd: NULL output or weights buffer");
    OM_REQUIRE(ctx, ld_qkv >= H * d && ld_o >= H * d, "om_attention_fwd: row strides %d / %d below H*D = %d", ld_qkv,
               ld_o, H * d);
    if (scale == 0.0f || scale != scale) scale = 1.0f / sqrtf((float)d);
    // S = scale * Q K^T + mask  -> p
    omg::Params ps = omg::dense_params(lq, lk, d, nullptr, 0, nullptr, 0, p, lk);
    ps.batch_div = H;
    head_view(ps, 0, q, lq, d, ld_qkv);
    head_view(ps, 1, k, lk, d, ld_qkv);
    ps.sc_outer = (int64_t)H * lq * lk;
    ps.sc_inner = (int64_t)lq * lk;
    ps.alpha = scale;
    ps.mask = mask;
    ps.mask_outer_stride = (mask && mask_batched) ? (int64_t)lq * lk : 0;
    s = omg::launch_dense(ctx, ps, false, true, B * H, "attention scores");
    if (s) return s;
    s = om_internal_softmax_rows(ctx, p, B * H * lq, lk);
    if (s) return s;
    // O = P V -> o in [B, Lq, H, D] rows of stride ld_o
    omg::Params po = omg::dense_params(lq, d, lk, nullptr, 0, nullptr, 0, o, ld_o);
    po.batch_div = H;
    score_view(po, 0, p, H, lq, lk);
    head_view(po, 1, v, lk, d, ld_qkv);
    po.sc_outer = (int64_t)lq * ld_o;
    po.sc_inner = d;
    return omg::launch_dense(ctx, po, false, false, B * H, "attention output");
}

om_status om_attention_fwd(om_ctx *ctx, const float *q, const float *k, const float *v, const float *mask,
                           int mask_batched, float *o, float *p, int B, int H, int lq, int lk, int d, float scale) {
    return om_attention_fwd_ld(ctx, q, k, v, H * d, mask, mask_batched, o, H * d, p, B, H, lq, lk, d, scale);
}

om_status om_attention_bwd_ld(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                              const float *p, const float *g, int ld_g, float *dq, float *dk, float *dv, int ld_d,
                              float *ds, int B, int H, int lq, int lk, int d, float scale, int acc) {
    OM_CHECK_CTX(ctx);
    om_status s = check(ctx, "om_attention_bwd", q, k, v, B, H, lq, lk, d);
    if (s) return s;
    OM_REQUIRE(ctx, p && g && ds, "om_attention_bwd: NULL weights, gradient or scratch");
    OM_REQUIRE(ctx, ld_qkv >= H * d && ld_g >= H * d && ld_d >= H * d,
               "om_attention_bwd: row strides %d / %d / %d below H*D = %d", ld_qkv, ld_g, ld_d, H * d);
    if (scale == 0.0f || scale != scale) scale = 1.0f / sqrtf((float)d);
    const int Z = B * H;
    if (dv) {  // dV = P^T dO : [Lk, D] = [Lq, Lk]^T [Lq, D]
        omg::Params pv = omg::dense_params(lk, d, lq, nullptr, 0, nullptr, 0, dv, ld_d);
        pv.batch_div = H;
        score_view(pv, 0, p, H, lq, lk);
        head_view(pv, 1, g, lq, d, ld_g);
        pv.sc_outer = (int64_t)lk * ld_d;
        pv.sc_inner = d;
        pv.accumulate = acc;
        s = omg::launch_dense(ctx, pv, true, false, Z, "attention dV");
        if (s) return s;
    }
    if (!dq && !dk) return OM_OK;
    {  // dP = dO V^T : [Lq, Lk] -> ds
        omg::Params pp = omg::dense_params(lq, lk, d, nullptr, 0, nullptr, 0, ds, lk);
        pp.batch_div = H;
        head_view(pp, 0, g, lq, d, ld_g);
        head_view(pp, 1, v, lk, d, ld_qkv);
        pp.sc_outer = (int64_t)H * lq * lk;
        pp.sc_inner = (int64_t)lq * lk;
        s = omg::launch_dense(ctx, pp, false, true, Z, "attention dP");
        if (s) return s;
    }
    s = om_internal_attn_ds(ctx, ds, p, Z * lq, lk, scale);
    if (s) return s;
    if (dq) {  // dQ = dS K : [Lq, D] = [Lq, Lk] [Lk, D]
        omg::Params pq = omg::dense_params(lq, d, lk, nullptr, 0, nullptr, 0, dq, ld_d);
        pq.batch_div = H;
        score_view(pq, 0, ds, H, lq, lk);
        head_view(pq, 1, k, lk, d, ld_qkv);
        pq.sc_outer = (int64_t)lq * ld_d;
        pq.sc_inner = d;
        pq.accumulate = acc;
        s = omg::launch_dense(ctx, pq, false, false, Z, "attention dQ");
        if (s) return s;
    }
    if (dk) {  // dK = dS^T Q : [Lk, D] = [Lq, Lk]^T [Lq, D]
        omg::Params pk = omg::dense_params(lk, d, lq, nullptr, 0, nullptr, 0, dk, ld_d);
        pk.batch_div = H;
        score_view(pk, 0, ds, H, lq, lk);
        head_view(pk, 1, q, lq, d, ld_qkv);
        pk.sc_outer = (int64_t)lk * ld_d;
        pk.sc_inner = d;
        pk.accumulate = acc;
        s = omg::launch_dense(ctx, pk, true, false, Z, "attention dK");
        if (s) return s;
    }
    return OM_OK;
}

om_status om_attention_bwd(om_ctx *ctx, const float *q, const float *k, const float *v, const float *p,
                           const float *g, float *dq, float *dk, float *dv, float *ds, int B, int H, int lq, int lk,
                           int d, float scale, int acc) {
    return om_attention_bwd_ld(ctx, q, k, v, H * d, p, g, H * d, dq, dk, dv, H * d, ds, B, H, lq, lk, d, scale, acc);
}

}  // extern "C"
