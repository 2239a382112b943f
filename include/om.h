/*
 * om.h — C ABI of libom_hip.so, the MI355X (gfx950) kernels of the OneModel training path.
 *
 * This is the boundary a host tape binds (the reference's C# tape through [LibraryImport], or this repository's C++
 * tape in onemodel-csharp_amd/train). Every entry point:
 *   - takes plain device pointers (float*, int32_t*) and sizes; no C++ or framework types cross the ABI;
 *   - is asynchronous on the context's HIP stream; only om_download, om_readback_wait and om_ctx_sync block;
 *   - returns om_status (OM_OK = 0) and leaves a message in om_last_error(ctx) on failure;
 *   - validates shapes and pointers on the host before launching, so a kernel never sees a shape it does not handle;
 *   - is deterministic: tiling, split-K and reduction orders depend only on the shape.
 * Arithmetic follows the reference's CPU training path (fp32 tensors, fp64 where the reference sums in double) within
 * 1e-5 scaled error; integer work (labels, pool indices, CTC alignment) is bit-exact, and so is the optimizer step
 * given the same gradient.
 *
 * Citations name the reference function (recursive-ai-oss/onemodel-csharp, file:line) each entry point replaces.
 */
#ifndef OM_H
#define OM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t om_status;
enum {
    OM_OK = 0,
    OM_E_ARG = 1,    /* bad shape, size or pointer: the reference's TensorShapeException / ArgumentException */
    OM_E_OOM = 2,    /* the arena or the device is out of memory */
    OM_E_DEVICE = 3, /* a HIP runtime error */
    OM_E_STATE = 4   /* the call is not valid in the context's current state (InvalidOperationException) */
};

typedef struct om_ctx om_ctx;

/* ---------------------------------------------------------------------------------------------- context */
/* One context per host thread and device; it owns one HIP stream and the arena. */
om_status om_ctx_create(int device, om_ctx **out);
om_status om_ctx_destroy(om_ctx *ctx);
om_status om_ctx_sync(om_ctx *ctx);
const char *om_last_error(om_ctx *ctx);
/* The context's hipStream_t, for callers that time or order work around the library's launches. */
void *om_ctx_stream(om_ctx *ctx);
/* Launch timing probe (measurement; no counterpart in the reference, for callers that report how long the parameter
 * gradients take inside real steps): while on, every om_param_grads_group call (and so om_linear_bwd_dw_group)
 * records a HIP event on the context's stream before its first launch and one after its last (at most 1024 calls per
 * series; none while a step graph is captured). om_ctx_probe(ctx, 1) starts a new series, om_ctx_probe(ctx, 0) stops
 * recording; om_ctx_probe_read waits for the stream and gives the number of calls recorded and their mean duration in
 * milliseconds (0 when there are none). */
om_status om_ctx_probe(om_ctx *ctx, int on);
om_status om_ctx_probe_read(om_ctx *ctx, int *calls, double *mean_ms);
/* How the GELU epilogues of products (om_linear_gelu_fwd, om_linear_gelu_fwd_slope, om_linear_bwd_dx_gelu) evaluate
 * erf and exp. OM_GELU_FAST (the default): erfc from the degree-9 Chebyshev fit of Numerical Recipes' erfcc
 * (fractional error below 1.2e-7) with the hardware reciprocal and exponential; GELU within 1.2e-7 max(1, |x|) of
 * the exact value and its slope within 2.2e-7, about 35 vector instructions per element, which lets the wide tiles
 * of the plain products carry the epilogue. OM_GELU_REFERENCE: the reference's polynomials (Transcendental.GeluErf,
 * Transcendental.cs:252; GeluGradBin, TrainElementwise.cs:59-85), bit for bit, about 180 instructions per element.
 * om_gelu_fwd and om_gelu_bwd follow the same mode. A step graph records the mode in force when it was captured. No
 * counterpart in the reference (whose GELU is the polynomial in both of its modes). */
enum { OM_GELU_FAST = 0, OM_GELU_REFERENCE = 1 };
om_status om_ctx_set_gelu(om_ctx *ctx, int mode);
/* Version of this ABI (major * 100 + minor). */
int om_abi_version(void);
/* 1 for a checked build (compiled with -DOM_CHECKED: every kernel's LDS, every om_alloc allocation and the context
 * scratch handed out filled with 0xFF bytes, a NaN for floats, so results computed from memory nothing wrote turn
 * into NaN; the reference's Checked configuration, BufferPool.cs:21-22), 0 for the product build. */
int om_build_checked(void);

/* ---------------------------------------------------------------------------------------------- arena */
/* Device memory in two regions, in the spirit of the reference's buffer lifetimes (ActivationScope.cs:18-106,
 * BufferPool.cs:26-161): PERSISTENT holds parameters, gradients and optimizer moments for the life of the context;
 * STEP holds a step's activations and temporary gradients and is rewound by om_step_reset at the step edge
 * (the ActivationScope.Dispose equivalent). Allocations are 256-byte aligned bump allocations; a step that outgrows
 * its slab chains another slab, so addresses handed out stay valid until the reset. */
enum { OM_REGION_PERSISTENT = 0, OM_REGION_STEP = 1 };
om_status om_arena_reserve(om_ctx *ctx, uint64_t persistent_bytes, uint64_t step_bytes);
om_status om_alloc(om_ctx *ctx, int region, uint64_t bytes, void **out);
om_status om_step_reset(om_ctx *ctx);
/* Bytes in use and reserved, per region. */
om_status om_arena_stats(om_ctx *ctx, int region, uint64_t *used, uint64_t *reserved);
/* Fault injection for callers' out-of-memory handling (no counterpart in the reference): from now on om_alloc in
 * `region` fails with OM_E_OOM, as if the device were full, when the bytes handed out since the region's last reset
 * (the step region: om_step_reset) would exceed `bytes`; 0 removes the limit. Nothing else changes. */
om_status om_arena_set_limit(om_ctx *ctx, int region, uint64_t bytes);
/* Host<->device copies at step edges (a region is the unit of transfer, ExecutionBackend.cs:8-13). */
om_status om_upload(om_ctx *ctx, void *dst_device, const void *src_host, uint64_t bytes);
om_status om_download(om_ctx *ctx, void *dst_host, const void *src_device, uint64_t bytes);
om_status om_copy(om_ctx *ctx, void *dst_device, const void *src_device, uint64_t bytes);
/* dst = 0 (Backprop.ZeroGrad, Engine.cs:77-91); a fill kernel, so it is safe inside a captured graph. */
om_status om_zero(om_ctx *ctx, void *dst_device, uint64_t bytes);
om_status om_fill(om_ctx *ctx, float *dst, float value, int64_t n);

/* ---------------------------------------------------------------------------------------------- staging */
/* Host data staging for the per-step batches a DataLoader builds (DataLoader.cs:35-90, Batching.cs:129-200 produce
 * them on the host): a ring of `slots` slots, each a pinned host buffer and a device buffer of slot_bytes, and a
 * copy stream of default priority. The producer writes a batch straight into the pinned buffer that
 * om_stager_begin returns (it waits for that buffer's previous upload to have read it), om_stager_commit queues the
 * upload behind the previous use of the slot's device buffer and returns the device address, om_stager_acquire
 * makes the context's stream wait for the upload before the step's launches, and om_stager_release, after the
 * step's last launch, frees the device buffer for the slot's next upload. The upload of batch k+1 thus runs under
 * step k. A slot can be begun again only after its batch was released (OM_E_STATE otherwise). No counterpart in
 * the reference's CPU path, whose batches are used where they are built. */
typedef struct om_stager om_stager;
om_status om_stager_create(om_ctx *ctx, uint64_t slot_bytes, int slots, om_stager **out);
om_status om_stager_destroy(om_stager *s);
uint64_t om_stager_slot_bytes(const om_stager *s);
om_status om_stager_begin(om_stager *s, void **host, int *slot);
om_status om_stager_commit(om_stager *s, int slot, uint64_t bytes, void **device);
om_status om_stager_acquire(om_stager *s, int slot);
om_status om_stager_release(om_stager *s, int slot);

/* Readback of a small device value (a step's loss) without waiting for the rest of the stream: om_readback_post
 * queues a copy of `bytes` (at most 64 KiB) from device memory into a pinned host buffer, a one-workgroup kernel on
 * the context's stream writing through the buffer's device mapping and then a sequence number, ordered after the
 * work already queued there; om_readback_wait polls that number, so it blocks
 * only until the copy has landed (and reports a stream error meanwhile), then copies the value to dst. Launches queued between the two keep the device busy while the host
 * returns with the value. No counterpart in the reference's CPU path, where the loss is a host float as soon as the
 * forward has run: its training step reads it there, before Backward and Step (TrainCase.cs:117-127). */
typedef struct om_readback om_readback;
om_status om_readback_create(om_ctx *ctx, uint64_t bytes, om_readback **out);
om_status om_readback_destroy(om_readback *r);
om_status om_readback_post(om_readback *r, const void *src_device, uint64_t bytes);
om_status om_readback_wait(om_readback *r, void *dst_host, uint64_t bytes);

/* ---------------------------------------------------------------------------------------------- step graphs */
/* A training step as one HIP graph: between om_graph_capture_begin and om_graph_capture_end the launches a caller
 * queues on the context's stream are recorded instead of run, and om_graph_launch replays them as one submission
 * (a step of small launches is bound by the host's per-launch cost otherwise).
 * Recorded launches keep the arguments they were recorded with (pointers, sizes, flags), except the values that
 * change from step to step, which the graph's kernels read from device memory that the graph's first node fills
 * from the om_step_values given to each om_graph_launch: the rate and Adam's two bias-correction scalars of
 * om_adam_step / om_adam_step_scaled (their by-value lr, step_size and sqrt_bc2 are ignored inside a capture, and
 * 1 - lr * weight_decay is formed on the device with the same float rounding), and the sequence number of the
 * capture's one readback post (om_readback_post, om_mse_fwd_post or om_xent_fwd_unit; om_graph_launch advances the readback as a
 * post would, so om_readback_wait works as after an eager post). A caller captures again whenever anything else
 * it passed would change.
 * Inside a capture, calls that would wait for the device or read host memory when the graph runs fail with
 * OM_E_STATE and leave the capture unusable (abort it): om_upload, om_download, om_ctx_sync, om_sgd_step (its rate
 * and first-step flag are host values), the stager calls, a second readback object, and growth of the context's
 * scratch (run one step outside a capture first, so scratch and arena have their steady size).
 * om_graph_launch waits, if need be, until the previous launch of the same graph has read its values.
 * No counterpart in the reference, whose step runs on the CPU (TrainCase.cs:114-127). */
typedef struct om_graph om_graph;
typedef struct {
    float lr, step_size, sqrt_bc2; /* as passed to om_adam_step for the step (om_adam_scalars) */
} om_step_values;
om_status om_graph_capture_begin(om_ctx *ctx);
om_status om_graph_capture_end(om_ctx *ctx, om_graph **out);
/* Ends a capture without a graph (after a failed call inside it); the stream runs launches again. */
om_status om_graph_capture_abort(om_ctx *ctx);
om_status om_graph_launch(om_graph *g, const om_step_values *v);
/* Waits for the graph's launches, then frees it. */
om_status om_graph_destroy(om_graph *g);

/* ---------------------------------------------------------------------------------------------- GEMM */
/* C[m,n] = op(A)[m,k] * op(B)[k,n] (+ bias[n]) on fp32 MFMA, for `batch` independent products. Row-major operands
 * with leading dimensions lda/ldb/ldc; trans_a means A is stored [k,m], trans_b means B is stored [n,k].
 * accumulate != 0 adds the product into C (C = C + AB, one rounding of the finished dot product), the leaf
 * accumulation of Engine.AccumulateLeaf (Engine.cs:292-328). Replaces Dense.Gemm / Kernels.Gemm.Run
 * (Dense.cs:12-49, Gemm.cs:48). Batch item z reads A at a + (z / batch_div) * sa_outer + (z % batch_div) * sa_inner
 * (likewise B, C), which addresses heads inside [batch, seq, heads, dim] activations without a permute copy. */
typedef struct {
    int32_t batch, batch_div;
    int64_t sa_outer, sa_inner, sb_outer, sb_inner, sc_outer, sc_inner;
} om_batch;
om_status om_gemm(om_ctx *ctx, int trans_a, int trans_b, int m, int n, int k, const float *a, int lda,
                  const float *b, int ldb, float *c, int ldc, const float *bias, int accumulate,
                  const om_batch *batch);

/* ---------------------------------------------------------------------------------------------- dense layers */
/* Ops.Linear forward (Ops.Layers.cs:715-733): y[rows,out] = x[rows,in] * w[out,in]^T + b[out] (b may be NULL). */
om_status om_linear_fwd(om_ctx *ctx, const float *x, const float *w, const float *b, float *y, int rows, int in,
                        int out);
/* 1 when om_linear_fwd / om_linear_bwd take their one-launch path for this shape (rows <= 256, out <= 32,
 * rows * in * out <= 2^21: a classifier head over a small batch, whose time is launch latency): the forward is one
 * launch, and om_linear_bwd computes dx, dw and db together in one launch, each output a single fmaf chain in
 * increasing k (the reference fast-mode Dense.Gemm's accumulation order) and db a double sum in increasing row. A
 * caller that groups weight gradients (om_linear_bwd_dw_group) should pass such layers to om_linear_bwd instead. */
int om_linear_small(int rows, int in, int out);
/* Linear backward = MatMul backward + Permute backward + bias SumTo (BackwardOps.cs:69-82, 107-118, 201-269):
 * dx = g w, dw = g^T x written directly as [out,in], db = fp64 column sums of g (computed inside the dW launch when
 * both are requested and the tile allows it). Each output pointer may be NULL; the acc_* flags add into the
 * destination instead of overwriting it (leaf accumulation). */
om_status om_linear_bwd(om_ctx *ctx, const float *g, const float *x, const float *w, float *dx, float *dw, float *db,
                        int rows, int in, int out, int acc_dx, int acc_dw, int acc_db);
/* Linear's input gradient plus a residual's gradient arriving at the same tensor (a post-LN block's sub-layer input,
 * which is also its residual): dx = (g w) + r, the bits of om_linear_bwd's dx followed by om_axpy(1, r, dx), with the
 * add in the product's epilogue. No counterpart as one call. */
om_status om_linear_bwd_dx_resid(om_ctx *ctx, const float *g, const float *w, const float *r, float *dx, int rows,
                                 int in, int out);
/* Linear followed by the residual Add of an encoder block (Ops.Layers.cs:715-733, then Ops.Add, Ops.cs:15-56):
 * y = resid + (x w^T + b), in that rounding order, in one launch. */
om_status om_linear_fwd_resid(om_ctx *ctx, const float *x, const float *w, const float *b, const float *resid,
                              float *y, int rows, int in, int out);
/* Linear followed by ReLU (Ops.Layers.cs:715-733, then Ops.Relu): y = relu(x w^T + b), bit for bit om_linear_fwd then
 * om_relu_fwd, with the ReLU applied in the product's epilogue (the one-launch small layers run the two launches).
 * No counterpart as one call; the ReLU's backward reads y. */
om_status om_linear_relu_fwd(om_ctx *ctx, const float *x, const float *w, const float *b, float *y, int rows, int in,
                             int out);
/* Its backward: the ReLU's rule (om_relu_bwd: g where y > 0, y the saved output) and then om_linear_bwd on that
 * gradient, with om_linear_bwd's arguments and accumulate flags. For a small batch whose product takes one launch,
 * dW and db without dx are one launch with the rule applied to g as it is read (the same values). */
om_status om_linear_relu_bwd(om_ctx *ctx, const float *g, const float *y, const float *x, const float *w, float *dx,
                             float *dw, float *db, int rows, int in, int out, int acc_dx, int acc_dw, int acc_db);
/* Linear followed by GELU (erf form, Ops.Nn.cs:86-112) in one launch: h = x w^T + b (the pre-activation GELU's
 * backward reads) and a = gelu(h), both [rows, out]. */
om_status om_linear_gelu_fwd(om_ctx *ctx, const float *x, const float *w, const float *b, float *h, float *a, int rows,
                             int in, int out);
/* The input gradient of Linear(GELU(h)) with respect to h in one launch: dh = GeluGradBin(g w, h)
 * (MatMul backward BackwardOps.cs:69-82, then GELU backward BackwardNn.cs:12-14); g is [rows, out], w [out, in],
 * h and dh [rows, in]. */
om_status om_linear_bwd_dx_gelu(om_ctx *ctx, const float *g, const float *w, const float *h, float *dh, int rows,
                                int in, int out);
/* The same pair with GELU's slope saved in place of the pre-activation: the forward writes a = gelu(h) and
 * s = 0.5 (1 + erf(h/sqrt2)) + h exp(-h^2/2) / sqrt(2 pi) (the factor GeluGradBin multiplies by, TrainElementwise.cs:
 * 59-85, rounded as there) from one erf evaluation; the backward is then dh = (g w) * s, bit for bit the
 * om_linear_bwd_dx_gelu result, with no transcendental left in its epilogue. a and s are [rows, out]. */
om_status om_linear_gelu_fwd_slope(om_ctx *ctx, const float *x, const float *w, const float *b, float *a, float *s,
                                   int rows, int in, int out);
om_status om_linear_bwd_dx_slope(om_ctx *ctx, const float *g, const float *w, const float *s, float *dh, int rows,
                                 int in, int out);
/* Weight (and bias) gradients of several Linear layers whose inputs share the row count, in one launch: item i gets
 * dw_i (+)= g_i^T x_i ([out_i, in_i], g_i [rows, out_i], x_i [rows, in_i]) and db_i (+)= fp64 column sums of g_i,
 * the MatMul and SumTo rules of om_linear_bwd (BackwardOps.cs:69-82, 201-269). Up to four items whose sizes are
 * multiples of 64 share one tile-exact launch and one split-K reduce (their tiles fill the device together instead
 * of each launch ramping up and down alone); other calls run the items one by one through om_linear_bwd. Either
 * way each item's result is a GEMM of the library within its tolerance; the grouped launch fixes its tile and split
 * from the group, so its bits may differ from a lone om_linear_bwd of the same item. dw or db may be NULL. */
typedef struct {
    const float *g;
    const float *x;
    float *dw;
    float *db;
    int32_t in, out, acc_dw, acc_db;
} om_linear_dw;
om_status om_linear_bwd_dw_group(om_ctx *ctx, int count, const om_linear_dw *items, int rows);
/* Two-stage column sums finished later: out[c] (+)= (float) of the fp64 sum over k < chunks of part[k * cols + c]
 * (lanes add every 64th chunk in increasing order, then a fixed butterfly: om_layernorm_bwd's own final order). */
typedef struct {
    const double *part;
    float *out;
    int32_t chunks, cols, acc;
} om_column_sum;
/* All parameter gradients a backward pass leaves to the end in one go: the Linear weight gradients of
 * om_linear_bwd_dw_group and up to 8 column sums (the dgamma/dbeta partials of om_layernorm_bwd_partials), the
 * column sums riding in the weight gradients' reduce launch. */
om_status om_param_grads_group(om_ctx *ctx, int n_dw, const om_linear_dw *dw, int rows, int n_cs,
                               const om_column_sum *cs);
/* Bias gradient alone: db[n] (+)= (float) sum over rows of g[row, n] in double (BackwardOps.SumTo). */
om_status om_colsum(om_ctx *ctx, const float *g, float *db, int rows, int cols, int accumulate);

/* ---------------------------------------------------------------------------------------------- elementwise */
/* ReluUn / ReluGradBin (TrainElementwise.cs:41-45, 93-98; Ops.cs:94-107; BackwardOps.cs:66-68). */
/* The CRNN's sequence head (Mean over axis 2 of x [B, C, H, W], then Permute(2, 0, 1)): y [W, B, C] bit for bit
 * om_mean_axis then om_permute, in one launch; the backward dx [B, C, H, W] (+)= g[w][b][c] / H, the bits of the
 * permute's and the mean's backward in turn. No counterpart as one call. */
om_status om_mean_permute_fwd(om_ctx *ctx, const float *x, float *y, int B, int C, int H, int W);
om_status om_mean_permute_bwd(om_ctx *ctx, const float *g, float *dx, int B, int C, int H, int W, int accumulate);
om_status om_relu_fwd(om_ctx *ctx, const float *x, float *y, int64_t n);
om_status om_relu_bwd(om_ctx *ctx, const float *g, const float *y, float *dx, int64_t n, int accumulate);
/* Ops.Gelu erf form and GeluGradBin (Ops.Nn.cs:86-112; TrainElementwise.cs:59-85; Transcendental.cs:167-263): the
 * reference's polynomials bit for bit under OM_GELU_REFERENCE, the fast pair of om_ctx_set_gelu otherwise. */
om_status om_gelu_fwd(om_ctx *ctx, const float *x, float *y, int64_t n);
om_status om_gelu_bwd(om_ctx *ctx, const float *g, const float *x, float *dx, int64_t n, int accumulate);
/* y = a + b, y = a - b, y = a * b (same shapes; Ops.cs:15-56). */
om_status om_add(om_ctx *ctx, const float *a, const float *b, float *y, int64_t n);
om_status om_sub(om_ctx *ctx, const float *a, const float *b, float *y, int64_t n);
om_status om_mul(om_ctx *ctx, const float *a, const float *b, float *y, int64_t n);
/* y[r][c] = x[r][c] + b[c] over [rows, cols]: Ops.Add with b broadcast over the rows (Ops.cs:15-56), the bias add of
 * Ops.Linear (Ops.Layers.cs:715-733) as the reference records it, a separate op after the MatMul. Its backward is
 * the identity for x and om_colsum (BackwardOps.SumTo) for b. */
om_status om_add_rows(om_ctx *ctx, const float *x, const float *b, float *y, int rows, int cols);
/* dst += src, or dst = src * alpha + dst (Engine.AddInto, Engine.cs:331-344; Neg backward is alpha = -1). */
om_status om_axpy(om_ctx *ctx, float alpha, const float *src, float *dst, int64_t n);
/* dst = src * alpha (a copy when alpha is 1). */
om_status om_scale(om_ctx *ctx, float alpha, const float *src, float *dst, int64_t n);
/* y = x.Permute(perm) made contiguous (rank <= 6): the Clone() of a permuted view, and with the inverse permutation
 * the Permute backward (BackwardOps.cs:107-118). accumulate adds into y. */
om_status om_permute(om_ctx *ctx, const float *x, float *y, int ndim, const int32_t *shape, const int32_t *perm,
                     int accumulate);
/* Losses.Mse = Mean(Mul(Sub(pred, target), same)) (Losses.cs:86-91; Ops.cs:23-56; Ops.Nn.cs:162-231): diff = pred -
 * target is saved, *loss (device) = (float)(sum in double of fl(diff*diff) / n). The backward is the chain's rounding
 * order: t = (g / (float)n) * diff, dpred = t + t (the two Mul emissions added, Engine.AddInto). */
om_status om_mse_fwd(om_ctx *ctx, const float *pred, const float *target, float *diff, float *loss, int64_t n);
/* The same, also writing dpred_unit = the backward's dpred for a unit upstream gradient (g = 1: t = (1 / (float)n) *
 * diff, t + t), so a loss that is the root of the backward needs no separate gradient launch. diff may be NULL (not
 * written): a caller that needs it later only off that path recomputes it with om_sub. */
om_status om_mse_fwd_unit(om_ctx *ctx, const float *pred, const float *target, float *diff, float *loss,
                          float *dpred_unit, int64_t n);
/* The same (dpred_unit or diff may be NULL, not both) with the loss also posted to rb, as om_readback_post(rb, loss, 4) would post
 * it, by the launch that finishes the loss's sum (which then writes the value to the pinned buffer, fences, and
 * writes the sequence number). No counterpart in the reference (whose loss is a host float after the forward): it
 * spares the loss's own readback launch. Waits for rb's previous post like om_readback_post. */
om_status om_mse_fwd_post(om_ctx *ctx, const float *pred, const float *target, float *diff, float *loss,
                          float *dpred_unit, int64_t n, om_readback *rb);
om_status om_mse_bwd(om_ctx *ctx, const float *g_scalar, const float *diff, float *dpred, int64_t n, int accumulate);
/* An encoder block's last Linear with its residual Add, followed by the MSE loss of its output against target
 * (Ops.Layers.cs:715-733, Ops.Add, then Losses.Mse, Losses.cs:86-91): y as om_linear_fwd_resid writes it, and the
 * loss, dpred_unit (and the post to rb when rb is not NULL) as om_mse_fwd_unit / om_mse_fwd_post of that y. The squared
 * differences are formed and summed in the product's epilogue (fp64 per wavefront, then one launch adds those
 * partials), so y, dpred_unit and each term are the same bits as the two calls and the loss differs from their
 * value only in the order of the fp64 additions. No counterpart as one call. */
om_status om_linear_fwd_resid_mse(om_ctx *ctx, const float *x, const float *w, const float *b, const float *resid,
                                  const float *target, float *y, float *dpred_unit, float *loss, int rows, int in,
                                  int out, om_readback *rb);

/* ---------------------------------------------------------------------------------------------- reductions */
/* Ops.Sum / Ops.Mean over all elements in double (Ops.Nn.cs:162-231); *out is a device float. */
om_status om_sum_all(om_ctx *ctx, const float *x, float *out, int64_t n, int mean);
/* The same, with the result also posted to rb as om_readback_post(rb, out, 4) would post it, by the launch that
 * finishes the sum (a loss that is a Mean: the step's readback without a copy launch of its own). Waits for rb's
 * previous post like om_readback_post. */
om_status om_sum_all_post(om_ctx *ctx, const float *x, float *out, int64_t n, int mean, om_readback *rb);
/* Mean over the middle axis of [outer, n, inner] (Ops.Nn.cs:186-231) and its backward: dx = g / n broadcast
 * (BackwardNn.cs:145-168). The backward reads g from device memory; g_scalar_index < 0 means g has [outer, inner]
 * values, otherwise it is one scalar at g[0] broadcast to everything (Mean over all elements). */
om_status om_mean_axis(om_ctx *ctx, const float *x, float *y, int outer, int n, int inner);
om_status om_mean_axis_bwd(om_ctx *ctx, const float *g, float *dx, int outer, int n, int inner, int accumulate);
om_status om_mean_all_bwd(om_ctx *ctx, const float *g_scalar, float *dx, int64_t n, int accumulate);
/* Ops.Relu followed by the mean over each row of [outer, n] (a conv block's ReLU and global average pool,
 * Ops.Layers.cs:463-472), in one pass: y[o] bit for bit om_relu_fwd then om_mean_axis(outer, n, 1). The backward
 * (mean backward then ReLU backward, BackwardNn.cs:145-168 and the Relu rule) reads the pre-activation x:
 * dx (+)= x > 0 ? g[o] / n : 0, bit for bit the two separate rules. No counterpart in the reference as one call. */
om_status om_relu_mean_rows(om_ctx *ctx, const float *x, float *y, int outer, int n);
om_status om_relu_mean_rows_bwd(om_ctx *ctx, const float *g, const float *x, float *dx, int outer, int n,
                                int accumulate);

/* ---------------------------------------------------------------------------------------------- normalisation */
/* Ops.LayerNorm (Ops.Layers.cs:109-141; NormKernels.cs:79-127): saves mean and 1/sigma per row. */
om_status om_layernorm_fwd(om_ctx *ctx, const float *x, const float *gamma, const float *beta, float *y, float *mean,
                           float *rstd, int rows, int cols, float eps);
/* LayerNormBackward (BackwardNn.cs:170-223): dx, and dgamma/dbeta as fp64 column sums (any may be NULL). */
om_status om_layernorm_bwd(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                           const float *rstd, float *dx, float *dgamma, float *dbeta, int rows, int cols, int acc_dx,
                           int acc_params);
/* The same with the input gradient's earlier part passed in: dx = dx_add + (this layer's dx), one rounding, into a
 * buffer other than dx_add — the AddInto of a residual gradient (Engine.cs:331-344) without first copying the
 * residual's buffer, which may still be read by a queued launch. */
om_status om_layernorm_bwd_add(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                               const float *rstd, const float *dx_add, float *dx, float *dgamma, float *dbeta, int rows,
                               int cols, int acc_params);
/* om_layernorm_bwd without any device allocation, for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc); no counterpart in the reference. The dgamma/dbeta fp64
 * partials (2 * ceil(rows / r) * cols doubles, r = 16 rows per chunk when cols is 384 or 768, else 8) go to the
 * calling context's own slot of one fixed device array per GPU (OM_NOALLOC_SLOTS slots of OM_NOALLOC_SCRATCH_BYTES,
 * held until the process ends). A context claims its slot on its first call and keeps it until om_ctx_destroy;
 * when every slot of the device is held by other live contexts the call fails with OM_E_STATE, and larger shapes are
 * refused with OM_E_ARG, both before anything is launched. The partials are rewritten by every call, so nothing has
 * to start at zero; calls on one context are ordered by its stream, and contexts never share a slot, so calls from
 * several contexts (threads, streams) on one GPU do not race. A graph captured with this call keeps using the slot
 * of the context it was captured on: replay it only while that context is alive (after om_ctx_destroy the slot may
 * go to another context). Results are om_layernorm_bwd's, bit for bit. */
#define OM_NOALLOC_SCRATCH_BYTES (8u << 20)
#define OM_NOALLOC_SLOTS 4
om_status om_layernorm_bwd_noalloc(om_ctx *ctx, const float *g, const float *x, const float *gamma,
                                   const float *mean, const float *rstd, float *dx, float *dgamma, float *dbeta,
                                   int rows, int cols, int acc_dx, int acc_params);
/* LayerNorm backward leaving dgamma/dbeta as fp64 partials: dx as om_layernorm_bwd (dx = dx_add + v when dx_add is
 * given, else accumulated when acc_dx, else written; dx may be NULL), and part_g / part_b (either may be NULL), each
 * [om_layernorm_bwd_chunks(rows, cols)][cols], to be finished by om_param_grads_group's column sums. */
int om_layernorm_bwd_chunks(int rows, int cols);
om_status om_layernorm_bwd_partials(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                                    const float *rstd, const float *dx_add, float *dx, int acc_dx, double *part_g,
                                    double *part_b, int rows, int cols);

/* ---------------------------------------------------------------------------------------------- softmax family */
/* Softmax.Rows (Softmax.cs:27-133) and its backward (BackwardNn.cs:26-52). */
om_status om_softmax_fwd(om_ctx *ctx, const float *x, float *y, int rows, int cols);
om_status om_softmax_bwd(om_ctx *ctx, const float *g, const float *y, float *dx, int rows, int cols, int accumulate);
/* Ops.LogSoftmax (Ops.Layers.cs:47-96) and backward (BackwardNn.cs:54-80). */
om_status om_logsoftmax_fwd(om_ctx *ctx, const float *x, float *y, int rows, int cols);
om_status om_logsoftmax_bwd(om_ctx *ctx, const float *g, const float *y, float *dx, int rows, int cols,
                            int accumulate);
/* Ops.NllLoss (Ops.Layers.cs:644-699) -> *loss (device float); a target outside [0,cols) that is not ignore_index
 * is reported through *bad_row (device int32, -1 when none), the reference's ArgumentOutOfRangeException. */
om_status om_nll_fwd(om_ctx *ctx, const float *logp, const int32_t *target, float *loss, int32_t *bad_row, int rows,
                     int cols, int mean, int ignore_index);
/* NllBackward (BackwardNn.cs:602-632): dlogp (+)= -scale at [i, target[i]] for every row whose target is not
 * ignore_index and 0 elsewhere, scale = g / max(1, count of such rows) with mean, else g (g_scalar a device float). */
om_status om_nll_bwd(om_ctx *ctx, const float *g_scalar, const int32_t *target, float *dlogp, int rows, int cols,
                     int mean, int ignore_index, int accumulate);
/* Fused softmax cross-entropy gradient = LogSoftmax backward of NllBackward (BackwardNn.cs:54-80, 602-632), in the
 * reference's rounding order: dlogits = d - exp(logp) * (float)sum(d), d = -g/count at the target. */
om_status om_xent_bwd(om_ctx *ctx, const float *g_scalar, const float *logp, const int32_t *target, float *dlogits,
                      int rows, int cols, int mean, int ignore_index, int accumulate);
/* Losses.CrossEntropy = NllLoss(LogSoftmax(logits)) (Losses.cs:20-40) forward, also writing dlogits_unit = the
 * om_xent_bwd result for a unit upstream gradient (g = 1, mean reduction), so a loss that is the root of the
 * backward needs no gradient launch of its own: logp, *loss and *bad_row as om_logsoftmax_fwd then om_nll_fwd give
 * them, bit for bit, and dlogits_unit bit for bit what om_xent_bwd(one, ...) writes. Two launches; with rb (may be
 * NULL) the second also posts the loss as om_readback_post(rb, loss, 4) would. No counterpart in the reference:
 * its loss and gradient are separate CPU passes. */
om_status om_xent_fwd_unit(om_ctx *ctx, const float *logits, const int32_t *target, float *logp, float *loss,
                           int32_t *bad_row, float *dlogits_unit, int rows, int cols, int ignore_index,
                           om_readback *rb);

/* ---------------------------------------------------------------------------------------------- attention */
/* Ops.Attention (Ops.Layers.cs:746-807) and AttentionBackward (BackwardNn.cs:636-701). q,o are [B,Lq,H,D] and
 * k,v [B,Lk,H,D] (the Linear outputs, heads interleaved; the reference's split/merge permutes become addressing),
 * mask is NULL, [Lq,Lk] (mask_batched 0) or [B,Lq,Lk] additive. The forward saves the weights P [B,H,Lq,Lk]
 * (HBM is plentiful; the reference recomputes them). The backward writes dq, dk, dv in the q/k/v layouts and uses
 * `ds` [B,H,Lq,Lk] as scratch. */
om_status om_attention_fwd(om_ctx *ctx, const float *q, const float *k, const float *v, const float *mask,
                           int mask_batched, float *o, float *p, int B, int H, int lq, int lk, int d, float scale);
om_status om_attention_bwd(om_ctx *ctx, const float *q, const float *k, const float *v, const float *p,
                           const float *g, float *dq, float *dk, float *dv, float *ds, int B, int H, int lq, int lk,
                           int d, float scale, int acc);

/* The same with explicit row strides (in floats): q/k/v rows ld_qkv apart (3*H*D when the three projections are one
 * packed [rows, 3*H*D] Linear output, so q, k, v are column offsets 0, H*D, 2*H*D into it), o rows ld_o apart, and in
 * the backward g rows ld_g and dq/dk/dv rows ld_d apart. The two entry points above are these with every stride H*D.
 * Same reference functions (Ops.Layers.cs:746-807, BackwardNn.cs:636-701; the packing replaces the q/k/v Linear
 * calls of MultiHeadAttention.Forward, Layers.cs:497-516). */
om_status om_attention_fwd_ld(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                              const float *mask, int mask_batched, float *o, int ld_o, float *p, int B, int H, int lq,
                              int lk, int d, float scale);
om_status om_attention_bwd_ld(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                              const float *p, const float *g, int ld_g, float *dq, float *dk, float *dv, int ld_d,
                              float *ds, int B, int H, int lq, int lk, int d, float scale, int acc);
/* Self-attention (Lq = Lk = L) as the reference computes it, with no saved weights: the forward returns O only, and
 * the backward recomputes S and P from q, k and the mask (AttentionBackward, BackwardNn.cs:636-701, recomputes them
 * the same way). For D = 32 and L in {64, 128} each is one fused kernel (scores, exact row softmax and the products
 * on chip); other shapes run the GEMM path with the scores in context scratch. Strides as in the _ld entry points. */
om_status om_attention_fwd_fused(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                 const float *mask, int mask_batched, float *o, int ld_o, int B, int H, int L, int d,
                                 float scale);
om_status om_attention_bwd_fused(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                 const float *mask, int mask_batched, const float *g, int ld_g, float *dq, float *dk,
                                 float *dv, int ld_d, int B, int H, int L, int d, float scale, int acc);
/* The same pair with the forward's row statistics kept for the backward (the reference keeps nothing and
 * recomputes, BackwardNn.cs:636-701): the forward writes O and stats (2 * B * H * L floats: each query's row maximum,
 * in log2 units, then the inverse row sum); the backward recomputes P = 2^(x - max) / sum from the statistics, takes
 * delta = rowsum(dO * O) from the forward's output o, and never writes a [B, H, L, L] tensor (dQ partials per block
 * of 64 keys go through context scratch and are summed in key-block order, so results are deterministic). For D = 32
 * and L in {64, 128} the kernels hold whole rows; for D in {32, 64} and longer L (a multiple of 64) they stream keys
 * (forward, online softmax) and queries (backward) through the workgroup in chunks of 64. Rows must be 16-byte
 * aligned; other shapes run the _fused entry points instead (the forward then leaves stats unwritten and the
 * backward recomputes). Results agree with the reference within its fp32 sums (1e-5). */
om_status om_attention_fwd_flash(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                 const float *mask, int mask_batched, float *o, int ld_o, float *stats, int B, int H,
                                 int L, int d, float scale);
om_status om_attention_bwd_flash(om_ctx *ctx, const float *q, const float *k, const float *v, int ld_qkv,
                                 const float *mask, int mask_batched, const float *o, int ld_o, const float *stats,
                                 const float *g, int ld_g, float *dq, float *dk, float *dv, int ld_d, int B, int H,
                                 int L, int d, float scale, int acc);
/* ---------------------------------------------------------------------------------------------- convolution, pooling */
/* Ops.Conv2d, groups 1, square stride/padding (Ops.Layers.cs:279-336; Conv.cs:54) as implicit GEMM on MFMA, and
 * ConvBackward (BackwardNn.cs:317-402): dx = col2im(W^T g) as an implicit GEMM over g, dw = g im2col(x) with a
 * deterministic split over images and pixels, db = fp64 sums. Output pointers may be NULL. */
om_status om_conv2d_fwd(om_ctx *ctx, const float *x, const float *w, const float *bias, float *y, int N, int Cin,
                        int H, int W, int Cout, int KH, int KW, int stride, int pad);
/* Ops.Conv2d followed by Ops.Relu, the ReLU applied in the convolution's epilogue (3x3, stride 1, padding 1; other
 * geometries run the two launches): y bit for bit om_conv2d_fwd then om_relu_fwd. No counterpart as one call. */
om_status om_conv2d_relu_fwd(om_ctx *ctx, const float *x, const float *w, const float *bias, float *y, int N,
                             int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad);
/* A conv stage's forward (Ops.Conv2d, Ops.Relu, then Ops.MaxPool2d with no padding): a = relu(conv(x) + b) as
 * om_conv2d_relu_fwd writes it, then y and idx as om_maxpool_fwd(a, ..., pkh, pkw, psh, psw, 0, 0) writes them, bit for
 * bit. Where the convolution sums input-channel splits in a pass of its own and the windows tile a exactly (stride
 * equal to the window), that pass also pools. No counterpart as one call. idx may be NULL. */
om_status om_conv2d_relu_pool_fwd(om_ctx *ctx, const float *x, const float *w, const float *bias, float *a, float *y,
                                  int32_t *idx, int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride,
                                  int pad, int pkh, int pkw, int psh, int psw);
om_status om_conv2d_bwd(om_ctx *ctx, const float *g, const float *x, const float *w, float *dx, float *dw, float *db,
                        int N, int Cin, int H, int W, int Cout, int KH, int KW, int stride, int pad, int acc_dx,
                        int acc_params);
/* Ops.MaxPool2d (Ops.cs:151-178; TensorKernels.cs:242-296): Int32 flat argmax, first wins, NaN wins; and
 * MaxPoolBackward (BackwardOps.cs:285-298): dx = 0, dx[idx] += g. */
om_status om_maxpool_fwd(om_ctx *ctx, const float *x, float *y, int32_t *idx, int N, int C, int H, int W, int KH,
                         int KW, int SH, int SW, int PH, int PW);
om_status om_maxpool_bwd(om_ctx *ctx, const float *g, const int32_t *idx, float *dx, int N, int C, int H, int W,
                         int OH, int OW, int KH, int KW, int SH, int SW, int PH, int PW, int accumulate);
/* MaxPoolBackward then the backward of the ReLU that produced the pool's input y, in one pass: dx (+)= the pooled
 * gradient where y > 0, else 0; bit for bit om_maxpool_bwd then om_relu_bwd. No counterpart as one call. */
om_status om_maxpool_relu_bwd(om_ctx *ctx, const float *g, const int32_t *idx, const float *y, float *dx, int N,
                              int C, int H, int W, int OH, int OW, int KH, int KW, int SH, int SW, int PH, int PW,
                              int accumulate);
/* Ops.AvgPool2d (Ops.Layers.cs:405-455) over `planes` = N*C planes of H x W: each output is its window's in-order
 * float sum divided by the window size (counting the zero padding when count_include_pad, else only real pixels);
 * and AvgPoolBackward (BackwardNn.cs:464-492), each input pixel gathering its windows' shares in the reference's
 * scatter order. Both bit-exact. Padding at most half the window. */
om_status om_avgpool2d_fwd(om_ctx *ctx, const float *x, float *y, int planes, int H, int W, int KH, int KW, int SH,
                           int SW, int PH, int PW, int count_include_pad);
om_status om_avgpool2d_bwd(om_ctx *ctx, const float *g, float *dx, int planes, int H, int W, int KH, int KW, int SH,
                           int SW, int PH, int PW, int count_include_pad, int accumulate);

/* ---------------------------------------------------------------------------------------------- normalisation, lookup */
/* Ops.BatchNorm2d (Ops.Layers.cs:158-246) over x [N, C, plane]. training != 0: batch mean and biased variance in
 * fp64, saved mean/inv = 1/sqrtf(var + eps) per channel, running statistics updated in place with the unbiased
 * variance: r = (float)((1 - momentum) * r + momentum * stat); training == 0: mean/inv from the running statistics.
 * y = ((x - mean) * inv) * gamma + beta. */
om_status om_batchnorm2d_fwd(om_ctx *ctx, const float *x, const float *gamma, const float *beta, float *running_mean,
                             float *running_var, float *y, float *mean, float *inv, int N, int C, int plane,
                             int training, float momentum, float eps);
/* BatchNormBackward (BackwardNn.cs:244-307) from the saved mean/inv: fp64 per-channel sums of g*xhat and g; dx may
 * be NULL; dgamma/dbeta may be NULL. */
om_status om_batchnorm2d_bwd(om_ctx *ctx, const float *g, const float *x, const float *gamma, const float *mean,
                             const float *inv, float *dx, float *dgamma, float *dbeta, int N, int C, int plane,
                             int training, int acc_dx, int acc_params);
/* Ops.Embedding, dense (Ops.Layers.cs:549-600): y[i] = table[ids[i]] for n_ids int32 ids in [0, rows) (an id out of
 * range reads nothing and gives NaN; the host validates ids before they are uploaded); and EmbeddingBackward's
 * dense branch (BackwardNn.cs:521-540): dtable row r = the sum of g rows of the positions holding r, in increasing
 * position order (rows never looked up, and padding_index, get 0). Bit-exact. */
om_status om_embedding_fwd(om_ctx *ctx, const float *table, const int32_t *ids, float *y, int64_t n_ids, int dim,
                           int rows);
om_status om_embedding_bwd(om_ctx *ctx, const float *g, const int32_t *ids, float *dtable, int64_t n_ids, int dim,
                           int rows, int padding_index, int accumulate);
/* Dropout.Forward in training mode (Layers.cs:341-368): y = x * mask with mask[i] = 1/(1-p) when
 * (Mix(Mix(seed + draw*G) + (i+1)*G) >> 40) / 2^24 >= p and 0 otherwise (SplitMix64's Mix, G = 0x9E3779B97F4A7C15,
 * draw = the module's count of masks drawn before this one). The backward (the Mul rule, dx = g * mask) recomputes
 * the mask from (seed, draw) instead of reading a stored one. p in [0, 1). Bit-exact. */
om_status om_dropout_fwd(om_ctx *ctx, const float *x, float *y, int64_t n, float p, uint64_t seed, int64_t draw);
om_status om_dropout_bwd(om_ctx *ctx, const float *g, float *dx, int64_t n, float p, uint64_t seed, int64_t draw,
                         int accumulate);

/* ---------------------------------------------------------------------------------------------- CTC */
/* Ops.CtcLoss (CtcLoss.cs:40-153) in double with the reference's exp/ln/logadd (Ctc.cs:515-616); reduction
 * 0 = None ([B] losses), 1 = Mean, 2 = Sum (a scalar). Both entry points validate on the host, from the host copies
 * of the lengths and targets, everything the kernels index with (input lengths within [0, T], target lengths summing
 * to n_targets, labels in [0, C) and not the blank, blank in [0, C)) and size their scratch from the host target
 * lengths. `lp` is [T,B,C] on the device; targets/in_len/tgt_len are device copies that must hold the same values as
 * the host arrays. om_ctc_bwd = CtcBackward (BackwardRecurrent.cs:253-296): dlp[t,b,c] (+)= -scale * exp(...), g on
 * the device. */
om_status om_ctc_fwd(om_ctx *ctx, const float *lp, const int32_t *targets, const int32_t *in_len,
                     const int32_t *tgt_len, const int32_t *h_in_len, const int32_t *h_tgt_len,
                     const int32_t *h_targets, int n_targets, int T, int B, int C, int blank, int reduction,
                     int zero_infinity, float *loss);
om_status om_ctc_bwd(om_ctx *ctx, const float *lp, const int32_t *targets, const int32_t *in_len,
                     const int32_t *tgt_len, const int32_t *h_in_len, const int32_t *h_tgt_len,
                     const int32_t *h_targets, int n_targets, const float *g, float *dlp, int T, int B, int C,
                     int blank, int reduction, int accumulate);
/* The same pair with each recursion run once (the values of om_ctc_fwd / om_ctc_bwd, bit for bit; the reference's
 * CtcBackward recomputes alpha and then runs beta, BackwardRecurrent.cs:253-296): om_ctc_fwd_tables also runs the beta
 * recursion, beside alpha on another wavefront, and keeps both tables in `tables` (device memory of at least
 * om_ctc_tables_bytes(T, B, max(tgt_len)) bytes, given as tables_bytes); om_ctc_bwd_tables forms the gradient from
 * them, with the same arguments as om_ctc_bwd, so the backward repeats neither recursion. */
uint64_t om_ctc_tables_bytes(int T, int B, int max_tgt_len);
om_status om_ctc_fwd_tables(om_ctx *ctx, const float *lp, const int32_t *targets, const int32_t *in_len,
                            const int32_t *tgt_len, const int32_t *h_in_len, const int32_t *h_tgt_len,
                            const int32_t *h_targets, int n_targets, int T, int B, int C, int blank, int reduction,
                            int zero_infinity, float *loss, double *tables, uint64_t tables_bytes);
om_status om_ctc_bwd_tables(om_ctx *ctx, const float *lp, const int32_t *targets, const int32_t *in_len,
                            const int32_t *tgt_len, const int32_t *h_in_len, const int32_t *h_tgt_len,
                            const int32_t *h_targets, int n_targets, const float *g, float *dlp, int T, int B, int C,
                            int blank, int reduction, int accumulate, const double *tables, uint64_t tables_bytes);

/* ---------------------------------------------------------------------------------------------- optimizer */
/* Adam.UpdateRange (Optimizers.cs:554-589) over n contiguous elements: the tape keeps parameters, gradients and
 * both moments each contiguous in the persistent region in Parameters() order, so one launch updates every
 * parameter (a run per contiguous group of parameters that have gradients). vmax is NULL unless AMSGrad.
 * step_size and sqrt_bc2 come from om_adam_scalars (Adam.BeginStep, Optimizers.cs:501-508). IEEE float, no fused
 * multiply-add: bit-identical to the reference's CPU update given the same gradient. */
om_status om_adam_step(om_ctx *ctx, float *p, const float *g, float *m, float *v, float *vmax, int64_t n, float lr,
                       float beta1, float beta2, float eps, float weight_decay, int decoupled, float step_size,
                       float sqrt_bc2);
/* Host helper: Adam.IntPow + BeginStep in double for step t (1-based). */
void om_adam_scalars(float lr, float beta1, float beta2, int64_t t, float *step_size, float *sqrt_bc2);
/* om_adam_step with GradClip.ClipNorm's scaling folded into the read of g: grad_scale is a device float (the coef
 * om_clip_grad_norm wrote) and every gradient element is used as g * c when c < 1, unchanged otherwise — the same
 * float product the reference's in-place scaling (Schedules.cs:70-76) stores before Adam reads it, so the update is
 * bit-identical to clip-then-step; the gradient buffer itself is left unscaled (one fewer pass over it). */
om_status om_adam_step_scaled(om_ctx *ctx, float *p, const float *g, float *m, float *v, float *vmax, int64_t n,
                              float lr, float beta1, float beta2, float eps, float weight_decay, int decoupled,
                              float step_size, float sqrt_bc2, const float *grad_scale);
/* Sgd.Update (Optimizers.cs, class Sgd) over n contiguous elements; buf may be NULL (no momentum); first != 0 on
 * the parameter's first step (the momentum buffer starts from the gradient). */
om_status om_sgd_step(om_ctx *ctx, float *p, const float *g, float *buf, int64_t n, float lr, float momentum,
                      float dampening, float weight_decay, int nesterov, int first);

/* ---------------------------------------------------------------------------------------------- gradient clipping */
/* GradClip.ClipNorm (Schedules.cs:22-100) over `count` gradient segments: grads[i] (device) holds lens[i] floats;
 * a NULL or empty segment is skipped, as a parameter without a gradient is (pass a row-sparse gradient's values).
 * The norm is the L2 norm (squares summed in fp64; the device sums in a fixed tree that depends only on the
 * segment lengths, within count·2^-53 relative of the reference's serial sum) or, with infinity_norm, the largest
 * |g| (a NaN wins). When the norm is finite and coef = (float)(max_norm / (norm + 1e-6)) < 1, every element becomes
 * g * coef. Asynchronous: the norm is written as float to *total (device, may be NULL) — om_download it to read the
 * value ClipNorm returns — and the coefficient to *coef (device, may be NULL; 1 when the norm is not finite).
 * scale_in_place = 0 leaves the gradients unscaled for om_adam_step_scaled (coef required then).
 * max_norm must be positive (OM_E_ARG, the reference's ArgumentOutOfRangeException). */
om_status om_clip_grad_norm(om_ctx *ctx, int count, float *const *grads, const int64_t *lens, float max_norm,
                            int infinity_norm, int scale_in_place, float *total, float *coef);
/* GradClip.ClipValue (Schedules.cs:119-149): every element clamped to [-clip_value, clip_value], NaN stays NaN;
 * bit-exact. clip_value must not be negative (OM_E_ARG). */
om_status om_clip_grad_value(om_ctx *ctx, int count, float *const *grads, const int64_t *lens, float clip_value);

#ifdef __cplusplus
}
#endif
#endif /* OM_H */
