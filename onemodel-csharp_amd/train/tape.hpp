// The host-side training tape: the MI355X build's stand-in for the reference's C# autograd layer
// (src/OneModel/Tensors/Autograd, src/OneModel.Training). It keeps the reference's surface and semantics —
// tensors that record a backward record per op, Tensor.Backward() over the records in reverse topological order with
// one pending gradient per record, leaf gradients that accumulate, ZeroGrad, modules registering parameters in order,
// losses, SGD/Adam/AdamW — and does every piece of arithmetic through the C ABI of libom_hip.so (include/om.h).
// No tensor data ever lives on the host: inputs cross at step edges, the loss crosses back at the end of a step.
#pragma once

#include <cstdint>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "om.h"

namespace omt {

// Errors raised inside the tape; the C ABI turns them into status codes and messages.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};
void check(om_ctx *ctx, om_status s, const char *what);

struct Record;
struct TensorImpl;
using Tensor = std::shared_ptr<TensorImpl>;
using RecordP = std::shared_ptr<Record>;

// A float32 tensor in device memory (row-major, contiguous), or an int32 one (labels, pool indices).
struct TensorImpl {
    std::vector<int> shape;
    int64_t numel = 0;
    float *data = nullptr;
    int32_t *idata = nullptr;
    bool requires_grad = false;
    RecordP grad_fn;  // null for leaves
    // Leaf gradient (persistent region, allocated with the parameter arena). `grad_exists` mirrors the reference's
    // non-empty Tensor.Grad; `grad_live` says the buffer holds this step's values (false right after ZeroGrad, whose
    // zero fill is deferred until something reads the gradient, so the first emission can overwrite).
    float *grad = nullptr;
    bool grad_exists = false;
    bool grad_live = false;
    std::string name;
    // The storage's version counter (Tensor.Version, Tensor.cs:190-191; TensorBuffer.Version): views share it, and
    // every in-place write to the storage raises it (touch), so a record that saved the tensor notices.
    std::shared_ptr<int64_t> version = std::make_shared<int64_t>(0);
    bool is_leaf() const { return !grad_fn; }
};
// An in-place write to t's storage (Tensor.MutableData, Tensor.cs:292-309): raises its version.
inline void touch(const Tensor &t) {
    if (t) ++*t->version;
}
// The tape's error code for TensorVersionException (Autograd.cs:188-191): a tensor saved for the backward pass was
// modified in place. The om_train.h ABI reports it as OMT_E_TENSOR_VERSION.
constexpr int kErrTensorVersion = 21;

class Engine;
// A backward record (BackwardRecord.cs:17-150): inputs in order and the rule that turns the output gradient into
// gradients for them.
struct Record {
    const char *op = "";
    std::vector<Tensor> inputs;
    std::function<void(Engine &, Record &, const float *g)> rule;
    // pending gradient of the output (Engine.cs:129-191)
    float *pending = nullptr;
    bool pending_borrowed = false;  // aliases another gradient; copy before writing into it
    int64_t out_numel = 0;
    uint64_t mark = 0;
    // Set when a backward pass has run through the record and freed what it saved (BackwardRecord.Release).
    bool released = false;
    // The tensors the rule reads, each with its storage version at the time it was saved (SavedTensor,
    // Autograd.cs:197-237); unpack_check() fails if any was written in place since.
    std::vector<std::pair<std::shared_ptr<int64_t>, int64_t>> saved;
    void save(const Tensor &t) {
        if (t) saved.emplace_back(t->version, *t->version);
    }
    void unpack_check() const;
    bool needs(int i) const { return inputs[i] && inputs[i]->requires_grad; }
};

// The device context and the step-scoped allocator.
class Device {
   public:
    explicit Device(int device);
    ~Device();
    om_ctx *ctx() const { return ctx_; }
    // Record structure of the ops and modules built on this device. false (the default): composite records (a
    // Linear with its bias, q|k|v as one product over colocated weights, the feed-forward sub-block, a conv stage,
    // fused losses) and the engine's grouped weight-gradient launches. true: exactly the reference's records, each
    // rule one C-ABI call run when the engine reaches it (a Linear is Reshape, MatMul with W.T(), Add of the bias,
    // Reshape, Ops.Layers.cs:715-733; MultiHeadAttention three Linears, the attention and one Linear,
    // Layers.cs:497-516; losses as Sub/Mul/Mean and LogSoftmax/NllLoss, Losses.cs:20-91). Views (Reshape, W.T(),
    // the head split/merge permutes) stay views: the kernels address them in place. Fixed before modules are built.
    bool per_op = false;
    float *step_floats(int64_t n);
    int32_t *step_ints(int64_t n);
    void *persistent(uint64_t bytes);
    // A persistent 1.0f: the seed gradient of every backward pass (written once, never written again).
    const float *one();
    void step_reset();
    void sync();
    // Loss readback folded into the loss's own launch: arm_loss_post(rb) offers rb to the next loss op that can post
    // its value itself (MSE); that op takes it (take_loss_post) and reports what it posted (loss_posted), so the
    // step posts the loss separately only when the offer was not taken for that very tensor.
    void arm_loss_post(om_readback *rb) {
        loss_rb_ = rb;
        loss_posted_ = nullptr;
    }
    om_readback *take_loss_post() {
        om_readback *r = loss_rb_;
        loss_rb_ = nullptr;
        return r;
    }
    void set_loss_posted(const float *p) { loss_posted_ = p; }
    const float *loss_posted() const { return loss_posted_; }

   private:
    om_ctx *ctx_ = nullptr;
    float *one_ = nullptr;
    om_readback *loss_rb_ = nullptr;
    const float *loss_posted_ = nullptr;
};

Device &dev();            // the device of the current thread's model (set by Model)
void set_dev(Device *d);  // installs it

Tensor make(const std::vector<int> &shape);                    // step-region float tensor
Tensor make_ints(const std::vector<int> &shape);               // step-region int32 tensor
int64_t numel_of(const std::vector<int> &shape);

// The reverse-mode engine (Engine.Execute, Engine.cs:124-207 and Emit/AccumulateLeaf/AddInto, Engine.cs:210-344).
class Engine {
   public:
    // Destination for a freshly computed gradient of input i: the producer's pending buffer or the leaf's gradient,
    // with *acc telling the kernel to add (C = C + v) instead of overwrite. nullptr when the input needs no gradient.
    float *dest(Record &r, int i, int *acc);
    // The same for kernels that can add an existing gradient themselves (out = addend + v): where dest would copy a
    // borrowed gradient still held elsewhere before adding into the copy, this returns a fresh buffer and hands the
    // borrowed one over as *addend (else *addend is NULL and the result is dest's).
    float *dest_add(Record &r, int i, int *acc, const float **addend);
    // Hands the incoming gradient itself on to input i (EmitAliased, Engine.cs:245-249): no copy unless it has to
    // be added to an existing gradient.
    void emit_alias(Record &r, int i, const float *g);
    // Queues a Linear layer's weight and bias gradients (dw (+)= g^T x, db (+)= column sums of g); queued items of
    // the same row count are launched together (om_linear_bwd_dw_group), up to four at a time, when the queue is
    // full, when another gradient is about to be added into one of their leaf gradients, and when the pass ends.
    // Until then g stays pinned: it counts as held, so no record writes into it in place.
    void queue_dw(const om_linear_dw &item, int rows);
    // Queues a two-stage column sum (LayerNorm's dgamma / dbeta partials in step memory), launched with the weight
    // gradients (om_param_grads_group).
    void queue_colsum(const om_column_sum &item);
    void flush_dw();
    void run(const Tensor &root);

   private:
    std::vector<om_linear_dw> dw_queue_;
    std::vector<om_column_sum> cs_queue_;
    int dw_rows_ = 0;
    // Leaf gradient ranges [begin, end) a queued item writes.
    std::vector<std::pair<const char *, const char *>> dw_ranges_;
    bool queued_leaf(const float *p) const {
        const char *c = reinterpret_cast<const char *>(p);
        for (const auto &r : dw_ranges_)
            if (c >= r.first && c < r.second) return true;
        return false;
    }

    // How many records hold each gradient buffer as their pending gradient during a backward pass (the record
    // running counts as a holder of its own gradient until its rule returns). A borrowed buffer whose only holder
    // is the record about to write into it is written in place instead of being copied first.
    std::unordered_map<const float *, int> holders_;
    bool sole_holder(const float *b) const {
        auto it = holders_.find(b);
        return it != holders_.end() && it->second == 1;
    }
};

void backward(const Tensor &root);  // Tensor.Backward() of a one-element tensor
void zero_grad(const std::vector<Tensor> &leaves);
// Materialises deferred zero fills (before the optimizer reads gradients).
void settle_grads(const std::vector<Tensor> &leaves);

// ------------------------------------------------------------------------------------------------ ops
// Each records a backward record when an input requires a gradient (the reference's Ops.*).
Tensor linear(const Tensor &x, const Tensor &w, const Tensor &b);
// relu(Linear(x)) as one record: one launch forward (the ReLU in the product's epilogue, the same bits as the pair).
Tensor linear_relu(const Tensor &x, const Tensor &w, const Tensor &b);
// resid + Linear(x) (Ops.Layers.cs:715-733 then Ops.Add): one launch forward, the residual's gradient is g itself.
Tensor linear_residual(const Tensor &x, const Tensor &w, const Tensor &b, const Tensor &resid);
// The feed-forward sub-block resid + Linear2(GELU(Linear1(x))) as one record (resid may be empty): forward is two
// launches (Linear1 with GELU in its epilogue, Linear2 with the residual in its epilogue); backward is Linear2's dW
// (with its bias gradient), the input gradient through GELU in one launch, then Linear1's backward.
Tensor ffn(const Tensor &x, const Tensor &w1, const Tensor &b1, const Tensor &w2, const Tensor &b2,
           const Tensor &resid);
// mse(ffn(x, w1, b1, w2, b2, resid), target) with the loss formed in the second product's epilogue (the same
// records; one launch for the product and the squared differences, one for the sum)
Tensor ffn_mse(const Tensor &x, const Tensor &w1, const Tensor &b1, const Tensor &w2, const Tensor &b2,
               const Tensor &resid, const Tensor &target);
Tensor relu(const Tensor &x);
// The pieces of the reference's per-op records: Ops.MatMul(x2d, W.T()) of x [rows, in] and w [out, in], one record
// whose rule is MatMul's backward with the W.T() view's Permute backward folded in (dW written as [out, in]);
// Ops.Add with b [cols] broadcast over the rows of x [rows, cols]; Sub, Mul (same shapes); Ops.Mean over all elements;
// Ops.NllLoss with the mean reduction and ignore index -100 over [N, C] log-probabilities.
Tensor matmul_wt(const Tensor &x, const Tensor &w);
Tensor add_rows(const Tensor &x, const Tensor &b);
Tensor sub(const Tensor &a, const Tensor &b);
Tensor mul(const Tensor &a, const Tensor &b);
Tensor mean_all(const Tensor &x);
Tensor nll_loss(const Tensor &logp, const Tensor &labels);
// Mean over axis 2 of [B, C, H, W] then Permute(2, 0, 1): [W, B, C], one record, the bits of the two ops.
Tensor mean_permute_seq(const Tensor &x);
Tensor gelu(const Tensor &x);
Tensor add(const Tensor &a, const Tensor &b);
Tensor layer_norm(const Tensor &x, const Tensor &gamma, const Tensor &beta, float eps);
// Multi-head attention core over Linear outputs q/k/v [B, L, H*D] (heads interleaved), additive mask [B, L, L] or
// empty; returns [B, L, H*D]. The reference's Reshape/Permute/Attention/Permute/Reshape with the permutes folded into
// the kernels' addressing.
Tensor attention_heads(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &mask, int heads);
// The q/k/v projections and the attention core of MultiHeadAttention (Layers.cs:497-516) in one record: when the
// three weights (and the three biases) sit back to back in the arena, the projections are one [rows, 3W] Linear
// (one GEMM forward, one dX GEMM over K = 3W, one dW GEMM over M = 3W, one bias sum in the backward) and attention
// reads q, k, v as column blocks of it; otherwise it is the three Linear calls and attention_heads.
Tensor attention_qkv(const Tensor &x, const Tensor &wq, const Tensor &bq, const Tensor &wk, const Tensor &bk,
                     const Tensor &wv, const Tensor &bv, const Tensor &mask, int heads);
Tensor reshape(const Tensor &x, const std::vector<int> &shape);
Tensor permute(const Tensor &x, const std::vector<int> &perm);
Tensor mean_axis(const Tensor &x, int axis);
Tensor log_softmax(const Tensor &x);
Tensor cross_entropy(const Tensor &logits, const Tensor &labels);  // Losses.CrossEntropy: NllLoss(LogSoftmax)
Tensor mse(const Tensor &pred, const Tensor &target);              // Losses.Mse: Mean((pred-target)^2)
Tensor conv2d(const Tensor &x, const Tensor &w, const Tensor &b, int stride, int pad);
Tensor max_pool2d(const Tensor &x, int kh, int kw, int sh, int sw);
// MaxPool2d(Relu(Conv2d(x))) (a CRNN stage, Layers.cs Conv2d / Relu / MaxPool2d) as one record: the ReLU runs in the
// convolution's epilogue, and the backward runs MaxPool's and Relu's rules in one pass before ConvBackward. The same
// arithmetic as the three ops, so the same bits.
Tensor conv2d_relu_pool(const Tensor &x, const Tensor &w, const Tensor &b, int stride, int pad, int kh, int kw, int sh,
                        int sw);
// Mean over each (H, W) plane of Relu(x), [N, C, H, W] -> [N, C] (a conv block's ReLU and GlobalAvgPool2d with its
// Flatten, Ops.Layers.cs:463-472) as one record: one pass forward, one backward; the same bits as the separate ops.
Tensor relu_mean_plane(const Tensor &x);
// The int arrays on the host; d_* are optional int tensors holding the same values on the device (a model's int
// inputs keep such a copy), which spare the step three uploads from pageable memory. They are saved for the backward
// like any tensor it reads, so an in-place write between forward and backward fails that backward.
Tensor ctc_loss(const Tensor &lp, const std::vector<int32_t> &targets, const std::vector<int32_t> &in_len,
                const std::vector<int32_t> &tgt_len, int blank, int reduction, const Tensor &d_targets = nullptr,
                const Tensor &d_in_len = nullptr, const Tensor &d_tgt_len = nullptr);
// Ops.AvgPool2d (Ops.Layers.cs:405-455), square window k, stride s, padding p.
Tensor avg_pool2d(const Tensor &x, int k, int s, int p, bool count_include_pad = true);
// Ops.BatchNorm2d (Ops.Layers.cs:158-246) with the module's running statistics (device, [C], updated in training).
Tensor batch_norm2d(const Tensor &x, const Tensor &gamma, const Tensor &beta, float *running_mean,
                    float *running_var, bool training, float momentum, float eps);
// Ops.Embedding, dense gradient (Ops.Layers.cs:549-600): ids is an Int32 tensor; the result is ids.shape + [dim].
Tensor embedding(const Tensor &table, const Tensor &ids, int padding_index);
// Dropout.Forward in training mode (Layers.cs:341-368) for mask number `draw` of the stream `seed`.
Tensor dropout(const Tensor &x, float p, uint64_t seed, int64_t draw);

// ------------------------------------------------------------------------------------------------ modules
// SplitMix64 (Generator.cs:10-48).
class Generator {
   public:
    explicit Generator(uint64_t seed) : s_(seed) {}
    uint64_t next_u64();
    float next_single();
    float uniform(float lo, float hi) { return lo + (hi - lo) * next_single(); }
    void fill_uniform(float lo, float hi, std::vector<float> &v);
    void fill_normal(std::vector<float> &v);  // benchmark inputs: Box-Muller in double
    void fill_ints(int32_t lo, int32_t hi, std::vector<int32_t> &v);

   private:
    uint64_t s_;
};

// NnModule (NnModule.cs): parameters in registration order, then children in registration order.
class Module {
   public:
    virtual ~Module() = default;
    Tensor param(const std::string &name, std::vector<int> shape, std::vector<float> init);
    template <class M>
    M *child(const std::string &name, std::unique_ptr<M> m) {
        M *p = m.get();
        children_.emplace_back(name, std::move(m));
        return p;
    }
    void named_parameters(std::vector<std::pair<std::string, Tensor>> &out, const std::string &prefix = "") const;
    // A float state buffer that is not a parameter (RegisterBuffer, NnModule.cs:54-65): device memory in the
    // persistent region, initialised from `init`.
    float *buffer(const std::string &name, const std::vector<float> &init);
    // An Int64 [1] buffer kept on the host (Dropout's count of masks drawn).
    void buffer_i64(const std::string &name, int64_t *host);
    struct BufferRef {
        float *dev = nullptr;      // float buffer in device memory
        int64_t *host = nullptr;   // or an Int64 [1] buffer on the host
        int64_t numel = 0;
    };
    void named_buffers(std::vector<std::pair<std::string, BufferRef>> &out, const std::string &prefix = "") const;
    // StateDict order (NnModule.cs:281-311): per module its own parameters, its own buffers, then its children.
    // Each entry is a parameter (tensor set) or a buffer.
    struct StateRef {
        std::string name;
        Tensor param;
        BufferRef buf;
    };
    void state(std::vector<StateRef> &out, const std::string &prefix = "") const;
    // Asks the arena to place these parameters back to back, in this order (values, gradients and moments alike),
    // so one kernel can treat them as one tensor. Parameters() order is unchanged.
    void colocate(std::vector<Tensor> group) { colocate_.push_back(std::move(group)); }
    void colocation_groups(std::vector<std::vector<Tensor>> &out) const;
    // Moves the host initial values out, in named_parameters() order, for the model to upload into its arena.
    void take_init(std::vector<std::vector<float>> &out);

   private:
    std::vector<std::pair<std::string, Tensor>> params_;
    std::vector<std::pair<std::string, BufferRef>> buffers_;
    std::vector<std::pair<std::string, std::unique_ptr<Module>>> children_;
    std::vector<std::vector<float>> init_;  // host values until the parameters are laid out in device memory
    std::vector<std::vector<Tensor>> colocate_;
};

class Linear : public Module {
   public:
    Linear(int in, int out, Generator &g, bool bias = true);
    Tensor operator()(const Tensor &x) const { return linear(x, w, b); }
    // relu(this(x)) as one record (linear_relu)
    Tensor relu_of(const Tensor &x) const { return dev().per_op ? relu(linear(x, w, b)) : linear_relu(x, w, b); }
    Tensor w, b;
};
class Conv2d : public Module {
   public:
    Conv2d(int cin, int cout, int k, Generator &g, int padding = 0, int stride = 1);
    Tensor operator()(const Tensor &x) const { return conv2d(x, w, b, stride, pad); }
    Tensor w, b;
    int stride, pad;
};
// BatchNorm2d (Layers.cs:202-238): weight 1, bias 0; buffers running_mean 0 and running_var 1.
class BatchNorm2d : public Module {
   public:
    explicit BatchNorm2d(int c, float momentum = 0.1f, float eps = 1e-5f);
    Tensor operator()(const Tensor &x) const { return batch_norm2d(x, w, b, rm, rv, training, momentum, eps); }
    Tensor w, b;
    float *rm, *rv;
    float momentum, eps;
    bool training = true;
};
// Embedding (Layers.cs:268-308): weight U(-sqrt(3), sqrt(3)) in row-major order, dense gradient.
class Embedding : public Module {
   public:
    Embedding(int count, int width, Generator &g, int padding_index = -1);
    Tensor operator()(const Tensor &ids) const { return embedding(w, ids, pad); }
    Tensor w;
    int pad;
};
// Dropout (Layers.cs:310-368): the mask stream is a pure function of (seed, masks drawn so far, index).
class Dropout : public Module {
   public:
    Dropout(float p, uint64_t seed);  // registers the buffer "draws" (Int64 [1])
    Tensor operator()(const Tensor &x) {
        if (!training || p == 0.0f) return x;
        return dropout(x, p, seed, draws++);
    }
    float p;
    uint64_t seed;
    int64_t draws = 0;
    bool training = true;
};
class LayerNorm : public Module {
   public:
    explicit LayerNorm(int n, float eps = 1e-5f);
    Tensor operator()(const Tensor &x) const { return layer_norm(x, w, b, eps); }
    Tensor w, b;
    float eps;
};
class MultiHeadAttention : public Module {
   public:
    MultiHeadAttention(int width, int heads, Generator &g);
    Tensor operator()(const Tensor &x, const Tensor &mask) const;
    // resid + MultiHeadAttention(x): the residual Add fused into the output projection.
    Tensor residual(const Tensor &x, const Tensor &mask, const Tensor &resid) const;
    Linear *q, *k, *v, *o;
    int heads;
};

// ------------------------------------------------------------------------------------------------ optimizers
// Optimizer.Step (Optimizers.cs:184-219) over a model's parameter arena.
class Optimizer {
   public:
    virtual ~Optimizer() = default;
    virtual void step() = 0;
    int64_t step_count = 0;
};

}  // namespace omt
