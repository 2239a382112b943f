// The tape: device and step allocator, the reverse-mode engine, and the recording ops.
#include "tape.hpp"

#include <cstdlib>

#include <cmath>
#include <cstring>

namespace omt {

void check(om_ctx *ctx, om_status s, const char *what) {
    if (s != OM_OK) throw Error(s, std::string(what) + ": " + om_last_error(ctx));
}

namespace {
thread_local Device *g_dev = nullptr;
uint64_t g_pass = 0;
}  // namespace

Device &dev() {
    if (!g_dev) throw Error(OM_E_STATE, "no device context is installed on this thread");
    return *g_dev;
}
void set_dev(Device *d) { g_dev = d; }

Device::Device(int device) {
    om_status s = om_ctx_create(device, &ctx_);
    if (s != OM_OK) throw Error(s, std::string("om_ctx_create: ") + om_last_error(nullptr));
    check(ctx_, om_arena_reserve(ctx_, 0, 1ull << 30), "om_arena_reserve");
}
Device::~Device() {
    if (ctx_) om_ctx_destroy(ctx_);
}
float *Device::step_floats(int64_t n) {
    void *p = nullptr;
    check(ctx_, om_alloc(ctx_, OM_REGION_STEP, (uint64_t)(n > 0 ? n : 1) * sizeof(float), &p), "om_alloc");
    return static_cast<float *>(p);
}
int32_t *Device::step_ints(int64_t n) {
    void *p = nullptr;
    check(ctx_, om_alloc(ctx_, OM_REGION_STEP, (uint64_t)(n > 0 ? n : 1) * sizeof(int32_t), &p), "om_alloc");
    return static_cast<int32_t *>(p);
}
void *Device::persistent(uint64_t bytes) {
    void *p = nullptr;
    check(ctx_, om_alloc(ctx_, OM_REGION_PERSISTENT, bytes, &p), "om_alloc");
    return p;
}
const float *Device::one() {
    if (!one_) {
        float *p = static_cast<float *>(persistent(sizeof(float)));
        check(ctx_, om_fill(ctx_, p, 1.0f, 1), "om_fill");
        one_ = p;
    }
    return one_;
}
void Device::step_reset() { check(ctx_, om_step_reset(ctx_), "om_step_reset"); }
void Device::sync() { check(ctx_, om_ctx_sync(ctx_), "om_ctx_sync"); }

int64_t numel_of(const std::vector<int> &shape) {
    int64_t n = 1;
    for (int d : shape) n *= d;
    return n;
}
Tensor make(const std::vector<int> &shape) {
    auto t = std::make_shared<TensorImpl>();
    t->shape = shape;
    t->numel = numel_of(shape);
    t->data = dev().step_floats(t->numel);
    return t;
}
Tensor make_ints(const std::vector<int> &shape) {
    auto t = std::make_shared<TensorImpl>();
    t->shape = shape;
    t->numel = numel_of(shape);
    t->idata = dev().step_ints(t->numel);
    return t;
}

static om_ctx *C() { return dev().ctx(); }
#define OMT(call) check(C(), (call), #call)

static std::string shape_str(const std::vector<int> &s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); i++) r += (i ? "," : "") + std::to_string(s[i]);
    return r + "]";
}
[[noreturn]] static void shape_error(const std::string &m) { throw Error(OM_E_ARG, m); }

// ------------------------------------------------------------------------------------------------ engine
void Record::unpack_check() const {
    for (const auto &s : saved)
        if (*s.first != s.second)
            throw Error(kErrTensorVersion, "A tensor saved for the backward pass was modified in place (saved at version " +
                                               std::to_string(s.second) + ", now " + std::to_string(*s.first) + ").");
}

void Engine::queue_dw(const om_linear_dw &item, int rows) {
    if (!item.dw && !item.db) return;
    if (!item.dw || item.out % 64 || item.in % 64) {
        // Never part of a grouped launch (it takes whole 64 x 64 tiles): run it now, so that it does not take one of
        // the four places of a group (a classifier head would otherwise push every later layer's products one place
        // along, splitting each layer's four over two launches).
        OMT(om_param_grads_group(C(), 1, &item, rows, 0, nullptr));
        return;
    }
    if (!dw_queue_.empty() && (rows != dw_rows_ || dw_queue_.size() == 4)) flush_dw();
    dw_queue_.push_back(item);
    dw_rows_ = rows;
    holders_[item.g]++;
    if (item.dw) {
        const char *b = reinterpret_cast<const char *>(item.dw);
        dw_ranges_.emplace_back(b, b + sizeof(float) * (uint64_t)item.in * item.out);
    }
    if (item.db) {
        const char *b = reinterpret_cast<const char *>(item.db);
        dw_ranges_.emplace_back(b, b + sizeof(float) * (uint64_t)item.out);
    }
}

void Engine::queue_colsum(const om_column_sum &item) {
    if (cs_queue_.size() == 8) flush_dw();
    cs_queue_.push_back(item);
    const char *b = reinterpret_cast<const char *>(item.out);
    dw_ranges_.emplace_back(b, b + sizeof(float) * (uint64_t)item.cols);
}

void Engine::flush_dw() {
    if (dw_queue_.empty() && cs_queue_.empty()) return;
    OMT(om_param_grads_group(C(), (int)dw_queue_.size(), dw_queue_.data(), dw_rows_, (int)cs_queue_.size(),
                             cs_queue_.data()));
    for (const om_linear_dw &it : dw_queue_) holders_[it.g]--;
    dw_queue_.clear();
    cs_queue_.clear();
    dw_ranges_.clear();
}

float *Engine::dest(Record &r, int i, int *acc) {
    *acc = 0;
    if (i >= (int)r.inputs.size() || !r.needs(i)) return nullptr;
    TensorImpl &x = *r.inputs[i];
    if (x.is_leaf()) {
        // AccumulateLeaf (Engine.cs:292-328): the first gradient creates Grad, later ones add into it.
        if (!x.grad) throw Error(OM_E_STATE, "leaf " + x.name + " requires a gradient but has no gradient buffer");
        if (queued_leaf(x.grad)) flush_dw();  // a queued launch writes this gradient first
        *acc = x.grad_live ? 1 : 0;
        x.grad_live = x.grad_exists = true;
        return x.grad;
    }
    Record &p = *x.grad_fn;
    if (!p.pending) {
        p.pending = dev().step_floats(x.numel);
        p.pending_borrowed = false;
        holders_[p.pending] = 1;
        return p.pending;
    }
    if (p.pending_borrowed) {
        if (sole_holder(p.pending)) {  // the lender is done with it: take it over
            p.pending_borrowed = false;
        } else {  // copy-on-write: the buffer is still another record's gradient
            float *nb = dev().step_floats(x.numel);
            OMT(om_copy(C(), nb, p.pending, sizeof(float) * (uint64_t)x.numel));
            holders_[p.pending]--;
            p.pending = nb;
            holders_[nb] = 1;
            p.pending_borrowed = false;
        }
    }
    *acc = 1;  // Engine.AddInto (Engine.cs:331-344)
    return p.pending;
}

float *Engine::dest_add(Record &r, int i, int *acc, const float **addend) {
    *addend = nullptr;
    if (i < (int)r.inputs.size() && r.needs(i) && !r.inputs[i]->is_leaf()) {
        Record &p = *r.inputs[i]->grad_fn;
        if (p.pending && p.pending_borrowed && !sole_holder(p.pending)) {
            // the borrowed gradient goes in as the addend; the result lands in a fresh buffer of this record's own
            float *nb = dev().step_floats(r.inputs[i]->numel);
            *addend = p.pending;
            holders_[p.pending]--;
            p.pending = nb;
            holders_[nb] = 1;
            p.pending_borrowed = false;
            *acc = 0;
            return nb;
        }
    }
    return dest(r, i, acc);
}

void Engine::emit_alias(Record &r, int i, const float *g) {
    if (i >= (int)r.inputs.size() || !r.needs(i)) return;
    TensorImpl &x = *r.inputs[i];
    uint64_t bytes = sizeof(float) * (uint64_t)x.numel;
    if (x.is_leaf()) {
        if (!x.grad) throw Error(OM_E_STATE, "leaf " + x.name + " requires a gradient but has no gradient buffer");
        if (queued_leaf(x.grad)) flush_dw();  // a queued launch writes this gradient first
        if (x.grad_live) {
            OMT(om_axpy(C(), 1.0f, g, x.grad, x.numel));
        } else {
            OMT(om_copy(C(), x.grad, g, bytes));
        }
        x.grad_live = x.grad_exists = true;
        return;
    }
    Record &p = *x.grad_fn;
    if (!p.pending) {
        p.pending = const_cast<float *>(g);
        p.pending_borrowed = true;
        holders_[g]++;
        return;
    }
    if (p.pending_borrowed && !sole_holder(p.pending)) {
        float *nb = dev().step_floats(x.numel);
        OMT(om_add(C(), p.pending, g, nb, x.numel));
        holders_[p.pending]--;
        p.pending = nb;
        holders_[nb] = 1;
        p.pending_borrowed = false;
        return;
    }
    p.pending_borrowed = false;
    OMT(om_axpy(C(), 1.0f, g, p.pending, x.numel));
}

void Engine::run(const Tensor &root) {
    // The seed gradient dL/dL = 1 is the device's persistent one; it is held as a borrowed buffer that is never
    // anyone's sole holding, so every gradient that would be added into it is copied first.
    float *g = const_cast<float *>(dev().one());
    if (root->is_leaf()) {
        Record tmp;
        tmp.inputs = {root};
        emit_alias(tmp, 0, g);
        return;
    }
    // Reverse topological order: iterative DFS post-order over input edges in input order (Engine.cs:130-158).
    uint64_t mark = ++g_pass;
    std::vector<Record *> order;
    std::vector<std::pair<Record *, size_t>> stack;
    root->grad_fn->mark = mark;
    stack.emplace_back(root->grad_fn.get(), 0);
    while (!stack.empty()) {
        Record *rec = stack.back().first;
        size_t next = stack.back().second;
        if (rec->released)
            throw Error(OM_E_STATE,
                        "Backward ran through a graph whose saved tensors were already freed by an earlier backward.");
        if (next < rec->inputs.size()) {
            stack.back().second = next + 1;
            const Tensor &x = rec->inputs[next];
            if (x && x->grad_fn && x->grad_fn->mark != mark) {
                x->grad_fn->mark = mark;
                stack.emplace_back(x->grad_fn.get(), 0);
            }
        } else {
            order.push_back(rec);
            stack.pop_back();
        }
    }
    holders_.clear();
    root->grad_fn->pending = g;
    root->grad_fn->pending_borrowed = true;
    holders_[g] = 1 << 30;
    for (size_t i = order.size(); i-- > 0;) {
        Record *r = order[i];
        float *gi = r->pending;
        r->pending = nullptr;
        if (!gi) continue;
        r->unpack_check();  // SavedTensor.Unpack's version check, before the rule reads anything
        r->rule(*this, *r, gi);
        holders_[gi]--;  // this record is done with its gradient
    }
    flush_dw();
    holders_.clear();
    // Release the records (BackwardRecord.Release): a second backward through this graph is an error.
    for (Record *r : order) {
        r->rule = nullptr;
        r->inputs.clear();
        r->saved.clear();
        r->released = true;
    }
}

void backward(const Tensor &root) {
    if (!root || !root->requires_grad) throw Error(OM_E_STATE, "Backward needs a tensor that requires gradients.");
    if (root->numel != 1) throw Error(OM_E_ARG, "Backward without a gradient needs a one-element tensor.");
    Engine e;
    e.run(root);
}

void zero_grad(const std::vector<Tensor> &leaves) {
    for (const Tensor &t : leaves)
        if (t->grad_exists) t->grad_live = false;  // the zero fill is deferred (settle_grads)
}
void settle_grads(const std::vector<Tensor> &leaves) {
    for (const Tensor &t : leaves)
        if (t->grad_exists && !t->grad_live) {
            OMT(om_zero(C(), t->grad, sizeof(float) * (uint64_t)t->numel));
            t->grad_live = true;
        }
}

// ------------------------------------------------------------------------------------------------ ops
static bool tracked(std::initializer_list<const Tensor *> xs) {
    for (const Tensor *x : xs)
        if (*x && (*x)->requires_grad) return true;
    return false;
}
// Records `op` on `out`. `saved` lists the tensors the rule reads (the reference's rec.Save slots); the output
// itself may be among them (Relu and LogSoftmax save their result).
static void attach(const Tensor &out, const char *op, std::vector<Tensor> inputs,
                   std::function<void(Engine &, Record &, const float *)> rule,
                   std::initializer_list<Tensor> saved = {}) {
    auto r = std::make_shared<Record>();
    r->op = op;
    r->inputs = std::move(inputs);
    r->rule = std::move(rule);
    r->out_numel = out->numel;
    for (const Tensor &t : saved) r->save(t);
    out->requires_grad = true;
    out->grad_fn = r;
}

// The Linear's backward from the gradient g of its output (inputs x, w and optionally b of record r): dx now, dW and
// db queued for the grouped weight-gradient launch, or all three in one launch for the small layers.
static void linear_backward(Engine &e, Record &r, const float *g, int rows, int in, int out) {
    int ax, aw, ab = 0;
    float *dx = e.dest(r, 0, &ax);
    if (om_linear_small(rows, in, out)) {  // dx, dw and db in one launch
        float *dw = e.dest(r, 1, &aw);
        float *db = r.inputs.size() > 2 ? e.dest(r, 2, &ab) : nullptr;
        OMT(om_linear_bwd(C(), g, r.inputs[0]->data, r.inputs[1]->data, dx, dw, db, rows, in, out, ax, aw, ab));
        return;
    }
    if (dx) OMT(om_linear_bwd(C(), g, r.inputs[0]->data, r.inputs[1]->data, dx, nullptr, nullptr, rows, in, out, ax, 0,
                              0));
    float *dw = e.dest(r, 1, &aw);
    float *db = r.inputs.size() > 2 ? e.dest(r, 2, &ab) : nullptr;
    e.queue_dw(om_linear_dw{g, r.inputs[0]->data, dw, db, in, out, aw, ab}, rows);
}

Tensor linear(const Tensor &x, const Tensor &w, const Tensor &b) {
    if (w->shape.size() != 2 || x->shape.empty() || x->shape.back() != w->shape[1])
        shape_error("Linear: input " + shape_str(x->shape) + " does not fit weights " + shape_str(w->shape) + " ([out, in]).");
    const int in = w->shape[1], out = w->shape[0];
    const int rows = (int)(x->numel / in);
    std::vector<int> ys = x->shape;
    ys.back() = out;
    if (dev().per_op) {  // Reshape, MatMul(x, W.T()), Add(bias), Reshape: Ops.Layers.cs:715-733
        Tensor y = matmul_wt(reshape(x, {rows, in}), w);
        if (b) y = add_rows(y, b);
        return reshape(y, ys);
    }
    Tensor y = make(ys);
    OMT(om_linear_fwd(C(), x->data, w->data, b ? b->data : nullptr, y->data, rows, in, out));
    if (tracked({&x, &w, &b})) {
        std::vector<Tensor> ins{x, w};
        if (b) ins.push_back(b);
        attach(y, "Linear", ins, [rows, in, out](Engine &e, Record &r, const float *g) {
            linear_backward(e, r, g, rows, in, out);
        }, {x, w});
    }
    return y;
}

// Linear then ReLU as one record (the pair of a conv stage's fused record, for dense layers): the forward is one
// launch with the ReLU in the product's epilogue; the backward applies the ReLU's rule (g where y > 0, from the
// saved output) and runs the Linear's backward on that gradient.
Tensor linear_relu(const Tensor &x, const Tensor &w, const Tensor &b) {
    if (w->shape.size() != 2 || x->shape.empty() || x->shape.back() != w->shape[1])
        shape_error("Linear: input " + shape_str(x->shape) + " does not fit weights " + shape_str(w->shape) + " ([out, in]).");
    const int in = w->shape[1], out = w->shape[0];
    const int rows = (int)(x->numel / in);
    std::vector<int> ys = x->shape;
    ys.back() = out;
    Tensor y = make(ys);
    OMT(om_linear_relu_fwd(C(), x->data, w->data, b ? b->data : nullptr, y->data, rows, in, out));
    if (tracked({&x, &w, &b})) {
        std::vector<Tensor> ins{x, w};
        if (b) ins.push_back(b);
        float *yd = y->data;
        attach(y, "LinearRelu", ins, [rows, in, out, yd](Engine &e, Record &r, const float *g) {
            if (!r.needs(0) && (in % 64 || out % 64) && !om_linear_small(rows, in, out)) {
                // dW and db only, of a product no grouped launch takes (it would run now anyway): om_linear_relu_bwd,
                // which applies the ReLU's rule as it reads g where the product is one launch
                int aw, ab = 0;
                float *dw = e.dest(r, 1, &aw);
                float *db = r.inputs.size() > 2 ? e.dest(r, 2, &ab) : nullptr;
                OMT(om_linear_relu_bwd(C(), g, yd, r.inputs[0]->data, r.inputs[1]->data, nullptr, dw, db, rows, in,
                                       out, 0, aw, ab));
                return;
            }
            const int64_t n = (int64_t)rows * out;
            float *gp = dev().step_floats(n);
            OMT(om_relu_bwd(C(), g, yd, gp, n, 0));
            linear_backward(e, r, gp, rows, in, out);
        }, {x, w, y});
    }
    return y;
}

Tensor relu(const Tensor &x) {
    Tensor y = make(x->shape);
    OMT(om_relu_fwd(C(), x->data, y->data, x->numel));
    if (tracked({&x})) {
        float *yd = y->data;
        int64_t n = x->numel;
        attach(y, "Relu", {x}, [yd, n](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            OMT(om_relu_bwd(C(), g, yd, dx, n, a));
        }, {y});
    }
    return y;
}

Tensor matmul_wt(const Tensor &x, const Tensor &w) {
    if (w->shape.size() != 2 || x->shape.size() != 2 || x->shape[1] != w->shape[1])
        shape_error("MatMul: " + shape_str(x->shape) + " does not fit the transposed weights " + shape_str(w->shape));
    const int rows = x->shape[0], in = w->shape[1], out = w->shape[0];
    Tensor y = make({rows, out});
    OMT(om_linear_fwd(C(), x->data, w->data, nullptr, y->data, rows, in, out));
    if (tracked({&x, &w}))
        attach(y, "MatMul", {x, w}, [rows, in, out](Engine &e, Record &r, const float *g) {
            // dA = g B^T and dB = A^T g (BackwardOps.cs:69-82) with B = W.T(): dW = g^T x, written as [out, in]
            int ax, aw;
            float *dx = e.dest(r, 0, &ax);
            float *dw = e.dest(r, 1, &aw);
            if (dx || dw)
                OMT(om_linear_bwd(C(), g, r.inputs[0]->data, r.inputs[1]->data, dx, dw, nullptr, rows, in, out, ax,
                                  aw, 0));
        }, {x, w});
    return y;
}

Tensor add_rows(const Tensor &x, const Tensor &b) {
    const int cols = b->numel > 0 ? (int)b->numel : 1;
    if (b->shape.size() != 1 || x->shape.empty() || x->shape.back() != cols)
        shape_error("Add: " + shape_str(b->shape) + " does not broadcast to " + shape_str(x->shape));
    const int rows = (int)(x->numel / cols);
    Tensor y = make(x->shape);
    OMT(om_add_rows(C(), x->data, b->data, y->data, rows, cols));
    if (tracked({&x, &b}))
        attach(y, "Add", {x, b}, [rows, cols](Engine &e, Record &r, const float *g) {
            e.emit_alias(r, 0, g);
            int a;
            float *db = e.dest(r, 1, &a);  // EmitSummed: SumTo over the broadcast rows in double
            if (db) OMT(om_colsum(C(), g, db, rows, cols, a));
        });
    return y;
}

Tensor sub(const Tensor &a, const Tensor &b) {
    if (a->shape != b->shape) shape_error("Sub: shapes " + shape_str(a->shape) + " and " + shape_str(b->shape) + " differ.");
    Tensor y = make(a->shape);
    OMT(om_sub(C(), a->data, b->data, y->data, a->numel));
    if (tracked({&a, &b})) {
        const int64_t n = a->numel;
        attach(y, "Sub", {a, b}, [n](Engine &e, Record &r, const float *g) {
            e.emit_alias(r, 0, g);
            int acc;
            float *d = e.dest(r, 1, &acc);  // Neg's rule: -g
            if (d) OMT(acc ? om_axpy(C(), -1.0f, g, d, n) : om_scale(C(), -1.0f, g, d, n));
        });
    }
    return y;
}

Tensor mul(const Tensor &a, const Tensor &b) {
    if (a->shape != b->shape) shape_error("Mul: shapes " + shape_str(a->shape) + " and " + shape_str(b->shape) + " differ.");
    Tensor y = make(a->shape);
    OMT(om_mul(C(), a->data, b->data, y->data, a->numel));
    if (tracked({&a, &b})) {
        const int64_t n = a->numel;
        attach(y, "Mul", {a, b}, [n](Engine &e, Record &r, const float *g) {
            // g * b to a, g * a to b (BackwardOps.cs:23-65); an emission into an existing gradient is added to it
            for (int i = 0; i < 2; i++) {
                int acc;
                float *d = e.dest(r, i, &acc);
                if (!d) continue;
                const float *other = r.inputs[1 - i]->data;
                if (!acc) {
                    OMT(om_mul(C(), g, other, d, n));
                } else {
                    float *t = dev().step_floats(n);
                    OMT(om_mul(C(), g, other, t, n));
                    OMT(om_axpy(C(), 1.0f, t, d, n));
                }
            }
        }, {a, b});
    }
    return y;
}

Tensor mean_all(const Tensor &x) {
    Tensor y = make({});
    if (om_readback *rb = dev().take_loss_post()) {  // the step's loss readback, when this Mean is the loss
        OMT(om_sum_all_post(C(), x->data, y->data, x->numel, 1, rb));
        dev().set_loss_posted(y->data);
    } else {
        OMT(om_sum_all(C(), x->data, y->data, x->numel, 1));
    }
    if (tracked({&x})) {
        const int64_t n = x->numel;
        attach(y, "Mean", {x}, [n](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            if (dx) OMT(om_mean_all_bwd(C(), g, dx, n, a));
        });
    }
    return y;
}

Tensor nll_loss(const Tensor &logp, const Tensor &labels) {
    if (logp->shape.size() != 2 || !labels->idata || labels->shape != std::vector<int>{logp->shape[0]})
        shape_error("NllLoss needs [N, C] log-probabilities and [N] Int32 targets, not " + shape_str(logp->shape) +
                    " and " + shape_str(labels->shape));
    const int rows = logp->shape[0], cols = logp->shape[1];
    Tensor loss = make({});
    OMT(om_nll_fwd(C(), logp->data, labels->idata, loss->data, nullptr, rows, cols, 1, -100));
    if (tracked({&logp})) {
        const int32_t *tg = labels->idata;
        attach(loss, "NllLoss", {logp}, [tg, rows, cols](Engine &e, Record &r, const float *g) {
            int a;
            float *d = e.dest(r, 0, &a);
            if (d) OMT(om_nll_bwd(C(), g, tg, d, rows, cols, 1, -100, a));
        }, {labels});
    }
    return loss;
}

Tensor gelu(const Tensor &x) {
    Tensor y = make(x->shape);
    OMT(om_gelu_fwd(C(), x->data, y->data, x->numel));
    if (tracked({&x})) {
        int64_t n = x->numel;
        attach(y, "Gelu", {x}, [n](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            OMT(om_gelu_bwd(C(), g, r.inputs[0]->data, dx, n, a));
        }, {x});
    }
    return y;
}

Tensor add(const Tensor &a, const Tensor &b) {
    if (a->shape != b->shape) shape_error("Add: shapes " + shape_str(a->shape) + " and " + shape_str(b->shape) + " differ.");
    Tensor y = make(a->shape);
    OMT(om_add(C(), a->data, b->data, y->data, a->numel));
    if (tracked({&a, &b}))
        attach(y, "Add", {a, b}, [](Engine &e, Record &r, const float *g) {
            e.emit_alias(r, 0, g);
            e.emit_alias(r, 1, g);
        });
    return y;
}

Tensor layer_norm(const Tensor &x, const Tensor &gamma, const Tensor &beta, float eps) {
    const int cols = x->shape.back();
    if (gamma->shape != std::vector<int>{cols} || beta->shape != std::vector<int>{cols})
        shape_error("LayerNorm over " + std::to_string(cols) + " features needs gamma and beta of shape [" +
                    std::to_string(cols) + "].");
    const int rows = (int)(x->numel / cols);
    Tensor y = make(x->shape);
    bool rec = tracked({&x, &gamma, &beta});
    float *mean = rec ? dev().step_floats(rows) : nullptr;
    float *rstd = rec ? dev().step_floats(rows) : nullptr;
    OMT(om_layernorm_fwd(C(), x->data, gamma->data, beta->data, y->data, mean, rstd, rows, cols, eps));
    if (rec && dev().per_op) {
        attach(y, "LayerNorm", {x, gamma, beta}, [rows, cols, mean, rstd](Engine &e, Record &r, const float *g) {
            // dx, dgamma and dbeta now, in one call (two when the parameter gradients' accumulation differs)
            int ax, ag, ab;
            float *dx = e.dest(r, 0, &ax);
            float *dg = e.dest(r, 1, &ag);
            float *db = e.dest(r, 2, &ab);
            const float *xd = r.inputs[0]->data, *gd = r.inputs[1]->data;
            if (!dg || !db || ag == ab) {
                OMT(om_layernorm_bwd(C(), g, xd, gd, mean, rstd, dx, dg, db, rows, cols, ax, dg ? ag : ab));
            } else {
                OMT(om_layernorm_bwd(C(), g, xd, gd, mean, rstd, dx, dg, nullptr, rows, cols, ax, ag));
                OMT(om_layernorm_bwd(C(), g, xd, gd, mean, rstd, nullptr, nullptr, db, rows, cols, 0, ab));
            }
        }, {x, gamma});
    } else if (rec)
        attach(y, "LayerNorm", {x, gamma, beta}, [rows, cols, mean, rstd](Engine &e, Record &r, const float *g) {
            // dx now; dgamma / dbeta as fp64 partials in step memory whose column sums are queued with the weight
            // gradients (om_param_grads_group)
            int ax, ag, ab;
            const float *dx_add = nullptr;
            float *dx = e.dest_add(r, 0, &ax, &dx_add);
            float *dg = e.dest(r, 1, &ag);
            float *db = e.dest(r, 2, &ab);
            const int chunks = om_layernorm_bwd_chunks(rows, cols);
            auto partials = [&]() { return reinterpret_cast<double *>(dev().step_floats(2 * (int64_t)chunks * cols)); };
            double *pg = dg ? partials() : nullptr;
            double *pb = db ? partials() : nullptr;
            OMT(om_layernorm_bwd_partials(C(), g, r.inputs[0]->data, r.inputs[1]->data, mean, rstd, dx_add, dx, ax, pg,
                                          pb, rows, cols));
            if (dg) e.queue_colsum(om_column_sum{pg, dg, chunks, cols, ag});
            if (db) e.queue_colsum(om_column_sum{pb, db, chunks, cols, ab});
        }, {x, gamma});
    return y;
}

Tensor attention_heads(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &mask, int heads) {
    if (q->shape.size() != 3 || k->shape != q->shape || v->shape != q->shape || heads < 1 || q->shape[2] % heads)
        shape_error("Attention needs [B, L, H*D] q/k/v of equal shape, got " + shape_str(q->shape));
    const int B = q->shape[0], L = q->shape[1], D = q->shape[2] / heads;
    if (D % 2) shape_error("Attention needs an even head dimension, got " + std::to_string(D));
    if (mask && mask->shape != std::vector<int>{B, L, L})
        shape_error("The mask must be [" + std::to_string(B) + "," + std::to_string(L) + "," + std::to_string(L) +
                    "], not " + shape_str(mask->shape));
    Tensor o = make(q->shape);
    const float *md = mask ? mask->data : nullptr;
    const int W = heads * D;
    float *st = dev().step_floats(2 * (int64_t)B * heads * L);  // per-query softmax statistics for the backward
    OMT(om_attention_fwd_flash(C(), q->data, k->data, v->data, W, md, 1, o->data, W, st, B, heads, L, D, 0.0f));
    const float *od = o->data;
    if (tracked({&q, &k, &v}))
        attach(o, "Attention", {q, k, v}, [md, st, od, B, heads, L, D, W](Engine &e, Record &r, const float *g) {
            int a[3];
            float *d[3];
            for (int i = 0; i < 3; i++) d[i] = e.dest(r, i, &a[i]);
            // one accumulate flag per call: outputs whose flag differs go through a temporary
            int common = a[0];
            float *tmp[3] = {nullptr, nullptr, nullptr};
            for (int i = 0; i < 3; i++)
                if (d[i] && a[i] != common) {
                    tmp[i] = dev().step_floats(r.inputs[i]->numel);
                }
            OMT(om_attention_bwd_flash(C(), r.inputs[0]->data, r.inputs[1]->data, r.inputs[2]->data, W, md, 1, od, W,
                                       st, g, W, tmp[0] ? tmp[0] : d[0], tmp[1] ? tmp[1] : d[1],
                                       tmp[2] ? tmp[2] : d[2], W, B, heads, L, D, 0.0f, common));
            for (int i = 0; i < 3; i++)
                if (tmp[i]) {
                    if (a[i]) OMT(om_axpy(C(), 1.0f, tmp[i], d[i], r.inputs[i]->numel));
                    else OMT(om_copy(C(), d[i], tmp[i], sizeof(float) * (uint64_t)r.inputs[i]->numel));
                }
        }, {q, k, v, mask});
    return o;
}

Tensor linear_residual(const Tensor &x, const Tensor &w, const Tensor &b, const Tensor &resid) {
    if (w->shape.size() != 2 || x->shape.empty() || x->shape.back() != w->shape[1])
        shape_error("Linear: input " + shape_str(x->shape) + " does not fit weights " + shape_str(w->shape) + " ([out, in]).");
    const int in = w->shape[1], out = w->shape[0];
    const int rows = (int)(x->numel / in);
    std::vector<int> ys = x->shape;
    ys.back() = out;
    if (resid->shape != ys) shape_error("Add: shapes " + shape_str(resid->shape) + " and " + shape_str(ys) + " differ.");
    Tensor y = make(ys);
    OMT(om_linear_fwd_resid(C(), x->data, w->data, b ? b->data : nullptr, resid->data, y->data, rows, in, out));
    if (tracked({&x, &w, &b, &resid})) {
        attach(y, "LinearAdd", {x, w, b, resid}, [rows, in, out](Engine &e, Record &r, const float *g) {
            int ax, aw, ab = 0;
            float *dx = e.dest(r, 0, &ax);
            if (dx) OMT(om_linear_bwd(C(), g, r.inputs[0]->data, r.inputs[1]->data, dx, nullptr, nullptr, rows, in, out,
                                      ax, 0, 0));
            float *dw = e.dest(r, 1, &aw);
            float *db = r.inputs[2] ? e.dest(r, 2, &ab) : nullptr;
            e.queue_dw(om_linear_dw{g, r.inputs[0]->data, dw, db, in, out, aw, ab}, rows);
            if (r.needs(3)) e.emit_alias(r, 3, g);  // Add backward: the residual gets g unchanged
        }, {x, w});
    }
    return y;
}

static void attach_mse(const Tensor &loss, const Tensor &pred, const Tensor &target, float *diff, float *unit,
                       int64_t n);

// The FeedForward record of y = Linear2(GELU(Linear1(x))) (+ resid): a is the GELU output, sl GELU's slope.
static void attach_ffn(const Tensor &y, const Tensor &x, const Tensor &w1, const Tensor &b1, const Tensor &w2,
                       const Tensor &b2, const Tensor &resid, float *a, float *sl, int rows, int d, int f, int o) {
    if (tracked({&x, &w1, &b1, &w2, &b2, &resid})) {
        attach(y, "FeedForward", {x, w1, b1, w2, b2, resid}, [sl, a, rows, d, f, o](Engine &e, Record &r, const float *g) {
            // The input-gradient chain (dh = (g W2) * GELU's slope, then dx = dh W1); both layers' weight and bias
            // gradients are queued for a grouped launch.
            int aw2, ab2 = 0;
            float *dw2 = e.dest(r, 3, &aw2);
            float *db2 = r.inputs[4] ? e.dest(r, 4, &ab2) : nullptr;
            om_linear_dw items[2];
            int n = 0;
            if (dw2 || db2) items[n++] = om_linear_dw{g, a, dw2, db2, f, o, aw2, ab2};
            const bool below = r.needs(0) || r.needs(1) || r.needs(2);
            bool folded = false;
            if (below) {
                float *dh = dev().step_floats((int64_t)rows * f);
                OMT(om_linear_bwd_dx_slope(C(), g, r.inputs[3]->data, sl, dh, rows, f, o));
                int ax, aw1, ab1 = 0;
                float *dx = e.dest(r, 0, &ax);
                float *dw1 = e.dest(r, 1, &aw1);
                float *db1 = r.inputs[2] ? e.dest(r, 2, &ab1) : nullptr;
                // the input is also the residual (a post-LN block) and its gradient starts here: the residual's
                // gradient g goes into the product's epilogue instead of a later add (the same bits)
                folded = dx && !ax && r.needs(5) && r.inputs[5].get() == r.inputs[0].get();
                if (folded)
                    OMT(om_linear_bwd_dx_resid(C(), dh, r.inputs[1]->data, g, dx, rows, d, f));
                else if (dx)
                    OMT(om_linear_bwd(C(), dh, r.inputs[0]->data, r.inputs[1]->data, dx, nullptr, nullptr, rows, d, f,
                                      ax, 0, 0));
                if (dw1 || db1) items[n++] = om_linear_dw{dh, r.inputs[0]->data, dw1, db1, d, f, aw1, ab1};
            }
            for (int i = 0; i < n; i++) e.queue_dw(items[i], rows);
            if (r.needs(5) && !folded) e.emit_alias(r, 5, g);
        }, {x, w1, w2});
    }
}

// Shapes of the feed-forward sub-block; returns rows, the widths d, f, o and the output shape.
static void ffn_shapes(const Tensor &x, const Tensor &w1, const Tensor &w2, const Tensor &resid, int &rows, int &d,
                       int &f, int &o, std::vector<int> &ys) {
    if (w1->shape.size() != 2 || w2->shape.size() != 2 || x->shape.empty() || x->shape.back() != w1->shape[1] ||
        w2->shape[1] != w1->shape[0])
        shape_error("FeedForward: input " + shape_str(x->shape) + " does not fit weights " + shape_str(w1->shape) +
                    " and " + shape_str(w2->shape));
    d = w1->shape[1];
    f = w1->shape[0];
    o = w2->shape[0];
    rows = (int)(x->numel / d);
    ys = x->shape;
    ys.back() = o;
    if (resid && resid->shape != ys)
        shape_error("Add: shapes " + shape_str(resid->shape) + " and " + shape_str(ys) + " differ.");
}

Tensor ffn(const Tensor &x, const Tensor &w1, const Tensor &b1, const Tensor &w2, const Tensor &b2,
           const Tensor &resid) {
    int rows, d, f, o;
    std::vector<int> ys;
    ffn_shapes(x, w1, w2, resid, rows, d, f, o, ys);
    float *a = dev().step_floats((int64_t)rows * f);   // GELU output, read by Linear2's weight gradient
    float *sl = dev().step_floats((int64_t)rows * f);  // GELU's slope at the pre-activation, all its backward needs
    OMT(om_linear_gelu_fwd_slope(C(), x->data, w1->data, b1 ? b1->data : nullptr, a, sl, rows, d, f));
    Tensor y = make(ys);
    if (resid) OMT(om_linear_fwd_resid(C(), a, w2->data, b2 ? b2->data : nullptr, resid->data, y->data, rows, f, o));
    else OMT(om_linear_fwd(C(), a, w2->data, b2 ? b2->data : nullptr, y->data, rows, f, o));
    attach_ffn(y, x, w1, b1, w2, b2, resid, a, sl, rows, d, f, o);
    return y;
}

Tensor ffn_mse(const Tensor &x, const Tensor &w1, const Tensor &b1, const Tensor &w2, const Tensor &b2,
               const Tensor &resid, const Tensor &target) {
    // One record pair, two launches fewer: the second product's epilogue also forms the loss's squared differences
    // and the unit gradient (om_linear_fwd_resid_mse). Taken when the loss's backward needs exactly what mse() keeps
    // for a tracked prediction and an untracked target (no diff); otherwise the two ops as they are.
    const bool fuse = resid && target && !target->requires_grad && tracked({&x, &w1, &b1, &w2, &b2, &resid});
    if (!fuse) return mse(ffn(x, w1, b1, w2, b2, resid), target);
    int rows, d, f, o;
    std::vector<int> ys;
    ffn_shapes(x, w1, w2, resid, rows, d, f, o, ys);
    if (target->shape != ys)
        shape_error("Mse: shapes " + shape_str(ys) + " and " + shape_str(target->shape) + " differ.");
    float *a = dev().step_floats((int64_t)rows * f);
    float *sl = dev().step_floats((int64_t)rows * f);
    OMT(om_linear_gelu_fwd_slope(C(), x->data, w1->data, b1 ? b1->data : nullptr, a, sl, rows, d, f));
    Tensor y = make(ys);
    const int64_t n = y->numel;
    float *unit = dev().step_floats(n);
    Tensor loss = make({});
    om_readback *rb = dev().take_loss_post();
    OMT(om_linear_fwd_resid_mse(C(), a, w2->data, b2 ? b2->data : nullptr, resid->data, target->data, y->data, unit,
                                loss->data, rows, f, o, rb));
    if (rb) dev().set_loss_posted(loss->data);
    attach_ffn(y, x, w1, b1, w2, b2, resid, a, sl, rows, d, f, o);
    attach_mse(loss, y, target, nullptr, unit, n);
    return loss;
}

Tensor attention_qkv(const Tensor &x, const Tensor &wq, const Tensor &bq, const Tensor &wk, const Tensor &bk,
                     const Tensor &wv, const Tensor &bv, const Tensor &mask, int heads) {
    const int64_t W = wq->shape.size() == 2 ? wq->shape[0] : 0;
    const int64_t WW = W * W;
    auto packed = [&](const float *a, const float *b, const float *c, int64_t n) {
        return a && b && c && b == a + n && c == b + n;
    };
    const bool square = W > 0 && wq->shape == std::vector<int>{(int)W, (int)W} && wk->shape == wq->shape &&
                        wv->shape == wq->shape && bq && bk && bv && bq->numel == W && bk->numel == W &&
                        bv->numel == W && x->shape.size() == 3 && x->shape[2] == W;
    if (!square || !packed(wq->data, wk->data, wv->data, WW) || !packed(bq->data, bk->data, bv->data, W))
        return attention_heads(linear(x, wq, bq), linear(x, wk, bk), linear(x, wv, bv), mask, heads);
    if (heads < 1 || W % heads) shape_error("Attention: width " + std::to_string(W) + " is not a multiple of the head count");
    const int B = x->shape[0], L = x->shape[1], D = (int)(W / heads), w = (int)W;
    if (D % 2) shape_error("Attention needs an even head dimension, got " + std::to_string(D));
    if (mask && mask->shape != std::vector<int>{B, L, L})
        shape_error("The mask must be [" + std::to_string(B) + "," + std::to_string(L) + "," + std::to_string(L) +
                    "], not " + shape_str(mask->shape));
    const int rows = B * L;
    // q | k | v as one Linear(W -> 3W): the weights [3W, W] and biases [3W] are the packed arena blocks.
    float *qkv = dev().step_floats((int64_t)rows * 3 * W);
    OMT(om_linear_fwd(C(), x->data, wq->data, bq->data, qkv, rows, w, 3 * w));
    Tensor o = make(x->shape);
    const float *md = mask ? mask->data : nullptr;
    float *st = dev().step_floats(2 * (int64_t)B * heads * L);  // per-query softmax statistics for the backward
    OMT(om_attention_fwd_flash(C(), qkv, qkv + W, qkv + 2 * W, 3 * w, md, 1, o->data, w, st, B, heads, L, D, 0.0f));
    const float *od = o->data;
    if (tracked({&x, &wq, &bq, &wk, &bk, &wv, &bv}))
        attach(o, "AttentionQKV", {x, wq, bq, wk, bk, wv, bv},
               [qkv, md, st, od, B, L, heads, D, w, rows, WW](Engine &e, Record &r, const float *g) {
                   const int64_t W = w;
                   float *dqkv = dev().step_floats((int64_t)rows * 3 * W);
                   OMT(om_attention_bwd_flash(C(), qkv, qkv + W, qkv + 2 * W, 3 * w, md, 1, od, w, st, g, w, dqkv,
                                              dqkv + W, dqkv + 2 * W, 3 * w, B, heads, L, D, 0.0f, 0));
                   int ax, a[6];
                   // x's gradient may already be a residual's gradient another record still holds (a post-LN
                   // layer's input feeds both the attention and the residual Add): it then goes in as the addend of
                   // the input-gradient product (dx = addend + dqkv W, the bits of the product added to it), which
                   // spares a copy of it before the add
                   const float *dx_add = nullptr;
                   float *dx = e.dest_add(r, 0, &ax, &dx_add);
                   float *d[6];
                   for (int i = 0; i < 6; i++) d[i] = e.dest(r, 1 + i, &a[i]);
                   // d = {dwq, dbq, dwk, dbk, dwv, dbv}: one dW / db launch when the three leaves' gradients are the
                   // packed blocks with one accumulate flag, else through a temporary added or copied into each.
                   auto direct = [&](int first, int64_t n) {
                       return d[first] && d[first + 2] && d[first + 4] && d[first + 2] == d[first] + n &&
                              d[first + 4] == d[first + 2] + n && a[first] == a[first + 2] && a[first] == a[first + 4];
                   };
                   const bool dw_direct = direct(0, WW), db_direct = direct(1, W);
                   const bool any_w = d[0] || d[2] || d[4], any_b = d[1] || d[3] || d[5];
                   float *dw = !any_w ? nullptr : dw_direct ? d[0] : dev().step_floats(3 * WW);
                   float *db = !any_b ? nullptr : db_direct ? d[1] : dev().step_floats(3 * W);
                   if (dx && dx_add) {
                       OMT(om_linear_bwd_dx_resid(C(), dqkv, r.inputs[1]->data, dx_add, dx, rows, w, 3 * w));
                       dx = nullptr;
                   }
                   if ((!any_w || dw_direct) && (!any_b || db_direct)) {
                       // the packed leaves' gradients directly: the input gradient now, dW and db queued
                       if (dx) OMT(om_linear_bwd(C(), dqkv, r.inputs[0]->data, r.inputs[1]->data, dx, nullptr, nullptr,
                                                 rows, w, 3 * w, ax, 0, 0));
                       e.queue_dw(om_linear_dw{dqkv, r.inputs[0]->data, dw, db, w, 3 * w, a[0], a[1]}, rows);
                       return;
                   }
                   OMT(om_linear_bwd(C(), dqkv, r.inputs[0]->data, r.inputs[1]->data, dx, dw, db, rows, w, 3 * w, ax,
                                     dw_direct ? a[0] : 0, db_direct ? a[1] : 0));
                   for (int i = 0; i < 6; i++) {
                       const bool isw = (i % 2) == 0;
                       if (!d[i] || (isw ? dw_direct : db_direct)) continue;
                       const int64_t n = isw ? WW : W;
                       const float *src = (isw ? dw : db) + (i / 2) * n;
                       if (a[i]) OMT(om_axpy(C(), 1.0f, src, d[i], n));
                       else OMT(om_copy(C(), d[i], src, sizeof(float) * (uint64_t)n));
                   }
               }, {x, wq, wk, wv, mask});
    return o;
}

Tensor reshape(const Tensor &x, const std::vector<int> &shape) {
    std::vector<int> s = shape;
    int64_t known = 1;
    int infer = -1;
    for (size_t i = 0; i < s.size(); i++) {
        if (s[i] == -1) infer = (int)i;
        else known *= s[i];
    }
    if (infer >= 0) s[infer] = (int)(x->numel / (known ? known : 1));
    if (numel_of(s) != x->numel) shape_error("Cannot reshape " + shape_str(x->shape) + " to " + shape_str(shape));
    auto y = std::make_shared<TensorImpl>();
    y->shape = s;
    y->numel = x->numel;
    y->data = x->data;  // a view: same memory, same version counter
    y->idata = x->idata;
    y->version = x->version;
    if (tracked({&x})) attach(y, "Reshape", {x}, [](Engine &e, Record &r, const float *g) { e.emit_alias(r, 0, g); });
    return y;
}

Tensor permute(const Tensor &x, const std::vector<int> &perm) {
    const int nd = (int)x->shape.size();
    if ((int)perm.size() != nd) shape_error("Permute: rank mismatch");
    std::vector<int> ys(nd), inv(nd);
    for (int i = 0; i < nd; i++) {
        ys[i] = x->shape[perm[i]];
        inv[perm[i]] = i;
    }
    Tensor y = make(ys);
    std::vector<int32_t> s32(x->shape.begin(), x->shape.end()), p32(perm.begin(), perm.end());
    OMT(om_permute(C(), x->data, y->data, nd, s32.data(), p32.data(), 0));
    if (tracked({&x})) {
        std::vector<int32_t> yshape(ys.begin(), ys.end()), inv32(inv.begin(), inv.end());
        attach(y, "Permute", {x}, [yshape, inv32, nd](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            OMT(om_permute(C(), g, dx, nd, yshape.data(), inv32.data(), a));
        });
    }
    return y;
}

Tensor mean_axis(const Tensor &x, int axis) {
    const int nd = (int)x->shape.size();
    int ax = axis < 0 ? axis + nd : axis;
    if (ax < 0 || ax >= nd) shape_error("Mean: axis out of range");
    int outer = 1, inner = 1, n = x->shape[ax];
    std::vector<int> ys;
    for (int i = 0; i < nd; i++) {
        if (i < ax) outer *= x->shape[i];
        if (i > ax) inner *= x->shape[i];
        if (i != ax) ys.push_back(x->shape[i]);
    }
    Tensor y = make(ys);
    OMT(om_mean_axis(C(), x->data, y->data, outer, n, inner));
    if (tracked({&x}))
        attach(y, "Mean", {x}, [outer, n, inner](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            OMT(om_mean_axis_bwd(C(), g, dx, outer, n, inner, a));
        });
    return y;
}

// Mean over axis 2 of x [B, C, H, W], then Permute(2, 0, 1) to [W, B, C], as one record (the CRNN's sequence head):
// one launch each way, the bits of the two ops.
Tensor mean_permute_seq(const Tensor &x) {
    if (x->shape.size() != 4) shape_error("Mean then Permute: input " + shape_str(x->shape) + " is not [B, C, H, W].");
    const int B = x->shape[0], Cc = x->shape[1], H = x->shape[2], W = x->shape[3];
    Tensor y = make({W, B, Cc});
    OMT(om_mean_permute_fwd(C(), x->data, y->data, B, Cc, H, W));
    if (tracked({&x}))
        attach(y, "MeanPermute", {x}, [B, Cc, H, W](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            if (dx) OMT(om_mean_permute_bwd(C(), g, dx, B, Cc, H, W, a));
        });
    return y;
}

Tensor log_softmax(const Tensor &x) {
    const int cols = x->shape.back();
    const int rows = (int)(x->numel / cols);
    Tensor y = make(x->shape);
    OMT(om_logsoftmax_fwd(C(), x->data, y->data, rows, cols));
    if (tracked({&x})) {
        float *yd = y->data;
        attach(y, "LogSoftmax", {x}, [yd, rows, cols](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            OMT(om_logsoftmax_bwd(C(), g, yd, dx, rows, cols, a));
        }, {y});
    }
    return y;
}

Tensor cross_entropy(const Tensor &logits, const Tensor &labels) {
    if (logits->shape.size() != 2 || !labels->idata || labels->shape != std::vector<int>{logits->shape[0]})
        shape_error("NllLoss needs [N, C] log-probabilities and [N] Int32 targets, not " + shape_str(logits->shape) +
                    " and " + shape_str(labels->shape));
    if (dev().per_op) return nll_loss(log_softmax(logits), labels);  // Losses.cs:20-40
    const int rows = logits->shape[0], cols = logits->shape[1];
    Tensor logp = make(logits->shape);
    Tensor loss = make({});
    const bool rec = tracked({&logits});
    // As for Mse: the gradient for a unit upstream gradient comes with the forward (and the loss posts itself when
    // the step offers its readback), since the loss is normally the backward's root, seeded with exactly that unit.
    float *unit = rec ? dev().step_floats(logits->numel) : nullptr;
    if (unit) {
        om_readback *rb = dev().take_loss_post();
        OMT(om_xent_fwd_unit(C(), logits->data, labels->idata, logp->data, loss->data, nullptr, unit, rows, cols, -100,
                             rb));
        if (rb) dev().set_loss_posted(loss->data);
    } else {
        OMT(om_logsoftmax_fwd(C(), logits->data, logp->data, rows, cols));
        OMT(om_nll_fwd(C(), logp->data, labels->idata, loss->data, nullptr, rows, cols, 1, -100));
    }
    if (rec) {
        float *lp = logp->data;
        const int32_t *tg = labels->idata;
        attach(loss, "CrossEntropy", {logits}, [lp, tg, rows, cols, unit](Engine &e, Record &r, const float *g) {
            if (g == dev().one()) {
                e.emit_alias(r, 0, unit);
                return;
            }
            int a;
            float *dz = e.dest(r, 0, &a);
            OMT(om_xent_bwd(C(), g, lp, tg, dz, rows, cols, 1, -100, a));
        }, {labels});
    }
    return loss;
}

Tensor mse(const Tensor &pred, const Tensor &target) {
    if (pred->shape != target->shape)
        shape_error("Mse: shapes " + shape_str(pred->shape) + " and " + shape_str(target->shape) + " differ.");
    if (dev().per_op) {  // Losses.Mse (Losses.cs:86-91): d = Sub(pred, target); Mean(Mul(d, d))
        Tensor d = sub(pred, target);
        return mean_all(mul(d, d));
    }
    const int64_t n = pred->numel;
    Tensor loss = make({});
    const bool rec = tracked({&pred, &target});
    // the gradient for a unit upstream gradient comes with the forward: the loss is normally the backward's root,
    // whose seed gradient is exactly that unit. diff is then kept only when the target needs a gradient; another
    // upstream gradient recomputes it (om_sub, the forward's own subtraction)
    float *unit = rec && pred->requires_grad ? dev().step_floats(n) : nullptr;
    float *diff = !unit || target->requires_grad ? dev().step_floats(n) : nullptr;
    if (om_readback *rb = dev().take_loss_post()) {
        OMT(om_mse_fwd_post(C(), pred->data, target->data, diff, loss->data, unit, n, rb));
        dev().set_loss_posted(loss->data);
    } else if (unit) {
        OMT(om_mse_fwd_unit(C(), pred->data, target->data, diff, loss->data, unit, n));
    } else {
        OMT(om_mse_fwd(C(), pred->data, target->data, diff, loss->data, n));
    }
    if (rec) attach_mse(loss, pred, target, diff, unit, n);
    return loss;
}

// The Mse record (Losses.cs:86-91) of a loss already computed: diff (may be NULL: recomputed with om_sub when needed)
// and the gradient for a unit upstream gradient (may be NULL).
static void attach_mse(const Tensor &loss, const Tensor &pred, const Tensor &target, float *diff, float *unit,
                       int64_t n) {
        attach(loss, "Mse", {pred, target}, [diff, unit, n](Engine &e, Record &r, const float *g) {
            const float *d = diff;
            if (!d && (g != dev().one() || r.needs(1))) {
                float *t = dev().step_floats(n);
                OMT(om_sub(C(), r.inputs[0]->data, r.inputs[1]->data, t, n));
                d = t;
            }
            if (unit && g == dev().one()) {
                e.emit_alias(r, 0, unit);
            } else {
                int a;
                float *dp = e.dest(r, 0, &a);
                if (dp) OMT(om_mse_bwd(C(), g, d, dp, n, a));
            }
            if (r.needs(1)) {  // Sub backward negates the second input's gradient
                float *t = dev().step_floats(n);
                OMT(om_mse_bwd(C(), g, d, t, n, 0));
                int b;
                float *dt = e.dest(r, 1, &b);
                if (b) OMT(om_axpy(C(), -1.0f, t, dt, n));
                else OMT(om_scale(C(), -1.0f, t, dt, n));
            }
        });
}

struct ConvGeom {
    int N, Cin, H, W, Cout, KH, KW, OH, OW, stride, pad;
};
static ConvGeom conv_geom(const Tensor &x, const Tensor &w, int stride, int pad) {
    if (x->shape.size() != 4 || w->shape.size() != 4 || w->shape[1] != x->shape[1])
        shape_error("Conv2d: weights " + shape_str(w->shape) + " do not fit input " + shape_str(x->shape));
    ConvGeom c{x->shape[0], x->shape[1], x->shape[2], x->shape[3], w->shape[0], w->shape[2], w->shape[3], 0, 0,
               stride, pad};
    c.OH = (c.H + 2 * pad - c.KH) / stride + 1;
    c.OW = (c.W + 2 * pad - c.KW) / stride + 1;
    if (c.OH < 1 || c.OW < 1) shape_error("Invalid convolution geometry for input " + shape_str(x->shape));
    return c;
}
// ConvBackward (BackwardNn.cs:317-402) of record r (inputs x, w[, b]) for the output gradient g.
static void conv_backward(Engine &e, Record &r, const float *g, const ConvGeom &c) {
    int ax, aw, ab = 0;
    float *dx = e.dest(r, 0, &ax);
    float *dw = e.dest(r, 1, &aw);
    float *db = r.inputs.size() > 2 ? e.dest(r, 2, &ab) : nullptr;
    if (dw && db && aw != ab) {
        if (!aw) OMT(om_zero(C(), dw, sizeof(float) * (uint64_t)r.inputs[1]->numel));
        if (!ab) OMT(om_zero(C(), db, sizeof(float) * (uint64_t)c.Cout));
        aw = ab = 1;
    }
    OMT(om_conv2d_bwd(C(), g, r.inputs[0]->data, r.inputs[1]->data, dx, dw, db, c.N, c.Cin, c.H, c.W, c.Cout, c.KH,
                      c.KW, c.stride, c.pad, ax, dw ? aw : ab));
}

Tensor conv2d(const Tensor &x, const Tensor &w, const Tensor &b, int stride, int pad) {
    const ConvGeom c = conv_geom(x, w, stride, pad);
    Tensor y = make({c.N, c.Cout, c.OH, c.OW});
    OMT(om_conv2d_fwd(C(), x->data, w->data, b ? b->data : nullptr, y->data, c.N, c.Cin, c.H, c.W, c.Cout, c.KH, c.KW,
                      stride, pad));
    if (tracked({&x, &w, &b})) {
        std::vector<Tensor> ins{x, w};
        if (b) ins.push_back(b);
        attach(y, "Conv2d", ins, [=](Engine &e, Record &r, const float *g) { conv_backward(e, r, g, c); }, {x, w});
    }
    return y;
}

Tensor conv2d_relu_pool(const Tensor &x, const Tensor &w, const Tensor &b, int stride, int pad, int kh, int kw, int sh,
                        int sw) {
    const ConvGeom c = conv_geom(x, w, stride, pad);
    const int PH = (c.OH - kh) / sh + 1, PW = (c.OW - kw) / sw + 1;
    if (PH < 1 || PW < 1) shape_error("MaxPool2d: window larger than the input");
    Tensor a = make({c.N, c.Cout, c.OH, c.OW});  // Relu(Conv2d(x))
    Tensor y = make({c.N, c.Cout, PH, PW});
    const bool rec = tracked({&x, &w, &b});
    int32_t *idx = rec ? dev().step_ints((int64_t)c.N * c.Cout * PH * PW) : nullptr;
    OMT(om_conv2d_relu_pool_fwd(C(), x->data, w->data, b ? b->data : nullptr, a->data, y->data, idx, c.N, c.Cin, c.H,
                                c.W, c.Cout, c.KH, c.KW, stride, pad, kh, kw, sh, sw));
    if (rec) {
        std::vector<Tensor> ins{x, w};
        if (b) ins.push_back(b);
        const float *ad = a->data;
        attach(y, "Conv2dReluMaxPool", ins, [=](Engine &e, Record &r, const float *g) {
            // MaxPool's rule then Relu's, in one pass, into the convolution's output gradient
            float *ga = dev().step_floats((int64_t)c.N * c.Cout * c.OH * c.OW);
            OMT(om_maxpool_relu_bwd(C(), g, idx, ad, ga, c.N, c.Cout, c.OH, c.OW, PH, PW, kh, kw, sh, sw, 0, 0, 0));
            conv_backward(e, r, ga, c);
        }, {x, w, a});
    }
    return y;
}

Tensor relu_mean_plane(const Tensor &x) {
    if (x->shape.size() != 4) shape_error("ReluMean needs an (N,C,H,W) input, not " + shape_str(x->shape));
    const int N = x->shape[0], Cc = x->shape[1], plane = x->shape[2] * x->shape[3];
    Tensor y = make({N, Cc});
    OMT(om_relu_mean_rows(C(), x->data, y->data, N * Cc, plane));
    if (tracked({&x})) {
        const float *xd = x->data;
        attach(y, "ReluMean", {x}, [=](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            if (dx) OMT(om_relu_mean_rows_bwd(C(), g, xd, dx, N * Cc, plane, a));
        }, {x});
    }
    return y;
}

Tensor max_pool2d(const Tensor &x, int kh, int kw, int sh, int sw) {
    if (x->shape.size() != 4) shape_error("MaxPool2d needs an (N,C,H,W) input, not " + shape_str(x->shape));
    const int N = x->shape[0], Cc = x->shape[1], H = x->shape[2], W = x->shape[3];
    const int OH = (H - kh) / sh + 1, OW = (W - kw) / sw + 1;
    Tensor y = make({N, Cc, OH, OW});
    bool rec = tracked({&x});
    int32_t *idx = rec ? dev().step_ints((int64_t)N * Cc * OH * OW) : nullptr;
    OMT(om_maxpool_fwd(C(), x->data, y->data, idx, N, Cc, H, W, kh, kw, sh, sw, 0, 0));
    if (rec)
        attach(y, "MaxPool2d", {x}, [=](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            OMT(om_maxpool_bwd(C(), g, idx, dx, N, Cc, H, W, OH, OW, kh, kw, sh, sw, 0, 0, a));
        });
    return y;
}

Tensor ctc_loss(const Tensor &lp, const std::vector<int32_t> &targets, const std::vector<int32_t> &in_len,
                const std::vector<int32_t> &tgt_len, int blank, int reduction, const Tensor &d_targets,
                const Tensor &d_in_len, const Tensor &d_tgt_len) {
    if (lp->shape.size() != 3) shape_error("CtcLoss needs log-probabilities [T,B,C], not " + shape_str(lp->shape));
    const int T = lp->shape[0], B = lp->shape[1], Cc = lp->shape[2];
    if ((int)in_len.size() != B || (int)tgt_len.size() != B)
        shape_error("Expected " + std::to_string(B) + " input and target lengths");
    const int32_t *dt = d_targets ? d_targets->idata : nullptr, *dil = d_in_len ? d_in_len->idata : nullptr,
                  *dtl = d_tgt_len ? d_tgt_len->idata : nullptr;
    auto upload = [&](const std::vector<int32_t> &h) {
        int32_t *d = dev().step_ints((int64_t)h.size());
        OMT(om_upload(C(), d, h.data(), sizeof(int32_t) * h.size()));
        return d;
    };
    if (!dt) dt = upload(targets);
    if (!dil) dil = upload(in_len);
    if (!dtl) dtl = upload(tgt_len);
    Tensor loss = reduction == 0 ? make({B}) : make({});
    if (!tracked({&lp})) {
        OMT(om_ctc_fwd(C(), lp->data, dt, dil, dtl, in_len.data(), tgt_len.data(), targets.data(),
                       (int)targets.size(), T, B, Cc, blank, reduction, 0, loss->data));
        return loss;
    }
    // the forward also runs the beta recursion (beside alpha) and keeps both tables for the backward, which then only
    // forms the gradient
    int max_tgt = 0;
    for (int32_t l : tgt_len) max_tgt = l > max_tgt ? l : max_tgt;
    const uint64_t tb = om_ctc_tables_bytes(T, B, max_tgt);
    double *tables = reinterpret_cast<double *>(dev().step_floats((int64_t)((tb + 3) / 4)));
    OMT(om_ctc_fwd_tables(C(), lp->data, dt, dil, dtl, in_len.data(), tgt_len.data(), targets.data(),
                          (int)targets.size(), T, B, Cc, blank, reduction, 0, loss->data, tables, tb));
    attach(loss, "CtcLoss", {lp}, [=](Engine &e, Record &r, const float *g) {
        int a;
        float *d = e.dest(r, 0, &a);
        OMT(om_ctc_bwd_tables(C(), r.inputs[0]->data, dt, dil, dtl, in_len.data(), tgt_len.data(), targets.data(),
                              (int)targets.size(), g, d, T, B, Cc, blank, reduction, a, tables, tb));
    }, {lp, d_targets, d_in_len, d_tgt_len});
    return loss;
}

Tensor avg_pool2d(const Tensor &x, int k, int s, int p, bool count_include_pad) {
    if (x->shape.size() != 4) shape_error("AvgPool2d needs an (N,C,H,W) input, not " + shape_str(x->shape));
    const int N = x->shape[0], Cc = x->shape[1], H = x->shape[2], W = x->shape[3];
    const int OH = (H + 2 * p - k) / s + 1, OW = (W + 2 * p - k) / s + 1;
    Tensor y = make({N, Cc, OH, OW});
    const int cip = count_include_pad ? 1 : 0;
    OMT(om_avgpool2d_fwd(C(), x->data, y->data, N * Cc, H, W, k, k, s, s, p, p, cip));
    if (tracked({&x}))
        attach(y, "AvgPool2d", {x}, [=](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            OMT(om_avgpool2d_bwd(C(), g, dx, N * Cc, H, W, k, k, s, s, p, p, cip, a));
        });
    return y;
}

Tensor batch_norm2d(const Tensor &x, const Tensor &gamma, const Tensor &beta, float *running_mean,
                    float *running_var, bool training, float momentum, float eps) {
    if (x->shape.size() != 4) shape_error("BatchNorm2d needs an (N,C,H,W) input, not " + shape_str(x->shape));
    const int N = x->shape[0], Cc = x->shape[1], plane = x->shape[2] * x->shape[3];
    if (gamma->numel != Cc || beta->numel != Cc)
        shape_error("BatchNorm2d over " + std::to_string(Cc) + " channels needs per-channel tensors");
    Tensor y = make(x->shape);
    float *mean = dev().step_floats(Cc), *inv = dev().step_floats(Cc);
    const int tr = training ? 1 : 0;
    OMT(om_batchnorm2d_fwd(C(), x->data, gamma->data, beta->data, running_mean, running_var, y->data, mean, inv, N,
                           Cc, plane, tr, momentum, eps));
    if (tracked({&x, &gamma, &beta}))
        attach(y, "BatchNorm", {x, gamma, beta}, [=](Engine &e, Record &r, const float *g) {
            int ax, ag, ab;
            float *dx = e.dest(r, 0, &ax), *dg = e.dest(r, 1, &ag), *db = e.dest(r, 2, &ab);
            const float *xd = r.inputs[0]->data, *gd = r.inputs[1]->data;
            if (!dg || !db || ag == ab) {
                OMT(om_batchnorm2d_bwd(C(), g, xd, gd, mean, inv, dx, dg, db, N, Cc, plane, tr, ax, dg ? ag : ab));
            } else {  // the two parameter gradients need different accumulation: one launch each
                OMT(om_batchnorm2d_bwd(C(), g, xd, gd, mean, inv, dx, dg, nullptr, N, Cc, plane, tr, ax, ag));
                OMT(om_batchnorm2d_bwd(C(), g, xd, gd, mean, inv, nullptr, nullptr, db, N, Cc, plane, tr, 0, ab));
            }
        }, {x, gamma});
    return y;
}

Tensor embedding(const Tensor &table, const Tensor &ids, int padding_index) {
    if (table->shape.size() != 2 || !ids->idata)
        shape_error("Embedding needs a [count, width] table and Int32 ids, not " + shape_str(table->shape));
    const int rows = table->shape[0], dim = table->shape[1];
    std::vector<int> ys = ids->shape;
    ys.push_back(dim);
    Tensor y = make(ys);
    const int64_t n = ids->numel;
    OMT(om_embedding_fwd(C(), table->data, ids->idata, y->data, n, dim, rows));
    if (tracked({&table})) {
        const int32_t *id = ids->idata;
        attach(y, "Embedding", {table}, [=](Engine &e, Record &r, const float *g) {
            int a;
            float *dt = e.dest(r, 0, &a);
            OMT(om_embedding_bwd(C(), g, id, dt, n, dim, rows, padding_index, a));
        }, {ids});
    }
    return y;
}

Tensor dropout(const Tensor &x, float p, uint64_t seed, int64_t draw) {
    Tensor y = make(x->shape);
    const int64_t n = x->numel;
    OMT(om_dropout_fwd(C(), x->data, y->data, n, p, seed, draw));
    if (tracked({&x}))
        attach(y, "Mul", {x}, [=](Engine &e, Record &r, const float *g) {
            int a;
            float *dx = e.dest(r, 0, &a);
            OMT(om_dropout_bwd(C(), g, dx, n, p, seed, draw, a));
        });
    return y;
}

}  // namespace omt
