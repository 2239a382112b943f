// Modules, the parameter arena, optimizers, the benchmark configurations and the C ABI of include/om_train.h.
#include <climits>
#include <cmath>
#include <cstring>
#include <deque>
#include <map>
#include <utility>

#include "checkpoint.hpp"
#include "om_train.h"
#include "schedules.hpp"
#include "tape.hpp"

namespace omt {

// ------------------------------------------------------------------------------------------------ generator
uint64_t Generator::next_u64() {
    // SplitMix64 (Steele, Lea and Flood 2014), as Generator.NextUInt64 (Generator.cs:27-31)
    uint64_t z = (s_ += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
float Generator::next_single() { return (float)(next_u64() >> 40) * (1.0f / 16777216.0f); }
void Generator::fill_uniform(float lo, float hi, std::vector<float> &v) {
    for (float &x : v) x = uniform(lo, hi);
}
void Generator::fill_normal(std::vector<float> &v) {
    for (float &x : v) {
        double u1 = ((double)(next_u64() >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(next_u64() >> 11) * (1.0 / 9007199254740992.0);
        x = (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
}
void Generator::fill_ints(int32_t lo, int32_t hi, std::vector<int32_t> &v) {
    uint64_t span = (uint64_t)(hi - lo);
    for (int32_t &x : v) x = lo + (int32_t)(next_u64() % span);
}

static float fan_in_bound(int fan_in) { return 1.0f / std::sqrt((float)fan_in); }  // Layers.cs:59

// ------------------------------------------------------------------------------------------------ modules
Tensor Module::param(const std::string &name, std::vector<int> shape, std::vector<float> init) {
    auto t = std::make_shared<TensorImpl>();
    t->shape = std::move(shape);
    t->numel = numel_of(t->shape);
    t->requires_grad = true;
    t->name = name;
    params_.emplace_back(name, t);
    init_.push_back(std::move(init));
    return t;
}
void Module::named_parameters(std::vector<std::pair<std::string, Tensor>> &out, const std::string &prefix) const {
    for (auto &p : params_) out.emplace_back(prefix + p.first, p.second);
    for (auto &c : children_) c.second->named_parameters(out, prefix + c.first + ".");
}
float *Module::buffer(const std::string &name, const std::vector<float> &init) {
    const uint64_t bytes = sizeof(float) * (init.empty() ? 1 : init.size());
    float *d = (float *)dev().persistent(bytes);
    if (!init.empty()) check(dev().ctx(), om_upload(dev().ctx(), d, init.data(), bytes), "buffer upload");
    BufferRef r;
    r.dev = d;
    r.numel = (int64_t)init.size();
    buffers_.emplace_back(name, r);
    return d;
}
void Module::buffer_i64(const std::string &name, int64_t *host) {
    BufferRef r;
    r.host = host;
    r.numel = 1;
    buffers_.emplace_back(name, r);
}
void Module::named_buffers(std::vector<std::pair<std::string, BufferRef>> &out, const std::string &prefix) const {
    for (auto &b : buffers_) out.emplace_back(prefix + b.first, b.second);
    for (auto &c : children_) c.second->named_buffers(out, prefix + c.first + ".");
}
void Module::state(std::vector<StateRef> &out, const std::string &prefix) const {
    for (auto &p : params_) out.push_back({prefix + p.first, p.second, {}});
    for (auto &b : buffers_) out.push_back({prefix + b.first, nullptr, b.second});
    for (auto &c : children_) c.second->state(out, prefix + c.first + ".");
}
void Module::colocation_groups(std::vector<std::vector<Tensor>> &out) const {
    for (auto &g : colocate_) out.push_back(g);
    for (auto &c : children_) c.second->colocation_groups(out);
}
void Module::take_init(std::vector<std::vector<float>> &out) {
    for (auto &v : init_) out.push_back(std::move(v));
    init_.clear();
    for (auto &c : children_) c.second->take_init(out);
}

Linear::Linear(int in, int out, Generator &g, bool bias) {
    float bd = fan_in_bound(in);
    std::vector<float> wv((size_t)in * out), bv(bias ? out : 0);
    g.fill_uniform(-bd, bd, wv);  // weight first, then bias (Layers.cs:59-64)
    if (bias) g.fill_uniform(-bd, bd, bv);
    w = param("weight", {out, in}, std::move(wv));
    if (bias) b = param("bias", {out}, std::move(bv));
}
Conv2d::Conv2d(int cin, int cout, int k, Generator &g, int padding, int stride_) : stride(stride_), pad(padding) {
    float bd = fan_in_bound(cin * k * k);
    std::vector<float> wv((size_t)cout * cin * k * k), bv(cout);
    g.fill_uniform(-bd, bd, wv);  // Layers.cs:105-110
    g.fill_uniform(-bd, bd, bv);
    w = param("weight", {cout, cin, k, k}, std::move(wv));
    b = param("bias", {cout}, std::move(bv));
}
BatchNorm2d::BatchNorm2d(int c, float momentum_, float eps_) : momentum(momentum_), eps(eps_) {
    if (c < 1) throw Error(OM_E_ARG, "BatchNorm2d needs at least one channel");
    w = param("weight", {c}, std::vector<float>(c, 1.0f));
    b = param("bias", {c}, std::vector<float>(c, 0.0f));
    rm = buffer("running_mean", std::vector<float>(c, 0.0f));
    rv = buffer("running_var", std::vector<float>(c, 1.0f));
}
Embedding::Embedding(int count, int width, Generator &g, int padding_index) : pad(padding_index) {
    if (count < 1 || width < 1) throw Error(OM_E_ARG, "Embedding needs at least one id and one column");
    std::vector<float> v((size_t)count * width);
    g.fill_uniform(-1.7320508f, 1.7320508f, v);  // Init.Uniform(g, sqrt(3), count, width), Layers.cs:11-21
    w = param("weight", {count, width}, std::move(v));
}
Dropout::Dropout(float p_, uint64_t seed_) : p(p_), seed(seed_) {
    if (!(p >= 0.0f && p < 1.0f)) throw Error(OM_E_ARG, "Dropout probability must be in [0, 1).");
    buffer_i64("draws", &draws);
}
LayerNorm::LayerNorm(int n, float eps_) : eps(eps_) {
    w = param("weight", {n}, std::vector<float>(n, 1.0f));  // Layers.cs:255-262
    b = param("bias", {n}, std::vector<float>(n, 0.0f));
}
MultiHeadAttention::MultiHeadAttention(int width, int heads_, Generator &g) : heads(heads_) {
    if (heads < 1 || width % heads) throw Error(OM_E_ARG, "Width must be divisible by the head count.");
    q = child("q", std::make_unique<Linear>(width, width, g));  // drawn q, k, v, o (Layers.cs:486-494)
    k = child("k", std::make_unique<Linear>(width, width, g));
    v = child("v", std::make_unique<Linear>(width, width, g));
    o = child("o", std::make_unique<Linear>(width, width, g));
    if (!dev().per_op) {
        colocate({q->w, k->w, v->w});  // one [3W, W] weight and one [3W] bias for the packed projection
        colocate({q->b, k->b, v->b});
    }
}
Tensor MultiHeadAttention::operator()(const Tensor &x, const Tensor &mask) const {
    // Layers.cs:497-516: q/k/v projections, split heads, attention, merge heads, output projection. The per-op records
    // are the three Linears, the attention over their outputs (the split and merge permutes are views the kernels
    // address in place) and the output Linear.
    if (dev().per_op) return (*o)(attention_heads((*q)(x), (*k)(x), (*v)(x), mask, heads));
    return (*o)(attention_qkv(x, q->w, q->b, k->w, k->b, v->w, v->b, mask, heads));
}
Tensor MultiHeadAttention::residual(const Tensor &x, const Tensor &mask, const Tensor &resid) const {
    if (dev().per_op) return add(resid, (*this)(x, mask));  // Ops.Add(input, attn)
    return linear_residual(attention_qkv(x, q->w, q->b, k->w, k->b, v->w, v->b, mask, heads), o->w, o->b, resid);
}

// Post-norm TransformerEncoderLayer (Layers.cs:523-578).
struct EncoderLayer : Module {
    MultiHeadAttention *attn;
    LayerNorm *norm1, *norm2;
    Linear *ff1, *ff2;
    Dropout *drop1 = nullptr, *drop2 = nullptr;  // only when dropout > 0 (seeds s and s + 1)
    EncoderLayer(int width, int heads, int ff, Generator &g, float dropout = 0.0f, uint64_t dropout_seed = 0) {
        attn = child("attn", std::make_unique<MultiHeadAttention>(width, heads, g));
        norm1 = child("norm1", std::make_unique<LayerNorm>(width));
        ff1 = child("ff1", std::make_unique<Linear>(width, ff, g));
        ff2 = child("ff2", std::make_unique<Linear>(ff, width, g));
        norm2 = child("norm2", std::make_unique<LayerNorm>(width));
        if (dropout > 0.0f) {
            drop1 = child("drop1", std::make_unique<Dropout>(dropout, dropout_seed));
            drop2 = child("drop2", std::make_unique<Dropout>(dropout, dropout_seed + 1));
        }
    }
    Tensor operator()(const Tensor &x, const Tensor &mask) const {
        if (dev().per_op) {  // TransformerEncoderLayer.Forward (Layers.cs:557-577) record for record
            Tensor a = (*attn)(x, mask);
            if (drop1) a = (*drop1)(a);
            Tensor x1 = (*norm1)(add(x, a));
            Tensor f = (*ff2)(gelu((*ff1)(x1)));
            if (drop2) f = (*drop2)(f);
            return (*norm2)(add(x1, f));
        }
        if (drop1) {  // norm1(x + drop1(attn(x))), norm2(x1 + drop2(ff2(gelu(ff1(x1)))))
            Tensor x1 = (*norm1)(add(x, (*drop1)((*attn)(x, mask))));
            return (*norm2)(add(x1, (*drop2)(ffn(x1, ff1->w, ff1->b, ff2->w, ff2->b, nullptr))));
        }
        // norm1(x + attn(x)), then norm2(x1 + ff2(gelu(ff1(x1)))), with the residual Adds and GELU fused into the
        // Linear launches
        Tensor x1 = (*norm1)(attn->residual(x, mask, x));
        return (*norm2)(ffn(x1, ff1->w, ff1->b, ff2->w, ff2->b, x1));
    }
};
// The C3 block: pre-norm, composed from the reference's pieces (children ln1, attn, ln2, ff1, ff2).
struct PreNormBlock : Module {
    LayerNorm *ln1, *ln2;
    MultiHeadAttention *attn;
    Linear *ff1, *ff2;
    PreNormBlock(int width, int heads, int ff, Generator &g) {
        ln1 = child("ln1", std::make_unique<LayerNorm>(width));
        attn = child("attn", std::make_unique<MultiHeadAttention>(width, heads, g));
        ln2 = child("ln2", std::make_unique<LayerNorm>(width));
        ff1 = child("ff1", std::make_unique<Linear>(width, ff, g));
        ff2 = child("ff2", std::make_unique<Linear>(ff, width, g));
    }
    Tensor operator()(const Tensor &x, const Tensor &mask) const {
        // h = x + attn(ln1(x)); y = h + ff2(gelu(ff1(ln2(h)))), the Adds and GELU fused into the Linear launches
        if (dev().per_op) {
            Tensor h = add(x, (*attn)((*ln1)(x), mask));
            return add(h, (*ff2)(gelu((*ff1)((*ln2)(h)))));
        }
        Tensor h = attn->residual((*ln1)(x), mask, x);
        return ffn((*ln2)(h), ff1->w, ff1->b, ff2->w, ff2->b, h);
    }
    // Losses.Mse of the block's output against target; the composite records form the loss in the last product
    Tensor mse_loss(const Tensor &x, const Tensor &mask, const Tensor &target) const {
        if (dev().per_op) return mse((*this)(x, mask), target);
        Tensor h = attn->residual((*ln1)(x), mask, x);
        return ffn_mse((*ln2)(h), ff1->w, ff1->b, ff2->w, ff2->b, h, target);
    }
};

}  // namespace omt

// ------------------------------------------------------------------------------------------------ model
using namespace omt;

struct Input {
    std::string name;
    Tensor t;                    // device copy (persistent region)
    std::vector<float> hf;       // host copy (float inputs)
    std::vector<int32_t> hi;     // host copy (int inputs)
    bool is_int = false;
    int32_t lo = INT32_MIN, hi_bound = INT32_MAX;  // int inputs: the values the model accepts, [lo, hi_bound)
    float *home_data = nullptr;                    // the input's own device buffer (a staged batch replaces it
    int32_t *home_idata = nullptr;                 // for one step)
    std::vector<int32_t> home_hi;                  // int inputs: the own host copy while a staged batch is active
    bool host_read = false;  // the step's launches take arguments from the host copy (a new value needs a new graph)
    void set_range(int32_t l, int32_t h) {
        lo = l;
        hi_bound = h;
    }
};

enum { OPT_SGD = 0, OPT_ADAM = 1, OPT_ADAMW = 2 };

struct omt_model {
    std::unique_ptr<Device> device;
    std::unique_ptr<Module> root;
    std::vector<std::pair<std::string, Tensor>> params;
    std::vector<Tensor> leaves;  // params + inputs that require gradients
    std::vector<int64_t> offset;
    std::vector<int> phys;  // parameter indices in arena order
    int64_t total = 0;
    float *pb = nullptr, *gb = nullptr, *mb = nullptr, *vb = nullptr;
    std::vector<Input> inputs;
    std::vector<std::pair<std::string, Module::BufferRef>> buffers;  // float buffers, named_buffers() order
    std::function<Tensor(omt_model &)> loss_fn;
    // Optimizer (Optimizers.cs): kind OPT_SGD, OPT_ADAM (L2 weight decay) or OPT_ADAMW (decoupled); the benchmark
    // configurations use AdamW(lr 1e-3, betas 0.9/0.999, eps 1e-8, wd 0.01).
    int opt_kind = OPT_ADAMW;
    float lr = 1e-3f, beta1 = 0.9f, beta2 = 0.999f, eps = 1e-8f, wd = 0.01f;
    float momentum = 0.0f, dampening = 0.0f;
    bool nesterov = false, amsgrad = false;
    float *vmaxb = nullptr;            // AMSGrad's running maximum of v (allocated when first asked for)
    std::vector<char> sgd_started;     // per parameter: its momentum buffer holds a value (Sgd starts it from g)
    int64_t step_count = 0;
    std::unique_ptr<LrSchedule> schedule;  // LrSchedule.Apply before every step when set
    float clip_max = 0.0f;                 // ClipNorm inside omt_step when > 0
    int clip_inf = 0;
    float *clip_buf = nullptr;             // device: [norm, coefficient] of the last ClipNorm
    std::map<std::string, int64_t> ckpt_extra;  // the extra values of the last checkpoint loaded
    // Host data staging: a batch packs the inputs in input order, each 256-byte aligned; committed batches wait in
    // `staged` until a step consumes the oldest.
    static constexpr int kStageSlots = 3;
    om_stager *stager = nullptr;
    om_readback *loss_rb = nullptr;  // the step's loss, read back while the backward and update still run
    std::vector<uint64_t> batch_off;
    uint64_t batch_bytes = 0;
    int begun_slot = -1;
    char *begun_host = nullptr;
    struct Staged {
        int slot;
        char *dev;
        std::vector<std::vector<int32_t>> ints;  // host copies of the int inputs (CTC reads its lengths on the host)
    };
    std::deque<Staged> staged;
    int active_slot = -1;
    // The loss of the last omt_forward, kept for omt_backward; its records are released by that backward, so a second
    // omt_backward runs through a released graph (Engine.cs:136-141). Dropped at the next step's start.
    Tensor graph_loss;
    // Step graphs (om_graph_*): with graph_on, omt_step runs one step as usual, captures the next into a HIP graph
    // (launched at once) and replays that graph afterwards, doing on the host only what a step changes there. Dropped
    // (captured again) when something a recorded launch depends on changes; never used with SGD (host-valued rate
    // and first-step flags), dropout (a new mask seed every step) or staged batches (new input addresses).
    bool graph_on = false;
    bool has_dropout = false;
    om_graph *graph = nullptr;
    int graph_warm = 0;          // steps run outside a graph since the graph was last dropped
    om_step_values last_vals{};  // what the last optimizer step passed to om_adam_step
    std::string err;

    Input &add_input(const std::string &name, std::vector<int> shape, std::vector<float> host, bool requires_grad) {
        Input in;
        in.name = name;
        in.t = std::make_shared<TensorImpl>();
        in.t->shape = std::move(shape);
        in.t->numel = numel_of(in.t->shape);
        in.t->data = (float *)device->persistent(sizeof(float) * (uint64_t)in.t->numel);
        in.home_data = in.t->data;
        in.t->name = name;
        check(device->ctx(), om_upload(device->ctx(), in.t->data, host.data(), sizeof(float) * host.size()), "upload");
        if (requires_grad) {
            in.t->requires_grad = true;
            in.t->grad = (float *)device->persistent(sizeof(float) * (uint64_t)in.t->numel);
            leaves.push_back(in.t);
        }
        in.hf = std::move(host);
        inputs.push_back(std::move(in));
        return inputs.back();
    }
    Input &add_int_input(const std::string &name, std::vector<int> shape, std::vector<int32_t> host) {
        Input in;
        in.name = name;
        in.is_int = true;
        in.t = std::make_shared<TensorImpl>();
        in.t->shape = std::move(shape);
        in.t->numel = numel_of(in.t->shape);
        in.t->idata = (int32_t *)device->persistent(sizeof(int32_t) * (uint64_t)(in.t->numel > 0 ? in.t->numel : 1));
        in.home_idata = in.t->idata;
        in.t->name = name;
        check(device->ctx(), om_upload(device->ctx(), in.t->idata, host.data(), sizeof(int32_t) * host.size()),
              "upload");
        in.hi = std::move(host);
        inputs.push_back(std::move(in));
        return inputs.back();
    }
    const Input &input(const std::string &name) const {
        for (auto &i : inputs)
            if (i.name == name) return i;
        throw Error(OM_E_ARG, "no input " + name);
    }
    Input &input(const std::string &name) { return const_cast<Input &>(std::as_const(*this).input(name)); }

    // Lays the parameters out contiguously (Parameters() order, 16-byte aligned) in four persistent blocks: values,
    // gradients, first and second moments; uploads the initial values once.
    void finalize(std::vector<std::vector<float>> &&init) {
        root->named_parameters(params);
        {
            std::vector<std::pair<std::string, Module::BufferRef>> all;
            root->named_buffers(all);
            for (auto &b : all)
                if (b.second.dev) buffers.push_back(b);
        }
        std::vector<std::vector<Tensor>> groups;
        root->colocation_groups(groups);
        // Physical order: Parameters() order, except that a colocation group is placed whole where its first member
        // would go. Every tensor starts 16-byte aligned; a group's members are only packed without gaps when their
        // sizes are multiples of four floats (the packed kernels check contiguity before relying on it).
        offset.assign(params.size(), -1);
        phys.clear();
        auto index_of = [&](const Tensor &t) {
            for (size_t i = 0; i < params.size(); i++)
                if (params[i].second == t) return (int)i;
            return -1;
        };
        int64_t off = 0;
        auto place = [&](int i) {
            offset[i] = off;
            off += (params[i].second->numel + 3) & ~int64_t(3);
            phys.push_back(i);
        };
        for (size_t i = 0; i < params.size(); i++) {
            if (offset[i] >= 0) continue;
            const std::vector<Tensor> *grp = nullptr;
            for (auto &g : groups)
                for (auto &t : g)
                    if (t == params[i].second) grp = &g;
            if (!grp) {
                place((int)i);
                continue;
            }
            for (auto &t : *grp) {
                int j = index_of(t);
                if (j >= 0 && offset[j] < 0) place(j);
            }
        }
        total = off;
        uint64_t bytes = sizeof(float) * (uint64_t)(total > 0 ? total : 4);
        om_ctx *c = device->ctx();
        pb = (float *)device->persistent(bytes);
        gb = (float *)device->persistent(bytes);
        mb = (float *)device->persistent(bytes);
        vb = (float *)device->persistent(bytes);
        std::vector<float> host((size_t)total, 0.0f);
        for (size_t i = 0; i < params.size(); i++) {
            if (init[i].size() != (size_t)params[i].second->numel) throw Error(OM_E_STATE, "init size mismatch");
            std::memcpy(host.data() + offset[i], init[i].data(), sizeof(float) * init[i].size());
            Tensor &t = params[i].second;
            t->name = params[i].first;
            t->data = pb + offset[i];
            t->grad = gb + offset[i];
            leaves.insert(leaves.begin() + (long)i, t);
        }
        sgd_started.assign(params.size(), 0);
        clip_buf = (float *)device->persistent(16);
        check(c, om_fill(c, clip_buf, std::nanf(""), 4), "clip slot");
        check(c, om_upload(c, pb, host.data(), bytes), "upload params");
        check(c, om_zero(c, gb, bytes), "zero grads");
        check(c, om_zero(c, mb, bytes), "zero m");
        check(c, om_zero(c, vb, bytes), "zero v");
        device->sync();
    }

    // Runs of physically consecutive parameters that have gradients, as (first element, length) in the arena: the
    // alignment gaps between them are zero in every block, and every per-element operation here (Adam, clipping)
    // keeps a zero parameter with a zero gradient and zero moments at zero and adds nothing to a norm.
    std::vector<std::pair<int64_t, int64_t>> live_runs() const {
        auto live = [&](size_t q) { return params[phys[q]].second->grad_exists && params[phys[q]].second->requires_grad; };
        std::vector<std::pair<int64_t, int64_t>> runs;
        size_t i = 0;
        while (i < phys.size()) {
            if (!live(i)) {
                i++;
                continue;
            }
            size_t j = i;
            while (j + 1 < phys.size() && live(j + 1)) j++;
            const int64_t beg = offset[phys[i]], end = offset[phys[j]] + params[phys[j]].second->numel;
            runs.emplace_back(beg, end - beg);
            i = j + 1;
        }
        return runs;
    }

    // Optimizer.Step (Optimizers.cs:184-219): LrSchedule.Apply when a schedule is attached, the rate check, then
    // one fused update per run of parameters that have gradients (a parameter without one is skipped, as in the
    // reference). Adam/AdamW: BeginStep scalars on the host (Optimizers.cs:501-508), UpdateRange on the device;
    // grad_scale is ClipNorm's device coefficient folded into the read of g (om_adam_step_scaled), or NULL.
    // SGD (class Sgd): runs are split where the momentum buffers' started state changes.
    void optimizer_step(const float *grad_scale = nullptr) {
        settle_grads(leaves);
        // the update writes the parameters in place (Tensor.MutableData in Optimizer.Step): a graph that saved one
        // of them can no longer run backward
        for (auto &p : params)
            if (p.second->grad_exists && p.second->requires_grad) touch(p.second);
        if (schedule) lr = schedule->lr_at(step_count);
        if (!std::isfinite(lr) || lr < 0.0f) throw Error(OM_E_ARG, "learning rate must be finite and not negative");
        om_ctx *c = device->ctx();
        if (opt_kind == OPT_SGD) {
            if (grad_scale) throw Error(OM_E_STATE, "SGD takes in-place clipped gradients");
            sgd_step();
            step_count++;
            return;
        }
        float ss, sq;
        om_adam_scalars(lr, beta1, beta2, step_count + 1, &ss, &sq);
        last_vals = om_step_values{lr, ss, sq};
        const int dec = opt_kind == OPT_ADAMW ? 1 : 0;
        for (auto [beg, n] : live_runs()) {
            float *vm = amsgrad ? vmaxb + beg : nullptr;
            if (grad_scale)
                check(c, om_adam_step_scaled(c, pb + beg, gb + beg, mb + beg, vb + beg, vm, n, lr, beta1, beta2, eps,
                                             wd, dec, ss, sq, grad_scale),
                      "om_adam_step_scaled");
            else
                check(c, om_adam_step(c, pb + beg, gb + beg, mb + beg, vb + beg, vm, n, lr, beta1, beta2, eps, wd,
                                      dec, ss, sq),
                      "om_adam_step");
        }
        step_count++;
    }
    void sgd_step() {
        om_ctx *c = device->ctx();
        const bool buf = momentum != 0.0f;
        size_t i = 0;
        while (i < phys.size()) {
            const Tensor &t = params[phys[i]].second;
            if (!(t->grad_exists && t->requires_grad)) {
                i++;
                continue;
            }
            const bool first = buf && !sgd_started[phys[i]];
            size_t j = i;
            while (j + 1 < phys.size()) {
                const Tensor &u = params[phys[j + 1]].second;
                if (!(u->grad_exists && u->requires_grad) || (buf && !sgd_started[phys[j + 1]]) != first) break;
                j++;
            }
            const int64_t beg = offset[phys[i]], n = offset[phys[j]] + params[phys[j]].second->numel - beg;
            check(c, om_sgd_step(c, pb + beg, gb + beg, buf ? mb + beg : nullptr, n, lr, momentum, dampening, wd,
                                 nesterov ? 1 : 0, first ? 1 : 0),
                  "om_sgd_step");
            for (size_t q = i; q <= j; q++) sgd_started[phys[q]] = 1;
            i = j + 1;
        }
    }
    // A new optimizer over Parameters() (its state starts empty: moments and momentum buffers zero, step count 0).
    void set_optimizer(int kind, float lr_, float b1, float b2, float eps_, float wd_, float mom, float damp,
                       bool nest, bool ams) {
        auto finite_nonneg = [](float v) { return std::isfinite(v) && v >= 0.0f; };
        if (kind != OPT_SGD && kind != OPT_ADAM && kind != OPT_ADAMW) throw Error(OM_E_ARG, "unknown optimizer kind");
        if (!finite_nonneg(lr_) || !finite_nonneg(wd_)) throw Error(OM_E_ARG, "rate and weight decay must be finite and not negative");
        if (kind == OPT_SGD) {
            if (!finite_nonneg(mom) || !finite_nonneg(damp)) throw Error(OM_E_ARG, "momentum and dampening must be finite and not negative");
            if (nest && (mom <= 0.0f || damp != 0.0f))
                throw Error(OM_E_ARG, "Nesterov momentum needs a positive momentum and zero dampening");
        } else {
            if (!(b1 >= 0.0f && b1 < 1.0f) || !(b2 >= 0.0f && b2 < 1.0f)) throw Error(OM_E_ARG, "betas must be in [0, 1)");
            if (!(eps_ > 0.0f) || !std::isfinite(eps_)) throw Error(OM_E_ARG, "epsilon must be positive and finite");
        }
        opt_kind = kind;
        lr = lr_;
        beta1 = b1;
        beta2 = b2;
        eps = eps_;
        wd = wd_;
        momentum = kind == OPT_SGD ? mom : 0.0f;
        dampening = kind == OPT_SGD ? damp : 0.0f;
        nesterov = kind == OPT_SGD && nest;
        amsgrad = kind != OPT_SGD && ams;
        om_ctx *c = device->ctx();
        const uint64_t bytes = sizeof(float) * (uint64_t)(total > 0 ? total : 4);
        if (amsgrad && !vmaxb) vmaxb = (float *)device->persistent(bytes);
        check(c, om_zero(c, mb, bytes), "zero moments");
        check(c, om_zero(c, vb, bytes), "zero moments");
        if (vmaxb) check(c, om_zero(c, vmaxb, bytes), "zero moments");
        sgd_started.assign(params.size(), 0);
        step_count = 0;
        device->sync();
    }

    // GradClip.ClipNorm / ClipValue over Parameters() (Schedules.cs:22-149) on the device; the norm and the
    // coefficient land in clip_buf. in_place = false leaves the gradients for optimizer_step(clip_buf + 1).
    void clip_norm(float max_norm, int infinity_norm, bool in_place) {
        settle_grads(leaves);
        std::vector<float *> ptrs;
        std::vector<int64_t> lens;
        for (auto [beg, n] : live_runs()) {
            ptrs.push_back(gb + beg);
            lens.push_back(n);
        }
        om_ctx *c = device->ctx();
        check(c, om_clip_grad_norm(c, (int)ptrs.size(), ptrs.data(), lens.data(), max_norm, infinity_norm,
                                   in_place ? 1 : 0, clip_buf, clip_buf + 1),
              "om_clip_grad_norm");
    }
    void clip_value(float bound) {
        settle_grads(leaves);
        std::vector<float *> ptrs;
        std::vector<int64_t> lens;
        for (auto [beg, n] : live_runs()) {
            ptrs.push_back(gb + beg);
            lens.push_back(n);
        }
        om_ctx *c = device->ctx();
        check(c, om_clip_grad_value(c, (int)ptrs.size(), ptrs.data(), lens.data(), bound), "om_clip_grad_value");
    }

    void batch_layout() {
        batch_off.clear();
        uint64_t off = 0;
        for (const Input &in : inputs) {
            batch_off.push_back(off);
            const uint64_t b = (uint64_t)in.t->numel * 4;
            off = (off + b + 255) & ~uint64_t(255);
        }
        batch_bytes = off > 0 ? off : 256;
    }
    void batch_begin(void **host) {
        if (begun_slot >= 0) throw Error(OM_E_STATE, "omt_batch_begin: the previous batch was not committed");
        if ((int)staged.size() >= kStageSlots)
            throw Error(OM_E_STATE, "omt_batch_begin: " + std::to_string(kStageSlots) + " batches already wait for a step");
        om_ctx *c = device->ctx();
        if (!stager) {
            batch_layout();
            check(c, om_stager_create(c, batch_bytes, kStageSlots, &stager), "om_stager_create");
        }
        void *h = nullptr;
        int slot = -1;
        check(c, om_stager_begin(stager, &h, &slot), "om_stager_begin");
        begun_slot = slot;
        begun_host = (char *)h;
        *host = h;
    }
    void batch_commit() {
        if (begun_slot < 0) throw Error(OM_E_STATE, "omt_batch_commit: no batch was begun");
        Staged st;
        st.slot = begun_slot;
        for (size_t i = 0; i < inputs.size(); i++) {
            const Input &in = inputs[i];
            if (!in.is_int) continue;
            const int32_t *v = reinterpret_cast<const int32_t *>(begun_host + batch_off[i]);
            for (int64_t k = 0; k < in.t->numel; k++)
                if (v[k] < in.lo || v[k] >= in.hi_bound)
                    throw Error(OM_E_ARG, "omt_batch_commit: " + in.name + "[" + std::to_string(k) + "] = " +
                                              std::to_string(v[k]) + " is out of range");
            st.ints.emplace_back(v, v + in.t->numel);
        }
        void *d = nullptr;
        check(device->ctx(), om_stager_commit(stager, begun_slot, batch_bytes, &d), "om_stager_commit");
        st.dev = (char *)d;
        begun_slot = -1;
        begun_host = nullptr;
        staged.push_back(std::move(st));
    }
    // At the start of a step: the oldest committed batch becomes the inputs (the stream waits for its upload).
    void take_batch() {
        if (staged.empty()) return;
        Staged st = std::move(staged.front());
        staged.pop_front();
        check(device->ctx(), om_stager_acquire(stager, st.slot), "om_stager_acquire");
        size_t k = 0;
        for (size_t i = 0; i < inputs.size(); i++) {
            Input &in = inputs[i];
            if (in.is_int) {
                in.t->idata = reinterpret_cast<int32_t *>(st.dev + batch_off[i]);
                in.home_hi = std::move(in.hi);
                in.hi = std::move(st.ints[k++]);
            } else {
                in.t->data = reinterpret_cast<float *>(st.dev + batch_off[i]);
            }
        }
        active_slot = st.slot;
    }
    // After the step's last launch: the slot's device copy is released and the inputs point home again. The inputs
    // point home even when the release fails.
    void return_batch() {
        if (active_slot < 0) return;
        const int slot = active_slot;
        active_slot = -1;
        for (Input &in : inputs) {
            if (in.is_int) {
                in.t->idata = in.home_idata;
                in.hi = std::move(in.home_hi);  // the host copy matches the device buffer it points at again
            } else {
                in.t->data = in.home_data;
            }
        }
        check(device->ctx(), om_stager_release(stager, slot), "om_stager_release");
    }
    // Returns the step's batch when the scope ends, also when the step throws (a failed step must not keep its
    // staging slot, or the ring runs dry after a few failures). keep() hands the batch on to a later backward.
    struct BatchScope {
        omt_model *m;
        bool armed = true;
        ~BatchScope() {
            if (!armed) return;
            try {
                m->return_batch();
            } catch (...) {  // the step's own error is the one reported
            }
        }
        void keep() { armed = false; }
        void done() {  // returns the batch now, reporting a failure
            armed = false;
            m->return_batch();
        }
    };
    // The start of every step: a batch still held by an omt_forward that no backward followed is returned, the
    // previous graph is dropped, step memory is rewound (ActivationScope.Dispose), the next batch is taken and the
    // gradients are zeroed (Optimizer.ZeroGrad).
    void begin_step() {
        graph_loss.reset();
        return_batch();
        device->step_reset();
        take_batch();
    }

    float forward_backward() {
        begin_step();
        BatchScope batch{this};
        zero_grad(leaves);
        Tensor loss = loss_fn(*this);
        backward(loss);
        batch.done();
        float v = 0.0f;
        check(device->ctx(), om_download(device->ctx(), &v, loss->data, sizeof(float)), "loss readback");
        return v;
    }
    // ZeroGrad and the forward alone; the graph and the batch are kept for backward_pass().
    float forward() {
        begin_step();
        BatchScope batch{this};
        zero_grad(leaves);
        Tensor loss = loss_fn(*this);
        float v = 0.0f;
        check(device->ctx(), om_download(device->ctx(), &v, loss->data, sizeof(float)), "loss readback");
        graph_loss = loss;
        batch.keep();
        return v;
    }
    // loss.Backward() of the last forward(). Its records are released afterwards, so a second call fails as the
    // reference's second Backward does; a saved tensor written in place since the forward fails with
    // TensorVersionException's code. The batch goes back either way.
    void backward_pass() {
        if (!graph_loss) throw Error(OM_E_STATE, "omt_backward: no forward pass to run backward through");
        BatchScope batch{this};
        backward(graph_loss);
        batch.done();
    }
    // ---------------------------------------------------------------------------------------------- checkpoints
    // The model's StateDict as checkpoint tensors (names, types, shapes), and the optimizer's kind, hyper-parameters
    // and StateTensors (Sgd: "initialized" Int32 flags then "momentum_buffer.i"; Adam/AdamW: "exp_avg.i",
    // "exp_avg_sq.i", and "max_exp_avg_sq.i" with AMSGrad; Optimizers.cs:88-160, 300-315, 440-470).
    std::vector<Module::StateRef> state_refs() const {
        std::vector<Module::StateRef> st;
        root->state(st);
        return st;
    }
    int param_index(const Tensor &t) const {
        for (size_t i = 0; i < params.size(); i++)
            if (params[i].second == t) return (int)i;
        throw Error(OM_E_STATE, "state tensor is not a parameter of the model");
    }
    std::vector<ckpt::Tensor> model_specs(const std::vector<Module::StateRef> &st) const {
        std::vector<ckpt::Tensor> out;
        for (const auto &r : st) {
            ckpt::Tensor t;
            t.name = r.name;
            if (r.param) {
                t.dims = r.param->shape;
            } else if (r.buf.host) {
                t.dtype = ckpt::I64;
                t.dims = {1};
            } else {
                t.dims = {(int)r.buf.numel};
            }
            out.push_back(std::move(t));
        }
        return out;
    }
    ckpt::Optimizer optimizer_spec() const {
        ckpt::Optimizer o;
        o.step = step_count;
        auto slot = [&](const char *nm) {
            for (size_t i = 0; i < params.size(); i++) {
                ckpt::Tensor t;
                t.name = std::string(nm) + "." + std::to_string(i);
                t.dims = params[i].second->shape;
                o.state.push_back(t);
                o.param_dims.push_back(t.dims);
            }
        };
        if (opt_kind == OPT_SGD) {
            o.kind = "sgd";
            o.hyper = {{"lr", lr}, {"momentum", momentum}, {"dampening", dampening}, {"weight_decay", wd},
                       {"nesterov", nesterov ? 1.0f : 0.0f}};
            ckpt::Tensor f;
            f.name = "initialized";
            f.dtype = ckpt::I32;
            f.dims = {(int)params.size()};
            o.state.push_back(f);
            o.param_dims.push_back({});
            if (momentum != 0.0f) slot("momentum_buffer");
        } else {
            o.kind = opt_kind == OPT_ADAMW ? "adamw" : "adam";
            o.hyper = {{"lr", lr}, {"beta1", beta1}, {"beta2", beta2}, {"epsilon", eps}, {"weight_decay", wd},
                       {"amsgrad", amsgrad ? 1.0f : 0.0f}};
            slot("exp_avg");
            slot("exp_avg_sq");
            if (amsgrad) slot("max_exp_avg_sq");
        }
        return o;
    }
    std::vector<float> host_block(float *block) const {
        std::vector<float> h((size_t)(total > 0 ? total : 4));
        check(device->ctx(), om_download(device->ctx(), h.data(), block, sizeof(float) * h.size()), "download");
        return h;
    }
    // Checkpoint.Save (Checkpoint.cs:80-138): one download per arena block, then the file in StateDict order.
    void save_checkpoint(const std::string &path, bool with_opt, const std::map<std::string, int64_t> &extra) {
        const auto st = state_refs();
        std::vector<ckpt::Tensor> model = model_specs(st);
        const std::vector<float> ph = host_block(pb);
        std::vector<std::vector<float>> bufs(st.size());
        for (size_t i = 0; i < st.size(); i++) {
            if (st[i].param) {
                model[i].data = ph.data() + offset[param_index(st[i].param)];
            } else if (st[i].buf.host) {
                model[i].data = st[i].buf.host;
            } else {
                bufs[i].resize((size_t)st[i].buf.numel);
                check(device->ctx(), om_download(device->ctx(), bufs[i].data(), st[i].buf.dev,
                                                 sizeof(float) * bufs[i].size()), "download");
                model[i].data = bufs[i].data();
            }
        }
        ckpt::Optimizer o;
        std::vector<float> mh, vh, xh;
        std::vector<int32_t> flags;
        if (with_opt) {
            o = optimizer_spec();
            mh = host_block(mb);
            if (opt_kind != OPT_SGD) vh = host_block(vb);
            if (amsgrad) xh = host_block(vmaxb);
            size_t k = 0;
            const size_t P = params.size();
            if (opt_kind == OPT_SGD) {
                flags.assign(sgd_started.begin(), sgd_started.end());
                o.state[k++].data = flags.data();
                if (momentum != 0.0f)
                    for (size_t i = 0; i < P; i++) o.state[k++].data = mh.data() + offset[i];
            } else {
                for (size_t i = 0; i < P; i++) o.state[k++].data = mh.data() + offset[i];
                for (size_t i = 0; i < P; i++) o.state[k++].data = vh.data() + offset[i];
                if (amsgrad)
                    for (size_t i = 0; i < P; i++) o.state[k++].data = xh.data() + offset[i];
            }
        }
        ckpt::save(path, model, with_opt ? &o : nullptr, extra);
    }
    // Optimizer.SetHyperParameters' checks (Optimizers.cs:320-330, 470-480): the fixed settings must equal the
    // target's, the rate and the weight decay must be finite and not negative.
    static std::string settings_ok(const std::map<std::string, float> &h, const ckpt::Optimizer &o) {
        auto rate_ok = [](float v) { return std::isfinite(v) && v >= 0.0f; };
        auto target = [&](const char *n) {
            for (auto &p : o.hyper)
                if (p.first == n) return p.second;
            return 0.0f;
        };
        if (o.kind == "sgd") {
            if (h.at("momentum") != target("momentum") || h.at("dampening") != target("dampening") ||
                (h.at("nesterov") != 0.0f) != (target("nesterov") != 0.0f))
                return "The saved momentum, dampening or nesterov setting differs from this optimizer's.";
        } else if (h.at("beta1") != target("beta1") || h.at("beta2") != target("beta2") ||
                   h.at("epsilon") != target("epsilon") || (h.at("amsgrad") != 0.0f) != (target("amsgrad") != 0.0f)) {
            return "The saved betas, epsilon or amsgrad setting differ from this optimizer's.";
        }
        if (!rate_ok(h.at("lr")) || !rate_ok(h.at("weight_decay"))) return "Value must be finite and not negative.";
        return "";
    }
    // Checkpoint.Load (Checkpoint.cs:151-331): everything is checked before the model changes; then one upload per
    // arena block and per buffer.
    bool load_checkpoint(const std::string &path, bool with_opt) {
        const auto st = state_refs();
        const std::vector<ckpt::Tensor> model = model_specs(st);
        ckpt::Optimizer o;
        if (with_opt) o = optimizer_spec();
        ckpt::Loaded L = ckpt::load(path, model, with_opt ? &o : nullptr, &settings_ok);
        om_ctx *c = device->ctx();
        std::vector<float> ph = host_block(pb);
        for (size_t i = 0; i < st.size(); i++) {
            const std::vector<char> &b = L.model[i];
            if (st[i].param) {
                std::memcpy(ph.data() + offset[param_index(st[i].param)], b.data(), b.size());
            } else if (st[i].buf.host) {
                std::memcpy(st[i].buf.host, b.data(), sizeof(int64_t));
            } else {
                check(c, om_upload(c, st[i].buf.dev, b.data(), b.size()), "upload");
            }
        }
        check(c, om_upload(c, pb, ph.data(), sizeof(float) * ph.size()), "upload");
        for (auto &p : params) touch(p.second);
        if (with_opt) {
            const size_t P = params.size();
            std::vector<float> mh(ph.size(), 0.0f), vh(ph.size(), 0.0f), xh;
            if (amsgrad) xh.assign(ph.size(), 0.0f);
            auto put = [&](std::vector<float> &blk, size_t i, const std::vector<char> &b) {
                if (!b.empty()) std::memcpy(blk.data() + offset[i], b.data(), b.size());  // [0]: zero state
            };
            size_t k = 0;
            if (opt_kind == OPT_SGD) {
                const std::vector<char> &f = L.state[k++];
                for (size_t i = 0; i < P; i++) {
                    int32_t v;
                    std::memcpy(&v, f.data() + 4 * i, 4);
                    sgd_started[i] = v != 0;
                }
                if (momentum != 0.0f)
                    for (size_t i = 0; i < P; i++) put(mh, i, L.state[k++]);
            } else {
                for (size_t i = 0; i < P; i++) put(mh, i, L.state[k++]);
                for (size_t i = 0; i < P; i++) put(vh, i, L.state[k++]);
                if (amsgrad)
                    for (size_t i = 0; i < P; i++) put(xh, i, L.state[k++]);
            }
            check(c, om_upload(c, mb, mh.data(), sizeof(float) * mh.size()), "upload");
            check(c, om_upload(c, vb, vh.data(), sizeof(float) * vh.size()), "upload");
            if (amsgrad) check(c, om_upload(c, vmaxb, xh.data(), sizeof(float) * xh.size()), "upload");
            lr = L.hyper.at("lr");
            wd = L.hyper.at("weight_decay");
            step_count = L.step;
        }
        ckpt_extra = L.extra;
        device->sync();
        return L.had_optimizer;
    }

    // One step. The loss is read back as the reference's step reads it, right after the forward (TrainCase.cs:
    // 117-127): its copy is queued behind the forward and the host waits for that copy alone, after queueing the
    // backward and the update, so those still run while the caller gets the value and queues the next step. Later
    // work on the context's stream is ordered after them.
    float step() {
        if (graphable()) {
            if (graph) return step_replay();
            if (graph_warm > 0) return step_capture();
        }
        const bool warmable = graphable();
        begin_step();
        BatchScope batch{this};
        step_body(batch);
        graph_warm = warmable ? graph_warm + 1 : 0;
        return wait_loss();
    }
    bool graphable() const {
        return graph_on && opt_kind != OPT_SGD && !has_dropout && staged.empty() && active_slot < 0 && begun_slot < 0;
    }
    // Drops the step graph; the next graphable step runs outside a graph and the one after it captures again.
    void graph_drop() {
        graph_warm = 0;
        if (!graph) return;
        om_graph *g = graph;
        graph = nullptr;
        check(device->ctx(), om_graph_destroy(g), "om_graph_destroy");
    }
    float wait_loss() {
        float v = 0.0f;
        check(device->ctx(), om_readback_wait(loss_rb, &v, sizeof(float)), "loss readback");
        return v;
    }
    // The step recorded into a graph and launched. If anything fails inside the capture, the capture is dropped,
    // the host state the step changed is put back, graphs are switched off for the model and the step runs as usual
    // (so a failure that is not the capture's own is reported by that run).
    float step_capture() {
        const int64_t count0 = step_count;
        const float lr0 = lr;
        begin_step();
        om_ctx *c = device->ctx();
        check(c, om_graph_capture_begin(c), "om_graph_capture_begin");
        om_graph *g = nullptr;
        try {
            BatchScope batch{this};
            step_body(batch);
            check(c, om_graph_capture_end(c, &g), "om_graph_capture_end");
        } catch (const Error &) {
            (void)om_graph_capture_abort(c);
            step_count = count0;
            lr = lr0;
            graph_on = false;
            graph_warm = 0;
            begin_step();
            BatchScope batch{this};
            step_body(batch);
            return wait_loss();
        }
        graph = g;
        check(c, om_graph_launch(g, &last_vals), "om_graph_launch");
        return wait_loss();
    }
    // A replay: on the host, what ZeroGrad + forward + backward + Step change there — step memory rewound, the
    // parameters' versions raised by the in-place update, the rate from the schedule, the step count — while the
    // graph does the device work with this step's rate and bias corrections.
    float step_replay() {
        begin_step();
        for (auto &p : params)
            if (p.second->grad_exists && p.second->requires_grad) touch(p.second);
        if (schedule) lr = schedule->lr_at(step_count);
        if (!std::isfinite(lr) || lr < 0.0f) throw Error(OM_E_ARG, "learning rate must be finite and not negative");
        float ss, sq;
        om_adam_scalars(lr, beta1, beta2, step_count + 1, &ss, &sq);
        last_vals = om_step_values{lr, ss, sq};
        check(device->ctx(), om_graph_launch(graph, &last_vals), "om_graph_launch");
        step_count++;
        return wait_loss();
    }
    // ZeroGrad, the forward with the loss posted for readback, loss.Backward() and optimizer.Step() (with ClipNorm
    // when set): the launches of one step, queued on the model's stream.
    void step_body(BatchScope &batch) {
        zero_grad(leaves);
        if (!loss_rb) check(device->ctx(), om_readback_create(device->ctx(), sizeof(float), &loss_rb), "readback");
        device->arm_loss_post(loss_rb);  // a loss op that posts its own value takes it (MSE)
        struct Disarm {  // the offer ends with the loss function, also when it throws
            Device *d;
            ~Disarm() { d->take_loss_post(); }
        };
        Tensor loss;
        {
            Disarm disarm{device.get()};
            loss = loss_fn(*this);
        }
        if (device->loss_posted() != loss->data)
            check(device->ctx(), om_readback_post(loss_rb, loss->data, sizeof(float)), "loss readback");
        backward(loss);
        batch.done();
        if (clip_max > 0.0f) {
            // Adam/AdamW read the coefficient in their update; SGD gets the gradients scaled in place
            const bool fold = opt_kind != OPT_SGD;
            clip_norm(clip_max, clip_inf, !fold);
            optimizer_step(fold ? clip_buf + 1 : nullptr);
        } else {
            optimizer_step();
        }
    }
};

// ------------------------------------------------------------------------------------------------ configurations
static uint64_t cfg_seed(int cfg, int index) { return 20261201ull + 100ull * (uint64_t)cfg + (uint64_t)index; }
static std::vector<float> normal(int cfg, int index, int64_t n) {
    Generator g(cfg_seed(cfg, index));
    std::vector<float> v((size_t)n);
    g.fill_normal(v);
    return v;
}
static std::vector<int32_t> ints(int cfg, int index, int64_t n, int lo, int hi) {
    Generator g(cfg_seed(cfg, index));
    std::vector<int32_t> v((size_t)n);
    g.fill_ints(lo, hi, v);
    return v;
}
static int pick(int v, int d) { return v > 0 ? v : d; }

static void build(omt_model &M, int cfg, const omt_scale &sc) {
    Generator g(cfg_seed(cfg, 0));
    if (cfg == 1) {
        const int B = pick(sc.batch, 64);
        struct Mlp : Module {
            Linear *l1, *l2;
        };
        auto m = std::make_unique<Mlp>();
        m->l1 = m->child("0", std::make_unique<Linear>(784, 256, g));
        m->l2 = m->child("2", std::make_unique<Linear>(256, 10, g));
        Mlp *mp = m.get();
        M.root = std::move(m);
        M.add_input("x", {B, 784}, normal(1, 1, (int64_t)B * 784), false);
        M.add_int_input("labels", {B}, ints(1, 2, B, 0, 10));
        M.loss_fn = [mp](omt_model &s) {
            return cross_entropy((*mp->l2)(mp->l1->relu_of(s.input("x").t)), s.input("labels").t);
        };
    } else if (cfg == 2) {
        const int B = pick(sc.batch, 32), HW = pick(sc.hw, 56);
        struct ConvNet : Module {
            Conv2d *conv;
            Linear *fc;
        };
        auto m = std::make_unique<ConvNet>();
        m->conv = m->child("0", std::make_unique<Conv2d>(64, 64, 3, g, 1));
        m->fc = m->child("4", std::make_unique<Linear>(64, 10, g));
        ConvNet *mp = m.get();
        M.root = std::move(m);
        M.add_input("x", {B, 64, HW, HW}, normal(2, 1, (int64_t)B * 64 * HW * HW), true);
        M.add_int_input("labels", {B}, ints(2, 2, B, 0, 10));
        M.loss_fn = [mp](omt_model &s) {
            // Relu, then GlobalAvgPool2d (Ops.Layers.cs:463-472: Reshape + Mean(axis 2) + Reshape) and Flatten, as
            // one record
            if (dev().per_op) {  // Relu, GlobalAvgPool2d (Reshape, Mean(axis 2), Reshape), Flatten
                Tensor a = relu((*mp->conv)(s.input("x").t));
                const int N = a->shape[0], Cc = a->shape[1], P = a->shape[2] * a->shape[3];
                Tensor gap = reshape(mean_axis(reshape(a, {N, Cc, P}), 2), {N, Cc, 1, 1});
                return cross_entropy((*mp->fc)(reshape(gap, {N, Cc})), s.input("labels").t);
            }
            Tensor gap = relu_mean_plane((*mp->conv)(s.input("x").t));
            return cross_entropy((*mp->fc)(gap), s.input("labels").t);
        };
    } else if (cfg == 3) {
        const int B = pick(sc.batch, 32), L = pick(sc.seq, 128), D = 384, H = 12, F = 1536;
        auto m = std::make_unique<PreNormBlock>(D, H, F, g);
        PreNormBlock *mp = m.get();
        M.root = std::move(m);
        M.add_input("x", {B, L, D}, normal(3, 1, (int64_t)B * L * D), false);
        M.add_input("target", {B, L, D}, normal(3, 2, (int64_t)B * L * D), false);
        std::vector<int32_t> len = ints(3, 3, B, L < 64 ? L : 64, L + 1);
        std::vector<float> mask((size_t)B * L * L, 0.0f);
        for (int b = 0; b < B; b++)
            for (int i = 0; i < L; i++)
                for (int j = len[b]; j < L; j++) mask[((size_t)b * L + i) * L + j] = -INFINITY;
        M.add_int_input("lengths", {B}, len);
        M.add_input("mask", {B, L, L}, std::move(mask), false);
        M.loss_fn = [mp](omt_model &s) {
            return mp->mse_loss(s.input("x").t, s.input("mask").t, s.input("target").t);
        };
    } else if (cfg == 4) {
        const int B = pick(sc.batch, 32);
        struct Crnn : Module {
            Conv2d *conv[4];
            Linear *head;
        };
        auto m = std::make_unique<Crnn>();
        const int ch[5] = {1, 32, 64, 128, 256};
        for (int i = 0; i < 4; i++)
            m->conv[i] = m->child(std::to_string(3 * i), std::make_unique<Conv2d>(ch[i], ch[i + 1], 3, g, 1));
        m->head = m->child("out", std::make_unique<Linear>(256, 37, g));
        Crnn *mp = m.get();
        M.root = std::move(m);
        Generator gx(cfg_seed(4, 1));
        std::vector<float> x((size_t)B * 32 * 128);
        gx.fill_uniform(0.0f, 1.0f, x);
        M.add_input("x", {B, 1, 32, 128}, std::move(x), false);
        std::vector<int32_t> tl = ints(4, 2, B, 1, 11);
        int64_t tot = 0;
        for (int32_t l : tl) tot += l;
        M.add_int_input("labels", {(int)tot}, ints(4, 3, tot, 1, 37));
        M.add_int_input("in_len", {B}, std::vector<int32_t>(B, 32));
        M.add_int_input("tgt_len", {B}, tl);
        for (const char *n : {"labels", "in_len", "tgt_len"}) M.input(n).host_read = true;  // CTC checks them on the host
        M.loss_fn = [mp](omt_model &s) {
            static const int pools[4][2] = {{2, 2}, {2, 2}, {2, 1}, {2, 1}};
            Tensor h = s.input("x").t;
            // Conv2d -> Relu -> MaxPool2d per stage, one record each
            for (int i = 0; i < 4; i++) {
                const Conv2d &cv = *mp->conv[i];
                if (dev().per_op)
                    h = max_pool2d(relu(cv(h)), pools[i][0], pools[i][1], pools[i][0], pools[i][1]);
                else
                    h = conv2d_relu_pool(h, cv.w, cv.b, cv.stride, cv.pad, pools[i][0], pools[i][1], pools[i][0],
                                         pools[i][1]);
            }
            // Mean(axis 2) [B, 256, T], then Permute(2, 0, 1): [T, B, 256]
            Tensor seq = dev().per_op ? permute(mean_axis(h, 2), {2, 0, 1}) : mean_permute_seq(h);
            Tensor lp = log_softmax((*mp->head)(seq));
            const Input &lb = s.input("labels"), &il = s.input("in_len"), &tl = s.input("tgt_len");
            return ctc_loss(lp, lb.hi, il.hi, tl.hi, 0, 1, lb.t, il.t, tl.t);
        };
    } else if (cfg == 5) {
        const int B = pick(sc.batch, 8), L = pick(sc.seq, 512), NL = pick(sc.layers, 4), D = 768, H = 12, F = 3072;
        struct Bert : Module {
            std::vector<EncoderLayer *> layers;
            Linear *head;
        };
        auto m = std::make_unique<Bert>();
        for (int i = 0; i < NL; i++)
            m->layers.push_back(m->child("layer" + std::to_string(i), std::make_unique<EncoderLayer>(D, H, F, g)));
        m->head = m->child("head", std::make_unique<Linear>(D, 9, g));
        Bert *mp = m.get();
        M.root = std::move(m);
        M.add_input("x", {B, L, D}, normal(5, 1, (int64_t)B * L * D), false);
        M.add_int_input("labels", {B * L}, ints(5, 2, (int64_t)B * L, 0, 9));
        M.loss_fn = [mp, B, L](omt_model &s) {
            Tensor h = s.input("x").t;
            for (EncoderLayer *l : mp->layers) h = (*l)(h, nullptr);
            return cross_entropy(reshape((*mp->head)(h), {B * L, 9}), s.input("labels").t);
        };
    } else if (cfg == 6) {
        // TrainCase.Mlp (TrainCase.cs:114-143): Linear(20,32) - ReLU - Linear(32,4), CE, SGD(0.05, momentum 0.9,
        // weight decay 1e-4); the batches come from the caller (omt_input_write) each step.
        const int B = pick(sc.batch, 32);
        Generator gm(1);
        struct Mlp : Module {
            Linear *l1, *l2;
        };
        auto m = std::make_unique<Mlp>();
        m->l1 = m->child("0", std::make_unique<Linear>(20, 32, gm));
        m->l2 = m->child("2", std::make_unique<Linear>(32, 4, gm));
        Mlp *mp = m.get();
        M.root = std::move(m);
        M.add_input("x", {B, 20}, std::vector<float>((size_t)B * 20, 0.0f), false);
        M.add_int_input("labels", {B}, std::vector<int32_t>(B, 0)).set_range(0, 4);
        M.loss_fn = [mp](omt_model &s) {
            return cross_entropy((*mp->l2)(mp->l1->relu_of(s.input("x").t)), s.input("labels").t);
        };
        M.opt_kind = OPT_SGD;
        M.lr = 0.05f;
        M.momentum = 0.9f;
        M.wd = 1e-4f;
    } else if (cfg == 7) {
        // TrainCase.Cnn (TrainCase.cs:145-183): Conv(1,4,3,p1) BN ReLU MaxPool(2) Conv(4,8,3,p1) BN ReLU AvgPool(2)
        // Flatten Linear(72,5), CE, AdamW(3e-3, wd 0.01), CosineLr(3e-3, 60) and ClipNorm(0.5) every step.
        const int B = pick(sc.batch, 8);
        Generator gm(2);
        struct Cnn : Module {
            Conv2d *c1, *c2;
            BatchNorm2d *bn1, *bn2;
            Linear *fc;
        };
        auto m = std::make_unique<Cnn>();
        m->c1 = m->child("0", std::make_unique<Conv2d>(1, 4, 3, gm, 1));
        m->bn1 = m->child("1", std::make_unique<BatchNorm2d>(4));
        m->c2 = m->child("4", std::make_unique<Conv2d>(4, 8, 3, gm, 1));
        m->bn2 = m->child("5", std::make_unique<BatchNorm2d>(8));
        m->fc = m->child("9", std::make_unique<Linear>(72, 5, gm));
        Cnn *mp = m.get();
        M.root = std::move(m);
        M.add_input("x", {B, 1, 12, 12}, std::vector<float>((size_t)B * 144, 0.0f), false);
        M.add_int_input("labels", {B}, std::vector<int32_t>(B, 0)).set_range(0, 5);
        M.loss_fn = [mp, B](omt_model &s) {
            Tensor h = max_pool2d(relu((*mp->bn1)((*mp->c1)(s.input("x").t))), 2, 2, 2, 2);
            h = avg_pool2d(relu((*mp->bn2)((*mp->c2)(h))), 2, 2, 0);
            return cross_entropy((*mp->fc)(reshape(h, {B, 72})), s.input("labels").t);
        };
        M.opt_kind = OPT_ADAMW;
        M.lr = 3e-3f;
        M.wd = 0.01f;
        omt_lr_schedule *cs = nullptr;
        check(nullptr, omt_lr_cosine(3e-3f, 60, 0.0f, &cs), "CosineLr");
        M.schedule = std::move(cs->s);
        omt_lr_free(cs);
        M.clip_max = 0.5f;
    } else if (cfg == 8 || cfg == 9) {
        // TrainCase.Encoder (TrainCase.cs:185-237): EncoderClassifier(vocab 11, width 16, 2 heads, FFN 32, 2 post-norm
        // layers, 2 classes) = Embedding, layers, Mean over the sequence, Linear; CE; Adam(2e-3);
        // WarmupLr(ConstantLr(2e-3), 10, 0.1). Configuration 9 is the same with dropout 0.1 in every layer (seed 77,
        // layer i's two streams 77 + 2i and 78 + 2i; CheckpointTests.cs:21-30).
        const int B = pick(sc.batch, 16), L = pick(sc.seq, 6), NL = pick(sc.layers, 2);
        const float drop = cfg == 9 ? 0.1f : 0.0f;
        M.has_dropout = drop > 0.0f;
        Generator gm(3);
        struct Classifier : Module {
            Embedding *emb;
            std::vector<EncoderLayer *> layers;
            Linear *cls;
        };
        auto m = std::make_unique<Classifier>();
        m->emb = m->child("emb", std::make_unique<Embedding>(11, 16, gm));
        for (int i = 0; i < NL; i++)
            m->layers.push_back(m->child("layer" + std::to_string(i),
                                         std::make_unique<EncoderLayer>(16, 2, 32, gm, drop, 77ull + 2ull * i)));
        m->cls = m->child("cls", std::make_unique<Linear>(16, 2, gm));
        Classifier *mp = m.get();
        M.root = std::move(m);
        M.add_int_input("ids", {B, L}, std::vector<int32_t>((size_t)B * L, 0)).set_range(0, 11);
        M.add_int_input("labels", {B}, std::vector<int32_t>(B, 0)).set_range(0, 2);
        M.loss_fn = [mp](omt_model &s) {
            Tensor h = (*mp->emb)(s.input("ids").t);
            for (EncoderLayer *l : mp->layers) h = (*l)(h, nullptr);
            return cross_entropy((*mp->cls)(mean_axis(h, 1)), s.input("labels").t);
        };
        M.opt_kind = OPT_ADAM;
        M.lr = 2e-3f;
        M.wd = 0.0f;
        omt_lr_schedule *cs = nullptr, *ws = nullptr;
        check(nullptr, omt_lr_constant(2e-3f, &cs), "ConstantLr");
        check(nullptr, omt_lr_warmup(cs, 10, 0.1f, &ws), "WarmupLr");
        M.schedule = std::move(ws->s);
        omt_lr_free(ws);
        omt_lr_free(cs);
    } else if (cfg == 10) {
        // A weight applied twice (the layer-level form of the reference's DiamondGraphSumsBothPaths,
        // BackwardEngineTests.cs:13-25): Linear(64,128) - ReLU - T - ReLU - T - ReLU - Linear(128,64), T one
        // Linear(128,128) whose gradient is the sum of both uses (AccumulateLeaf, Engine.cs:292-328), CE, AdamW.
        const int B = pick(sc.batch, 256);
        struct Tied : Module {
            Linear *l1, *t, *l2;
        };
        auto m = std::make_unique<Tied>();
        m->l1 = m->child("0", std::make_unique<Linear>(64, 128, g));
        m->t = m->child("1", std::make_unique<Linear>(128, 128, g));
        m->l2 = m->child("2", std::make_unique<Linear>(128, 64, g));
        Tied *mp = m.get();
        M.root = std::move(m);
        M.add_input("x", {B, 64}, normal(10, 1, (int64_t)B * 64), false);
        M.add_int_input("labels", {B}, ints(10, 2, B, 0, 64));
        M.loss_fn = [mp](omt_model &s) {
            Tensor h = relu((*mp->l1)(s.input("x").t));
            h = relu((*mp->t)(relu((*mp->t)(h))));
            return cross_entropy((*mp->l2)(h), s.input("labels").t);
        };
    } else {
        throw Error(OM_E_ARG, "unknown configuration " + std::to_string(cfg));
    }
}

// ------------------------------------------------------------------------------------------------ C ABI
static std::string g_create_err;
void omt::set_global_error(const std::string &msg) { g_create_err = msg; }

template <class F>
static om_status guard(omt_model *m, F f) {
    try {
        if (m) set_dev(m->device.get());
        f();
        return OM_OK;
    } catch (const Error &e) {
        if (m) m->err = e.what();
        else g_create_err = e.what();
        return e.code;
    } catch (const ckpt::Failure &e) {
        if (m) m->err = e.what();
        else g_create_err = e.what();
        return OMT_E_CKPT_BAD_HEADER + (int)e.kind;
    } catch (const std::exception &e) {
        if (m) m->err = e.what();
        else g_create_err = e.what();
        return OM_E_STATE;
    }
}

extern "C" {

om_status omt_config_create(int device, int cfg, const omt_scale *scale, omt_model **out) {
    return omt_config_create_records(device, cfg, scale, OMT_RECORDS_FUSED, out);
}

om_status omt_config_create_records(int device, int cfg, const omt_scale *scale, int records, omt_model **out) {
    if (!out) return OM_E_ARG;
    *out = nullptr;
    if (records != OMT_RECORDS_FUSED && records != OMT_RECORDS_PER_OP) {
        g_create_err = "omt_config_create_records: records must be OMT_RECORDS_FUSED or OMT_RECORDS_PER_OP";
        return OM_E_ARG;
    }
    auto *m = new omt_model();
    om_status s = guard(nullptr, [&] {
        m->device = std::make_unique<Device>(device);
        m->device->per_op = records == OMT_RECORDS_PER_OP;
        set_dev(m->device.get());
        omt_scale sc{0, 0, 0, 0};
        if (scale) sc = *scale;
        build(*m, cfg, sc);
        std::vector<std::vector<float>> init;
        m->root->take_init(init);
        m->finalize(std::move(init));
    });
    if (s != OM_OK) {
        delete m;
        return s;
    }
    *out = m;
    return OM_OK;
}

void omt_destroy(omt_model *m) {
    if (!m) return;
    set_dev(m->device.get());
    if (m->graph) om_graph_destroy(m->graph);
    if (m->stager) om_stager_destroy(m->stager);
    if (m->loss_rb) om_readback_destroy(m->loss_rb);
    m->root.reset();
    m->params.clear();
    m->leaves.clear();
    m->inputs.clear();
    m->device.reset();
    set_dev(nullptr);
    delete m;
}

const char *omt_last_error(omt_model *m) { return m ? m->err.c_str() : g_create_err.c_str(); }

float omt_lr(omt_model *m) { return m ? m->lr : std::nanf(""); }
om_status omt_set_lr(omt_model *m, float lr) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        if (!std::isfinite(lr) || lr < 0.0f) throw Error(OM_E_ARG, "omt_set_lr: rate must be finite and not negative");
        m->lr = lr;
    });
}
om_status omt_set_lr_schedule(omt_model *m, const omt_lr_schedule *s) {
    if (!m) return OM_E_ARG;
    m->schedule = (s && s->s) ? s->s->clone() : nullptr;
    return OM_OK;
}
om_status omt_clip_grad_norm(omt_model *m, float max_norm, int infinity_norm, float *norm) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        if (!(max_norm > 0.0f)) throw Error(OM_E_ARG, "ClipNorm: the maximum norm must be positive");
        m->clip_norm(max_norm, infinity_norm, true);
        if (norm)
            check(m->device->ctx(), om_download(m->device->ctx(), norm, m->clip_buf, sizeof(float)), "norm readback");
    });
}
om_status omt_clip_grad_value(omt_model *m, float clip_value) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        if (!(clip_value >= 0.0f)) throw Error(OM_E_ARG, "ClipValue: the bound must not be negative");
        m->clip_value(clip_value);
    });
}
om_status omt_set_clip(omt_model *m, float max_norm, int infinity_norm) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        if (!(max_norm >= 0.0f)) throw Error(OM_E_ARG, "omt_set_clip: max_norm must be positive (or 0 to switch off)");
        m->graph_drop();  // the clip launches are part of the recorded step
        m->clip_max = max_norm;
        m->clip_inf = infinity_norm;
    });
}
om_status omt_last_grad_norm(omt_model *m, float *norm) {
    if (!m || !norm) return OM_E_ARG;
    return guard(m, [&] {
        check(m->device->ctx(), om_download(m->device->ctx(), norm, m->clip_buf, sizeof(float)), "norm readback");
    });
}

om_status omt_step(omt_model *m, float *loss) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        float v = m->step();
        if (loss) *loss = v;
    });
}
om_status omt_set_step_graph(omt_model *m, int on) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        m->graph_drop();
        m->graph_on = on != 0;
    });
}
int omt_step_graph_ready(omt_model *m) { return m && m->graph && m->graphable() ? 1 : 0; }
om_status omt_set_gelu(omt_model *m, int mode) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        check(m->device->ctx(), om_ctx_set_gelu(m->device->ctx(), mode), "om_ctx_set_gelu");
        m->graph_drop();  // recorded launches carry the old epilogue
    });
}
om_status omt_forward_backward(omt_model *m, float *loss) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        float v = m->forward_backward();
        settle_grads(m->leaves);
        if (loss) *loss = v;
    });
}
om_status omt_forward(omt_model *m, float *loss) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        float v = m->forward();
        if (loss) *loss = v;
    });
}
om_status omt_backward(omt_model *m) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        m->backward_pass();
        settle_grads(m->leaves);
    });
}
om_status omt_optimizer_step(omt_model *m) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        m->optimizer_step();
        m->device->sync();
    });
}
om_ctx *omt_ctx(omt_model *m) { return m ? m->device->ctx() : nullptr; }

int omt_param_count(omt_model *m) { return m ? (int)m->params.size() : 0; }
om_status omt_param_info(omt_model *m, int i, char *name, int cap, int *ndim, int32_t *dims) {
    if (!m || i < 0 || i >= (int)m->params.size()) return OM_E_ARG;
    const auto &p = m->params[i];
    if (name && cap > 0) {
        std::strncpy(name, p.first.c_str(), (size_t)cap - 1);
        name[cap - 1] = 0;
    }
    if (ndim) *ndim = (int)p.second->shape.size();
    if (dims)
        for (size_t d = 0; d < p.second->shape.size(); d++) dims[d] = p.second->shape[d];
    return OM_OK;
}
static float *param_block(omt_model *m, int which) {
    return which == 0 ? m->pb : which == 1 ? m->gb : which == 2 ? m->mb : which == 3 ? m->vb : nullptr;
}
om_status omt_param_read(omt_model *m, int i, int which, float *host, int64_t numel) {
    if (!m || i < 0 || i >= (int)m->params.size() || !param_block(m, which) || !host) return OM_E_ARG;
    return guard(m, [&] {
        if (numel != m->params[i].second->numel) throw Error(OM_E_ARG, "omt_param_read: wrong element count");
        if (which == 1) settle_grads(m->leaves);
        check(m->device->ctx(), om_download(m->device->ctx(), host, param_block(m, which) + m->offset[i],
                                            sizeof(float) * (uint64_t)numel), "download");
    });
}
om_status omt_param_write(omt_model *m, int i, int which, const float *host, int64_t numel) {
    if (!m || i < 0 || i >= (int)m->params.size() || !param_block(m, which) || !host) return OM_E_ARG;
    return guard(m, [&] {
        if (numel != m->params[i].second->numel) throw Error(OM_E_ARG, "omt_param_write: wrong element count");
        check(m->device->ctx(), om_upload(m->device->ctx(), param_block(m, which) + m->offset[i], host,
                                          sizeof(float) * (uint64_t)numel), "upload");
        if (which == 0) touch(m->params[i].second);
        m->device->sync();
    });
}
int64_t omt_step_count(omt_model *m) { return m ? m->step_count : -1; }

om_status omt_checkpoint_save(omt_model *m, const char *path, int with_optimizer, int n_extra,
                              const char *const *extra_keys, const int64_t *extra_values) {
    if (!m || !path || !*path || n_extra < 0 || (n_extra > 0 && (!extra_keys || !extra_values))) return OM_E_ARG;
    return guard(m, [&] {
        std::map<std::string, int64_t> extra;
        for (int i = 0; i < n_extra; i++) {
            if (!extra_keys[i]) throw Error(OM_E_ARG, "omt_checkpoint_save: NULL extra key");
            extra[extra_keys[i]] = extra_values[i];
        }
        m->save_checkpoint(path, with_optimizer != 0, extra);
    });
}
om_status omt_checkpoint_load(omt_model *m, const char *path, int with_optimizer, int *had_optimizer) {
    if (!m || !path || !*path) return OM_E_ARG;
    return guard(m, [&] {
        m->graph_drop();
        const bool had = m->load_checkpoint(path, with_optimizer != 0);
        if (had_optimizer) *had_optimizer = had ? 1 : 0;
    });
}
int omt_checkpoint_extra_count(omt_model *m) { return m ? (int)m->ckpt_extra.size() : 0; }
om_status omt_checkpoint_extra(omt_model *m, int i, char *key, int cap, int64_t *value) {
    if (!m || i < 0 || i >= (int)m->ckpt_extra.size()) return OM_E_ARG;
    auto it = m->ckpt_extra.begin();
    std::advance(it, i);
    if (key && cap > 0) {
        std::strncpy(key, it->first.c_str(), (size_t)cap - 1);
        key[cap - 1] = 0;
    }
    if (value) *value = it->second;
    return OM_OK;
}
om_status omt_checkpoint_check(const char *path, const omt_tensor_spec *model, int n_model) {
    if (!path || n_model < 0 || (n_model > 0 && !model)) return OM_E_ARG;
    return guard(nullptr, [&] {
        std::vector<ckpt::Tensor> target;
        for (int i = 0; i < n_model; i++) {
            ckpt::Tensor t;
            if (!model[i].name || model[i].dtype < 0 || model[i].dtype > 2 || model[i].ndim < 0 ||
                (model[i].ndim > 0 && !model[i].dims))
                throw Error(OM_E_ARG, "omt_checkpoint_check: bad target entry " + std::to_string(i));
            t.name = model[i].name;
            t.dtype = (ckpt::DType)model[i].dtype;
            t.dims.assign(model[i].dims, model[i].dims + model[i].ndim);
            target.push_back(std::move(t));
        }
        ckpt::load(path, target, nullptr);
    });
}

om_status omt_set_optimizer(omt_model *m, int kind, float lr, float beta1, float beta2, float eps, float weight_decay,
                            float momentum, float dampening, int nesterov, int amsgrad) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        m->graph_drop();  // new optimizer state and kind
        m->set_optimizer(kind, lr, beta1, beta2, eps, weight_decay, momentum, dampening, nesterov != 0, amsgrad != 0);
    });
}

uint64_t omt_batch_bytes(omt_model *m) {
    if (!m) return 0;
    if (m->batch_off.empty()) m->batch_layout();
    return m->batch_bytes;
}
om_status omt_batch_layout(omt_model *m, int i, uint64_t *offset, uint64_t *bytes) {
    if (!m || i < 0 || i >= (int)m->inputs.size()) return OM_E_ARG;
    if (m->batch_off.empty()) m->batch_layout();
    if (offset) *offset = m->batch_off[i];
    if (bytes) *bytes = (uint64_t)m->inputs[i].t->numel * 4;
    return OM_OK;
}
om_status omt_batch_begin(omt_model *m, void **host) {
    if (!m || !host) return OM_E_ARG;
    return guard(m, [&] { m->batch_begin(host); });
}
om_status omt_batch_commit(omt_model *m) {
    if (!m) return OM_E_ARG;
    return guard(m, [&] {
        m->graph_drop();  // staged steps replace the inputs' addresses
        m->batch_commit();
    });
}
int omt_batch_queued(omt_model *m) { return m ? (int)m->staged.size() : 0; }

int omt_buffer_count(omt_model *m) { return m ? (int)m->buffers.size() : 0; }
om_status omt_buffer_info(omt_model *m, int i, char *name, int cap, int64_t *numel) {
    if (!m || i < 0 || i >= (int)m->buffers.size()) return OM_E_ARG;
    if (name && cap > 0) {
        std::strncpy(name, m->buffers[i].first.c_str(), (size_t)cap - 1);
        name[cap - 1] = 0;
    }
    if (numel) *numel = m->buffers[i].second.numel;
    return OM_OK;
}
om_status omt_buffer_read(omt_model *m, int i, float *host, int64_t numel) {
    if (!m || i < 0 || i >= (int)m->buffers.size() || !host) return OM_E_ARG;
    return guard(m, [&] {
        if (numel != m->buffers[i].second.numel) throw Error(OM_E_ARG, "omt_buffer_read: wrong element count");
        check(m->device->ctx(), om_download(m->device->ctx(), host, m->buffers[i].second.dev,
                                            sizeof(float) * (uint64_t)numel), "download");
    });
}
om_status omt_buffer_write(omt_model *m, int i, const float *host, int64_t numel) {
    if (!m || i < 0 || i >= (int)m->buffers.size() || !host) return OM_E_ARG;
    return guard(m, [&] {
        if (numel != m->buffers[i].second.numel) throw Error(OM_E_ARG, "omt_buffer_write: wrong element count");
        check(m->device->ctx(), om_upload(m->device->ctx(), m->buffers[i].second.dev, host,
                                          sizeof(float) * (uint64_t)numel), "upload");
        m->device->sync();
    });
}

int omt_input_count(omt_model *m) { return m ? (int)m->inputs.size() : 0; }
om_status omt_input_info(omt_model *m, int i, char *name, int cap, int *is_int, int *ndim, int32_t *dims) {
    if (!m || i < 0 || i >= (int)m->inputs.size()) return OM_E_ARG;
    const Input &in = m->inputs[i];
    if (name && cap > 0) {
        std::strncpy(name, in.name.c_str(), (size_t)cap - 1);
        name[cap - 1] = 0;
    }
    if (is_int) *is_int = in.is_int ? 1 : 0;
    if (ndim) *ndim = (int)in.t->shape.size();
    if (dims)
        for (size_t d = 0; d < in.t->shape.size(); d++) dims[d] = in.t->shape[d];
    return OM_OK;
}
om_status omt_input_read(omt_model *m, int i, void *host, int64_t numel) {
    if (!m || i < 0 || i >= (int)m->inputs.size() || !host) return OM_E_ARG;
    const Input &in = m->inputs[i];
    if (numel != in.t->numel) return OM_E_ARG;
    if (in.is_int) std::memcpy(host, in.hi.data(), sizeof(int32_t) * (size_t)numel);
    else std::memcpy(host, in.hf.data(), sizeof(float) * (size_t)numel);
    return OM_OK;
}
om_status omt_input_write(omt_model *m, int i, const void *host, int64_t numel) {
    if (!m || i < 0 || i >= (int)m->inputs.size() || !host) return OM_E_ARG;
    return guard(m, [&] {
        Input &in = m->inputs[i];
        if (numel != in.t->numel) throw Error(OM_E_ARG, "omt_input_write: wrong element count for " + in.name);
        if (in.host_read) m->graph_drop();
        if (in.is_int) {
            const int32_t *v = static_cast<const int32_t *>(host);
            for (int64_t k = 0; k < numel; k++)
                if (v[k] < in.lo || v[k] >= in.hi_bound)
                    throw Error(OM_E_ARG, "omt_input_write: " + in.name + "[" + std::to_string(k) + "] = " +
                                              std::to_string(v[k]) + " is out of range");
            std::memcpy(in.hi.data(), v, sizeof(int32_t) * (size_t)numel);
            check(m->device->ctx(), om_upload(m->device->ctx(), in.t->idata, v, sizeof(int32_t) * (uint64_t)numel),
                  "upload");
        } else {
            std::memcpy(in.hf.data(), host, sizeof(float) * (size_t)numel);
            check(m->device->ctx(), om_upload(m->device->ctx(), in.t->data, host, sizeof(float) * (uint64_t)numel),
                  "upload");
        }
        touch(in.t);
    });
}
om_status omt_input_grad(omt_model *m, int i, float *host, int64_t numel) {
    if (!m || i < 0 || i >= (int)m->inputs.size() || !host) return OM_E_ARG;
    return guard(m, [&] {
        const Input &in = m->inputs[i];
        if (!in.t->grad || numel != in.t->numel) throw Error(OM_E_ARG, "input has no gradient of that size");
        settle_grads(m->leaves);
        check(m->device->ctx(), om_download(m->device->ctx(), host, in.t->grad, sizeof(float) * (uint64_t)numel),
              "download");
    });
}

void omt_generate(uint64_t seed, int kind, float lo, float hi, void *out, int64_t n) {
    Generator g(seed);
    if (kind == 2) {
        std::vector<int32_t> v((size_t)n);
        g.fill_ints((int32_t)lo, (int32_t)hi, v);
        std::memcpy(out, v.data(), sizeof(int32_t) * (size_t)n);
    } else {
        std::vector<float> v((size_t)n);
        if (kind == 0) g.fill_uniform(lo, hi, v);
        else g.fill_normal(v);
        std::memcpy(out, v.data(), sizeof(float) * (size_t)n);
    }
}

}  // extern "C"
