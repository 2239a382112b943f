/*
 * om_train.h — C ABI of libom_train.so, the C++ training tape that sits above libom_hip.so (include/om.h).
 *
 * The reference keeps its tape in C# (RecursiveAI.OneModel.Training over the tensor layer's autograd); this image has
 * no .NET toolchain, so the tape is restated in C++ with the reference's surface: modules that register parameters in
 * order (NnModule.cs:54-165), ops that record backward records, Tensor.Backward() (Engine.cs:21-207), losses
 * (Losses.cs), ZeroGrad and SGD/Adam/AdamW Step() (Optimizers.cs:184-608). A model here is one of the benchmark's
 * training configurations, built on the device with its synthetic inputs; this ABI is what tests and bench.py drive.
 *
 * Conventions as in om.h: status codes (0 = OK), messages from omt_last_error, no C++ types across the boundary.
 */
#ifndef OM_TRAIN_H
#define OM_TRAIN_H

#include <stdint.h>

#include "om.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct omt_model omt_model;

/* Configuration sizes; 0 keeps the configuration's default (batch, sequence length / image side, layer count). */
typedef struct {
    int32_t batch, seq, layers, hw;
} omt_scale;

/* Builds configuration `cfg` (1 = MLP 784-256-10, 2 = conv block, 3 = MiniLM-shaped pre-LN block, 4 = CRNN + CTC,
 * 5 = BERT-base-shaped 4-layer stack) on `device`: parameters from the SplitMix64 generator in registration order
 * (Kaiming-uniform +-1/sqrt(fan_in), LayerNorm 1/0), synthetic inputs from seed 20261201 + 100*cfg + index, and an
 * AdamW(lr 1e-3, betas 0.9/0.999, eps 1e-8, wd 0.01) over the parameter arena.
 * Configurations 6-8 are the models of the reference's training-curve tests (TrainCase.cs:114-237), whose batches
 * the caller supplies each step with omt_input_write: 6 = MLP 20-32-4 with SGD(0.05, momentum 0.9, wd 1e-4);
 * 7 = conv/BatchNorm/pool net with AdamW(3e-3, wd 0.01), CosineLr(3e-3, 60) and ClipNorm(0.5) inside omt_step;
 * 8 = Embedding + 2 post-norm encoder layers + mean + Linear with Adam(2e-3) and WarmupLr(ConstantLr(2e-3), 10, 0.1);
 * 9 = configuration 8 with dropout 0.1 after attention and feed-forward in every layer (seeds 77 + 2i, 78 + 2i);
 * 10 = MLP 64-128-[128]-[128]-64 whose middle Linear is applied twice, so its gradient sums two uses
 * (BackwardEngineTests.cs:13-25 at layer level), CE, AdamW(1e-3, wd 0.01), batch 256. */
om_status omt_config_create(int device, int cfg, const omt_scale *scale, omt_model **out);
/* The same with a choice of record structure. OMT_RECORDS_FUSED (what omt_config_create builds): composite records
 * that a C# drop-in would need as module-level fused ops (a Linear with its bias in one record, q|k|v as one product
 * over weights the arena lays out side by side, the feed-forward sub-block with its GELU and residual, a conv stage
 * with its ReLU and max pool, MSE and cross-entropy as one record each) and weight gradients queued by the engine and
 * launched together. OMT_RECORDS_PER_OP: exactly the records the reference's ops and modules create, each rule one
 * C-ABI call made when Engine.Execute reaches it (Engine.cs:160-191), no queue, no colocation: Linear = Reshape,
 * MatMul(x, W.T()), Add(bias), Reshape (Ops.Layers.cs:715-733); MultiHeadAttention = three Linears, Attention, one
 * Linear (Layers.cs:497-516); Conv2d, Relu and MaxPool2d apart; Mean then Permute; Mse = Sub, Mul, Mean and
 * CrossEntropy = LogSoftmax, NllLoss (Losses.cs:20-91). Views stay views (the kernels address the reshaped, transposed
 * and head-permuted tensors in place). Both build the same parameters in the same order from the same generator. */
enum { OMT_RECORDS_FUSED = 0, OMT_RECORDS_PER_OP = 1 };
om_status omt_config_create_records(int device, int cfg, const omt_scale *scale, int records, omt_model **out);
void omt_destroy(omt_model *m);
const char *omt_last_error(omt_model *m); /* m may be NULL for creation errors */

/* One training step: ZeroGrad, forward, loss.Backward(), optimizer.Step(). *loss is the forward's loss, read where
 * the reference's step reads it (TrainCase.cs:117-127): the call returns once that value has landed on the host,
 * with the backward and the update queued behind it on the model's stream (omt_ctx). Every later call that touches
 * the model's memory is ordered after them; om_ctx_sync(omt_ctx(m)) waits for them. */
om_status omt_step(omt_model *m, float *loss);
/* Step graphs (om_graph_*, include/om.h) for omt_step: with `on`, the next omt_step runs as usual, the one after it
 * is recorded into a HIP graph and launched, and later ones replay that graph, with only the host-side effects of
 * a step (rate from the schedule, step count, parameter versions) done on the host; results are bit-identical to
 * omt_step without graphs. The graph is dropped and recorded again after omt_set_optimizer, omt_set_clip,
 * omt_checkpoint_load, omt_batch_commit (staged steps run without a graph), and omt_input_write of an input whose
 * host copy the step reads (configuration 4's lengths and labels). SGD and dropout models always run without one.
 * No counterpart in the reference (its step runs on the CPU); for callers whose step is bound by launch overhead. */
om_status omt_set_step_graph(omt_model *m, int on);
/* 1 when the next omt_step will replay a recorded graph. */
int omt_step_graph_ready(omt_model *m);
/* om_ctx_set_gelu on the model's context (OM_GELU_FAST, the default, or OM_GELU_REFERENCE for the reference's GELU
 * polynomials bit for bit in the feed-forward products' epilogues); a recorded step graph is dropped. */
om_status omt_set_gelu(omt_model *m, int mode);
/* ZeroGrad, forward and backward only (gradients are left in the arena). */
om_status omt_forward_backward(omt_model *m, float *loss);
/* The same two halves as separate calls, for callers that act between them: omt_forward runs ZeroGrad and the
 * forward, reads the loss and keeps the graph (and the step's staged batch); omt_backward runs loss.Backward() over
 * it (Tensor.Backward, Engine.cs:21-207). Records are released by the backward, so a second omt_backward on the same
 * forward fails with OM_E_STATE (Engine.cs:136-141). A tensor the graph saved that was written in place since the
 * forward (omt_param_write of a value, omt_input_write, omt_optimizer_step, omt_checkpoint_load) makes omt_backward
 * fail with OMT_E_TENSOR_VERSION before any gradient is written for its record (SavedTensor.Unpack, Autograd.cs:
 * 222-237). The next omt_forward / omt_step drops the graph. */
enum { OMT_E_TENSOR_VERSION = 21 /* TensorVersionException (Autograd.cs:188-191) */ };
om_status omt_forward(omt_model *m, float *loss);
om_status omt_backward(omt_model *m);
/* optimizer.Step() alone, on the gradients currently in the arena. */
om_status omt_optimizer_step(omt_model *m);
/* The model's om_ctx (its stream orders every launch of the step). */
om_ctx *omt_ctx(omt_model *m);

/* Parameters in Parameters() order. which: 0 value, 1 gradient, 2 first moment, 3 second moment. */
int omt_param_count(omt_model *m);
om_status omt_param_info(omt_model *m, int i, char *name, int name_cap, int *ndim, int32_t *dims);
om_status omt_param_read(omt_model *m, int i, int which, float *host, int64_t numel);
om_status omt_param_write(omt_model *m, int i, int which, const float *host, int64_t numel);
/* Optimizer step count (Optimizer.StepCount). */
int64_t omt_step_count(omt_model *m);

/* Named inputs ("x", "target", "labels", "lengths", "mask", "in_len", "tgt_len"): float or int32 host copies.
 * is_int reports the element type; omt_input_read copies numel elements. */
int omt_input_count(omt_model *m);
om_status omt_input_info(omt_model *m, int i, char *name, int name_cap, int *is_int, int *ndim, int32_t *dims);
om_status omt_input_read(omt_model *m, int i, void *host, int64_t numel);
/* Gradient of an input that requires one (C2's image), after a backward. */
om_status omt_input_grad(omt_model *m, int i, float *host, int64_t numel);
/* Replaces input i with numel host values (float, or int32 for an int input, which must lie in the range the
 * model accepts: labels below the class count, ids below the vocabulary), uploaded on the model's stream ahead of
 * the next step: the per-step batch of a training loop (TrainCase.cs:77-96 builds its batches on the host). */
om_status omt_input_write(omt_model *m, int i, const void *host, int64_t numel);

/* Staged batches (om_stager, include/om.h): a batch packs the model's inputs in input order, input i at byte
 * `offset` (256-byte aligned) with `bytes` bytes (float32 or int32 elements). omt_batch_begin hands out a pinned
 * host buffer of omt_batch_bytes to fill in place; omt_batch_commit checks the int inputs' ranges and queues the
 * upload on the copy stream; the next omt_step / omt_forward_backward takes the oldest committed batch as its
 * inputs (after its upload) and releases it after its last launch, so committing batch k+1 before running step k
 * overlaps its upload with step k. Up to 3 batches may wait. Without a committed batch a step reads the inputs as
 * last written by omt_input_write (which a staged batch does not change). */
uint64_t omt_batch_bytes(omt_model *m);
om_status omt_batch_layout(omt_model *m, int i, uint64_t *offset, uint64_t *bytes);
om_status omt_batch_begin(omt_model *m, void **host);
om_status omt_batch_commit(omt_model *m);
int omt_batch_queued(omt_model *m);

/* Named float state buffers that are not parameters (NnModule.RegisterBuffer, NnModule.cs:54-65): BatchNorm2d's
 * running_mean and running_var, in named_buffers() order ("1.running_mean", ...). */
int omt_buffer_count(omt_model *m);
om_status omt_buffer_info(omt_model *m, int i, char *name, int name_cap, int64_t *numel);
om_status omt_buffer_read(omt_model *m, int i, float *host, int64_t numel);
om_status omt_buffer_write(omt_model *m, int i, const float *host, int64_t numel);

/* Replaces the model's optimizer with a new one over Parameters() (fresh state: zero moments and momentum buffers,
 * step count 0): kind 0 = Sgd(lr, momentum, dampening, weight_decay, nesterov) (Optimizers.cs:270-330), 1 = Adam
 * (L2 weight decay added to g), 2 = AdamW (decoupled decay) (Optimizers.cs:374-608), with betas, eps and amsgrad.
 * Arguments the reference rejects return OM_E_ARG. Configurations 1-5 default to AdamW(1e-3, 0.9, 0.999, 1e-8, 0.01);
 * 6-8 to the optimizers of the reference's training-curve cases (omt_config_create). */
om_status omt_set_optimizer(omt_model *m, int kind, float lr, float beta1, float beta2, float eps, float weight_decay,
                            float momentum, float dampening, int nesterov, int amsgrad);

/* ------------------------------------------------------------------------------------------ checkpoints */
/* Checkpoint errors (CheckpointErrorKind, Checkpoint.cs:11-24), returned by the calls below. */
enum {
    OMT_E_CKPT_BAD_HEADER = 16,        /* header missing, malformed or inconsistent with the file length */
    OMT_E_CKPT_BAD_MANIFEST = 17,      /* manifest not the expected JSON, or a field missing or out of range */
    OMT_E_CKPT_BAD_TENSOR = 18,        /* a tensor entry outside the data region or sized unlike its shape */
    OMT_E_CKPT_MISMATCH = 19,          /* well-formed but not the model's (or optimizer's) state */
    OMT_E_CKPT_UNSUPPORTED_STREAM = 20 /* not a regular, seekable file */
};
/* Checkpoint.Save (Checkpoint.cs:55-138): the ONEMCKPT file of the model's StateDict (parameters and buffers per
 * module, then children) and, with with_optimizer, the optimizer's kind, step count, hyper-parameters (float bit
 * patterns) and state tensors; n_extra integer values by key (written in key order). Written to path + ".tmp",
 * then renamed. The same state always writes the same bytes. */
om_status omt_checkpoint_save(omt_model *m, const char *path, int with_optimizer, int n_extra,
                              const char *const *extra_keys, const int64_t *extra_values);
/* Checkpoint.Load (Checkpoint.cs:151-331): checks the whole file against the model (and, with with_optimizer, its
 * optimizer: kind, fixed settings, state shapes) before changing anything, then restores parameters, buffers,
 * optimizer state, rate, weight decay and step count. *had_optimizer (may be NULL) says whether the file holds
 * optimizer state; a file without it fails with OMT_E_CKPT_MISMATCH when with_optimizer is set. */
om_status omt_checkpoint_load(omt_model *m, const char *path, int with_optimizer, int *had_optimizer);
/* The extra values of the last checkpoint loaded, in key order. */
int omt_checkpoint_extra_count(omt_model *m);
om_status omt_checkpoint_extra(omt_model *m, int i, char *key, int key_cap, int64_t *value);
/* Host only, no device: checks a checkpoint file against a model-state target given as (name, dtype 0 = f32,
 * 1 = i32, 2 = i64, shape) entries in state order, exactly as a model-only omt_checkpoint_load would, and returns
 * its status (message: omt_last_error(NULL)). For tools that vet a file before a device is involved. */
typedef struct {
    const char *name;
    int32_t dtype;
    int32_t ndim;
    const int32_t *dims;
} omt_tensor_spec;
om_status omt_checkpoint_check(const char *path, const omt_tensor_spec *model, int n_model);

/* Host helper with no device: the SplitMix64 generator of the tape (for cross-checks against the reference's
 * Generator): kind 0 = uniform [lo, hi), 1 = benchmark normal, 2 = ints in [lo, hi). */
void omt_generate(uint64_t seed, int kind, float lo, float hi, void *out, int64_t n);

/* ------------------------------------------------------------------------------------------ learning rate */
/* Optimizer.LearningRate (Optimizers.cs:30-60): the rate the next step uses. */
float omt_lr(omt_model *m);
om_status omt_set_lr(omt_model *m, float lr);

/* LrSchedule and its subclasses (Schedules.cs:151-422): pure functions of the step count, IEEE double in the
 * reference's order, so rates are the reference's bit for bit. Arguments the reference rejects with
 * ArgumentOutOfRangeException return OM_E_ARG (message: omt_last_error(NULL)). Host only, no device. */
typedef struct omt_lr_schedule omt_lr_schedule;
om_status omt_lr_constant(float lr, omt_lr_schedule **out);                                     /* ConstantLr */
om_status omt_lr_step(float base_lr, int64_t step_size, float gamma, omt_lr_schedule **out);    /* StepLr */
om_status omt_lr_cosine(float base_lr, int64_t total_steps, float min_lr, omt_lr_schedule **out); /* CosineLr */
/* WarmupLr over a copy of `after` (the caller keeps and frees its own). */
om_status omt_lr_warmup(const omt_lr_schedule *after, int64_t warmup_steps, float start_factor,
                        omt_lr_schedule **out);
om_status omt_lr_warmup_cosine(float base_lr, int64_t warmup_steps, int64_t total_steps, float floor_fraction,
                               omt_lr_schedule **out);                                          /* WarmupCosineLr */
om_status omt_lr_onecycle(float max_lr, int64_t total_steps, float pct_start, float div_factor,
                          float final_div_factor, omt_lr_schedule **out);                       /* OneCycleLr */
void omt_lr_free(omt_lr_schedule *s);
/* LrSchedule.LrAt(step); NaN for a NULL schedule. */
float omt_lr_at(const omt_lr_schedule *s, int64_t step);
/* LrSchedule.Cos: cos(pi * t) for t in [0, 1] (clamped), from + - * / only. */
double omt_lr_cos(double t);
/* LrSchedule.Apply before every optimizer step of the model: the rate becomes s(step count). The model keeps a
 * copy; NULL detaches (the rate then stays where it is). */
om_status omt_set_lr_schedule(omt_model *m, const omt_lr_schedule *s);

/* ------------------------------------------------------------------------------------------ gradient clipping */
/* GradClip.ClipNorm(model.Parameters(), max_norm, infinity_norm) (Schedules.cs:22-100) on the gradients now in the
 * arena, in place, on the device (om_clip_grad_norm). *norm (host, may be NULL) receives the norm ClipNorm returns;
 * asking for it waits for the device. */
om_status omt_clip_grad_norm(omt_model *m, float max_norm, int infinity_norm, float *norm);
/* GradClip.ClipValue(model.Parameters(), clip_value) (Schedules.cs:119-149), in place on the device. */
om_status omt_clip_grad_value(omt_model *m, float clip_value);
/* Makes omt_step run ClipNorm between the backward and the optimizer step (max_norm 0 switches it off). The scaling
 * is folded into AdamW's read of the gradients (om_adam_step_scaled), so the step's parameters and moments equal
 * backward + omt_clip_grad_norm + omt_optimizer_step bit for bit while the gradients stay unscaled. */
om_status omt_set_clip(omt_model *m, float max_norm, int infinity_norm);
/* The norm the last clipped omt_step computed (waits for the device; NaN before the first one). */
om_status omt_last_grad_norm(omt_model *m, float *norm);

#ifdef __cplusplus
}
#endif
#endif /* OM_TRAIN_H */
