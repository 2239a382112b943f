// The reference's checkpoint file (Checkpoint.cs:48-649; layout in its docs/training.md section 6): a 64-byte
// header ("ONEMCKPT", version 1), a compact UTF-8 JSON manifest, and the state tensors as raw little-endian
// elements at 64-byte-aligned offsets of the data region. This part is host code only: it turns lists of named
// tensors into a file and back, checking an untrusted file completely before anything is handed to the caller.
#pragma once

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace omt {
namespace ckpt {

// CheckpointErrorKind (Checkpoint.cs:11-24).
enum Kind { BadHeader = 0, BadManifest = 1, BadTensor = 2, Mismatch = 3, UnsupportedStream = 4 };
struct Failure : std::runtime_error {
    Kind kind;
    Failure(Kind k, const std::string &m) : std::runtime_error(m), kind(k) {}
};

enum DType { F32 = 0, I32 = 1, I64 = 2 };
inline int elem_size(DType t) { return t == I64 ? 8 : 4; }

// A named tensor of the state: its type and shape, and (when writing) its host bytes.
struct Tensor {
    std::string name;
    DType dtype = F32;
    std::vector<int> dims;
    const void *data = nullptr;  // writing only: little-endian elements, numel * elem_size bytes
    int64_t numel() const {
        int64_t n = 1;
        for (int d : dims) n *= d;
        return n;
    }
    int64_t bytes() const { return numel() * elem_size(dtype); }
};

// An optimizer as a checkpoint sees it (Optimizer.Kind, HyperParameters(), StateTensors, StepCount).
struct Optimizer {
    std::string kind;                                   // "sgd", "adam", "adamw"
    std::vector<std::pair<std::string, float>> hyper;   // in HyperParameters() order
    std::vector<Tensor> state;                          // in StateTensors order
    std::vector<std::vector<int>> param_dims;           // per state entry: its parameter's shape, or empty for flags
    int64_t step = 0;
};

// Writes the file (to path + ".tmp", then renamed over path). extra: integer values, written in key order.
void save(const std::string &path, const std::vector<Tensor> &model, const Optimizer *opt,
          const std::map<std::string, int64_t> &extra);

// What a load produced, after every check passed.
struct Loaded {
    bool had_optimizer = false;
    std::map<std::string, int64_t> extra;
    std::vector<std::vector<char>> model;  // bytes per model tensor, in target order
    // When optimizer state was asked for: bytes per state entry (empty for a state saved as [0], i.e. zero),
    // the step count and the hyper-parameters by name.
    std::vector<std::vector<char>> state;
    int64_t step = 0;
    std::map<std::string, float> hyper;
};

// Reads and checks `path` against the target model state (names, types, shapes in order) and, when `opt` is given,
// the target optimizer (kind, hyper-parameter names, state names/types/shapes). `settings_ok` vets the saved
// hyper-parameters (fixed settings equal, rates valid) and returns an error message or "" (a Mismatch).
// Throws Failure with the reference's kind for the first failed check, in the reference's order.
Loaded load(const std::string &path, const std::vector<Tensor> &model, const Optimizer *opt,
            std::string (*settings_ok)(const std::map<std::string, float> &, const Optimizer &) = nullptr);

}  // namespace ckpt
}  // namespace omt
