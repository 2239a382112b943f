// Host-only driver for the sanitizer run of the checkpoint reader and writer (tests/test_sanitized_host.py): built
// with AddressSanitizer and UndefinedBehaviorSanitizer from onemodel-csharp_amd/train/checkpoint.cpp, it checks
// every file named on the command line against the reference's hostile-test target (a Linear(2, 2) with bias:
// weight [2,2] then bias [2], CheckpointHostileTests.cs:13-16) and prints one line per file, "OK" or the failure's
// CheckpointErrorKind; then it writes a checkpoint with optimizer state and extra values, reads it back and checks
// the round trip. Any sanitizer report ends the process with a non-zero status.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "checkpoint.hpp"

using namespace omt::ckpt;

static const char *kind_name(Kind k) {
    switch (k) {
        case BadHeader: return "BadHeader";
        case BadManifest: return "BadManifest";
        case BadTensor: return "BadTensor";
        case Mismatch: return "Mismatch";
        case UnsupportedStream: return "UnsupportedStream";
    }
    return "?";
}

static std::vector<Tensor> target() {
    Tensor w, b;
    w.name = "weight";
    w.dims = {2, 2};
    b.name = "bias";
    b.dims = {2};
    return {w, b};
}

static int round_trip(const std::string &path) {
    const float w[4] = {1, 2, 3, 4}, b[2] = {5, 6}, m[6] = {0.5f, 0, 0, 0, 0, -1}, v[6] = {0.25f, 0, 0, 0, 0, 2};
    std::vector<Tensor> model = target();
    model[0].data = w;
    model[1].data = b;
    Optimizer opt;
    opt.kind = "adamw";
    opt.hyper = {{"lr", 1e-3f}, {"beta1", 0.9f}, {"beta2", 0.999f}, {"eps", 1e-8f}, {"weight_decay", 0.01f}};
    Tensor mw = model[0], mb = model[1], vw = model[0], vb = model[1];
    mw.name = "weight.m", mb.name = "bias.m", vw.name = "weight.v", vb.name = "bias.v";
    mw.data = m, mb.data = m + 4, vw.data = v, vb.data = v + 4;
    opt.state = {mw, mb, vw, vb};
    opt.param_dims = {{2, 2}, {2}, {2, 2}, {2}};
    opt.step = 7;
    save(path, model, &opt, {{"epoch", 3}, {"batch", 11}});
    Loaded l = load(path, target(), &opt);
    if (!l.had_optimizer || l.step != 7 || l.extra.at("epoch") != 3 || l.extra.at("batch") != 11) return 1;
    if (l.model.size() != 2 || memcmp(l.model[0].data(), w, 16) || memcmp(l.model[1].data(), b, 8)) return 1;
    if (l.state.size() != 4 || memcmp(l.state[0].data(), m, 16) || memcmp(l.state[3].data(), v + 4, 8)) return 1;
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s round-trip-path [checkpoint ...]\n", argv[0]);
        return 2;
    }
    for (int i = 2; i < argc; i++) {
        try {
            load(argv[i], target(), nullptr);
            printf("OK\n");
        } catch (const Failure &f) {
            printf("%s\n", kind_name(f.kind));
        } catch (const std::exception &e) {
            printf("error %s\n", e.what());
        }
    }
    const int rt = round_trip(argv[1]);
    printf("round-trip %s\n", rt ? "FAILED" : "OK");
    return rt;
}
