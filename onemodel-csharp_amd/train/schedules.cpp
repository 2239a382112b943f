// Learning-rate schedules of the reference (Schedules.cs:151-422) and their C ABI (include/om_train.h).
// Each constructor keeps its float arguments widened to double, as the reference's fields do, and rejects the
// arguments the reference rejects with ArgumentOutOfRangeException (OM_E_ARG here).
#include "schedules.hpp"

#include <algorithm>
#include <cmath>

#include "om_train.h"

namespace omt {
namespace {

int64_t clamp_step(int64_t s) { return s < 0 ? 0 : s; }

class ConstantLr final : public LrSchedule {
   public:
    explicit ConstantLr(float lr) : lr_(lr) {}
    float lr_at(int64_t) const override { return lr_; }
    std::unique_ptr<LrSchedule> clone() const override { return std::make_unique<ConstantLr>(*this); }

   private:
    float lr_;
};

// base * gamma^floor(step / stepSize), the power by binary exponentiation in double.
class StepLr final : public LrSchedule {
   public:
    StepLr(float base, int64_t step_size, float gamma) : base_(base), step_size_(step_size), gamma_(gamma) {}
    float lr_at(int64_t step) const override {
        int64_t n = clamp_step(step) / step_size_;
        double r = base_, b = gamma_;
        for (; n > 0; n >>= 1) {
            if (n & 1) r *= b;
            b *= b;
        }
        return (float)r;
    }
    std::unique_ptr<LrSchedule> clone() const override { return std::make_unique<StepLr>(*this); }

   private:
    double base_;
    int64_t step_size_;
    double gamma_;
};

// min + (base - min) * (1 + cos(pi * step / total)) / 2, held at min from step `total` on.
class CosineLr final : public LrSchedule {
   public:
    CosineLr(float base, int64_t total, float min_lr) : base_(base), min_(min_lr), total_(total) {}
    float lr_at(int64_t step) const override {
        const int64_t s = clamp_step(step);
        const double t = s >= total_ ? 1.0 : (double)s / (double)total_;
        return (float)(min_ + (base_ - min_) * (1.0 + cos_pi(t)) / 2.0);
    }
    std::unique_ptr<LrSchedule> clone() const override { return std::make_unique<CosineLr>(*this); }

   private:
    double base_, min_;
    int64_t total_;
};

// Linear warm-up from start * r0 to r0 (r0 = the inner schedule's first rate), then the inner schedule counted from
// the end of the warm-up.
class WarmupLr final : public LrSchedule {
   public:
    WarmupLr(std::unique_ptr<LrSchedule> after, int64_t warmup, float start)
        : after_(std::move(after)), warmup_(warmup), start_(start) {}
    WarmupLr(const WarmupLr &o) : after_(o.after_->clone()), warmup_(o.warmup_), start_(o.start_) {}
    float lr_at(int64_t step) const override {
        const int64_t s = clamp_step(step);
        if (s >= warmup_) return after_->lr_at(s - warmup_);
        const double r0 = after_->lr_at(0);
        return (float)(r0 * (start_ + (1.0 - start_) * ((double)s / (double)warmup_)));
    }
    std::unique_ptr<LrSchedule> clone() const override { return std::make_unique<WarmupLr>(*this); }

   private:
    std::unique_ptr<LrSchedule> after_;
    int64_t warmup_;
    double start_;
};

// base * (s + 1) / warmup during the warm-up, then base * (floor + (1 - floor) * (1 + cos(pi * p)) / 2) with
// p = (s - warmup) / max(1, total - warmup), capped at 1.
class WarmupCosineLr final : public LrSchedule {
   public:
    WarmupCosineLr(float base, int64_t warmup, int64_t total, float floor_fraction)
        : base_(base), warmup_(warmup), total_(total), floor_(floor_fraction) {}
    float lr_at(int64_t step) const override {
        const int64_t s = clamp_step(step);
        if (s < warmup_) return (float)(base_ * (double)(s + 1) / (double)warmup_);
        const double p = std::min(1.0, (double)(s - warmup_) / (double)std::max<int64_t>(1, total_ - warmup_));
        return (float)(base_ * (floor_ + ((1.0 - floor_) * 0.5 * (1.0 + cos_pi(p)))));
    }
    std::unique_ptr<LrSchedule> clone() const override { return std::make_unique<WarmupCosineLr>(*this); }

   private:
    double base_;
    int64_t warmup_, total_;
    double floor_;
};

// One-cycle (Smith and Topin): half-cosine rise from max/div to max over the first pct of the steps, then a
// half-cosine fall to max/div/final_div.
class OneCycleLr final : public LrSchedule {
   public:
    OneCycleLr(float max_lr, int64_t total, float pct_start, float div_factor, float final_div_factor)
        : max_(max_lr),
          initial_((double)max_lr / (double)div_factor),
          min_(initial_ / (double)final_div_factor),
          up_end_((double)pct_start * (double)total - 1.0),
          down_end_((double)total - 1.0) {}
    float lr_at(int64_t step) const override {
        double s = (double)clamp_step(step);
        if (s > down_end_) s = down_end_;
        return s <= up_end_ ? (float)anneal(initial_, max_, s / up_end_)
                            : (float)anneal(max_, min_, (s - up_end_) / (down_end_ - up_end_));
    }
    std::unique_ptr<LrSchedule> clone() const override { return std::make_unique<OneCycleLr>(*this); }

   private:
    static double anneal(double start, double end, double pct) {
        return end + (start - end) / 2.0 * (cos_pi(pct) + 1.0);
    }
    double max_, initial_, min_, up_end_, down_end_;
};

om_status reject(const char *msg) {
    set_global_error(msg);
    return OM_E_ARG;
}

om_status give(std::unique_ptr<LrSchedule> s, omt_lr_schedule **out) {
    if (!out) return reject("omt_lr_*: out is NULL");
    *out = new omt_lr_schedule{std::move(s)};
    return OM_OK;
}

}  // namespace

// Symmetry about t = 1/2 reduces the argument to [0, pi/2]; the Maclaurin series of cos to degree 26 (truncation
// below 1e-21 there) is summed by Horner's rule from the highest term: r <- 1 - a^2 / ((2k-1)(2k)) * r, k = 13..1.
double LrSchedule::cos_pi(double t) {
    if (!(t > 0.0)) return 1.0;
    if (t >= 1.0) return -1.0;
    double sign = 1.0, y = t;
    if (y > 0.5) {
        sign = -1.0;
        y = 1.0 - y;
    }
    const double a = 3.14159265358979323846 * y;
    const double a2 = a * a;
    double r = 1.0;
    for (int k = 13; k >= 1; k--) r = 1.0 - a2 / ((2.0 * k - 1.0) * (2.0 * k)) * r;
    return sign * r;
}

}  // namespace omt

using namespace omt;

extern "C" {

om_status omt_lr_constant(float lr, omt_lr_schedule **out) { return give(std::make_unique<ConstantLr>(lr), out); }

om_status omt_lr_step(float base_lr, int64_t step_size, float gamma, omt_lr_schedule **out) {
    if (step_size < 1) return reject("StepLr: stepSize must be at least 1");
    return give(std::make_unique<StepLr>(base_lr, step_size, gamma), out);
}

om_status omt_lr_cosine(float base_lr, int64_t total_steps, float min_lr, omt_lr_schedule **out) {
    if (total_steps < 1) return reject("CosineLr: totalSteps must be at least 1");
    return give(std::make_unique<CosineLr>(base_lr, total_steps, min_lr), out);
}

om_status omt_lr_warmup(const omt_lr_schedule *after, int64_t warmup_steps, float start_factor,
                        omt_lr_schedule **out) {
    if (!after || !after->s) return reject("WarmupLr: the inner schedule is NULL");
    if (warmup_steps < 1) return reject("WarmupLr: warmupSteps must be at least 1");
    return give(std::make_unique<WarmupLr>(after->s->clone(), warmup_steps, start_factor), out);
}

om_status omt_lr_warmup_cosine(float base_lr, int64_t warmup_steps, int64_t total_steps, float floor_fraction,
                               omt_lr_schedule **out) {
    if (warmup_steps < 1) return reject("WarmupCosineLr: warmupSteps must be at least 1");
    if (total_steps <= warmup_steps) return reject("WarmupCosineLr: totalSteps must exceed warmupSteps");
    // ThrowIfNegative / ThrowIfGreaterThan(1): a NaN passes both, as in the reference.
    if (floor_fraction < 0.0f) return reject("WarmupCosineLr: floorFraction must not be negative");
    if (floor_fraction > 1.0f) return reject("WarmupCosineLr: floorFraction must not exceed 1");
    return give(std::make_unique<WarmupCosineLr>(base_lr, warmup_steps, total_steps, floor_fraction), out);
}

om_status omt_lr_onecycle(float max_lr, int64_t total_steps, float pct_start, float div_factor,
                          float final_div_factor, omt_lr_schedule **out) {
    if (total_steps < 2) return reject("OneCycleLr: totalSteps must be at least 2");
    if (!(pct_start > 0.0f && pct_start < 1.0f)) return reject("OneCycleLr: pctStart must be in (0, 1)");
    return give(std::make_unique<OneCycleLr>(max_lr, total_steps, pct_start, div_factor, final_div_factor), out);
}

void omt_lr_free(omt_lr_schedule *s) { delete s; }

float omt_lr_at(const omt_lr_schedule *s, int64_t step) {
    return (s && s->s) ? s->s->lr_at(step) : std::nanf("");
}

double omt_lr_cos(double t) { return LrSchedule::cos_pi(t); }

}  // extern "C"
