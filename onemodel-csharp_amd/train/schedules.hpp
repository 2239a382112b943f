// Learning-rate schedules (Schedules.cs:151-422): pure functions from the number of optimizer steps taken to a rate,
// in IEEE double with the reference's operation order (no fused multiply-add: built with -ffp-contract=off), so the
// rates equal the reference's bit for bit on every platform.
#pragma once

#include <cstdint>
#include <memory>
#include <string>

namespace omt {

class LrSchedule {
   public:
    virtual ~LrSchedule() = default;
    // The rate for the step with index `step` (0 for the first); a negative step counts as 0.
    virtual float lr_at(int64_t step) const = 0;
    virtual std::unique_ptr<LrSchedule> clone() const = 0;
    // cos(pi * t) for t in [0, 1] (clamped) from + - * / only: LrSchedule.Cos (Schedules.cs:171-203).
    static double cos_pi(double t);
};

// Sets the message omt_last_error(NULL) returns (errors raised before a model exists).
void set_global_error(const std::string &msg);

}  // namespace omt

struct omt_lr_schedule {
    std::unique_ptr<omt::LrSchedule> s;
};
