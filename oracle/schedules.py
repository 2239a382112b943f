"""TEST INFRASTRUCTURE ONLY: the reference's learning-rate schedules restated in Python (Schedules.cs:151-422).

Python floats are IEEE doubles and every operation below is one IEEE operation in the reference's order, so these are
the reference's rates bit for bit. The reference's constructor arguments are C# floats widened to double; `f32()`
does that widening here. Only tests/ import this module; the product's schedules are C++ (libom_train.so).
"""
from __future__ import annotations

import numpy as np


def f32(x):
    """A C# float argument, widened to double."""
    return float(np.float32(x))


def cos_pi(t):
    """LrSchedule.Cos (Schedules.cs:171-203): cos(pi*t) on [0, 1] (clamped) by symmetry about 1/2 and the Maclaurin
    series to degree 26, Horner form."""
    if not t > 0.0:
        return 1.0
    if t >= 1.0:
        return -1.0
    sign, y = 1.0, t
    if y > 0.5:
        sign, y = -1.0, 1.0 - y
    a = 3.14159265358979323846 * y
    a2 = a * a
    r = 1.0
    for k in range(13, 0, -1):
        r = 1.0 - a2 / ((2.0 * k - 1.0) * (2.0 * k)) * r
    return sign * r


def _clamp(step):
    return 0 if step < 0 else step


class Constant:
    """ConstantLr (Schedules.cs:208-219)."""

    def __init__(self, lr):
        self.lr = np.float32(lr)

    def lr_at(self, step):
        return self.lr


class Step:
    """StepLr (Schedules.cs:222-258): base * gamma^floor(step/stepSize) by binary exponentiation in double."""

    def __init__(self, base, step_size, gamma=0.1):
        if step_size < 1:
            raise ValueError("stepSize")
        self.base, self.step_size, self.gamma = f32(base), int(step_size), f32(gamma)

    def lr_at(self, step):
        n = _clamp(step) // self.step_size
        r, b = self.base, self.gamma
        while n > 0:
            if n & 1:
                r *= b
            b *= b
            n >>= 1
        return np.float32(r)


class Cosine:
    """CosineLr (Schedules.cs:264-290)."""

    def __init__(self, base, total, min_lr=0.0):
        if total < 1:
            raise ValueError("totalSteps")
        self.base, self.min, self.total = f32(base), f32(min_lr), int(total)

    def lr_at(self, step):
        s = _clamp(step)
        t = 1.0 if s >= self.total else s / self.total
        return np.float32(self.min + (self.base - self.min) * (1.0 + cos_pi(t)) / 2.0)


class Warmup:
    """WarmupLr (Schedules.cs:297-330): linear rise from startFactor*r0 to r0, then the inner schedule from its step 0."""

    def __init__(self, after, warmup, start_factor=0.0):
        if after is None:
            raise ValueError("after")
        if warmup < 1:
            raise ValueError("warmupSteps")
        self.after, self.warmup, self.start = after, int(warmup), f32(start_factor)

    def lr_at(self, step):
        s = _clamp(step)
        if s >= self.warmup:
            return self.after.lr_at(s - self.warmup)
        r0 = float(self.after.lr_at(0))
        return np.float32(r0 * (self.start + (1.0 - self.start) * (s / self.warmup)))


class WarmupCosine:
    """WarmupCosineLr (Schedules.cs:338-375)."""

    def __init__(self, base, warmup, total, floor=0.0):
        if warmup < 1:
            raise ValueError("warmupSteps")
        if total <= warmup:
            raise ValueError("totalSteps")
        if floor < 0 or floor > 1:
            raise ValueError("floorFraction")
        self.base, self.warmup, self.total, self.floor = f32(base), int(warmup), int(total), f32(floor)

    def lr_at(self, step):
        s = _clamp(step)
        if s < self.warmup:
            return np.float32(self.base * float(s + 1) / self.warmup)
        p = min(1.0, float(s - self.warmup) / max(1, self.total - self.warmup))
        return np.float32(self.base * (self.floor + ((1.0 - self.floor) * 0.5 * (1.0 + cos_pi(p)))))


class OneCycle:
    """OneCycleLr (Schedules.cs:381-422)."""

    def __init__(self, max_lr, total, pct_start=0.3, div_factor=25.0, final_div_factor=1e4):
        if total < 2:
            raise ValueError("totalSteps")
        if not (np.float32(pct_start) > 0 and np.float32(pct_start) < 1):
            raise ValueError("pctStart")
        self.max = f32(max_lr)
        self.initial = f32(max_lr) / f32(div_factor)
        self.min = self.initial / f32(final_div_factor)
        self.up_end = f32(pct_start) * float(total) - 1.0
        self.down_end = float(total) - 1.0

    @staticmethod
    def _anneal(start, end, pct):
        return end + (start - end) / 2.0 * (cos_pi(pct) + 1.0)

    def lr_at(self, step):
        s = float(_clamp(step))
        if s > self.down_end:
            s = self.down_end
        if s <= self.up_end:
            return np.float32(self._anneal(self.initial, self.max, s / self.up_end))
        return np.float32(self._anneal(self.max, self.min, (s - self.up_end) / (self.down_end - self.up_end)))
