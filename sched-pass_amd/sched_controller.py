"""sched_controller.py -- the closed-loop controller that turns timer rows into
pi (reference python/sched_controller.py:30-177), GPU-free.

Three stages per step, as in the reference:
  1. estimate: an online least-squares fit cost = alpha * kv_len + beta over
     observed per-request cost (the timer rows), an EWMA residual per request,
     and an EWMA congestion index gamma = measured / predicted makespan;
  2. order: LPT (longest predicted first), SRPT (shortest first) or EDF
     (least slack deadline - elapsed - predicted first);
  3. damp: keep the previously published order unless the new one improves
     the order-quality scalar (total completion time, the sum of prefix sums
     of the ordered costs) by more than a dead-band fraction.

Stage 3 follows the reference literally: the gain is old minus new total
completion time. SRPT minimises that scalar, so a better SRPT order is
republished; LPT maximises it, so once an LPT order is published a new LPT
ranking never shows a positive gain and the published order is kept (the
reference behaves the same way; its serving path recomputes orders without
this class). The class drives any object with the plane's write interface
(set_order / set_num_tasks / push), such as sched_rt.SchedPlane.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class CostFit:
    """Running sums for the least-squares line cost = alpha * x + beta
    (python/sched_controller.py:30-54)."""
    n: int = 0
    sx: float = 0.0
    sy: float = 0.0
    sxx: float = 0.0
    sxy: float = 0.0

    def add(self, x: float, y: float) -> None:
        self.n += 1
        self.sx += x
        self.sy += y
        self.sxx += x * x
        self.sxy += x * y

    def coeffs(self) -> tuple[float, float]:
        """(alpha, beta). With fewer than two points, or all x equal, the fit
        is the proportional one through the origin (or 1, 0 with no data)."""
        proportional = (self.sy / self.sx, 0.0) if self.sx > 0 else (1.0, 0.0)
        if self.n < 2:
            return proportional
        det = self.n * self.sxx - self.sx * self.sx
        if det <= 0:
            return proportional
        alpha = (self.n * self.sxy - self.sx * self.sy) / det
        beta = (self.sy - alpha * self.sx) / self.n
        return alpha, beta


# Kept for callers that use the reference's private name.
_Fit = CostFit


@dataclass
class SchedControlPlane:
    """Per-step estimator + policy (python/sched_controller.py:57-177)."""

    policy: str = "lpt"          # lpt | srpt | edf
    ewma: float = 0.25           # residual / congestion smoothing
    deadband: float = 0.02       # minimum relative gain to republish an order
    _fit: CostFit = field(default_factory=CostFit)
    _resid: dict = field(default_factory=dict)
    _gamma: float = 1.0
    _last_order: list = field(default_factory=list)

    # -- estimation --------------------------------------------------------
    def observe(self, rids, kv_lens, cycles) -> None:
        """Fold one step's per-request costs in; non-positive costs mean the
        request was not measured this step and are skipped."""
        for rid, length, cost in zip(rids, kv_lens, cycles):
            if cost <= 0:
                continue
            self._fit.add(float(length), float(cost))
            err = float(cost) - self.predict_one(length)
            prev = self._resid.get(rid, 0.0)
            self._resid[rid] = (1 - self.ewma) * prev + self.ewma * err

    def observe_step(self, predicted_makespan: float, measured_makespan: float) -> None:
        """Congestion index: EWMA of measured / predicted step time."""
        if predicted_makespan > 0 and measured_makespan > 0:
            ratio = measured_makespan / predicted_makespan
            self._gamma = (1 - self.ewma) * self._gamma + self.ewma * ratio

    def predict_one(self, kv_len: float, rid=None) -> float:
        alpha, beta = self._fit.coeffs()
        t = alpha * float(kv_len) + beta
        if rid is not None:
            t += self._resid.get(rid, 0.0)
        return max(t, 0.0)

    @property
    def gamma(self) -> float:
        return self._gamma

    def uncertainty(self, rids, kv_lens) -> float:
        """Mean |residual| over mean prediction; a request never observed
        counts its whole prediction as doubt. 1.0 when nothing is predicted."""
        preds, doubt = [], []
        for rid, length in zip(rids, kv_lens):
            p = self.predict_one(length)
            preds.append(p)
            doubt.append(abs(self._resid[rid]) if rid in self._resid else p)
        if not preds:
            return 1.0
        mean_pred = sum(preds) / len(preds)
        return (sum(doubt) / len(doubt)) / mean_pred if mean_pred > 0 else 1.0

    # -- ordering with hysteresis -------------------------------------------
    def order(self, rids, kv_lens, deadlines=None, elapsed=None) -> list[int]:
        """Batch indices in service order under the policy, damped."""
        t_hat = [self.predict_one(length, rid) for rid, length in zip(rids, kv_lens)]
        idx = list(range(len(t_hat)))
        if self.policy == "lpt":
            new = sorted(idx, key=lambda i: -t_hat[i])
        elif self.policy == "srpt":
            new = sorted(idx, key=lambda i: t_hat[i])
        elif self.policy == "edf":
            if deadlines is None:
                raise ValueError("edf needs deadlines")
            el = elapsed if elapsed is not None else [0.0] * len(idx)
            new = sorted(idx, key=lambda i: deadlines[i] - el[i] - t_hat[i])
        else:
            raise ValueError(f"unknown policy {self.policy!r}")
        if len(self._last_order) == len(new):
            gain = self._span(t_hat, self._last_order) - self._span(t_hat, new)
            if gain < self.deadband * max(self._span(t_hat, new), 1e-9):
                return self._last_order
        self._last_order = new
        return new

    @staticmethod
    def _span(t_hat, order) -> float:
        """Total completion time of `order`: the sum of its prefix sums."""
        done = total = 0.0
        for i in order:
            done += t_hat[i]
            total += done
        return total

    # -- one serving step ---------------------------------------------------
    def step(self, plane, rids, kv_lens, cycles=None, deadlines=None, elapsed=None) -> list[int]:
        """Fold the measurements, order, write the plane, return the order."""
        if cycles is not None:
            self.observe(rids, kv_lens, cycles)
        order = self.order(rids, kv_lens, deadlines, elapsed)
        plane.set_order(order)
        plane.set_num_tasks(len(order))
        plane.push()
        return order


def task_costs_per_request(timer_rows, num_requests: int, num_kv_heads: int) -> list[float]:
    """Fold per-task timer rows (task = request * Hkv + head) into per-request
    cost, the reference's tile -> request scatter_add
    (python/sched_sglang_plugin.py:362-375)."""
    rows = [float(x) for x in timer_rows[:num_requests * num_kv_heads]]
    return [sum(rows[r * num_kv_heads:(r + 1) * num_kv_heads]) for r in range(num_requests)]


def task_order_from_requests(request_order, num_kv_heads: int) -> list[int]:
    """Expand a request order to the kernels' task order (all kv-heads of a
    request consecutively)."""
    return [r * num_kv_heads + h for r in request_order for h in range(num_kv_heads)]


class RequestPlane:
    """Presents a task-indexed plane (task = request * Hkv + head) to the
    controller, which orders requests: orders and task counts are expanded
    to all kv-heads of each request before they reach the plane."""

    def __init__(self, plane, num_kv_heads: int):
        self.plane = plane
        self.num_kv_heads = int(num_kv_heads)

    def set_order(self, request_order) -> None:
        self.plane.set_order(task_order_from_requests(request_order, self.num_kv_heads))

    def set_num_tasks(self, n: int) -> None:
        self.plane.set_num_tasks(int(n) * self.num_kv_heads)

    def push(self) -> None:
        self.plane.push()
