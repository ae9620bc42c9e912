"""sched_controller.py -- closed-loop control of the task order from the
residency timer, GPU-free.

Public surface of reference python/sched_controller.py:30-177:
SchedControlPlane(policy, ewma, deadband) with observe / observe_step /
predict_one / gamma / uncertainty / order / step, the policies lpt | srpt | edf
and the dead-band that keeps a published order unless a new one predicts a
real gain. It drives any object with the plane's write interface (set_order /
set_num_tasks / push), such as sched_rt.SchedPlane.

The internals are this module's own:

- CostModel: the linear cost model t = alpha * kv_len + beta, held as the
  normal equations of least squares (a 2x2 Gram matrix of [kv_len, 1] and
  its moment vector against the measured cost) and updated one whole step at
  a time with numpy. An optional forgetting factor (`forget` < 1) weights
  recent steps more, for costs per token that drift when co-runners take
  bandwidth; forget = 1 (the default) is the plain least-squares fit.
- RequestTable: per-request state (EWMA residual, whether it was ever
  measured) in numpy arrays behind a rid -> slot map, so a step's lookups and
  updates are array operations.
- A step's residuals are taken against the fit that already includes the
  whole step, so the estimate does not depend on the order in which the
  step's requests are listed.
- OrderGate: the hysteresis. An order's quality is its predicted total
  completion time, the dot product of the costs in service order with
  (n, n-1, ..., 1); the gate republishes only when the new order lowers it
  by more than `deadband` of the new total. (SRPT minimises this scalar, so a
  better SRPT order always passes; LPT maximises it, so a published LPT
  order is kept until the batch changes size. The serving hooks recompute
  orders without the gate.)
"""
from __future__ import annotations

import numpy as np


class CostModel:
    """Least-squares line cost = alpha * x + beta over (x, cost) samples.

    Degenerate data falls back to the proportional fit cost = alpha * x
    (alpha = sum(cost) / sum(x)): fewer than two samples, or every x equal.
    With no data at all the model is cost = x."""

    def __init__(self, forget: float = 1.0):
        if not 0.0 < forget <= 1.0:
            raise ValueError("forget must be in (0, 1]")
        self.forget = float(forget)
        self.gram = np.zeros((2, 2))   # sum of [x, 1]^T [x, 1]
        self.moment = np.zeros(2)      # sum of [x, 1]^T cost
        self.samples = 0               # samples seen (not discounted)
        self._coef = None              # (alpha, beta) of the current sums

    def add(self, x, cost) -> None:
        """Fold one step's samples in (arrays of equal length)."""
        x = np.asarray(x, np.float64).ravel()
        y = np.asarray(cost, np.float64).ravel()
        if x.size == 0:
            return
        a = np.stack([x, np.ones_like(x)], axis=1)
        self.gram = self.forget * self.gram + a.T @ a
        self.moment = self.forget * self.moment + a.T @ y
        self.samples += x.size
        self._coef = None

    def coefficients(self) -> tuple[float, float]:
        """(alpha, beta), solved once per change of the sums (a serving
        loop predicts every re-plan and folds samples one step in 8)."""
        if self._coef is None:
            self._coef = self._solve()
        return self._coef

    def _solve(self) -> tuple[float, float]:
        sum_x, sum_y = self.gram[0, 1], self.moment[1]
        proportional = (float(sum_y / sum_x), 0.0) if sum_x > 0 else (1.0, 0.0)
        if self.samples < 2:
            return proportional
        det = float(np.linalg.det(self.gram))
        if det <= 1e-12 * self.gram[0, 0] * self.gram[1, 1]:
            return proportional
        alpha, beta = np.linalg.solve(self.gram, self.moment)
        return float(alpha), float(beta)

    def predict(self, x) -> np.ndarray:
        alpha, beta = self.coefficients()
        return alpha * np.asarray(x, np.float64) + beta


class RequestTable:
    """EWMA residual and 'ever measured' flag per request id."""

    def __init__(self):
        self.slot_of: dict = {}
        self.resid = np.zeros(64)
        self.seen = np.zeros(64, bool)
        self._last = (None, None)   # (rids as a tuple, their slots): a batch repeats

    def slots(self, rids, create: bool = False) -> np.ndarray:
        """Slot of each rid (-1 for one never measured, unless create)."""
        # One cached list: slots are only created here, so the cached lookup
        # is current unless it holds -1 entries and this call creates slots.
        key = tuple(rids)
        if key == self._last[0] and (not create or (self._last[1] >= 0).all()):
            return self._last[1]
        out = self._lookup(key, create)
        self._last = (key, out)
        return out

    def _lookup(self, rids, create: bool) -> np.ndarray:
        out = np.empty(len(rids), np.int64)
        for i, rid in enumerate(rids):
            s = self.slot_of.get(rid, -1)
            if s < 0 and create:
                s = len(self.slot_of)
                self.slot_of[rid] = s
                if s >= self.resid.size:
                    grow = self.resid.size
                    self.resid = np.concatenate([self.resid, np.zeros(grow)])
                    self.seen = np.concatenate([self.seen, np.zeros(grow, bool)])
            out[i] = s
        return out

    def residuals(self, rids) -> np.ndarray:
        s = self.slots(rids)
        return np.where(s >= 0, self.resid[np.maximum(s, 0)], 0.0)

    def measured(self, rids) -> np.ndarray:
        s = self.slots(rids)
        return (s >= 0) & self.seen[np.maximum(s, 0)]

    def blend(self, rids, err: np.ndarray, weight: float) -> None:
        """resid <- (1 - weight) * resid + weight * err for each rid (a rid
        listed twice is blended twice, in list order)."""
        s = self.slots(rids, create=True)
        if np.unique(s).size == s.size:
            self.resid[s] = (1.0 - weight) * self.resid[s] + weight * err
        else:
            for k, e in zip(s, err):
                self.resid[k] = (1.0 - weight) * self.resid[k] + weight * e
        self.seen[s] = True


class OrderGate:
    """Hysteresis on the published order."""

    def __init__(self, deadband: float):
        self.deadband = float(deadband)
        self.published: np.ndarray | None = None

    @staticmethod
    def total_completion(cost: np.ndarray, order: np.ndarray) -> float:
        n = order.size
        return float(np.dot(cost[order], np.arange(n, 0, -1, dtype=np.float64)))

    def decide(self, cost: np.ndarray, candidate: np.ndarray) -> np.ndarray:
        held = self.published
        if held is not None and held.size == candidate.size:
            new_total = self.total_completion(cost, candidate)
            gain = self.total_completion(cost, held) - new_total
            if gain < self.deadband * max(new_total, 1e-9):
                return held
        self.published = candidate
        return candidate


class SchedControlPlane:
    """Per-step estimator + policy for a batch of (rid, kv_len) requests."""

    POLICIES = ("lpt", "srpt", "edf")

    def __init__(self, policy: str = "lpt", ewma: float = 0.25, deadband: float = 0.02,
                 forget: float = 1.0):
        self.policy = policy
        self.ewma = float(ewma)
        self.model = CostModel(forget)
        self.requests = RequestTable()
        self.gate = OrderGate(deadband)
        self._gamma = 1.0
        # advanced by every change of the predictions (observe): a caller
        # holding a decision made from predict / uncertainty compares it
        self.version = 0

    @property
    def deadband(self) -> float:
        return self.gate.deadband

    @deadband.setter
    def deadband(self, v: float) -> None:
        self.gate.deadband = float(v)

    # -- estimation ------------------------------------------------------------
    def observe(self, rids, kv_lens, cycles) -> None:
        """Fold one step's measured per-request cost in. A cost <= 0 means the
        request was not measured this step; it is left out."""
        rids = list(rids)
        x = np.asarray(kv_lens, np.float64).ravel()
        y = np.asarray(cycles, np.float64).ravel()
        if not (len(rids) == x.size == y.size):
            raise ValueError("rids, kv_lens and cycles must have the same length")
        keep = y > 0
        if not keep.any():
            return
        x, y = x[keep], y[keep]
        kept = [r for r, k in zip(rids, keep) if k]
        self.version += 1
        self.model.add(x, y)
        self.requests.blend(kept, y - np.maximum(self.model.predict(x), 0.0), self.ewma)

    def observe_step(self, predicted_makespan: float, measured_makespan: float) -> None:
        """Congestion index gamma: EWMA of measured / predicted step time."""
        if predicted_makespan > 0 and measured_makespan > 0:
            ratio = measured_makespan / predicted_makespan
            self._gamma += self.ewma * (ratio - self._gamma)

    @property
    def gamma(self) -> float:
        return self._gamma

    def coefficients(self) -> tuple[float, float]:
        """(alpha, beta) of the current cost fit."""
        return self.model.coefficients()

    def residuals(self, rids) -> np.ndarray:
        """EWMA residual per request (0 for one never measured)."""
        return self.requests.residuals(list(rids))

    def predict(self, rids, kv_lens) -> np.ndarray:
        """Predicted cost per request: fit + its residual, clipped at 0."""
        t = self.model.predict(np.asarray(kv_lens, np.float64).ravel())
        return np.maximum(t + self.requests.residuals(list(rids)), 0.0)

    def predict_one(self, kv_len: float, rid=None) -> float:
        t = float(self.model.predict(float(kv_len)))
        if rid is not None:
            t += float(self.requests.residuals([rid])[0])
        return max(t, 0.0)

    def uncertainty(self, rids, kv_lens) -> float:
        """Mean doubt over mean fitted prediction: a measured request's doubt
        is |its residual|, an unmeasured one's its whole prediction. 1.0 when
        there is nothing to predict."""
        rids = list(rids)
        if not rids:
            return 1.0
        pred = np.maximum(self.model.predict(np.asarray(kv_lens, np.float64).ravel()), 0.0)
        doubt = np.where(self.requests.measured(rids),
                         np.abs(self.requests.residuals(rids)), pred)
        mean_pred = float(pred.mean())
        return float(doubt.mean()) / mean_pred if mean_pred > 0 else 1.0

    # -- ordering ----------------------------------------------------------------
    def order(self, rids, kv_lens, deadlines=None, elapsed=None) -> list[int]:
        """Batch indices in service order under the policy (ties keep batch
        order), passed through the hysteresis gate."""
        cost = self.predict(rids, kv_lens)
        if self.policy == "lpt":
            key = -cost
        elif self.policy == "srpt":
            key = cost
        elif self.policy == "edf":
            if deadlines is None:
                raise ValueError("edf needs deadlines")
            el = np.zeros(cost.size) if elapsed is None else np.asarray(elapsed, np.float64)
            key = np.asarray(deadlines, np.float64) - el - cost   # slack
        else:
            raise ValueError(f"unknown policy {self.policy!r}")
        candidate = np.argsort(key, kind="stable")
        return [int(i) for i in self.gate.decide(cost, candidate)]

    def clear_published(self) -> None:
        """Forget the published order (the next order() publishes freely)."""
        self.gate.published = None

    # -- one serving step ----------------------------------------------------------
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
    """Per-task timer rows (task = request * Hkv + head) summed per request,
    the reference's tile -> request fold (python/sched_sglang_plugin.py:
    362-375)."""
    n = num_requests * num_kv_heads
    rows = np.zeros(n)
    got = np.asarray(timer_rows[:n], np.float64)
    rows[:got.size] = got
    return rows.reshape(num_requests, num_kv_heads).sum(axis=1).tolist()


def task_order_from_requests(request_order, num_kv_heads: int) -> list[int]:
    """A request order expanded to the kernels' task order (all kv-heads of a
    request consecutively)."""
    r = np.asarray(request_order, np.int64)
    return (r[:, None] * num_kv_heads + np.arange(num_kv_heads)[None, :]).ravel().tolist()


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
