"""Parity measures shared by the GPU tests.

Two measures, both asserted:

- mixed form, |a - r| <= tol * (1 + |r|) per element: the reference's own
  check (test/paged_decode.cu:268-274, :448-454);
- norm-relative per output row, ||a - r||_2 / ||r||_2 <= tol over the head
  dim of each (request, head) row: the relative tolerance the bf16 / fp32
  targets are stated in. At the measured workloads' output scale (V ~
  N(0, 1/128) averaged over thousands of tokens, |r| ~ 2e-3) the mixed form
  alone would admit an output off by 100%; the row measure does not.

Rows whose reference is not finite (the 0/0 of an empty context) are left
out; a reference row of norm 0 is compared in absolute terms.
"""
import numpy as np

TOL_F32 = 1e-5   # fp32 KV
TOL_BF16 = 2e-3  # bf16 / fp16 / fp8 KV


def _pair(a, r):
    a = np.asarray(a.detach().cpu() if hasattr(a, "detach") else a, np.float64)
    r = np.asarray(r.detach().cpu() if hasattr(r, "detach") else r, np.float64)
    if a.shape != r.shape:
        raise ValueError(f"shape mismatch {a.shape} vs {r.shape}")
    return a, r


def mixed_err(a, r) -> float:
    """max |a - r| / (1 + |r|) over the finite reference elements."""
    a, r = _pair(a, r)
    fin = np.isfinite(r)
    if not fin.any():
        return 0.0
    return float(np.max(np.abs(a[fin] - r[fin]) / (1 + np.abs(r[fin]))))


def row_rel_errs(a, r) -> np.ndarray:
    """||a - r|| / ||r|| of every row over the last axis (rows with a
    non-finite reference dropped; a zero reference row gives ||a - r||)."""
    a, r = _pair(a, r)
    d = r.shape[-1] if r.ndim else 1
    a = a.reshape(-1, d)
    r = r.reshape(-1, d)
    keep = np.isfinite(r).all(axis=1)
    a, r = a[keep], r[keep]
    diff = a - r
    num = np.sqrt(np.einsum("ij,ij->i", diff, diff)) if diff.size else np.zeros(0)
    den = np.sqrt(np.einsum("ij,ij->i", r, r)) if r.size else np.zeros(0)
    out = np.where(den > 0, num / np.where(den > 0, den, 1.0), num)
    # a NaN in the kernel output on a finite reference row is an error
    return np.where(np.isfinite(out), out, np.inf)


def row_rel_err(a, r) -> float:
    e = row_rel_errs(a, r)
    return float(e.max()) if e.size else 0.0


def par_err(a, r, what="") -> float:
    """max(mixed, row-relative): `par_err(a, r) <= tol` asserts both
    measures. Prints both (the worst values of the call)."""
    m = mixed_err(a, r)
    n = row_rel_err(a, r)
    print(f"  parity{' ' + what if what else ''}: mixed {m:.3g}, row-relative {n:.3g}",
          flush=True)
    return max(m, n)


def check(a, r, tol, what="") -> tuple:
    """Assert both measures within tol; print the worst values. Returns
    (mixed, row-relative)."""
    m = mixed_err(a, r)
    n = row_rel_err(a, r)
    print(f"{what}: mixed {m:.3g}, row-relative {n:.3g} (tol {tol:g})")
    assert m <= tol, f"{what}: mixed error {m} > {tol}"
    assert n <= tol, f"{what}: row-relative error {n} > {tol}"
    return m, n
