"""The parity measures themselves (tests/parity.py), pinned on the CPU: each
plausible kernel mistake at the measured workloads' output scale must fail
the row-relative check, and rounding-level noise must pass it."""
import numpy as np
import pytest

from parity import TOL_BF16, check, mixed_err, row_rel_err, row_rel_errs


def c2_scale_output(seed=0):
    """An output of the 64 x 2048 Llama-3-8B step's scale: every element the
    mean of 2048 values of V ~ N(0, 1/128), i.e. N(0, (0.088/45)^2)."""
    rng = np.random.default_rng(seed)
    return rng.normal(0.0, (128 ** -0.5) / np.sqrt(2048), size=(64, 32, 128))


def test_mixed_form_alone_misses_a_20pct_error_at_this_scale():
    r = c2_scale_output()
    assert np.abs(r).max() < 1e-2
    assert mixed_err(1.2 * r, r) <= TOL_BF16      # the reference's form passes it
    assert abs(row_rel_err(1.2 * r, r) - 0.2) < 1e-12


@pytest.mark.parametrize("mistake", ["scaled_1.5", "zeroed_row", "rolled_dims",
                                     "swapped_heads", "nan", "sign"])
def test_row_relative_check_fails_on_planted_mistakes(mistake):
    r = c2_scale_output(1)
    a = r.copy()
    if mistake == "scaled_1.5":
        a = 1.5 * r
    elif mistake == "zeroed_row":
        a[5, 7, :] = 0.0
    elif mistake == "rolled_dims":
        a[3, 2] = np.roll(r[3, 2], 1)
    elif mistake == "swapped_heads":
        a[0, [0, 1]] = r[0, [1, 0]]
    elif mistake == "nan":
        a[9, 9, 9] = np.nan
    elif mistake == "sign":
        a[10, 4] = -r[10, 4]
    with pytest.raises(AssertionError):
        check(a, r, TOL_BF16, mistake)


def test_rounding_level_noise_passes():
    r = c2_scale_output(2)
    rng = np.random.default_rng(3)
    # bf16 rounding of every probability: ~2^-9 relative per term, averaged
    a = r * (1 + rng.normal(0, 2e-4, size=r.shape))
    m, n = check(a, r, TOL_BF16, "noise")
    assert n < 1e-3


def test_rows_and_nonfinite_reference():
    r = np.array([[1.0, 0.0], [np.nan, np.nan], [0.0, 0.0]])
    a = np.array([[1.0, 1e-3], [5.0, 5.0], [0.0, 0.0]])
    e = row_rel_errs(a, r)
    assert e.shape == (2,)                       # the NaN reference row is dropped
    assert abs(e[0] - 1e-3) < 1e-15
    assert e[1] == 0.0                           # zero row compared absolutely
    assert row_rel_err(np.array([[0.0, 2e-3]]), np.zeros((1, 2))) == pytest.approx(2e-3)
