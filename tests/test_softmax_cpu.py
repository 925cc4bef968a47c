"""SoftmaxCPU (CPU execution provider op of the same domain).

Reference: csrc/softmax_cpu/softmax_cpu_ort.cpp:20-114.  The product entry
point (xm_softmax_cpu, C++) is compared bit for bit with the oracle's fp32 C
restatement (same operations, same order), and the oracle is pinned by
closed forms: uniform lines give exactly fl(1/n), integer shifts leave the
result unchanged, huge inputs do not overflow, and the reference's
"inv_sum = 0 unless sum > 0" branch shows up when a NaN poisons the sum.
"""

import numpy as np
import pytest

import xmetai_onnx_plugins as xp
from oracle import cref, numpy_ref

F32 = np.float32


def _rand(shape, seed, scale=4.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(F32)


@pytest.mark.parametrize("shape,axis", [((7,), -1), ((3, 5), 0), ((3, 5), 1), ((2, 3, 33), -1),
                                        ((2, 3, 33), 1), ((4, 1, 6), 1), ((2, 2, 3, 5), -3),
                                        ((1, 1000), -1), ((9, 17, 3), 0)])
def test_product_bitwise_equals_oracle(shape, axis):
    x = _rand(shape, seed=len(shape) * 7 + axis)
    y = xp.softmax_cpu(x, axis)
    ref = cref.softmax_cpu(x, axis, dtype=np.float32)
    assert y.dtype == F32 and y.shape == x.shape
    assert np.array_equal(y, ref)


@pytest.mark.parametrize("axis", [-1, 0, 1])
def test_oracle_matches_textbook_fp64(axis):
    x = _rand((4, 6, 5), seed=3)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis, keepdims=True))
    want = e / e.sum(axis, keepdims=True)
    for impl in (cref.softmax_cpu(x, axis, dtype=np.float32), cref.softmax_cpu(x, axis, dtype=np.float64),
                 numpy_ref.softmax_cpu(x, axis)):
        np.testing.assert_allclose(impl, want, rtol=2e-6, atol=1e-9)


@pytest.mark.parametrize("n", [1, 2, 3, 7, 10, 1000])
def test_uniform_line_is_exact_reciprocal(n):
    x = np.full((2, n), 3.25, F32)
    y = xp.softmax_cpu(x)
    assert np.array_equal(y, np.full_like(x, F32(1) / F32(n)))
    assert np.array_equal(cref.softmax_cpu(x), y)


def test_integer_shift_invariance_is_exact():
    x = np.random.default_rng(5).integers(-20, 20, size=(6, 11)).astype(F32)
    assert np.array_equal(xp.softmax_cpu(x), xp.softmax_cpu(x + F32(7)))


def test_large_inputs_do_not_overflow():
    y = xp.softmax_cpu(np.array([[1000.0, 1000.0], [3.0e38, -3.0e38]], F32))
    assert np.array_equal(y, np.array([[0.5, 0.5], [1.0, 0.0]], F32))


def test_underflow_gives_one_hot():
    y = xp.softmax_cpu(np.array([0.0, -200.0, -300.0], F32))
    assert np.array_equal(y, np.array([1.0, 0.0, 0.0], F32))


def test_nan_poisons_sum_and_zeroes_line():
    # max ignores the NaN (std::max keeps the running maximum), exp(NaN) is
    # NaN, the sum is NaN, so inv_sum = 0 (reference :75): finite entries
    # become 0 and the NaN stays NaN.
    x = np.array([[1.0, np.nan, 0.0], [0.0, 1.0, 2.0]], F32)
    y = xp.softmax_cpu(x)
    assert y[0, 0] == 0.0 and np.isnan(y[0, 1]) and y[0, 2] == 0.0
    assert np.array_equal(y[1], cref.softmax_cpu(x[1:])[0])
    assert np.array_equal(y, cref.softmax_cpu(x), equal_nan=True)


def test_infinities():
    x = np.array([[np.inf, 0.0], [-np.inf, -np.inf], [-np.inf, 0.0]], F32)
    y = xp.softmax_cpu(x)
    # +inf: inf - inf = NaN -> sum NaN -> inv 0; all -inf: -inf - -inf = NaN everywhere
    assert np.isnan(y[0, 0]) and y[0, 1] == 0.0
    assert np.isnan(y[1]).all()
    assert np.array_equal(y[2], np.array([0.0, 1.0], F32))
    assert np.array_equal(y, cref.softmax_cpu(x), equal_nan=True)


def test_empty_input_skips_axis_check():
    x = np.zeros((0, 4), F32)
    assert xp.softmax_cpu(x, axis=9).shape == (0, 4)


@pytest.mark.parametrize("shape,axis", [((3, 4), 2), ((3, 4), -3), ((), -1)])
def test_axis_out_of_range(shape, axis):
    x = np.ones(shape, F32)
    with pytest.raises(xp.XmError, match="SoftmaxCPU axis out of range") as e:
        xp.softmax_cpu(x, axis)
    assert e.value.status == xp.XM_ERR_INVALID_ARGUMENT


def test_oracle_plants_detected():
    # a wrong axis or a missing max-subtraction must fail the textbook check
    x = _rand((3, 4), seed=11, scale=30.0)
    good = cref.softmax_cpu(x, 1)
    assert not np.allclose(cref.softmax_cpu(x, 0), good)
    naive = np.exp(x) / np.exp(x).sum(1, keepdims=True)
    assert not np.array_equal(naive.astype(F32), good) or np.isfinite(naive).all()
