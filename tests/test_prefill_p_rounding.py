"""CPU check of the error bound the prefill tests allow for rounding P to
fp16: for weights p_i = 2^(s_i - m) with m the maximum of the first 32
scores (so the key that sets m has p = 1 and the row sum l >= 1) and every
p_i below 2^15, the output o = sum_i fp16(p_i) v_i / l (l the sum of the
unrounded p_i, as the kernel keeps it in fp32) differs from the exact
sum_i p_i v_i / l by at most (2^-11 + K 2^-25) max|v| for K keys.  numpy's
float16 conversion rounds to nearest even with subnormals, as gfx950's
v_cvt_pk_f16_f32 does (checked on the GPU with an in-bounds probe).  The
cases include the adversarial ones: every rounding error of one sign with V
of the same sign, weights just below fp16's normal range, and weights near
the 2^15 headroom."""

import numpy as np
import pytest


def _bound_holds(scores, v):
    K = scores.shape[0]
    m = scores[:32].max()
    p = np.exp2(scores - m)
    assert p.max() < 2.0 ** 15 and np.isclose(p[:32].max(), 1.0)
    l = p.sum()
    exact = (p[:, None] * v).sum(0) / l
    p16 = p.astype(np.float16).astype(np.float64)
    got = (p16[:, None] * v).sum(0) / l
    bound = (2.0 ** -11 + K * 2.0 ** -25) * np.abs(v).max()
    err = np.abs(got - exact).max()
    assert err <= bound, (err, bound)
    return err / bound


@pytest.mark.parametrize("seed", range(6))
def test_random_rows(seed):
    rng = np.random.default_rng(seed)
    K = int(rng.integers(33, 5000))
    scores = rng.normal(0.0, [0.5, 4.0, 12.0, 30.0, 2.0, 8.0][seed], K)
    scores = np.minimum(scores, scores[:32].max() + 14.9)  # the pass without redo keeps p < 2^15
    v = rng.normal(0.0, 2.0, (K, 16))
    _bound_holds(scores, v)


def test_aligned_errors_reach_most_of_the_bound():
    """Every weight rounds up by nearly its relative maximum and V is constant:
    the error approaches 2^-11 of max|V| and stays within the bound."""
    # p = 1 + 2^-11 - tiny rounds up to 1 + 2^-10 in fp16: relative error ~2^-11
    K = 4096
    frac = np.log2(1.0 + 2.0 ** -11 + 2.0 ** -20)
    scores = np.full(K, frac - 1.0)  # p = 0.5 * (1 + 2^-11 + ...) for every key but the first
    scores[0] = 0.0
    v = np.ones((K, 4))
    ratio = _bound_holds(scores, v)
    assert ratio > 0.4


def test_weights_just_below_the_normal_range():
    """Many weights of ~0.75 * 2^-14 (fp16 subnormals, absolute rounding 2^-25)
    against one weight of 1."""
    K = 20000
    scores = np.full(K, np.log2(0.75 * 2.0 ** -14 + 0.37 * 2.0 ** -24))
    scores[0] = 0.0
    v = np.ones((K, 4))
    _bound_holds(scores, v)


def test_weights_near_the_headroom():
    """A later key 2^14.9 heavier than the first 32: finite in fp16 and within
    the bound."""
    rng = np.random.default_rng(9)
    K = 300
    scores = rng.normal(0.0, 1.0, K)
    scores[200] = scores[:32].max() + 14.9
    v = rng.normal(0.0, 3.0, (K, 8))
    _bound_holds(scores, v)
