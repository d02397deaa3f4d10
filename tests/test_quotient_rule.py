"""The arithmetic rule the DynamicQuantizeLinear quantize pass uses in place of a division
(tmh_quant_ops.hip, k_dql_quantize_reduce): rint(x * rcp), rcp = 1 / sc rounded once, equals
rint of the rounded quotient x / sc whenever x * rcp lies further than |x * rcp| 2^-21 from every
half-integer; nearer, the kernel divides. Checked here in f32 (numpy's f32 division and product
round once, to nearest even) against the quotient itself, over values placed within a few ulps of
every half-integer the quantization reaches and over uniform values, for scales across twelve
decades; without the fallback to the division the near-half values do round differently, so the
check has something to catch."""

import numpy as np


def _rule(x, sc):
    with np.errstate(over="ignore", invalid="ignore"):
        return _rule_f32(x, sc)


def _rule_f32(x, sc):
    rcp = np.float32(np.float32(1.0) / sc)
    q0 = (x * rcp).astype(np.float32)
    frac = (q0 - np.floor(q0)).astype(np.float32)
    near = ~(np.abs(frac - np.float32(0.5)) > np.abs(q0) * np.float32(2.0 ** -21))
    return np.rint(q0), near


def test_quotient_rule_matches_the_rounded_quotient():
    rng = np.random.default_rng(20261202)
    mismatches = without_fallback = 0
    for _ in range(40):
        sc = np.float32(abs(rng.standard_normal()) * 10.0 ** int(rng.integers(-8, 4)) / 255 + 1e-30)
        k = rng.integers(-256, 256, 20000).astype(np.float32)
        half = ((k + np.float32(0.5)) * sc).astype(np.float32)
        x = [half]
        for steps in (1, 2, 3):
            for d in (np.float32(np.inf), np.float32(-np.inf)):
                v = half
                for _ in range(steps):
                    v = np.nextafter(v, d).astype(np.float32)
                x.append(v)
        x.append((rng.uniform(-256, 256, 20000) * sc).astype(np.float32))
        x = np.concatenate(x)
        exact = np.rint((x / sc).astype(np.float32))
        fast, near = _rule(x, sc)
        mismatches += int(np.count_nonzero(np.where(near, exact, fast) != exact))
        without_fallback += int(np.count_nonzero(fast != exact))
    assert mismatches == 0
    assert without_fallback > 0


def test_quotient_rule_falls_back_where_the_product_is_not_finite():
    sc = np.float32(1e-45)  # a subnormal scale: 1 / sc overflows to infinity
    x = np.array([0.0, 1e-45, -2e-45, 3e-45], np.float32)
    _fast, near = _rule(x, sc)
    assert near.all()
