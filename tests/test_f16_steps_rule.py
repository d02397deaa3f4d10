"""The arithmetic rule the QMoE final sum uses for f16 rows (tmh_moe.hip, moe_combine): a product
or a sum of two f16 values computed in f32 and rounded to f16 (the oracle's steps, each value
rounded to the input type after every operation) has the bits of the same operation rounded once,
straight to f16 (what v_pk_mul_f16 and v_pk_add_f16 compute). The exact result of each operation
is formed in f64 (a product of two f16 values needs 22 bits; a sum at most 11 plus the 40
binades between the largest and the smallest f16, both within f64's 53), then rounded once to
f16, and twice, through f32. Checked over every sign and exponent pairing and random
significands, over operands placed so that the exact result lies next to an f16 rounding tie, and
with a double rounding through a coarser format (13 significant bits in place of f32) as the planted mistake
the check must catch."""

import numpy as np


def _all_f16(rng, n):
    bits = rng.integers(0, 1 << 16, n, dtype=np.uint32).astype(np.uint16)
    x = bits.view(np.float16)
    return x[np.isfinite(x)]


def _round_bits(x64, p):
    """x rounded to p significant bits (nearest, ties to even), in f64."""
    m, e = np.frexp(x64)
    return np.ldexp(np.rint(np.ldexp(m, p)), e - p)


def _check(a, b, op):
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        exact = a64 * b64 if op == "mul" else a64 + b64
        once = exact.astype(np.float16)
        twice = exact.astype(np.float32).astype(np.float16)
    same = (once.view(np.uint16) == twice.view(np.uint16)) | (np.isnan(once) & np.isnan(twice))
    return same, exact


def test_products_and_sums_round_the_same_through_f32():
    rng = np.random.default_rng(20261203)
    for op in ("mul", "add"):
        for _ in range(8):
            a, b = _all_f16(rng, 1 << 20), _all_f16(rng, 1 << 20)
            n = min(a.size, b.size)
            same, _exact = _check(a[:n], b[:n], op)
            assert same.all(), op


def _ties(rng):
    """Positive f16 values of normal range and their f16 ulps."""
    big = np.abs(_all_f16(rng, 1 << 16)).astype(np.float64)
    big = big[(big > 2.0 ** -14) & (big < 2.0 ** 15)]
    return big, np.spacing(big.astype(np.float16)).astype(np.float64)


def test_operands_next_to_f16_ties():
    """Sums whose exact value lies on an f16 tie or just beside it: a second operand of half an
    f16 ulp of the first plus or minus down to its own last bit (2^-1 .. 2^-10 of that ulp), and
    operands from half an ulp down through 40 binades below it."""
    rng = np.random.default_rng(7)
    big, ulp = _ties(rng)
    offsets = [0.5 + sgn * 2.0 ** -g for g in range(2, 11) for sgn in (1.0, -1.0)]
    offsets += [0.5 * 2.0 ** -g for g in range(0, 41)]
    for off in offsets:
        for sign in (1.0, -1.0):
            b = (sign * ulp * off).astype(np.float16)
            keep = np.isfinite(b) & (b != 0)
            same, _exact = _check(big[keep].astype(np.float16), b[keep], "add")
            assert same.all(), off


def test_a_coarser_intermediate_format_is_caught():
    """Rounding first to 13 significant bits (two more than f16) and then to f16 does change
    sums that lie just above an f16 tie, so the checks above compare roundings that can differ
    there."""
    rng = np.random.default_rng(11)
    big, ulp = _ties(rng)
    differ = 0
    for g in range(3, 8):
        exact = big + (ulp * (0.5 + 2.0 ** -g)).astype(np.float16).astype(np.float64)
        once = exact.astype(np.float16)
        coarse = _round_bits(exact, 13).astype(np.float16)
        differ += int((once.view(np.uint16) != coarse.view(np.uint16)).sum())
    assert differ > 0
