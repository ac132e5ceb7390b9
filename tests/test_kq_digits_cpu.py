"""The K/IQ digit kernels' activation arithmetic, restated in numpy and held to
its error bound (no GPU).

The digit row, pipelined and K-split kernels (kq_device.h: dg_scale,
stage_run_dg, put_record_dg) turn each 32-value activation block into
16-bit integers: c = 32638 / max|x| (the reciprocal and the product each
rounded to f32), Z = round-half-even(x * c) through the bits of
F = f32(1.5 * 2^23 + x * c), split into two signed bytes z0 = sext(byte 0 of
F), z1 = sext(byte 1 of F + 128), with the unit u = f32(1 / c).  The GPU
tests compare the kernels with the oracle within the parity bar; these
tests pin the arithmetic itself:
  * the two bytes always rebuild Z and |Z| <= 32638, so z1 never leaves
    [-128, 127] (a 32639th unit would);
  * rounding error per value is at most 1.54e-5 of its block's largest |x|,
    and a row's error at most 8.7e-5 |w| |x| -- reached within 10% by a
    construction that puts every small value on a half unit and every
    weight on its error's sign, which a power-of-two scale of at most 2^14
    units (the largest two signed-byte digits hold for every block) fails.
"""
import numpy as np
import pytest

UNITS = 32638.0
BOUND_VALUE = 1.54e-5  # per value, of the block's largest |x|
BOUND_ROW = 8.7e-5     # per row, of |w| |x|


def f32(v):
    return np.asarray(v, dtype=np.float64).astype(np.float32)


def stage_block(x):
    """One 32-value block as the kernels stage it: (Z, z0, z1, unit)."""
    x = f32(x)
    m = np.float32(np.max(np.abs(x)))
    with np.errstate(divide="ignore"):
        r = np.float32(1.0) / m if m > 0 else np.float32(np.inf)
    c = min(np.float32(UNITS * np.float64(r)), np.float32(2.0 ** 126))
    u = np.float32(1.0 / np.float64(c))
    # fma(x, c, 1.5 * 2^23): the exact product plus the constant, rounded once
    F = f32(x.astype(np.float64) * np.float64(c) + 12582912.0).view(np.uint32)
    Z = F.astype(np.int64) - 0x4B400000
    b0 = (F & 0xFF).astype(np.int64)
    b1 = (((F + 128) >> 8) & 0xFF).astype(np.int64)
    z0 = np.where(b0 >= 128, b0 - 256, b0)
    z1 = np.where(b1 >= 128, b1 - 256, b1)
    return Z, z0, z1, u


def stage(x):
    blocks = [stage_block(x[i:i + 32]) for i in range(0, x.size, 32)]
    Z = np.concatenate([b[0] for b in blocks])
    z0 = np.concatenate([b[1] for b in blocks])
    z1 = np.concatenate([b[2] for b in blocks])
    u = np.repeat(np.array([b[3] for b in blocks], dtype=np.float64), 32)
    return Z, z0, z1, u


CASES = {
    "normal": lambda rng: rng.standard_normal(4096),
    "all at the block max": lambda rng: np.repeat(rng.choice([-1.0, 1.0], 128) * rng.uniform(0.5, 2.0, 128), 32),
    "one outlier per block": lambda rng: np.where(np.arange(4096) % 32 == 5, 1e4, rng.standard_normal(4096)),
    "wide binades": lambda rng: rng.standard_normal(4096) * 10.0 ** rng.integers(-30, 30, 4096),
    "tiny": lambda rng: rng.standard_normal(4096) * 1e-30,
    "huge": lambda rng: rng.standard_normal(4096) * 1e30,
    "zeros and signs": lambda rng: rng.choice([-0.0, 0.0, 1.0, -1.0], 4096),
}


@pytest.mark.parametrize("case", list(CASES))
def test_digits_rebuild_z_within_range(case):
    rng = np.random.default_rng(7)
    x = f32(CASES[case](rng))
    Z, z0, z1, u = stage(x)
    assert np.all(np.abs(Z) <= UNITS)
    assert np.all((z0 >= -128) & (z0 <= 127) & (z1 >= -128) & (z1 <= 127))
    assert np.array_equal(z0 + 256 * z1, Z)


@pytest.mark.parametrize("case", list(CASES))
def test_rounding_error_per_value(case):
    rng = np.random.default_rng(11)
    x = f32(CASES[case](rng)).astype(np.float64)
    Z, _, _, u = stage(x)
    m = np.repeat(np.abs(x).reshape(-1, 32).max(axis=1), 32)
    err = np.abs(x - Z * u)
    assert np.all(err <= BOUND_VALUE * m + 1e-300)


def half_unit_row(rng, nblocks):
    """The bound's worst case: per block one value at the block maximum m
    (it sets the scale and rounds exactly) and 31 small values on half units
    (each rounds by half a unit, as much as any value can), weights on the
    sign of each error so the row's error adds up without cancellation.
    Then max|x| ~ |x_b| and sum |w_i| = sqrt(32) |w_b|: both inequalities of
    the bound are near equalities."""
    m = rng.uniform(0.5, 2.0, nblocks)
    k = rng.integers(-3, 3, (nblocks, 32)).astype(np.float64)
    x = (k + 0.5) * (m / UNITS)[:, None]
    x[:, 0] = m
    return x.reshape(-1)


def test_row_error_bound_is_tight():
    rng = np.random.default_rng(3)
    x = f32(half_unit_row(rng, 256)).astype(np.float64)
    Z, _, _, u = stage(x)
    e = x - Z * u
    w = np.sign(e)
    err = abs(np.dot(w, e))
    scale = np.linalg.norm(w) * np.linalg.norm(x)
    assert err <= BOUND_ROW * scale
    # 31 half units per block against the bound's 32: within 10%
    assert err >= 0.9 * BOUND_ROW * scale


def test_looser_scales_would_miss_the_row_bound():
    """The same construction against a power-of-two scale of 2^13-2^14 units
    (the largest power of two that keeps two signed-byte digits for every
    block maximum) -- what the 32638-unit scale avoids."""
    rng = np.random.default_rng(5)
    nblocks = 256
    m = rng.uniform(0.5, 2.0, nblocks)
    unit = 2.0 ** (np.floor(np.log2(m)) - 13)  # max maps into [2^13, 2^14)
    k = rng.integers(-3, 3, (nblocks, 32)).astype(np.float64)
    x = (k + 0.5) * unit[:, None]
    x[:, 0] = m
    x = x.reshape(-1)
    e = np.full(x.size, 0.5) * np.repeat(unit, 32)
    e[::32] = 0.0
    w = np.ones(x.size)
    assert np.dot(w, e) > BOUND_ROW * np.linalg.norm(w) * np.linalg.norm(x)
