"""The activation quantizer's rounding identity (CPU).

The persistent decode kernel rounds a code as the truncation of
x + copysign(0.5 - 2^-25, x) in float32 instead of calling roundf (round half
away from zero, the reference's std::round in build_lut, TenzoEngine.cpp:34,
and compute_logits, :1668). This checks the identity on every float around
each integer and half-integer of the code range and on random floats."""
import numpy as np

H = np.float32(0.49999997)  # 0.5 - 2**-25, the float just below 0.5


def trick(x):
    x = np.asarray(x, np.float32)
    t = (x + np.copysign(H, x)).astype(np.float32)  # one float32 add, round to nearest even
    return np.trunc(t).astype(np.int64)


def roundf_ref(x):
    x = np.asarray(x, np.float32).astype(np.float64)  # exact
    return (np.sign(x) * np.floor(np.abs(x) + 0.5)).astype(np.int64)


def test_h_is_the_float_below_half():
    assert H == np.nextafter(np.float32(0.5), np.float32(0))
    assert float(H) == 0.5 - 2.0 ** -25


def test_around_integers_and_halves():
    bits = []
    for k in range(-260, 261):
        for c in (np.float32(k), np.float32(k + 0.5)):
            b = np.float32(c).view(np.int32)
            bits.append(np.arange(b - 4096, b + 4097, dtype=np.int64))
    b = np.concatenate(bits)
    b = b[(b >= -2**31) & (b < 2**31)].astype(np.int64)
    x = b.astype(np.int32).view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) < 256)]
    assert len(x) > 4_000_000
    np.testing.assert_array_equal(trick(x), roundf_ref(x))


def test_special_values():
    x = np.array([0.0, -0.0, 0.49999997, -0.49999997, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5,
                  31.0, -31.0, 30.5, -30.5, 127.5, -127.5, 1e-30, -1e-30,
                  2.0**22 + 0.5, -(2.0**22 + 0.5), 2.0**23 - 1, -(2.0**23 - 1)], np.float32)
    np.testing.assert_array_equal(trick(x), roundf_ref(x))


def test_random_floats():
    rng = np.random.default_rng(7)
    b = rng.integers(0, 0x43800000, size=20_000_000, dtype=np.int64)  # |x| < 256
    x = b.astype(np.int32).view(np.float32)
    x = np.where(rng.integers(0, 2, size=x.size) == 1, -x, x).astype(np.float32)
    np.testing.assert_array_equal(trick(x), roundf_ref(x))
