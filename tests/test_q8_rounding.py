"""The quantizer's round-half-away step (q8_round_code in
remora-lab_amd/csrc/rkv_device.h) as an identity on f32, checked on the CPU.

The reference rounds the scaled value with Rust's f32::round, half away from
zero, then `as i32` and clamps to [-127, 127] (har/crates/r4kv/src/quant.rs:63;
har/crates/har-serve/src/attention.rs:25-42).  The device computes
trunc(x + copysign(0x1.fffffep-2, x)) in f32 (round-to-nearest-even add), then
clamps and truncates.  numpy's float32 add rounds to nearest even as the GPU
does, so the identity is checked here on every f32 that can reach the
quantizer's rounding (|x| <= 127 * (1 + 2^-23) after scaling by 1/d), with
samples beyond it.
"""
import numpy as np
import pytest

C = np.frombuffer(np.uint32(0x3EFFFFFF).tobytes(), np.float32)[0]  # 0.5 - 2^-25


def device_round(x):
    """trunc(x + copysign(C, x)) in f32, clamped to [-127, 127]; NaN -> 0."""
    x = np.asarray(x, np.float32)
    y = (x + np.copysign(C, x).astype(np.float32)).astype(np.float32)
    out = np.trunc(np.clip(y, np.float32(-127), np.float32(127)))
    return np.where(np.isnan(y), 0.0, out)


def reference_round(x):
    """f32::round (half away from zero) as i32, clamped to [-127, 127]; NaN -> 0."""
    x64 = np.asarray(x, np.float32).astype(np.float64)
    r = np.sign(x64) * np.floor(np.abs(x64) + 0.5)  # exact in f64 for f32 inputs
    return np.where(np.isnan(x64), 0.0, np.clip(r, -127, 127))


def test_constant_is_the_largest_float_below_one_half():
    assert C < np.float32(0.5)
    assert np.nextafter(C, np.float32(1)) == np.float32(0.5)


def test_every_float_from_a_quarter_to_128():
    # below 0.25, x + C < 0.75 rounds to nothing that truncates to 1
    lo = np.float32(0.25).view(np.uint32)
    hi = np.float32(128.0).view(np.uint32)
    step = 1 << 24
    for s in range(int(lo), int(hi) + 1, step):
        x = np.arange(s, min(s + step, int(hi) + 1), dtype=np.uint32).view(np.float32)
        for sign in (1, -1):
            xs = (sign * x).astype(np.float32)
            got, want = device_round(xs), reference_round(xs)
            bad = np.nonzero(got != want)[0]
            assert bad.size == 0, (xs[bad[:4]], got[bad[:4]], want[bad[:4]])


@pytest.mark.parametrize("lo,hi", [(0.0, 0.25), (128.0, 2.0 ** 31)])
def test_sampled_ranges(lo, hi):
    rng = np.random.default_rng(11)
    u0, u1 = np.float32(lo).view(np.uint32), np.float32(hi).view(np.uint32)
    x = rng.integers(int(u0), int(u1), 4_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for xs in (x, -x):
        assert np.array_equal(device_round(xs), reference_round(xs))


def test_ties_and_special_values():
    ties = np.arange(-127.5, 128.0, 1.0, dtype=np.float32)  # every k + 0.5 in range
    assert np.array_equal(device_round(ties), reference_round(ties))
    assert np.array_equal(device_round(ties), np.clip(np.sign(ties) * np.ceil(np.abs(ties)), -127, 127))
    special = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-45, -1e-45, 3.4e38, -3.4e38,
                        0.49999997, -0.49999997, 0.5, -0.5, 126.5, -126.5, 127.49999, 127.5], np.float32)
    assert np.array_equal(device_round(special), reference_round(special))
