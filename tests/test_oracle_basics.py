"""bfloat16 / float16 rounding of the oracle: exact known values and torch's conversion."""

import numpy as np
import torch

import oracle


def test_round_bf16_known_values():
    one = np.float32(1.0)
    ulp = np.float32(2.0**-7)  # bf16 spacing at 1.0
    x = np.array(
        [
            1.0,
            1.0 + 2.0**-8,          # exactly half an ulp above 1 -> ties to even (1.0)
            1.0 + 3 * 2.0**-8,      # half an ulp above 1 + ulp -> ties to even (1 + 2 ulp)
            1.0 + 2.0**-8 + 2.0**-20,  # just above the tie -> rounds up
            -2.5,
            0.0,
            65504.0,
        ],
        np.float32,
    )
    want = np.array(
        [one, one, one + 2 * ulp, one + ulp, -2.5, 0.0, 65536.0], np.float32
    )
    np.testing.assert_array_equal(oracle.round_bf16(x), want)


def test_round_bf16_specials():
    x = np.array([np.inf, -np.inf, np.nan], np.float32)
    r = oracle.round_bf16(x)
    assert r[0] == np.inf and r[1] == -np.inf and np.isnan(r[2])


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(100_000) * np.exp(rng.uniform(-30, 30, 100_000))).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(oracle.round_bf16(x), want)


def test_round_f16_known_values():
    one = np.float32(1.0)
    ulp = np.float32(2.0**-10)  # fp16 spacing at 1.0
    x = np.array(
        [
            1.0 + 2.0**-11,              # half an ulp above 1 -> ties to even (1.0)
            1.0 + 3 * 2.0**-11,          # half an ulp above 1 + ulp -> ties to even (1 + 2 ulp)
            1.0 + 2.0**-11 + 2.0**-20,   # just above the tie -> rounds up
            2.0**-24,                    # smallest subnormal half
            2.0**-25,                    # half of it -> ties to even (0)
            1.5 * 2.0**-24,              # 1.5 subnormal steps -> ties to even (2 steps)
            65504.0,                     # largest finite half
            65519.0,                     # below the overflow threshold -> 65504
            65520.0,                     # the threshold (a tie with 2^16) -> inf
            -3.25,
        ],
        np.float32,
    )
    want = np.array(
        [one, one + 2 * ulp, one + ulp, 2.0**-24, 0.0, 2.0**-23, 65504.0, 65504.0, np.inf, -3.25],
        np.float32,
    )
    np.testing.assert_array_equal(oracle.round_f16(x), want)


def test_round_f16_specials_and_dispatch():
    x = np.array([np.inf, -np.inf, np.nan], np.float32)
    r = oracle.round_f16(x)
    assert r[0] == np.inf and r[1] == -np.inf and np.isnan(r[2])
    y = np.array([1.0 + 2.0**-9, 0.1], np.float32)
    np.testing.assert_array_equal(oracle.round_to(y, "bf16"), oracle.round_bf16(y))
    np.testing.assert_array_equal(oracle.round_to(y, "f16"), oracle.round_f16(y))
    assert oracle.round_to(y, "f32") is y


def test_round_f16_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100_000) * np.exp(rng.uniform(-20, 12, 100_000))).astype(np.float32)
    want = torch.from_numpy(x).to(torch.float16).to(torch.float32).numpy()
    np.testing.assert_array_equal(oracle.round_f16(x), want)
