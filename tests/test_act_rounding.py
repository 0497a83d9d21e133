"""The device activation quantizers' rounding formulas (swarmllm_amd/csrc/qmm_device.h):
q8k_code, trunc(clamp(t + copysign(0.49999997, t), -128.49, 127.49)), gives
the reference's Q8_K code for t = iscale * x (BlockQ8K::from_float,
vendor/candle/candle-core/src/quantized/k_quants.rs:2917-2920: t.round() half
away from zero, .min(127.) with NaN -> 127, `as i8`); q8_0_code, the same
rounding through v_cvt_i32_f32 and a clamp, gives its Q8_0 code
(BlockQ8_0::from_float, :1262-1265: t.round() as i8, NaN -> 0).

Two checks: a numpy restatement over the places a rounding formula can go
wrong (every float within 64 ulps of each half-integer and integer in
[-130, 130], the special values, a random sample of bit patterns), and the
exhaustive C check of both over all 2^32 floats (about 10 s on 8 threads)."""
import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def reference_codes(t: np.ndarray) -> np.ndarray:
    t64 = t.astype(np.float64)  # exact: half away from zero in double
    with np.errstate(invalid="ignore"):
        r = np.sign(t64) * np.floor(np.abs(t64) + 0.5)
        m = np.where(np.isnan(r), 127.0, np.minimum(r, 127.0))
        return np.clip(m, -128.0, 127.0).astype(np.int64)


def device_codes(t: np.ndarray) -> np.ndarray:
    t = t.astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        s = t + np.copysign(np.float32(0.49999997), t)  # float32 add, round to nearest even
        c = np.fmax(np.fmin(s, np.float32(127.49)), np.float32(-128.49))
    return np.trunc(c).astype(np.int64)


def neighbourhoods() -> np.ndarray:
    centres = np.concatenate([np.arange(-130, 131) + 0.5, np.arange(-130, 131)]).astype(np.float32)
    out = [centres]
    up, down = centres.copy(), centres.copy()
    for _ in range(64):
        up = np.nextafter(up, np.float32(np.inf))
        down = np.nextafter(down, np.float32(-np.inf))
        out += [up.copy(), down.copy()]
    return np.concatenate(out)


def test_constant_is_the_float_below_one_half():
    assert np.float32(0.49999997) == np.nextafter(np.float32(0.5), np.float32(0))


def test_formula_matches_reference_near_ties_and_integers():
    t = neighbourhoods()
    assert np.array_equal(device_codes(t), reference_codes(t))


def test_formula_special_values_and_random_bits():
    special = np.array([0.0, -0.0, np.nan, -np.nan, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45, -1e-45,
                        127.5, -128.5, 128.0, -129.0, 127.49999, -128.49998], dtype=np.float32)
    rng = np.random.default_rng(0)
    t = np.concatenate([special, rng.integers(0, 2**32, 4_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    assert np.array_equal(device_codes(t), reference_codes(t))
    assert device_codes(np.array([np.nan], np.float32))[0] == 127


def test_exhaustive_over_all_floats(tmp_path):
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "act_rounding"
    subprocess.run([cc, "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(HERE, "act_rounding_exhaustive.c"), "-lm"], check=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("0 mismatches")
