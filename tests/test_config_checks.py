"""The full-size parity checks of tests/test_hip_configs.py, checked themselves on the CPU.

They run here against the device-flavoured plan on the oracle (`cpu_devplan`: split sums, row
groups, attention steps, device fusion), at reduced sizes, and must pass; and the comparison
helpers must fail on the mistakes they exist to catch (a moment 10 % off on a leaf whose values
are all far below 1, a bias update a third too large, a missing bias correction), while passing
rounding-level differences that AdamW amplifies where a gradient is near zero.
"""

import numpy as np
import pytest

from rustautograd_amd import workloads

from conftest import DEVPLAN
from helpers import close_rel, updates_agree
from test_hip_configs import full_check

ADAMW = {"lr": 3e-4, "weight_decay": 0.01, "b1": 0.9, "b2": 0.999, "eps": 1e-8}


def test_checks_pass_on_the_device_plan_small_gpt():
    cfg = workloads.GPT_CONFIGS["C3"]._replace(batch=4, block=16, layers=2)
    step, state = workloads.gpt_train_step(cfg)
    full_check(step, state, 2, key_bias_d=cfg.d, device=DEVPLAN, standard=False)


def test_checks_pass_on_the_device_plan_small_mlp():
    step, state = workloads.mlp_train_step(workloads.MLPConfig(batch=64, d_in=32, hidden=64))
    full_check(step, state, 2, device=DEVPLAN, standard=False)


def _adamw_step(p, g, count=1.0, scale_update=1.0, unbias=True):
    """One AdamW step in float32 from zero moments: (new, mu, nu, count)."""
    f = np.float32
    mu = f(1 - 0.9) * g
    nu = f(1 - 0.999) * (g * g)
    c1, c2 = (f(1 - 0.9 ** count), f(1 - 0.999 ** count)) if unbias else (f(1), f(1))
    direction = (mu / c1) / (np.sqrt(nu / c2) + f(1e-8)) + f(0.01) * p
    return (p - f(ADAMW["lr"] * scale_update) * direction).astype(np.float32), mu, nu, count


def _gradients(seed, n=4096):
    r = np.random.default_rng(seed)
    g = (r.normal(size=n) * 1e-3).astype(np.float32)
    g[::97] *= np.float32(1e-6)  # elements near zero, as a sum over many cancelling terms gives
    return g


def test_update_check_passes_rounding_noise_that_adamw_amplifies():
    p = np.random.default_rng(1).normal(size=4096).astype(np.float32) * np.float32(0.02)
    g = _gradients(2)
    noise = (np.random.default_rng(3).normal(size=g.size) * 1e-6 * np.abs(g).max()).astype(np.float32)
    hip, cpu = _adamw_step(p, g + noise), _adamw_step(p, g)
    # A plain comparison of the updates fails: near-zero gradients flip sign under the noise.
    with pytest.raises(AssertionError):
        close_rel(hip[0] - p, cpu[0] - p, 1e-4, "plain")
    updates_agree(p, hip, cpu, 1e-4, "noise", ADAMW)
    close_rel(hip[1], cpu[1], 1e-4, "mu")
    close_rel(hip[2], cpu[2], 1e-4, "nu")


def test_update_check_catches_a_bias_update_a_third_too_large():
    p = np.zeros(768, np.float32)
    g = _gradients(4, 768)
    with pytest.raises(AssertionError):
        updates_agree(p, _adamw_step(p, g, scale_update=1.33), _adamw_step(p, g), 1e-4, "bias", ADAMW)


def test_update_check_catches_a_missing_bias_correction():
    p = np.random.default_rng(5).normal(size=1024).astype(np.float32)
    g = _gradients(6, 1024)
    hip = _adamw_step(p, g, count=3.0, unbias=False)
    with pytest.raises(AssertionError):
        updates_agree(p, hip, _adamw_step(p, g, count=3.0), 1e-4, "unbias", ADAMW)


def test_relative_check_catches_a_ten_percent_error_on_tiny_values():
    nu = (np.random.default_rng(7).random(1000) * 1e-9).astype(np.float32)
    bad = nu.copy()
    bad[17] *= np.float32(1.1)
    with pytest.raises(AssertionError):
        close_rel(bad, nu, 1e-4, "nu")
    close_rel(nu, nu, 1e-4, "nu")
