"""Pins of the fused producer ops' oracle (oracle/fused.py): against the reference C
(`mx_rms_norm`, `mx_silu_mul`, app/native/src/mx_fused_ops.c:6-42) through the committed
fixtures and live where oracle/_ref is built, and against closed forms.

Tolerance: the reference sums squares in a SIMD order of its compiler's choosing and calls libm's
expf, so agreement is to a few float32 ulps: 1e-6 relative per element."""

import numpy as np
import pytest
from scipy.special import expit

from oracle import fused as F
from tests.conftest import GOLDEN

RTOL = 1e-6


@pytest.fixture(scope="module")
def fused_cases():
    with np.load(GOLDEN / "fused_cases.npz") as z:
        return {k: z[k] for k in z.files}


def test_rms_norm_matches_reference_fixture(fused_cases) -> None:
    c = fused_cases
    got = F.rms_norm(c["rms_x"], c["rms_w"], float(c["rms_eps"][0]))
    np.testing.assert_allclose(got, c["rms_y"], rtol=RTOL, atol=0)
    assert np.all(c["rms_y"][1] == 0) and np.all(got[1] == 0)  # the zero row


def test_silu_mul_matches_reference_fixture(fused_cases) -> None:
    c = fused_cases
    got = F.silu_mul(c["silu_g"], c["silu_u"])
    np.testing.assert_allclose(got, c["silu_y"], rtol=RTOL, atol=1e-37)


def test_rms_norm_constant_row_closed_form() -> None:
    """A row of c: sum of squares is exactly dim * c^2 for c = 3/4, so out = c / sqrt(c^2 + eps)
    * w (a dropped mean, eps or weight term fails this)."""
    dim, c, eps = 1024, 0.75, 1e-5
    w = np.linspace(0.5, 1.5, dim, dtype=np.float32)
    got = F.rms_norm(np.full((1, dim), c, np.float32), w, eps)[0]
    want = c / np.sqrt(c * c + eps) * w.astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=4e-7)


def test_rms_norm_scale_invariant_without_eps() -> None:
    """With eps = 0, scaling x by a power of two scales the sum, mean and root exactly, so the
    result is unchanged bit for bit."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 512), dtype=np.float32)
    w = rng.standard_normal(512, dtype=np.float32)
    base = F.rms_norm(x, w, 0.0)
    for s in (2.0 ** -7, 8.0, 2.0 ** 20):
        assert np.array_equal(F.rms_norm(x * np.float32(s), w, 0.0), base)


def test_rms_norm_unit_rms_rows() -> None:
    """Each output row of a unit weight has mean square 1 (up to eps)."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((4, 2048), dtype=np.float32) * np.float32(7)
    y = F.rms_norm(x, np.ones(2048, np.float32), 0.0).astype(np.float64)
    np.testing.assert_allclose(np.mean(y * y, axis=1), 1.0, rtol=1e-5)


def test_silu_mul_special_values() -> None:
    g = np.array([0.0, 30.0, 90.0, -90.0, 1.0], np.float32)
    u = np.array([5.0, 2.0, -1.0, 3.0, 1.0], np.float32)
    y = F.silu_mul(g, u)
    assert y[0] == 0.0 and y[1] == np.float32(60.0) and y[2] == np.float32(-90.0)
    assert y[3] == 0.0
    np.testing.assert_allclose(y[4], 1.0 / (1.0 + np.exp(-1.0)), rtol=2e-7)


def test_silu_mul_against_expit() -> None:
    rng = np.random.default_rng(3)
    g = rng.standard_normal(10000).astype(np.float32) * np.float32(6)
    u = rng.standard_normal(10000).astype(np.float32)
    want = g.astype(np.float64) * expit(g.astype(np.float64)) * u
    np.testing.assert_allclose(F.silu_mul(g, u), want, rtol=1e-6, atol=1e-30)


@pytest.mark.parametrize("rows,dim", [(1, 256), (3, 4096), (2, 14336)])
def test_fused_oracle_against_live_reference(ref, rows, dim) -> None:
    rng = np.random.default_rng(rows * dim)
    x = rng.standard_normal((rows, dim), dtype=np.float32)
    w = rng.standard_normal(dim, dtype=np.float32)
    np.testing.assert_allclose(F.rms_norm(x, w, 1e-6), ref.rms_norm(x, w, 1e-6), rtol=RTOL)
    g = rng.standard_normal((rows, dim), dtype=np.float32) * np.float32(5)
    np.testing.assert_allclose(F.silu_mul(g, x), ref.silu_mul(g, x), rtol=RTOL, atol=1e-37)
