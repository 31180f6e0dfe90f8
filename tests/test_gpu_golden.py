"""The HIP kernels against the reference C kernel's own outputs (golden fixtures written by
tests/golden/make_golden.py): within the tolerance for every type, bit-equal for the K-quants and
Q8_0 (the kernels reproduce the reference's integer dots and its fp32 fold steps)."""

import numpy as np
import pytest

from oracle import dequant as D
from tests.test_golden import CONFIG_KEYS, SMALL, SMALL_KEYS, TYPES, config_case, small_case
from tests.test_gpu_kernels import assert_within_tolerance, bits, dev, host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("key", SMALL_KEYS)
def test_small_goldens(gpu, key) -> None:
    t, w, x, y, n, k = small_case(key)
    got = host(gpu.matmul(t, dev(w), dev(x), n, k))
    assert_within_tolerance(got, y)
    if t != D.IQ4_XS:
        assert np.array_equal(bits(got), bits(y))


@pytest.mark.parametrize("key", CONFIG_KEYS)
def test_config_goldens(gpu, key) -> None:
    t, w, x, rows, y, n, k = config_case(key)
    got = host(gpu.matmul(t, dev(w), dev(x), n, k))[:, rows]
    assert_within_tolerance(got, y)
    if t != D.IQ4_XS:
        assert np.array_equal(bits(got), bits(y))


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "iq4_xs"])
def test_dequant_goldens(gpu, name) -> None:
    w, v = SMALL[f"deq_{name}_w"], SMALL[f"deq_{name}_v"]
    got = host(gpu.dequantize(dev(w), TYPES[name])).reshape(8, 512)
    assert np.array_equal(got, v)
    if name == "q4_k":  # the others may differ from the reference route in the sign of zeros
        assert np.array_equal(bits(got), bits(v))
