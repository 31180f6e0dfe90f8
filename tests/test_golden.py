"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the reference's
own C kernels): the regenerated synthetic inputs must still be the fixture's bytes, the oracle
must reproduce the reference outputs bit for bit, and the numpy dequant must reproduce the
reference's dequantized values (Q6_K, IQ4_XS: equal values; the reference's routes may produce
+0.0 where numpy's product gives -0.0)."""

import hashlib

import numpy as np
import pytest

from matricxon_amd import synthetic as S
from oracle import dequant as D
from tests.conftest import GOLDEN

SMALL = np.load(GOLDEN / "small_cases.npz")
CONFIG = np.load(GOLDEN / "config_cases.npz")
TYPES = {"q8_0": D.Q8_0, "q4_k": D.Q4_K, "q6_k": D.Q6_K, "iq4_xs": D.IQ4_XS}
SMALL_KEYS = sorted(k[:-2] for k in SMALL.files if k.endswith("_y"))
CONFIG_KEYS = sorted(k[:-5] for k in CONFIG.files if k.endswith("_meta"))


def small_case(key: str):
    t = TYPES[key.rsplit("_", 1)[0]] if not key.startswith("q6_k_wide") else D.Q6_K
    w, x, y = SMALL[key + "_w"], SMALL[key + "_x"], SMALL[key + "_y"]
    return t, w, x, y, y.shape[1], x.shape[1]


def config_case(key: str):
    t, n, k, m, wseed, xseed = (int(v) for v in CONFIG[key + "_meta"])
    w = S.packed_weight(t, n, k, seed=wseed)
    x = S.activations(m, k, seed=xseed)
    wsha, xsha = CONFIG[key + "_sha"]
    assert hashlib.sha256(w.tobytes()).hexdigest() == wsha, "weight generator changed"
    assert hashlib.sha256(x.tobytes()).hexdigest() == xsha, "activation generator changed"
    return t, w, x, CONFIG[key + "_rows"], CONFIG[key + "_y"], n, k


@pytest.mark.parametrize("key", SMALL_KEYS)
def test_oracle_reproduces_small_goldens(oracle, key) -> None:
    t, w, x, y, n, k = small_case(key)
    assert np.array_equal(oracle.gemm(t, w, x, n, k), y)


@pytest.mark.parametrize("key", [k for k in CONFIG_KEYS if not k.startswith("cfg3")])
def test_oracle_reproduces_config_goldens(oracle, key) -> None:
    t, w, x, rows, y, n, k = config_case(key)
    assert np.array_equal(oracle.gemm(t, w[rows], x, len(rows), k), y)


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "iq4_xs"])
def test_numpy_dequant_reproduces_reference_values(name) -> None:
    w, v = SMALL[f"deq_{name}_w"], SMALL[f"deq_{name}_v"]
    got = D.dequantize_matrix(TYPES[name], w, 8, 512)
    assert np.array_equal(got, v)
    if name == "q4_k":  # Q6_K and the one-hot IQ4_XS route may differ in the sign of zeros
        assert np.array_equal(got.view(np.uint32), v.view(np.uint32))
