"""Pins the numpy dequant restatement (oracle/dequant.py) against things it did not derive from:
the reference's own C kernels compiled from their sources (oracle/_ref), the reference's
one-block Q8_0 known answer, IEEE half decoding on all 65536 bit patterns, an independent C
restatement, and closed-form special cases. A dropped term, a swapped nibble half, a wrong
scale index or a transposed block layout fails at least one of these."""

import numpy as np
import pytest

from matricxon_amd import synthetic as S
from oracle import dequant as D

TYPES = [D.Q8_0, D.Q4_K, D.Q6_K, D.IQ4_XS]


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_q8_0_known_answer() -> None:
    """tests/unit/test_dequant_kernels.py:46-59 of the reference: d = 0.5, qs = -16..15."""
    block = np.frombuffer(np.float16(0.5).tobytes() + np.arange(-16, 16, dtype=np.int8).tobytes(),
                          dtype=np.uint8)
    out = D.dequantize(D.Q8_0, block)
    assert np.array_equal(out, np.arange(-16, 16, dtype=np.float32) * np.float32(0.5))


def test_half_decoding_all_patterns(oracle) -> None:
    """Q8_0 with qs = 1 returns d itself: the numpy and the C restatements must widen every
    finite half (subnormals included) to the IEEE value."""
    h = np.arange(1 << 16, dtype=np.uint16)
    finite = ~np.isinf(h.view(np.float16)) & ~np.isnan(h.view(np.float16))
    h = h[finite]
    blocks = np.zeros((h.size, 34), dtype=np.uint8)
    blocks[:, 0:2] = h.view(np.uint8).reshape(-1, 2)
    blocks[:, 2] = 1
    expect = h.view(np.float16).astype(np.float32)
    got_np = D.dequantize(D.Q8_0, blocks).reshape(-1, 32)[:, 0]
    got_c = oracle.dequantize(D.Q8_0, blocks, h.size).reshape(-1, 32)[:, 0]
    assert np.array_equal(bits(got_np), bits(expect))
    assert np.array_equal(bits(got_c), bits(expect))
    # subnormal halves really are in the set
    assert np.any((h & 0x7C00) == 0) and np.any(expect[(h & 0x7C00) == 0] != 0)


@pytest.mark.parametrize("ggml_type", TYPES)
def test_numpy_and_c_restatements_agree_bitwise(oracle, ggml_type: int) -> None:
    w = S.packed_weight(ggml_type, 24, 1024, seed=100 + ggml_type)
    n_blocks = w.size // D.GEOMETRY[ggml_type][1]
    assert np.array_equal(bits(D.dequantize(ggml_type, w)),
                          bits(oracle.dequantize(ggml_type, w, n_blocks)))


def test_q4_k_matches_reference_dequant_rows_bitwise(ref_nofma) -> None:
    """The reference's mx_dequant_rows computes (d*sc)*u - dmin*m for Q4_K, the numpy order."""
    w = S.packed_weight(D.Q4_K, 40, 2048, seed=7)
    want = ref_nofma.dequant_rows(D.Q4_K, w, np.arange(40), 2048)
    assert np.array_equal(bits(D.dequantize_matrix(D.Q4_K, w, 40, 2048)), bits(want))


def test_q6_k_matches_reference_dequant_rows(ref_nofma) -> None:
    """The reference's mx_dequant_rows evaluates (d*sc)*(q+32) - d*(32*sc): equal values, but it
    yields +0.0 where numpy's (d*sc)*(q) gives -0.0 (q = 0 with sc < 0, or d*sc < 0 times 0)."""
    w = S.packed_weight(D.Q6_K, 40, 2048, seed=8, sc_low=-128, sc_high=127)
    want = ref_nofma.dequant_rows(D.Q6_K, w, np.arange(40), 2048)
    got = D.dequantize_matrix(D.Q6_K, w, 40, 2048)
    assert np.array_equal(got, want)
    differ = bits(got) != bits(want)
    assert np.all(got[differ] == 0.0)


def test_iq4_xs_matches_reference_on_one_hot_activations(ref) -> None:
    """The reference's IQ4_XS dot on raw floats (mx_dot_f32.c:32-58) with x = e_k returns the
    dequantized weight W[:, k] exactly (one product dl*grid, every other term is 0)."""
    n, k = 12, 512
    w = S.packed_weight(D.IQ4_XS, n, k, seed=9)
    got = ref.gemm(D.IQ4_XS, w, np.eye(k, dtype=np.float32), n, k).T
    assert np.array_equal(D.dequantize_matrix(D.IQ4_XS, w, n, k), got)


def test_q4_k_special_cases() -> None:
    rng = np.random.default_rng(0)
    blk = S.blocks_q4_k(rng, 4)
    blk[0, 0:2] = 0  # d = 0: every value is -(dmin * m)
    blk[1, 16:] = 0  # all q = 0: the same
    out = D.dequantize(D.Q4_K, blk).reshape(4, 8, 32)
    sc, mn = D.k4_scales_mins(blk[:, 4:16])
    dmin = blk[:, 2:4].copy().view("<f2").astype(np.float32).reshape(-1)
    for b in (0, 1):
        for s in range(8):
            want = -(dmin[b] * np.float32(mn[b, s]))
            assert np.all(out[b, s] == want)
    # scale/min unpacking round-trips through the packer
    sc2, mn2 = D.k4_scales_mins(D.pack_k4_scales_mins(sc, mn))
    assert np.array_equal(sc, sc2) and np.array_equal(mn, mn2)


def test_q6_k_zero_code_and_offsets() -> None:
    rng = np.random.default_rng(1)
    blk = S.blocks_q6_k(rng, 2)
    blk[0, 0:192] = 0x00  # u = 0 everywhere: value = (d*sc) * -32
    blk[1, 0:128] = 0x00  # ql = 0 and qh = 0b10101010: u = 32, q = 0 everywhere
    blk[1, 128:192] = 0xAA
    out = D.dequantize(D.Q6_K, blk).reshape(2, 16, 16)
    d = blk[:, 208:210].copy().view("<f2").astype(np.float32).reshape(-1)
    sc = blk[:, 192:208].view(np.int8).astype(np.float32)
    for s in range(16):
        assert np.all(out[0, s] == (d[0] * sc[0, s]) * np.float32(-32.0))
    assert np.all(out[1] == 0.0)
    assert np.array_equal(D.q6_k_codes(blk)[1], np.full(256, 32))


def test_iq4_xs_grid_and_scale() -> None:
    rng = np.random.default_rng(2)
    blk = S.blocks_iq4_xs(rng, 1)
    # ls = 33 for every sub-block: scales_l nibbles 1, scales_h bits 0b10 -> 1 | 2 << 4 = 33
    blk[0, 2:4] = np.frombuffer(np.uint16(0xAAAA).tobytes(), dtype=np.uint8)
    blk[0, 4:8] = 0x11
    blk[0, 8:] = np.array([(i % 16) | ((15 - i % 16) << 4) for i in range(128)], dtype=np.uint8)
    out = D.dequantize(D.IQ4_XS, blk).reshape(8, 32)
    d = blk[:, 0:2].copy().view("<f2").astype(np.float32)[0, 0]
    for ib in range(8):
        assert np.array_equal(out[ib, :16], d * D.IQ4_GRID[np.arange(16)])
        assert np.array_equal(out[ib, 16:], d * D.IQ4_GRID[15 - np.arange(16)])
