"""CPU checks of the GEMM tile layout (tests/_gemm_layout.py): the layout is a
permutation of the GGUF bytes, and the kernel's way of forming its B operands
from it gives back the oracle's dequantised weights (no reference
counterpart: the layout is this library's own)."""

import numpy as np
import pytest

import _gemm_layout as GL
import _oracle as O


@pytest.mark.parametrize("N,K", [(64, 64), (128, 256), (192, 1024)])
def test_layout_is_a_permutation(N, K):
    n = N * K // 32 * 18
    perm = GL.pack_layout(np.arange(n, dtype=np.int64), N, K)
    assert np.array_equal(np.sort(perm), np.arange(n))


@pytest.mark.parametrize("N,K", [(64, 64), (128, 256)])
def test_operands_from_layout_match_dequantisation(N, K):
    g = np.random.default_rng(N + K)
    W = O.make_q4_0(g, N, K)
    got = GL.dequant_from_layout(GL.pack_layout(W, N, K), N, K)
    assert np.array_equal(got, O.dequant_q4_0(W, N, K).astype(np.float64))


def test_a_wrong_byte_order_is_caught():
    # the same emulation over a layout without the 0, 2, 1, 3 order mixes up
    # neighbouring values: the check above would fail for it
    g = np.random.default_rng(3)
    W = O.make_q4_0(g, 64, 64)
    saved = GL.ORDER.copy()
    try:
        GL.ORDER[:] = np.arange(8)
        bad = GL.dequant_from_layout(GL.pack_layout(W, 64, 64), 64, 64)
    finally:
        GL.ORDER[:] = saved
    assert not np.array_equal(bad, O.dequant_q4_0(W, 64, 64).astype(np.float64))
