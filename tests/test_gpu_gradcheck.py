"""Finite-difference gradcheck of the host modules (the reference's own test
method, reference tests/gradcheck.c), run through tests/_build/libgradcheck.so."""
from __future__ import annotations

import ctypes
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "_build" / "libgradcheck.so"


def test_module_gradcheck(L):
    assert LIB.exists(), f"{LIB} missing: run __graft_entry__.build()"
    gc = ctypes.CDLL(str(LIB))
    gc.nn_gradcheck_run.restype = ctypes.c_int
    gc.nn_gradcheck_run.argtypes = [ctypes.c_int]
    fails = gc.nn_gradcheck_run(1)
    assert fails == 0, f"{fails} module(s) failed the gradcheck"


def test_sequential_chain_matches_modules_called_by_hand(L):
    """The Sequential container (src/sequential.c:31-118 semantics) against
    the same modules called one by one: bit-identical output, input gradient
    and parameter gradients, ParamList in module order, input copied."""
    gc = ctypes.CDLL(str(LIB))
    gc.nn_chaincheck_run.restype = ctypes.c_int
    assert gc.nn_chaincheck_run() == 0


def test_sequential_views_stay_aligned_after_odd_links(L):
    """A chain whose first link is 3 floats wide at batch 3, ahead of an
    implicit-GEMM convolution (which needs its input 16-byte aligned): the
    chain's output and gradients equal the modules run by hand, bit for bit,
    and no launcher records an error."""
    print("[case] Sequential with an odd-width link before a conv", flush=True)
    gc = ctypes.CDLL(str(LIB))
    gc.nn_chaincheck_odd_run.restype = ctypes.c_int
    assert gc.nn_chaincheck_odd_run() == 0


# Shapes whose GroupNorms take the streaming kernels (with the shift fused
# into GN2 at 8 channels per group; the block's own add and pixel sum at 4),
# and an EDM block whose convolutions take the implicit-GEMM kernels with the
# fused epilogues.
DIR_CASES = [(0, 16, 32, 32, 256, 32, 128), (0, 64, 32, 32, 128, 32, 64), (1, 16, 32, 32, 128, 0, 512)]
DIR_IDS = ["ddpm-streaming-shift-fused", "ddpm-streaming-cpg4", "edm-implicit-fused"]
DIR_BAR = 2e-3


@pytest.mark.parametrize("case", DIR_CASES, ids=DIR_IDS)
def test_block_directional_gradcheck(L, case):
    """The blocks' backward at sizes where per-element finite differences
    drown in fp32 noise: per input group (block input, embedding, each
    parameter tensor) the directional derivative along a random direction over
    the whole group, analytic <grad, d> against central differences of
    L = <out, g> summed in double (eps = 1e-2).  The bar 2e-3 is relative to
    max(|<grad, d>|, sqrt(sum (grad_i d_i)^2)): the truncation and rounding
    error is ~1e-4 there, while a wrong or dropped gradient term is off by
    orders of magnitude more."""
    kind, B, H, W, C, G, emb = case
    print(f"[case] directional gradcheck {case}", flush=True)
    worst = _dircheck(case, 1.0)
    print(f"directional gradcheck {case}: worst rel error {worst:.2e}", flush=True)
    assert worst <= DIR_BAR


def _dircheck(case, ana_scale):
    gc = ctypes.CDLL(str(LIB))
    gc.nn_dircheck_block.restype = ctypes.c_double
    gc.nn_dircheck_block.argtypes = [ctypes.c_int] * 7 + [ctypes.c_double, ctypes.c_int]
    return gc.nn_dircheck_block(*case, ana_scale, 1)


def test_block_directional_gradcheck_sees_a_half_percent_error(L):
    """The same check with every analytic gradient scaled by 1.005 (done in the
    harness, after the backward): the bar must reject it, so a gradient that is
    0.5% off anywhere would not pass."""
    print("[case] directional gradcheck sensitivity", flush=True)
    worst = _dircheck(DIR_CASES[0], 1.005)
    print(f"directional gradcheck with gradients x 1.005: worst rel error {worst:.2e}", flush=True)
    assert worst > DIR_BAR
