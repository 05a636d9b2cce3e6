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
