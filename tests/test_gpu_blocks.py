"""The fused diffusion blocks (conv_residual and cond_conv_residual, host/blocks.c)
against the reference's composition of the same launchers with the same
parameters (reference src/conv_residual.c:21-66, src/cond_conv_residual.c:
22-62): out, grad_in, every parameter gradient and the embedding gradient.
The DDPM sides differ only where the fused GroupNorm+SiLU recomputes the
pre-activation and uses the fast activation form: bar 1e-5 relative to
max(|ref|, rms(ref)) (measured: <= 3e-6), and for the embedding path's
reduced outputs (the pixel sum dc of GN2's input gradient, conv1's and the
projection's gradients, the embedding gradient) relative to at least the
scale sqrt(sum terms^2) of what they add.  At one channel per group that floor
is what the comparison rests on: GN2 then removes every per-(sample, channel)
shift, so those gradients are exactly zero and both sides return rounding
noise of the size eps * sqrt(n) * terms.  The EDM fused pair recomputes
x (c + 1) with the same operations and reduces grad_cond with the same kernel,
so its results are bit-identical.  The C side is tests/blockcheck.c in
_build/libgradcheck.so; it also times both sides (printed)."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "_build" / "libgradcheck.so"
BAR = 1e-5


@pytest.fixture(scope="module")
def bc(L):
    assert LIB.exists(), f"{LIB} missing: run __graft_entry__.build()"
    lib = C.CDLL(str(LIB))
    lib.nn_blockcheck_ddpm.argtypes = [C.c_int] * 7 + [C.POINTER(C.c_float)]
    lib.nn_blockcheck_ddpm.restype = C.c_double
    lib.nn_blockcheck_edm.argtypes = [C.c_int] * 5 + [C.c_float, C.c_int, C.POINTER(C.c_float)]
    lib.nn_blockcheck_edm.restype = C.c_double
    lib.nn_blockcheck_ddpm_graph.argtypes = [C.c_int] * 7 + [C.POINTER(C.c_float)]
    lib.nn_blockcheck_ddpm_graph.restype = C.c_int
    lib.nn_blockcheck_edm_graph.argtypes = [C.c_int] * 5 + [C.c_float, C.c_int, C.POINTER(C.c_float)]
    lib.nn_blockcheck_edm_graph.restype = C.c_int
    return lib


@pytest.mark.parametrize("shape", [(2, 8, 8, 32, 8, 16), (16, 32, 32, 256, 32, 128)],
                         ids=["small", "streaming-gn"])
def test_ddpm_block_graph_replay(bc, shape):
    """The fused DDPM block's forward + backward (lent workspaces, implicit
    convolutions, streaming GroupNorm at the larger shape, rocBLAS for the
    time projection) captured into one HIP graph: every replay reproduces the
    eager output, input gradient and embedding gradient bit for bit, with an
    eager forward on the same buffers between replays."""
    print(f"[case] DDPM block graph {shape}", flush=True)
    ms = (C.c_float * 2)()
    bad = bc.nn_blockcheck_ddpm_graph(*shape, 4, ms)
    print(f"DDPM block {shape} as a graph: eager fwd+bwd {ms[0]:.3f} ms, graph replay {ms[1]:.3f} ms", flush=True)
    assert bad == 0, "capture failed" if bad < 0 else f"{bad} replays differ from eager"


@pytest.mark.parametrize("shape", [(2, 8, 8, 16, 12), (128, 32, 32, 128, 512)], ids=["small", "cfg2"])
def test_edm_block_graph_replay(bc, shape):
    """The fused EDM block (weight-normalised convolutions with a lent
    workspace, the modulate + MP-SiLU pair, mp_sum) as one HIP graph: every
    replay bit-identical to eager."""
    print(f"[case] EDM block graph {shape}", flush=True)
    ms = (C.c_float * 2)()
    bad = bc.nn_blockcheck_edm_graph(*shape, 0.3, 4, ms)
    print(f"EDM block {shape} as a graph: eager fwd+bwd {ms[0]:.3f} ms, graph replay {ms[1]:.3f} ms", flush=True)
    assert bad == 0, "capture failed" if bad < 0 else f"{bad} replays differ from eager"


# The reference DDPM model's three levels (ddpm/ddpm.ini: channels 32, 64,
# 128, 32 groups, emb_dim 64, batch 8, 28x28 images halved per level): 1, 2
# and 4 channels per group, where GN2 adds the embedding in place and the
# plain GroupNorm kernels run; and a 4-channels-per-group block large enough
# for the streaming GroupNorm, whose shift forward the fused kernels refuse.
DDPM_SHAPES = [(2, 8, 8, 32, 8, 16), (16, 32, 32, 256, 32, 128),
               (8, 28, 28, 32, 32, 64), (8, 14, 14, 64, 32, 64), (8, 7, 7, 128, 32, 64),
               (64, 32, 32, 128, 32, 64)]
DDPM_IDS = ["small", "streaming-gn", "ref-level0-cpg1", "ref-level1-cpg2", "ref-level2-cpg4", "streaming-cpg4"]


@pytest.mark.parametrize("shape", DDPM_SHAPES, ids=DDPM_IDS)
def test_ddpm_block_matches_reference_composition(bc, shape):
    print(f"[case] DDPM block {shape}", flush=True)
    ms = (C.c_float * 2)()
    worst = bc.nn_blockcheck_ddpm(*shape, 3, ms)
    print(f"DDPM block {shape}: max rel diff {worst:.3e}; fwd+bwd fused {ms[0]:.3f} ms, "
          f"reference composition {ms[1]:.3f} ms", flush=True)
    assert worst <= BAR


@pytest.mark.parametrize("shape", [(2, 8, 8, 16, 12), (128, 32, 32, 128, 512)], ids=["small", "cfg2"])
def test_edm_block_matches_reference_composition(bc, shape):
    print(f"[case] EDM block {shape}", flush=True)
    ms = (C.c_float * 2)()
    worst = bc.nn_blockcheck_edm(*shape, 0.3, 3, ms)
    print(f"EDM block {shape}: max rel diff {worst:.3e}; fwd+bwd fused {ms[0]:.3f} ms, "
          f"reference composition {ms[1]:.3f} ms", flush=True)
    assert worst == 0.0


@pytest.mark.parametrize("geom", [(128, 32, 32, 128, 128, 3, 1, 1, 0), (128, 32, 32, 128, 128, 3, 1, 1, 1),
                                  (16, 64, 64, 256, 256, 3, 1, 1, 0)],
                         ids=["cfg3", "cfg3-mp", "ddpm-256"])
def test_conv_module_implicit_vs_gemm_path(bc, geom):
    """The conv2d module's two paths (implicit GEMMs on the matrix cores vs
    im2col + rocBLAS GEMMs + col2im) agree on y, grad_in and the parameter
    gradients within the reduction bar (different fp32 summation orders of the
    same products, relative to max(|v|, rms(v))); both paths' times are
    printed."""
    bc.nn_convcheck.argtypes = [C.c_int] * 10 + [C.POINTER(C.c_float)]
    bc.nn_convcheck.restype = C.c_double
    print(f"[case] conv module paths {geom}", flush=True)
    ms = (C.c_float * 4)()
    worst = bc.nn_convcheck(*geom, 3, ms)
    print(f"conv2d {geom}: max rel diff {worst:.3e}; forward implicit {ms[0]:.3f} ms vs im2col+rocBLAS {ms[1]:.3f} ms;"
          f" backward implicit {ms[2]:.3f} ms vs im2col+rocBLAS+col2im {ms[3]:.3f} ms", flush=True)
    assert worst <= 1e-5
