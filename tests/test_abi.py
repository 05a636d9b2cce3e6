"""The drop-in boundary, checked without a GPU: the library loads, exports every
function include/*.h declares, and refuses impossible arguments on the host
(reference launchers: src/nn.h:348-466) before any device work is queued."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _exported(lib_path: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_library_exports_every_declared_function(nn):
    declared = set(nn.header_functions())
    assert len(declared) > 60, sorted(declared)
    exported = _exported(nn.LIB_PATH)
    missing = sorted(declared - exported)
    assert not missing, f"declared in include/*.h but not exported: {missing}"


def test_reference_launcher_set_is_declared(nn):
    """Every on-path launcher of the reference's extern "C" block (src/nn.h:348-466)."""
    ref_names = {
        "launch_add_bias", "launch_bias_grad", "launch_sgd_step", "launch_activation_forward",
        "launch_activation_backward", "launch_adam_step", "launch_weight_normalize",
        "launch_weight_normalize_backward", "launch_scale_by_scalar", "launch_mp_sum", "launch_weighted_sum",
        "launch_mp_cat", "launch_mp_channel_cat", "launch_mp_channel_split", "launch_mp_fourier",
        "launch_sinusoidal", "launch_layernorm_forward", "launch_layernorm_backward",
        "launch_groupnorm_forward", "launch_groupnorm_backward", "launch_im2col", "launch_col2im",
        "launch_spatial_add", "launch_spatial_reduce_sum", "launch_spatial_modulate",
        "launch_spatial_modulate_backward",
    }
    assert ref_names <= set(nn.header_functions())


def test_launchers_keep_reference_argument_order(nn):
    """Argument lists of the reference-named launchers: same count and kinds
    (pointer / int / float), with the stream last."""
    text = (ROOT / "include" / "nn_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    sig = {m.group(1): [a.strip() for a in m.group(2).split(",")]
           for m in re.finditer(r"void\s+(launch_\w+)\s*\(([^;]*)\)\s*;", text)}
    expect = {
        # kinds per argument: p = pointer, i = int, f = float, s = stream (reference nn.h:348-466)
        "launch_groupnorm_forward": "ppppppiiiifs",
        "launch_groupnorm_backward": "ppppppppiiiis",
        "launch_layernorm_forward": "ppppppiifs",
        "launch_layernorm_backward": "ppppppppiis",
        "launch_activation_forward": "ppiis",
        "launch_activation_backward": "pppiis",
        "launch_adam_step": "ppppffffffis",
        "launch_weight_normalize": "piifs",
        "launch_weight_normalize_backward": "ppppiis",
        "launch_weighted_sum": "pppffis",
        "launch_mp_sum": "pppfis",
        "launch_mp_cat": "pppfiiis",
        "launch_mp_channel_cat": "pppfiiis",
        "launch_mp_channel_split": "pppfiiis",
        "launch_mp_fourier": "ppppiis",
        "launch_sinusoidal": "ppiifs",
        "launch_im2col": "ppiiiiiiiiis",
        "launch_col2im": "ppiiiiiiiiis",
        "launch_add_bias": "ppiis",
        "launch_bias_grad": "ppiis",
        "launch_sgd_step": "ppfis",
        "launch_scale_by_scalar": "ppis",
        "launch_spatial_add": "ppiiiis",
        "launch_spatial_reduce_sum": "ppiiis",
        "launch_spatial_modulate": "pppiiiis",
        "launch_spatial_modulate_backward": "pppppiiiis",
    }

    def kind(a: str) -> str:
        if "hipStream_t" in a:
            return "s"
        if "*" in a:
            return "p"
        if a.startswith("float"):
            return "f"
        return "i"  # int and the Activation enum

    for name, k in expect.items():
        got = "".join(kind(a) for a in sig[name])
        assert got == k, (name, got, k)


def test_reference_call_sites_compile_against_the_header():
    """tests/refcalls.c: the reference's launcher prototypes (src/nn.h:354-456)
    with the stream re-typed to hipStream_t, each launcher of include/nn_hip.h
    assigned to a pointer of that exact type, and call sites written as the
    reference's host modules write them (src/groupnorm.c:16, 27,
    src/layernorm.c:16, 26, src/activation.c:12, 21, src/mp_linear.c:16-38,
    src/conv2d.c:24-64, src/optimizer.c:58, 66, src/ema.c:32, ...), compiled
    with -Werror: no compatibility header, no cast."""
    cmd = ["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROOT / 'include'}", "-I/opt/rocm/include", str(ROOT / "tests" / "refcalls.c")]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]


def test_host_refusals_record_an_error(nn):
    """Shapes the kernels cannot take are refused on the host and recorded in
    the error record (the reference would launch and read out of bounds).
    Each case must be refused by the host check itself, before any launch:
    the pointers are dummies that a kernel would fault on, so the test checks
    for the refusal's own code and message (a launch that failed for another
    reason, such as no device here, would not match)."""
    L = nn.lib()
    L.last_error()  # clear
    dummy = ctypes.c_void_p(16)  # never dereferenced: the shape check comes first
    cases = [
        ("launch_groupnorm_forward", (dummy, dummy, dummy, dummy, dummy, dummy, 1, 4, 10, 4, 1e-5, None),
         "is not divisible by G"),
        ("launch_groupnorm_act_forward", (dummy, dummy, dummy, dummy, dummy, dummy, 1, 4, 8, 4, 1e-5, 99, None),
         "unknown activation 99"),
        ("launch_layernorm_forward", (dummy, dummy, dummy, dummy, dummy, dummy, 2, 0, 1e-5, None), "bad shape"),
        # K = 0 (an H_out that does not match H, K, stride and pad is not refused:
        # the reference trusts it too, and the kernels bounds-check the image side)
        ("launch_im2col", (dummy, dummy, 1, 4, 4, 2, 0, 1, 1, 4, 4, None), "bad geometry"),
        ("launch_sinusoidal", (dummy, dummy, 2, 1, 9.2, None), "bad shape"),
        ("launch_weight_normalize", (dummy, -1, 4, 1e-4, None), "bad shape"),
    ]
    for name, args, text in cases:
        with pytest.raises(nn.NnHipError, match=f"{name}: error 1: {name}: .*{text}"):
            L.call(name, *args)
    code, _ = L.last_error()
    assert code == 0  # the record is cleared by each read


def test_zero_sized_calls_are_no_ops(nn):
    L = nn.lib()
    null = None
    L.launch_activation_forward(null, null, 0, nn.ACT_SILU, None)
    L.launch_weighted_sum(null, null, null, 1.0, 2.0, 0, None)
    L.launch_mp_fourier(null, null, null, null, 0, 16, None)
    L.launch_im2col(null, null, 0, 4, 4, 2, 3, 1, 1, 4, 4, None)
    assert L.last_error()[0] == 0


@pytest.mark.parametrize("hw,c", [(2048, 128), (1024, 128), (4096, 256), (49, 6), (5000, 3), (7, 192)])
def test_spatial_workspace_grows_with_batch(nn, hw, c):
    """A workspace sized for a batch must serve every smaller batch (the host
    modules size theirs for the largest batch), so the reported size may never
    fall as the batch grows; the segment count per sample alone does not give
    that (b * ceil(2048 / b) is 2142 at b = 102 and 2060 at b = 103)."""
    L = nn.lib()
    sizes = [L.nnhip_spatial_reduce_workspace(b, hw, c) for b in range(1, 300)]
    assert all(a <= b for a, b in zip(sizes, sizes[1:])), sizes


@pytest.mark.parametrize("c", [4, 48, 64, 256, 1000])
def test_layernorm_workspace_grows_with_batch(nn, c):
    L = nn.lib()
    sizes = [L.nnhip_layernorm_backward_workspace(b, c) for b in list(range(1, 200)) + [4095, 4096, 4097, 65536]]
    assert all(a <= b for a, b in zip(sizes, sizes[1:])), sizes
