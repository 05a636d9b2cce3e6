"""Python binding of the MI355X fused-layer-kernel library (lib/libnnhip.so).

The library is the product: gfx950 HIP kernels behind the C-ABI launch layer
of ``include/nn_hip.h`` (the reference's ``launch_*`` entry points, reference
src/nn.h:348-466) plus the C host modules of ``include/nn_modules.h``.  This
module only binds that C-ABI with ctypes so that Python tests and the bench
can drive it; device memory, copies, streams and events come from the
library's own plumbing (``include/nn_hip_rt.h``), so no other GPU runtime is
loaded into the process.  Every launcher call is followed by a read of the
library's error record and raises :class:`NnHipError` on failure.

The package directory name is not a Python identifier; load it with
``load_package()`` from the repository root helpers (tests/conftest.py,
bench.py, __graft_entry__.py) which import it as ``cuda_c_diffusion_amd``.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
LIB_PATH = PKG_DIR / "lib" / "libnnhip.so"
INCLUDE_DIR = REPO_DIR / "include"

# Activation kinds (reference src/nn.h:178-183)
ACT_IDENTITY, ACT_RELU, ACT_GELU, ACT_SILU, ACT_TANH, ACT_MP_SILU = range(6)
ACT_NAMES = {"identity": 0, "relu": 1, "gelu": 2, "silu": 3, "tanh": 4, "mp_silu": 5}


class NnHipError(RuntimeError):
    """A launcher refused its arguments or a HIP call failed."""


P = C.c_void_p
I = C.c_int
F = C.c_float
SZ = C.c_size_t
LL = C.c_longlong

# name -> (restype, argtypes, is_launcher)
_SIGS = {
    # runtime plumbing (nn_hip_rt.h)
    "nnhip_get_last_error": (I, [C.c_char_p, I], False),
    "nnhip_launch_allocations": (C.c_ulonglong, [], False),
    "nnhip_rng_seed": (None, [P, C.c_uint64], False),
    "nnhip_fill_normal": (I, [P, P, SZ, F, F], False),
    "nnhip_fill_uniform": (I, [P, P, SZ], False),
    "nnhip_device_count": (I, [], False),
    "nnhip_set_device": (I, [I], False),
    "nnhip_device_info": (I, [C.c_char_p, I], False),
    "nnhip_malloc": (P, [SZ], False),
    "nnhip_free": (I, [P], False),
    "nnhip_memcpy_htod": (I, [P, P, SZ], False),
    "nnhip_memcpy_dtoh": (I, [P, P, SZ], False),
    "nnhip_memcpy_dtod": (I, [P, P, SZ], False),
    "nnhip_memset": (I, [P, I, SZ], False),
    "nnhip_memset_async": (I, [P, I, SZ, P], False),
    "nnhip_device_synchronize": (I, [], False),
    "nnhip_stream_create": (P, [], False),
    "nnhip_stream_destroy": (I, [P], False),
    "nnhip_stream_scratch_release": (None, [P], False),
    "nnhip_graph_capture_begin": (I, [P], False),
    "nnhip_graph_capture_end": (P, [P], False),
    "nnhip_graph_launch": (I, [P, P], False),
    "nnhip_graph_destroy": (I, [P], False),
    "nnhip_stream_synchronize": (I, [P], False),
    "nnhip_event_create": (P, [], False),
    "nnhip_event_destroy": (I, [P], False),
    "nnhip_event_record": (I, [P, P], False),
    "nnhip_event_synchronize": (I, [P], False),
    "nnhip_event_elapsed_ms": (F, [P, P], False),
    "nnhip_copy_f32": (None, [P, P, SZ, P], True),
    "nnhip_fill_f32": (None, [P, F, SZ, P], True),
    "launch_spatial_add": (None, [P, P, I, I, I, I, P], True),
    "launch_spatial_reduce_sum": (None, [P, P, I, I, I, P], True),
    "launch_spatial_modulate": (None, [P, P, P, I, I, I, I, P], True),
    "launch_spatial_modulate_backward": (None, [P, P, P, P, P, I, I, I, I, P], True),
    "launch_spatial_modulate_act_forward": (None, [P, P, P, I, I, I, I, I, P], True),
    "launch_spatial_modulate_act_backward": (None, [P, P, P, P, P, I, I, I, I, I, P, P], True),
    "launch_spatial_reduce_sum_ws": (None, [P, P, I, I, I, P, P], True),
    "nnhip_spatial_reduce_workspace": (SZ, [I, I, I], False),
    "launch_conv2d_forward_implicit": (None, [P, P, P, P, P] + [I] * 10 + [P], True),
    "nnhip_conv2d_implicit_supported": (I, [I, I], False),
    "launch_conv2d_input_grad_implicit": (None, [P, P, P, P] + [I] * 7 + [P], True),
    "nnhip_conv2d_input_grad_implicit_supported": (I, [I] * 5, False),
    "launch_conv2d_weight_grad_implicit": (None, [P, P, P] + [I] * 10 + [P, P], True),
    "nnhip_conv2d_wgrad_implicit_supported": (I, [I, I], False),
    "nnhip_conv2d_wgrad_workspace": (SZ, [I] * 6, False),
    "launch_conv2d_forward_implicit_fused": (None, [P, P, P, P, P] + [I] * 10 + [P, P], True),
    "launch_conv2d_input_grad_implicit_fused": (None, [P, P, P, P] + [I] * 7 + [P, P], True),
    # launch layer (nn_hip.h)
    "launch_add_bias": (None, [P, P, I, I, P], True),
    "launch_bias_grad": (None, [P, P, I, I, P], True),
    "launch_sgd_step": (None, [P, P, F, I, P], True),
    "launch_activation_forward": (None, [P, P, I, I, P], True),
    "launch_activation_backward": (None, [P, P, P, I, I, P], True),
    "launch_adam_step": (None, [P, P, P, P, F, F, F, F, F, F, I, P], True),
    "launch_weight_normalize": (None, [P, I, I, F, P], True),
    "launch_weight_normalize_backward": (None, [P, P, P, P, I, I, P], True),
    "launch_weight_normalize_backward_ws": (None, [P, P, P, P, I, I, P, P], True),
    "nnhip_weight_normalize_backward_workspace": (SZ, [I], False),
    "launch_scale_by_scalar": (None, [P, P, I, P], True),
    "launch_mp_sum": (None, [P, P, P, F, I, P], True),
    "launch_weighted_sum": (None, [P, P, P, F, F, I, P], True),
    "launch_mp_cat": (None, [P, P, P, F, I, I, I, P], True),
    "launch_mp_channel_cat": (None, [P, P, P, F, I, I, I, P], True),
    "launch_mp_channel_split": (None, [P, P, P, F, I, I, I, P], True),
    "launch_mp_fourier": (None, [P, P, P, P, I, I, P], True),
    "launch_sinusoidal": (None, [P, P, I, I, F, P], True),
    "launch_layernorm_forward": (None, [P, P, P, P, P, P, I, I, F, P], True),
    "launch_layernorm_backward": (None, [P, P, P, P, P, P, P, P, I, I, P], True),
    "launch_groupnorm_forward": (None, [P, P, P, P, P, P, I, I, I, I, F, P], True),
    "launch_groupnorm_backward": (None, [P, P, P, P, P, P, P, P, I, I, I, I, P], True),
    "launch_im2col": (None, [P, P, I, I, I, I, I, I, I, I, I, P], True),
    "launch_col2im": (None, [P, P, I, I, I, I, I, I, I, I, I, P], True),
    "launch_groupnorm_act_forward": (None, [P, P, P, P, P, P, I, I, I, I, F, I, P], True),
    "launch_groupnorm_act_backward": (None, [P, P, P, P, P, P, P, P, P, I, I, I, I, I, P], True),
    "nnhip_groupnorm_forward_workspace": (SZ, [I, I, I, I], False),
    "nnhip_groupnorm_backward_workspace": (SZ, [I, I, I, I], False),
    "nnhip_groupnorm_workspace_status": (I, [P], False),
    "launch_groupnorm_act_forward_ws": (None, [P, P, P, P, P, P, I, I, I, I, F, I, P, P], True),
    "nnhip_layernorm_backward_workspace": (SZ, [I, I], False),
    "launch_groupnorm_act_backward_ws": (None, [P, P, P, P, P, P, P, P, P, I, I, I, I, I, P, P], True),
    "launch_groupnorm_act_backward_noalloc": (None, [P, P, P, P, P, P, P, P, P, I, I, I, I, I, P], True),
    "launch_groupnorm_act_shift_forward_ws": (None, [P, P, P, P, P, P, P, I, I, I, I, F, I, P, P], True),
    "launch_groupnorm_act_shift_backward_ws": (None, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, P, P], True),
    "nnhip_groupnorm_shift_backward_workspace": (SZ, [I, I, I, I], False),
    "nnhip_groupnorm_shift_supported": (I, [I, I, I, I, I], False),
    "launch_layernorm_backward_ws": (None, [P, P, P, P, P, P, P, P, I, I, P, P], True),
    "launch_col2im_set": (None, [P, P, I, I, I, I, I, I, I, I, I, P], True),
    "nnhip_multi_tensor_plan_create": (P, [P, I], True),
    "nnhip_multi_tensor_plan_destroy": (None, [P], False),
    "launch_adam_ema_step": (None, [P, F, F, F, F, F, F, F, F, P], True),
    "launch_ema_update": (None, [P, F, F, P], True),
}


class NnTensorSlot(C.Structure):
    """Mirror of NnTensorSlot in include/nn_hip.h."""

    _fields_ = [("p", P), ("m", P), ("v", P), ("g", P), ("shadow", P), ("n", LL)]


class NnConvFusion(C.Structure):
    """Mirror of NnConvFusion in include/nn_hip.h (pass C.addressof(f))."""

    _fields_ = [("res", P), ("res_w", C.c_float), ("out_w", C.c_float), ("cond", P), ("y2", P),
                ("act_in", P), ("act", C.c_int)]


def header_functions() -> list[str]:
    """Every function name declared in include/*.h (the exported C-ABI)."""
    names: list[str] = []
    for h in sorted(INCLUDE_DIR.glob("*.h")):
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = text.replace("\\\n", " ")  # join macro continuation lines
        text = re.sub(r"^\s*#[^\n]*", "", text, flags=re.M)
        for m in re.finditer(r"\b([A-Za-z_][A-Za-z0-9_]*)\s*\(([^;{}]*)\)\s*;", text):
            name = m.group(1)
            if name in ("if", "while", "for", "return", "sizeof"):
                continue
            if m.group(2).lstrip().startswith("*"):  # function-pointer member: void (*f)(...)
                continue
            names.append(name)
    return names


class Lib:
    """Loaded libnnhip.so with checked launchers and device-memory helpers."""

    def __init__(self, path: Path | str = LIB_PATH):
        path = Path(path)
        if not path.exists():
            raise NnHipError(
                f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')"
            )
        self.path = path
        self.dll = C.CDLL(str(path), mode=C.RTLD_GLOBAL)
        for name, (res, args, _) in _SIGS.items():
            fn = getattr(self.dll, name)
            fn.restype = res
            fn.argtypes = args
        self._buf = C.create_string_buffer(1024)

    # ---- errors ----
    def last_error(self) -> tuple[int, str]:
        code = self.dll.nnhip_get_last_error(self._buf, len(self._buf))
        return code, self._buf.value.decode(errors="replace")

    def check(self, what: str = "") -> None:
        code, msg = self.last_error()
        if code:
            raise NnHipError(f"{what or 'nnhip'}: error {code}: {msg}")

    def call(self, name: str, *args):
        res = getattr(self.dll, name)(*args)
        if _SIGS[name][2]:
            self.check(name)
        return res

    def __getattr__(self, name: str):
        if name in _SIGS:
            return lambda *a: self.call(name, *a)
        raise AttributeError(name)

    # ---- device ----
    def device_count(self) -> int:
        return int(self.dll.nnhip_device_count())

    def device_info(self) -> dict:
        buf = C.create_string_buffer(512)
        rc = self.dll.nnhip_device_info(buf, 512)
        if rc:
            raise NnHipError(f"nnhip_device_info: {rc}")
        name, arch, cus, mem = buf.value.decode().split("|")
        return {"name": name, "arch": arch, "cus": int(cus), "mem_bytes": int(mem)}

    def sync(self) -> None:
        rc = self.dll.nnhip_device_synchronize()
        if rc:
            raise NnHipError(f"hipDeviceSynchronize failed: {rc}")

    def alloc(self, n_floats: int) -> "DeviceArray":
        return DeviceArray(self, int(n_floats))

    def to_device(self, host: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(host, dtype=np.float32)
        d = DeviceArray(self, a.size)
        d.upload(a)
        return d


class DeviceArray:
    """fp32 device buffer owned by Python (freed on close / garbage collection)."""

    def __init__(self, lib: Lib, n: int):
        self.lib = lib
        self.n = n
        self.ptr = lib.dll.nnhip_malloc(max(n, 1) * 4)
        if not self.ptr:
            raise NnHipError(f"hipMalloc of {n} floats failed")

    @property
    def p(self) -> int:
        return self.ptr

    def offset(self, k: int) -> int:
        """Device address of element k (for sub-tensor and misalignment tests)."""
        return self.ptr + 4 * int(k)

    def upload(self, host: np.ndarray) -> None:
        a = np.ascontiguousarray(host, dtype=np.float32)
        assert a.size <= self.n
        rc = self.lib.dll.nnhip_memcpy_htod(self.ptr, a.ctypes.data, a.nbytes)
        if rc:
            raise NnHipError(f"hipMemcpy H2D failed: {rc}")

    def download(self, n: int | None = None, shape=None) -> np.ndarray:
        n = self.n if n is None else n
        out = np.empty(n, dtype=np.float32)
        rc = self.lib.dll.nnhip_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes)
        if rc:
            raise NnHipError(f"hipMemcpy D2H failed: {rc}")
        return out.reshape(shape) if shape is not None else out

    def fill_bytes(self, value: int = 0) -> None:
        rc = self.lib.dll.nnhip_memset(self.ptr, value, self.n * 4)
        if rc:
            raise NnHipError(f"hipMemset failed: {rc}")

    def close(self) -> None:
        if self.ptr:
            self.lib.dll.nnhip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_LIB: Lib | None = None


def lib() -> Lib:
    """The process-wide loaded library (loaded on first use)."""
    global _LIB
    if _LIB is None:
        _LIB = Lib()
    return _LIB


def make_plan(L: Lib, slots: list[dict]) -> int:
    """Build an NnMultiTensorPlan from dicts with keys p, m, v, g, shadow, n."""
    arr = (NnTensorSlot * max(len(slots), 1))()
    for i, s in enumerate(slots):
        arr[i] = NnTensorSlot(s.get("p"), s.get("m"), s.get("v"), s.get("g"), s.get("shadow"), int(s["n"]))
    plan = L.call("nnhip_multi_tensor_plan_create", C.cast(arr, P), len(slots))
    if not plan:
        L.check("nnhip_multi_tensor_plan_create")
        raise NnHipError("plan creation failed")
    return plan


def mp_sum_weights(t: float) -> tuple[float, float]:
    """Host-float mp_sum weights exactly as the launcher forms them (kernels.cu:363-364)."""
    f = np.float32
    t = f(t)
    d = np.sqrt(f(f(f(1) - t) * f(f(1) - t)) + f(t * t), dtype=np.float32)
    return float(f(f(1) - t) / d), float(f(t / d))


def env_flag(name: str) -> bool:
    return os.environ.get(name, "") not in ("", "0")
