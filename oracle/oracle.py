"""numpy wrappers over oracle/_build/liboracle.so (the CPU restatement).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the reported CPU baseline.
Each wrapper names the oracle.c function (and through it the reference lines)
it calls.  Arrays are float32, C-contiguous, NHWC.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "liboracle.so"

P, I, F, LL = C.c_void_p, C.c_int, C.c_float, C.c_longlong
_SIGS = {
    "orc_pade_tanh": (F, [F]),
    "orc_pade_sigmoid": (F, [F]),
    "orc_act": (F, [F, I]),
    "orc_act_grad": (F, [F, I]),
    "orc_activation_forward": (None, [P, P, LL, I]),
    "orc_activation_backward": (None, [P, P, P, LL, I]),
    "orc_weighted_sum": (None, [P, P, P, F, F, LL]),
    "orc_mp_sum_weights": (None, [F, P, P]),
    "orc_mp_cat_weights": (None, [F, I, I, P, P]),
    "orc_mp_cat": (None, [P, P, P, F, F, LL, I, I]),
    "orc_mp_split": (None, [P, P, P, F, F, LL, I, I]),
    "orc_scale_by_scalar": (None, [P, F, LL]),
    "orc_add_bias": (None, [P, P, LL, I]),
    "orc_bias_grad": (None, [P, P, LL, I]),
    "orc_sgd_step": (None, [P, P, F, LL]),
    "orc_adam_step": (None, [P, P, P, P, F, F, F, F, F, F, LL]),
    "orc_adam_bias_corrections": (None, [F, F, I, P, P]),
    "orc_groupnorm_forward": (None, [P, P, P, P, P, P, I, I, I, I, F, I]),
    "orc_groupnorm_backward": (None, [P, P, P, P, P, P, P, P, P, I, I, I, I, I]),
    "orc_layernorm_forward": (None, [P, P, P, P, P, P, LL, I, F]),
    "orc_layernorm_backward": (None, [P, P, P, P, P, P, P, P, LL, I]),
    "orc_weight_normalize": (None, [P, I, I, F]),
    "orc_weight_normalize_backward": (None, [P, P, F, P, I, I]),
    "orc_mp_fourier": (None, [P, P, P, P, I, I]),
    "orc_sinusoidal": (None, [P, P, I, I, F]),
    "orc_im2col": (None, [P, P, I, I, I, I, I, I, I, I, I]),
    "orc_col2im": (None, [P, P, I, I, I, I, I, I, I, I, I]),
    "orc_spatial_add": (None, [P, P, I, I, I]),
    "orc_spatial_reduce_sum": (None, [P, P, I, I, I]),
    "orc_spatial_modulate": (None, [P, P, P, I, I, I]),
    "orc_spatial_modulate_backward": (None, [P, P, P, P, P, I, I, I]),
    "orc_spatial_modulate_act_forward": (None, [P, P, P, I, I, I, I]),
    "orc_spatial_modulate_act_backward": (None, [P, P, P, P, P, I, I, I, I]),
    "orc_set_threads": (None, [I]),
    "orc_get_threads": (I, []),
    "orc_groupnorm_forward_f32": (None, [P, P, P, P, P, P, I, I, I, I, F, I]),
    "orc_groupnorm_backward_f32": (None, [P, P, P, P, P, P, P, P, P, I, I, I, I, I]),
}

_dll = None


def dll():
    global _dll
    if _dll is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        d = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(d, name)
            fn.restype = res
            fn.argtypes = args
        _dll = d
    return _dll


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


# ---------------- scalar / elementwise ----------------
def pade_tanh(x: float) -> float:
    return dll().orc_pade_tanh(x)


def act_forward(x, act: int) -> np.ndarray:
    x = _f(x)
    out = np.empty_like(x)
    dll().orc_activation_forward(_p(out), _p(x), x.size, act)
    return out


def act_backward(gout, z, act: int) -> np.ndarray:
    gout, z = _f(gout), _f(z)
    out = np.empty_like(z)
    dll().orc_activation_backward(_p(out), _p(gout), _p(z), z.size, act)
    return out


def weighted_sum(a, b, wa: float, wb: float) -> np.ndarray:
    a, b = _f(a), _f(b)
    out = np.empty_like(a)
    dll().orc_weighted_sum(_p(out), _p(a), _p(b), wa, wb, a.size)
    return out


def mp_sum_weights(t: float) -> tuple[float, float]:
    wa, wb = C.c_float(), C.c_float()
    dll().orc_mp_sum_weights(t, C.byref(wa), C.byref(wb))
    return wa.value, wb.value


def mp_cat_weights(t: float, na: int, nb: int) -> tuple[float, float]:
    wa, wb = C.c_float(), C.c_float()
    dll().orc_mp_cat_weights(t, na, nb, C.byref(wa), C.byref(wb))
    return wa.value, wb.value


def mp_cat(a, b, t: float) -> np.ndarray:
    """a [R, Na], b [R, Nb] -> [R, Na+Nb]"""
    a, b = _f(a), _f(b)
    R, Na = a.shape[0], a.shape[-1]
    Nb = b.shape[-1]
    wa, wb = mp_cat_weights(t, Na, Nb)
    out = np.empty((R, Na + Nb), np.float32)
    dll().orc_mp_cat(_p(out), _p(a), _p(b), wa, wb, R, Na, Nb)
    return out


def mp_split(g, Ca: int, Cb: int, t: float) -> tuple[np.ndarray, np.ndarray]:
    g = _f(g)
    R = g.size // (Ca + Cb)
    wa, wb = mp_cat_weights(t, Ca, Cb)
    ga = np.empty((R, Ca), np.float32)
    gb = np.empty((R, Cb), np.float32)
    dll().orc_mp_split(_p(ga), _p(gb), _p(g), wa, wb, R, Ca, Cb)
    return ga, gb


def scale_by_scalar(x, s: float) -> np.ndarray:
    x = _f(x).copy()
    dll().orc_scale_by_scalar(_p(x), s, x.size)
    return x


def add_bias(Y, b) -> np.ndarray:
    Y, b = _f(Y).copy(), _f(b)
    dll().orc_add_bias(_p(Y), _p(b), Y.size // b.size, b.size)
    return Y


def bias_grad(g, N: int) -> np.ndarray:
    g = _f(g)
    out = np.empty(N, np.float32)
    dll().orc_bias_grad(_p(out), _p(g), g.size // N, N)
    return out


def sgd_step(p, g, lr: float) -> np.ndarray:
    p, g = _f(p).copy(), _f(g)
    dll().orc_sgd_step(_p(p), _p(g), lr, p.size)
    return p


def adam_bias_corrections(b1: float, b2: float, t: int) -> tuple[float, float]:
    bc1, bc2 = C.c_float(), C.c_float()
    dll().orc_adam_bias_corrections(b1, b2, t, C.byref(bc1), C.byref(bc2))
    return bc1.value, bc2.value


def adam_step(p, m, v, g, lr, b1, b2, eps, bc1, bc2):
    """In-place copy semantics: returns new (p, m, v)."""
    p, m, v, g = _f(p).copy(), _f(m).copy(), _f(v).copy(), _f(g)
    dll().orc_adam_step(_p(p), _p(m), _p(v), _p(g), lr, b1, b2, eps, bc1, bc2, p.size)
    return p, m, v


# ---------------- normalisation ----------------
def groupnorm_forward(x, gamma, beta, G: int, eps: float = 1e-5, act: int = 0):
    """x [B, HW, C] -> (y, mu [B*G], rstd [B*G])"""
    x, gamma, beta = _f(x), _f(gamma), _f(beta)
    B, HW, Cc = x.shape
    y = np.empty_like(x)
    mu = np.empty(B * G, np.float32)
    rs = np.empty(B * G, np.float32)
    dll().orc_groupnorm_forward(_p(y), _p(mu), _p(rs), _p(x), _p(gamma), _p(beta), B, HW, Cc, G, eps, act)
    return y, mu, rs


def groupnorm_backward(dy, x, gamma, beta, mu, rstd, G: int, act: int = 0):
    dy, x, gamma, beta, mu, rstd = map(_f, (dy, x, gamma, beta, mu, rstd))
    B, HW, Cc = x.shape
    dx = np.empty_like(x)
    gg = np.empty(Cc, np.float32)
    gb = np.empty(Cc, np.float32)
    dll().orc_groupnorm_backward(_p(dx), _p(gg), _p(gb), _p(dy), _p(x), _p(gamma), _p(beta), _p(mu),
                                 _p(rstd), B, HW, Cc, G, act)
    return dx, gg, gb


def groupnorm_forward_f32(x, gamma, beta, G: int, eps: float = 1e-5, act: int = 0):
    x, gamma, beta = _f(x), _f(gamma), _f(beta)
    B, HW, Cc = x.shape
    y = np.empty_like(x)
    mu = np.empty(B * G, np.float32)
    rs = np.empty(B * G, np.float32)
    dll().orc_groupnorm_forward_f32(_p(y), _p(mu), _p(rs), _p(x), _p(gamma), _p(beta), B, HW, Cc, G, eps, act)
    return y, mu, rs


def groupnorm_backward_f32(dy, x, gamma, beta, mu, rstd, G: int, act: int = 0):
    dy, x, gamma, beta, mu, rstd = map(_f, (dy, x, gamma, beta, mu, rstd))
    B, HW, Cc = x.shape
    dx = np.empty_like(x)
    gg = np.empty(Cc, np.float32)
    gb = np.empty(Cc, np.float32)
    dll().orc_groupnorm_backward_f32(_p(dx), _p(gg), _p(gb), _p(dy), _p(x), _p(gamma), _p(beta), _p(mu),
                                     _p(rstd), B, HW, Cc, G, act)
    return dx, gg, gb


def layernorm_forward(x, gamma, beta, eps: float = 1e-5):
    x, gamma, beta = _f(x), _f(gamma), _f(beta)
    R, Cc = x.shape
    y = np.empty_like(x)
    mu = np.empty(R, np.float32)
    rs = np.empty(R, np.float32)
    dll().orc_layernorm_forward(_p(y), _p(mu), _p(rs), _p(x), _p(gamma), _p(beta), R, Cc, eps)
    return y, mu, rs


def layernorm_backward(dy, x, gamma, mu, rstd):
    dy, x, gamma, mu, rstd = map(_f, (dy, x, gamma, mu, rstd))
    R, Cc = x.shape
    dx = np.empty_like(x)
    gg = np.empty(Cc, np.float32)
    gb = np.empty(Cc, np.float32)
    dll().orc_layernorm_backward(_p(dx), _p(gg), _p(gb), _p(dy), _p(x), _p(gamma), _p(mu), _p(rstd), R, Cc)
    return dx, gg, gb


# ---------------- weight norm ----------------
def weight_normalize(W, eps: float = 1e-4) -> np.ndarray:
    W = _f(W).copy()
    dll().orc_weight_normalize(_p(W), W.shape[0], W.shape[1], eps)
    return W


def weight_normalize_backward(gW, Wn, gain: float, g_gain_in: float = 0.0):
    gW, Wn = _f(gW).copy(), _f(Wn)
    gg = np.array([g_gain_in], np.float32)
    dll().orc_weight_normalize_backward(_p(gW), _p(Wn), gain, _p(gg), Wn.shape[0], Wn.shape[1])
    return gW, float(gg[0])


# ---------------- embeddings ----------------
def mp_fourier(x, freqs, phases) -> np.ndarray:
    x, freqs, phases = _f(x), _f(freqs), _f(phases)
    out = np.empty((x.size, freqs.size), np.float32)
    dll().orc_mp_fourier(_p(out), _p(x), _p(freqs), _p(phases), x.size, freqs.size)
    return out


def sinusoidal(t, Cc: int, log_max_period: float) -> np.ndarray:
    t = _f(t)
    out = np.empty((t.size, Cc), np.float32)
    dll().orc_sinusoidal(_p(out), _p(t), t.size, Cc, log_max_period)
    return out


# ---------------- conv ----------------
def conv_out(H: int, K: int, stride: int, pad: int) -> int:
    return (H + 2 * pad - K) // stride + 1


def im2col(im, K: int, stride: int, pad: int) -> np.ndarray:
    im = _f(im)
    B, H, W, Cc = im.shape
    Ho, Wo = conv_out(H, K, stride, pad), conv_out(W, K, stride, pad)
    col = np.empty((B * Ho * Wo, K * K * Cc), np.float32)
    dll().orc_im2col(_p(col), _p(im), B, H, W, Cc, K, stride, pad, Ho, Wo)
    return col


def col2im(col, shape, K: int, stride: int, pad: int, init=None) -> np.ndarray:
    col = _f(col)
    B, H, W, Cc = shape
    Ho, Wo = conv_out(H, K, stride, pad), conv_out(W, K, stride, pad)
    out = np.zeros(shape, np.float32) if init is None else _f(init).copy()
    dll().orc_col2im(_p(out), _p(col), B, H, W, Cc, K, stride, pad, Ho, Wo)
    return out


def spatial_add(x, v) -> np.ndarray:
    """x [B, HW, C] + v [B, C] broadcast over HW (orc_spatial_add)."""
    out = _f(x).copy()
    B, HW, Cc = out.shape
    dll().orc_spatial_add(_p(out), _p(_f(v)), B, HW, Cc)
    return out


def spatial_reduce_sum(x) -> np.ndarray:
    """[B, HW, C] -> [B, C] sums over HW (orc_spatial_reduce_sum, double accumulation)."""
    x = _f(x)
    B, HW, Cc = x.shape
    out = np.empty((B, Cc), np.float32)
    dll().orc_spatial_reduce_sum(_p(out), _p(x), B, HW, Cc)
    return out


def spatial_modulate(x, cond) -> np.ndarray:
    x = _f(x)
    B, HW, Cc = x.shape
    out = np.empty_like(x)
    dll().orc_spatial_modulate(_p(out), _p(x), _p(_f(cond)), B, HW, Cc)
    return out


def spatial_modulate_backward(gout, x, cond) -> tuple[np.ndarray, np.ndarray]:
    gout, x = _f(gout), _f(x)
    B, HW, Cc = x.shape
    gin, gc = np.empty_like(x), np.empty((B, Cc), np.float32)
    dll().orc_spatial_modulate_backward(_p(gin), _p(gc), _p(gout), _p(x), _p(_f(cond)), B, HW, Cc)
    return gin, gc


def spatial_modulate_act_forward(x, cond, act: int) -> np.ndarray:
    x = _f(x)
    B, HW, Cc = x.shape
    out = np.empty_like(x)
    dll().orc_spatial_modulate_act_forward(_p(out), _p(x), _p(_f(cond)), B, HW, Cc, act)
    return out


def spatial_modulate_act_backward(gout, x, cond, act: int) -> tuple[np.ndarray, np.ndarray]:
    gout, x = _f(gout), _f(x)
    B, HW, Cc = x.shape
    gin, gc = np.empty_like(x), np.empty((B, Cc), np.float32)
    dll().orc_spatial_modulate_act_backward(_p(gin), _p(gc), _p(gout), _p(x), _p(_f(cond)), B, HW, Cc, act)
    return gin, gc


def set_threads(n: int) -> None:
    dll().orc_set_threads(n)


def get_threads() -> int:
    return dll().orc_get_threads()
