"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is independent of the oracle's own formulas: coefficients derived
again from the continued fraction, torch on the CPU where the maths coincide
(group_norm, layer_norm, autograd, unfold/fold, Adam, lerp), closed forms and
invariants, brute force on tiny integer-valued inputs, and the reference's own
finite-difference gradcheck (reference tests/gradcheck.c:15-21, 51-56).
A planted mistake (dropped term, wrong sign or index, swapped operand) fails
at least one of them.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import TOL, rel_err

torch.set_num_threads(4)

IDENT, RELU, GELU, SILU, TANH, MP_SILU = range(6)


# ---------------------------------------------------------------------------
# Pade tanh (reference src/kernels.cu:6-17)
# ---------------------------------------------------------------------------
def _poly_mul(a, b):
    out = [Fraction(0)] * (len(a) + len(b) - 1)
    for i, x in enumerate(a):
        for j, y in enumerate(b):
            out[i + j] += x * y
    return out


def _poly_add(a, b):
    n = max(len(a), len(b))
    return [(a[i] if i < len(a) else 0) + (b[i] if i < len(b) else 0) for i in range(n)]


def test_pade_coefficients_from_lambert_continued_fraction():
    """tanh x = x / (1 + x^2/(3 + x^2/(5 + ... + x^2/13))) (Lambert's continued
    fraction cut after the 13): as N/D in u = x^2, scaled so that the
    denominator's constant is 135135, gives the constants of kernels.cu:8-9."""
    num, den = [Fraction(13)], [Fraction(1)]  # the tail 13 as num/den
    for k in (11, 9, 7, 5, 3, 1):
        # k + u / (num/den) = (k*num + u*den) / num
        new_num = _poly_add([Fraction(k) * c for c in num], [Fraction(0)] + den)
        num, den = new_num, num
    # tanh = x * den / num
    scale = Fraction(135135) / num[0]
    p = [c * scale for c in den]
    q = [c * scale for c in num]
    assert p == [135135, 17325, 378, 1]
    assert q == [135135, 62370, 3150, 28]


def test_pade_tanh_properties(orc):
    xs = np.linspace(-2, 2, 401, dtype=np.float32)
    t = np.array([orc.pade_tanh(float(v)) for v in xs])
    assert np.max(np.abs(t - np.tanh(xs.astype(np.float64)))) < 2e-6
    # odd, clamped, saturates at exactly +-1 for large |x|
    assert all(orc.pade_tanh(float(v)) == -orc.pade_tanh(float(-v)) for v in xs)
    assert orc.pade_tanh(30.0) == 1.0 and orc.pade_tanh(-30.0) == -1.0
    assert orc.pade_tanh(0.0) == 0.0


@pytest.mark.parametrize("act,torch_fn", [
    (SILU, F.silu),
    (GELU, lambda v: F.gelu(v, approximate="tanh")),
    (TANH, torch.tanh),
    (RELU, F.relu),
    (IDENT, lambda v: v),
])
def test_activation_forward_vs_torch_where_pade_is_exact(orc, rng, act, torch_fn):
    """|v| <= 2: the Pade forms agree with the exact functions to ~1e-6."""
    v = rng.uniform(-2, 2, 4096).astype(np.float32)
    got = orc.act_forward(v, act)
    ref = torch_fn(torch.from_numpy(v).double()).numpy()
    assert np.max(np.abs(got - ref)) < 3e-6


def test_mp_silu_is_silu_over_0596(orc, rng):
    v = rng.uniform(-6, 6, 2048).astype(np.float32)
    a = orc.act_forward(v, MP_SILU).astype(np.float64)
    b = orc.act_forward(v, SILU).astype(np.float64) / 0.596
    assert np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-3)) < 1e-6


@pytest.mark.parametrize("act,torch_fn", [
    (SILU, F.silu),
    (GELU, lambda v: F.gelu(v, approximate="tanh")),
    (TANH, torch.tanh),
])
def test_activation_backward_vs_torch_autograd(orc, rng, act, torch_fn):
    """act'(z) with |z| <= 1.5 against torch's autograd of the exact function."""
    z = rng.uniform(-1.5, 1.5, 2048).astype(np.float32)
    g = rng.standard_normal(2048).astype(np.float32)
    got = orc.act_backward(g, z, act)
    zt = torch.from_numpy(z).double().requires_grad_(True)
    torch_fn(zt).backward(torch.from_numpy(g).double())
    assert np.max(np.abs(got - zt.grad.numpy())) < 2e-5


def test_silu_backward_uses_pade_sigmoid_not_its_own_derivative(orc):
    """Reference kernels.cu:49-56: s(1+z(1-s)) with s the Pade sigmoid; for
    z << 0 the Pade SiLU is exactly 0 but s > 0 keeps a tiny nonzero slope."""
    z = np.float32(-12.0)
    assert orc.act_forward(np.array([z]), SILU)[0] == 0.0
    s = orc.dll().orc_pade_sigmoid(float(z))
    expect = np.float32(s) * (np.float32(1) + z * (np.float32(1) - np.float32(s)))
    assert orc.act_backward(np.ones(1, np.float32), np.array([z]), SILU)[0] == np.float32(expect)


# ---------------------------------------------------------------------------
# GroupNorm (reference src/kernels.cu:622-717), LayerNorm (:491-567)
# ---------------------------------------------------------------------------
def _torch_gn_nhwc(x, gamma, beta, G, eps=1e-5):
    B, HW, C = x.shape
    xt = torch.from_numpy(x).double().permute(0, 2, 1).reshape(B, C, HW, 1)
    return xt, lambda xt_, g_, b_: F.group_norm(xt_, G, g_, b_, eps).reshape(B, C, HW).permute(0, 2, 1)


@pytest.mark.parametrize("shape", [(2, 36, 8, 4), (3, 35, 64, 8), (2, 16, 96, 3)])
def test_groupnorm_forward_backward_vs_torch(orc, rng, shape):
    B, HW, C, G = shape
    x = rng.standard_normal((B, HW, C)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    dy = rng.standard_normal((B, HW, C)).astype(np.float32)
    y, mu, rs = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, IDENT)
    xt, gn = _torch_gn_nhwc(x, gamma, beta, G)
    xt.requires_grad_(True)
    gt = torch.from_numpy(gamma).double().requires_grad_(True)
    bt = torch.from_numpy(beta).double().requires_grad_(True)
    yt = gn(xt, gt, bt)
    assert rel_err(y, yt.detach().numpy()) <= TOL
    yt.backward(torch.from_numpy(dy).double())
    dx, gg, gb = orc.groupnorm_backward(dy, x, gamma, beta, mu, rs, G, IDENT)
    dxt = xt.grad.reshape(B, C, HW).permute(0, 2, 1).numpy()
    assert rel_err(dx, dxt) <= TOL
    assert rel_err(gg, gt.grad.numpy(), floor=1.0) <= TOL
    assert rel_err(gb, bt.grad.numpy(), floor=1.0) <= TOL


@pytest.mark.parametrize("act", [0, 3], ids=["identity", "silu"])
def test_groupnorm_f32_baseline_within_summation_bounds(orc, rng, act):
    """The CPU baseline's fp32 transcription (serial fp32 sums, E[x^2]-mu^2,
    one serial loop per channel for dgamma/dbeta, as src/kernels.cu:622-717)
    computes what the double oracle computes, within the worst-case error of
    recursive fp32 summation (u = 2^-24): the bench times correct code.  A
    wrong sign, index or a dropped row is off by O(1); for the channel sums
    the bound is tight enough that one dropped term of typical size fails."""
    B, H, W, C, G = 8, 32, 32, 128, 32  # BASELINE cfg1
    HW, cpg = H * W, C // G
    x = rng.standard_normal((B, HW, C), dtype=np.float32)
    dy = rng.standard_normal((B, HW, C), dtype=np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    u = 2.0 ** -24
    n = HW * cpg  # terms per group sum
    N = B * HW    # terms per channel sum
    y, mu, rs = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, act)
    y32, mu32, rs32 = orc.groupnorm_forward_f32(x, gamma, beta, G, 1e-5, act)
    xg = x.reshape(B, HW, G, cpg).astype(np.float64)
    abs_mean = np.mean(np.abs(xg), axis=(1, 3)).ravel()  # sum|x| / n per (b, g)
    assert np.all(np.abs(mu32.astype(np.float64) - mu) <= (n + 2) * u * abs_mean)
    assert rel_err(rs32, rs) <= n * u
    assert rel_err(y32, y) <= n * u
    dx, gg, gb = orc.groupnorm_backward(dy, x, gamma, beta, mu, rs, G, act)
    dx32, gg32, gb32 = orc.groupnorm_backward_f32(dy, x, gamma, beta, mu, rs, G, act)
    assert rel_err(dx32, dx) <= n * u
    m = np.repeat(mu.reshape(B, G), cpg, axis=1)[:, None, :].astype(np.float64)
    r = np.repeat(rs.reshape(B, G), cpg, axis=1)[:, None, :].astype(np.float64)
    xh = (x - m) * r
    d = dy if act == 0 else orc.act_backward(dy, (gamma * xh + beta).astype(np.float32), act).reshape(x.shape)
    d = d.astype(np.float64)
    # first-order bound of recursive summation in the port's order (b, then
    # hw, per channel): u * (sum_k |partial sum k| + sum |terms|) (Higham,
    # Accuracy and Stability of Numerical Algorithms, 4.2), plus the rounding
    # of each term; tight enough that one dropped term of typical size fails
    for terms, got, ref in ((d * xh, gg32, gg), (d, gb32, gb)):
        t = terms.reshape(N, C)
        bound = u * (np.sum(np.abs(np.cumsum(t, axis=0)), axis=0) + 3 * np.sum(np.abs(t), axis=0))
        assert np.all(np.abs(got.astype(np.float64) - ref) <= bound), float(np.max(np.abs(got - ref) / bound))
        dropped = np.abs(t).mean(axis=0)
        assert np.all(bound < dropped), "bound too loose to see one dropped term"


def test_groupnorm_closed_forms(orc, rng):
    B, HW, C, G = 2, 64, 32, 4
    x = (3.0 + 2.0 * rng.standard_normal((B, HW, C))).astype(np.float32)
    y, mu, rs = orc.groupnorm_forward(x, np.ones(C, np.float32), np.zeros(C, np.float32), G, 1e-5, IDENT)
    yg = y.reshape(B, HW, G, C // G).transpose(0, 2, 1, 3).reshape(B * G, -1).astype(np.float64)
    xg = x.reshape(B, HW, G, C // G).transpose(0, 2, 1, 3).reshape(B * G, -1).astype(np.float64)
    var = xg.var(axis=1)
    assert np.max(np.abs(yg.mean(axis=1))) < 1e-5
    np.testing.assert_allclose(yg.var(axis=1), var / (var + 1e-5), rtol=1e-5)
    np.testing.assert_allclose(mu, xg.mean(axis=1), rtol=1e-6)
    # dx sums to zero over every group when gamma is constant
    dy = rng.standard_normal((B, HW, C)).astype(np.float32)
    dx, _, gb = orc.groupnorm_backward(dy, x, np.full(C, 1.5, np.float32), np.zeros(C, np.float32), mu, rs, G,
                                       IDENT)
    dxg = dx.reshape(B, HW, G, C // G).transpose(0, 2, 1, 3).reshape(B * G, -1).astype(np.float64)
    assert np.max(np.abs(dxg.sum(axis=1))) < 1e-3
    np.testing.assert_allclose(gb, dy.astype(np.float64).sum(axis=(0, 1)), rtol=1e-6, atol=1e-5)


def test_groupnorm_g1_single_pixel_equals_layernorm(orc, rng):
    """Two reference formulas (E[x^2]-mu^2 for GN, two-pass for LN) agree."""
    R, C = 16, 64
    x = rng.standard_normal((R, 1, C)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    y1, mu1, rs1 = orc.groupnorm_forward(x, gamma, beta, 1, 1e-5, IDENT)
    y2, mu2, rs2 = orc.layernorm_forward(x.reshape(R, C), gamma, beta, 1e-5)
    assert rel_err(y1.reshape(R, C), y2) <= TOL
    assert rel_err(rs1, rs2) <= TOL


def test_layernorm_forward_backward_vs_torch(orc, rng):
    R, C = 37, 48
    x = (0.5 + rng.standard_normal((R, C))).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    dy = rng.standard_normal((R, C)).astype(np.float32)
    y, mu, rs = orc.layernorm_forward(x, gamma, beta, 1e-5)
    xt = torch.from_numpy(x).double().requires_grad_(True)
    gt = torch.from_numpy(gamma).double().requires_grad_(True)
    bt = torch.from_numpy(beta).double().requires_grad_(True)
    yt = F.layer_norm(xt, (C,), gt, bt, 1e-5)
    assert rel_err(y, yt.detach().numpy()) <= TOL
    yt.backward(torch.from_numpy(dy).double())
    dx, gg, gb = orc.layernorm_backward(dy, x, gamma, mu, rs)
    assert rel_err(dx, xt.grad.numpy()) <= TOL
    assert rel_err(gg, gt.grad.numpy(), floor=1.0) <= TOL
    assert rel_err(gb, bt.grad.numpy(), floor=1.0) <= TOL


# ---------------------------------------------------------------------------
# Reference gradcheck method on the oracle's own backward functions
# (reference tests/gradcheck.c: EPS 1e-3, ATOL 1e-2, rtol 2e-2, 20 samples)
# ---------------------------------------------------------------------------
EPS, ATOL, RTOL, K = 1e-3, 1e-2, 2e-2, 20


def _fd_check(rng, f, x, analytic, what):
    """L(x) = <f(x), g> in double; central difference on K sampled indices."""
    flat = x.reshape(-1)
    idx = rng.choice(flat.size, size=min(K, flat.size), replace=False)
    worst = 0.0
    for i in idx:
        keep = flat[i]
        flat[i] = keep + EPS
        lp = f(x)
        flat[i] = keep - EPS
        lm = f(x)
        flat[i] = keep
        num = (lp - lm) / (2 * EPS)
        ana = float(analytic.reshape(-1)[i])
        worst = max(worst, abs(num - ana) / (ATOL + RTOL * (abs(num) + abs(ana))))
    assert worst <= 1.0, f"{what}: violation ratio {worst:.3f}"


@pytest.mark.parametrize("act", [IDENT, SILU, GELU, TANH, MP_SILU])  # ReLU's kink defeats finite differences
def test_groupnorm_act_gradcheck(orc, rng, act):
    B, HW, C, G = 2, 36, 8, 4  # the reference gradcheck shape (gradcheck.c:301)
    x = rng.standard_normal((B, HW, C)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    g = rng.standard_normal((B, HW, C)).astype(np.float32)

    def loss_x(xx):
        return float(np.sum(orc.groupnorm_forward(xx, gamma, beta, G, 1e-5, act)[0].astype(np.float64) * g))

    _, mu, rs = orc.groupnorm_forward(x, gamma, beta, G, 1e-5, act)
    dx, gg, gb = orc.groupnorm_backward(g, x, gamma, beta, mu, rs, G, act)
    _fd_check(rng, loss_x, x, dx, "dx")
    gcopy = gamma.copy()
    _fd_check(rng, lambda gm: float(np.sum(orc.groupnorm_forward(x, gm, beta, G, 1e-5, act)[0].astype(np.float64) * g)),
              gcopy, gg, "dgamma")
    bcopy = beta.copy()
    _fd_check(rng, lambda bt: float(np.sum(orc.groupnorm_forward(x, gamma, bt, G, 1e-5, act)[0].astype(np.float64) * g)),
              bcopy, gb, "dbeta")


def test_layernorm_gradcheck(orc, rng):
    R, C = 2, 16  # layernorm(16), gradcheck.c:300
    x = rng.standard_normal((R, C)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(C)).astype(np.float32)
    g = rng.standard_normal((R, C)).astype(np.float32)
    _, mu, rs = orc.layernorm_forward(x, gamma, beta, 1e-5)
    dx, gg, gb = orc.layernorm_backward(g, x, gamma, mu, rs)
    _fd_check(rng, lambda xx: float(np.sum(orc.layernorm_forward(xx, gamma, beta, 1e-5)[0].astype(np.float64) * g)),
              x, dx, "dx")
    _fd_check(rng, lambda gm: float(np.sum(orc.layernorm_forward(x, gm, beta, 1e-5)[0].astype(np.float64) * g)),
              gamma.copy(), gg, "dgamma")


def test_weight_norm_backward_gradcheck(orc, rng):
    """W -> gain * normalize(W) (mp_linear.c:12-18 with the GEMM replaced by a
    fixed cotangent M); the reference backward projects M tangentially."""
    n_in, n_out, gain = 12, 8, 1.3
    W = rng.standard_normal((n_in, n_out)).astype(np.float32)
    M = rng.standard_normal((n_in, n_out)).astype(np.float32)
    Wn = orc.weight_normalize(W, 0.0)
    # on the sphere the forced normalisation is idempotent; d/dW at W=Wn
    gW, g_gain = orc.weight_normalize_backward(M, Wn, gain)

    def loss(w):
        return float(np.sum(gain * orc.weight_normalize(w, 0.0).astype(np.float64) * M))

    _fd_check(rng, loss, Wn.copy(), gW, "gW")
    # gain gradient: d/dgain <gain*Wn, M> = <Wn, M>
    assert abs(g_gain - float(np.sum(Wn.astype(np.float64) * M))) < 1e-4


# ---------------------------------------------------------------------------
# Weight normalisation closed forms (reference src/kernels.cu:255-297)
# ---------------------------------------------------------------------------
def test_weight_normalize_closed_forms(orc, rng):
    W = rng.standard_normal((1152, 128)).astype(np.float32)
    ss = np.sum(W.astype(np.float64) ** 2, axis=0)
    Wn = orc.weight_normalize(W, 1e-4)
    norms = np.sqrt(np.sum(Wn.astype(np.float64) ** 2, axis=0))
    np.testing.assert_allclose(norms, np.sqrt(ss / (ss + 1e-4)), rtol=2e-6)
    # repeated forwards converge to |W_j|^2 = 1 - eps
    for _ in range(50):
        Wn = orc.weight_normalize(Wn, 1e-4)
    np.testing.assert_allclose(np.sum(Wn.astype(np.float64) ** 2, axis=0), 1 - 1e-4, rtol=2e-6)
    # the gradient is tangential: <gW_j, Wn_j> ~ 0 for unit columns
    Wu = orc.weight_normalize(W, 0.0)
    M = rng.standard_normal(W.shape).astype(np.float32)
    gW, g_gain = orc.weight_normalize_backward(M, Wu, 2.0, 5.0)
    dots = np.sum(gW.astype(np.float64) * Wu, axis=0)
    assert np.max(np.abs(dots)) < 1e-3
    # the gain gradient is accumulated onto the incoming value (atomicAdd in kernels.cu:293)
    assert abs(g_gain - (5.0 + float(np.sum(M.astype(np.float64) * Wu)))) < 1e-3


# ---------------------------------------------------------------------------
# Magnitude-preserving sums and concatenation
# ---------------------------------------------------------------------------
def test_mp_weights(orc):
    wa, wb = orc.mp_sum_weights(0.3)
    assert abs(wa * wa + wb * wb - 1) < 1e-6
    assert abs(wa - 0.9191450) < 1e-6 and abs(wb - 0.3939193) < 1e-6
    ca, cb = orc.mp_cat_weights(0.3, 128, 128)
    assert abs((128 * ca * ca + 128 * cb * cb) / 256 - 1) < 1e-6
    assert abs(ca - 1.2998674) < 1e-6 and abs(cb - 0.5570860) < 1e-6
    ca, cb = orc.mp_cat_weights(0.5, 64, 192)
    assert abs((64 * ca * ca + 192 * cb * cb) / 256 - 1) < 1e-6
    # t = 0.5 with equal widths is a plain concat scaled by 1
    ca, cb = orc.mp_cat_weights(0.5, 16, 16)
    assert abs(ca - 1) < 1e-6 and abs(cb - 1) < 1e-6


def test_mp_cat_and_split_brute_force(orc, rng):
    R, Na, Nb = 7, 3, 5
    a = rng.standard_normal((R, Na)).astype(np.float32)
    b = rng.standard_normal((R, Nb)).astype(np.float32)
    wa, wb = orc.mp_cat_weights(0.3, Na, Nb)
    out = orc.mp_cat(a, b, 0.3)
    ref = np.concatenate([np.float32(wa) * a, np.float32(wb) * b], axis=1)
    assert np.array_equal(out, ref)
    g = rng.standard_normal((R, Na + Nb)).astype(np.float32)
    ga, gb = orc.mp_split(g, Na, Nb, 0.3)
    assert np.array_equal(ga, np.float32(wa) * g[:, :Na])
    assert np.array_equal(gb, np.float32(wb) * g[:, Na:])


def test_weighted_sum_and_small_elementwise(orc, rng):
    a = rng.standard_normal(1000).astype(np.float32)
    b = rng.standard_normal(1000).astype(np.float32)
    out = orc.weighted_sum(a, b, 0.25, -2.0)
    assert np.array_equal(out, np.float32(0.25) * a + np.float32(-2.0) * b)
    assert np.array_equal(orc.scale_by_scalar(a, 3.0), a * np.float32(3.0))
    Y = rng.standard_normal((9, 5)).astype(np.float32)
    bias = rng.standard_normal(5).astype(np.float32)
    assert np.array_equal(orc.add_bias(Y, bias), Y + bias)
    np.testing.assert_allclose(orc.bias_grad(Y, 5), Y.astype(np.float64).sum(axis=0), rtol=1e-6)
    assert np.array_equal(orc.sgd_step(a, b, 0.1), a - np.float32(0.1) * b)


# ---------------------------------------------------------------------------
# Embeddings (reference src/kernels.cu:385-394, 444-456)
# ---------------------------------------------------------------------------
def test_mp_fourier_special_values_and_unit_power(orc, rng):
    phases = np.array([0.0, 0.25, 0.5, 0.125], np.float32)
    out = orc.mp_fourier(np.zeros(1, np.float32), np.ones(4, np.float32), phases)
    np.testing.assert_allclose(out[0], np.sqrt(2) * np.cos(2 * np.pi * phases.astype(np.float64)), atol=2e-6)
    # E[out^2] = 1 for random frequencies and phases
    x = rng.standard_normal(64).astype(np.float32)
    f = rng.standard_normal(4096).astype(np.float32)
    ph = rng.uniform(0, 1, 4096).astype(np.float32)
    out = orc.mp_fourier(x, f, ph)
    assert abs(float(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 0.02


def test_mp_fourier_closed_form_products(orc):
    """out[b,k] = sqrt(2) cos(2 pi x[b] f[k]) at phase 0, with x[b] f[k] an exact
    number of eighth (and one sixteenth) turns, so every entry is a closed-form
    constant: 0, +-1, +-sqrt(2) or sqrt(2) cos(pi/8).  Batch 5 != C 4 and both
    x and f vary, so an oracle that dropped x, added x + f or read x[k] f[b]
    misses this table (reference src/kernels.cu:385-394)."""
    r2, c16 = np.sqrt(2.0), np.sqrt(2.0) * np.cos(np.pi / 8)
    x = np.array([0.25, 0.5, 0.125, 0.75, -0.25], np.float32)
    f = np.array([1.0, 2.0, 4.0, 0.5], np.float32)
    want = np.array([
        [0.0, -r2, r2, 1.0],      # x f = 1/4, 1/2, 1, 1/8 turns
        [-r2, r2, r2, 0.0],       # 1/2, 1, 2, 1/4
        [1.0, 0.0, -r2, c16],     # 1/8, 1/4, 1/2, 1/16
        [0.0, -r2, r2, -1.0],     # 3/4, 3/2, 3, 3/8
        [0.0, -r2, r2, 1.0],      # -1/4, -1/2, -1, -1/8
    ])
    # The float argument 6.28318530718f * (x f + phase) is off 2 pi (x f + phase)
    # by at most ~1.6e-6 rad at 3.75 turns, hence the 5e-6 tolerance on entries
    # of size sqrt(2); every planted mistake moves an entry by O(1).
    out = orc.mp_fourier(x, f, np.zeros(4, np.float32))
    assert out.shape == (5, 4)
    np.testing.assert_allclose(out, want, atol=5e-6)
    # the phase adds whole and fractional turns to x f
    ph = np.array([0.25, 0.5, 0.75, 0.0], np.float32)
    want_ph = np.array([
        [-r2, r2, 0.0, 1.0],      # 1/2, 1, 7/4, 1/8 turns
        [0.0, -r2, 0.0, 0.0],     # 3/4, 3/2, 11/4, 1/4
        [-1.0, 0.0, 0.0, c16],    # 3/8, 3/4, 5/4, 1/16
        [r2, r2, 0.0, -1.0],      # 1, 2, 15/4, 3/8
        [r2, r2, 0.0, 1.0],       # 0, 0, -1/4, -1/8
    ])
    out = orc.mp_fourier(x, f, ph)
    np.testing.assert_allclose(out, want_ph, atol=5e-6)


def test_mp_fourier_rows_follow_x_columns_follow_f(orc, rng):
    """Permuting x permutes the output rows, permuting (f, phase) together
    permutes its columns, bit for bit; changing one x changes only its row."""
    x = rng.standard_normal(7).astype(np.float32)
    f = rng.standard_normal(11).astype(np.float32)
    ph = rng.uniform(0, 1, 11).astype(np.float32)
    out = orc.mp_fourier(x, f, ph)
    px, pf = rng.permutation(7), rng.permutation(11)
    assert np.array_equal(orc.mp_fourier(x[px], f, ph), out[px])
    assert np.array_equal(orc.mp_fourier(x, f[pf], ph[pf]), out[:, pf])
    x2 = x.copy()
    x2[3] += np.float32(0.37)
    out2 = orc.mp_fourier(x2, f, ph)
    rows = np.any(out2 != out, axis=1)
    assert rows.tolist() == [False, False, False, True, False, False, False]


def test_sinusoidal_special_values(orc):
    C, L = 256, float(np.float32(np.log(10000.0)))
    out = orc.sinusoidal(np.zeros(1, np.float32), C, L)
    assert np.all(out[0, :128] == 0) and np.all(out[0, 128:] == 1)
    t = np.array([1.0, 17.0, 999.0], np.float32)
    out = orc.sinusoidal(t, C, L)
    # j = 0 has frequency exactly 1
    np.testing.assert_allclose(out[:, 0], np.sin(t.astype(np.float64)), atol=1e-7)
    np.testing.assert_allclose(out[:, 128], np.cos(t.astype(np.float64)), atol=1e-7)
    # frequencies are 10000^(-j/half) (to float rounding of the exponent argument)
    j = np.arange(128)
    f = np.exp(-np.float64(L) * j / 128)
    np.testing.assert_allclose(out[0, :128], np.sin(f), rtol=1e-6, atol=1e-7)
    assert np.all(np.abs(out) <= 1)


# ---------------------------------------------------------------------------
# im2col / col2im (reference src/kernels.cu:750-816)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("geom", [(2, 6, 6, 3, 3, 1, 1), (1, 7, 5, 4, 3, 2, 1), (2, 5, 5, 4, 1, 1, 0),
                                  (1, 8, 8, 2, 4, 2, 1)])
def test_im2col_vs_torch_unfold(orc, rng, geom):
    B, H, W, C, K, s, p = geom
    im = rng.uniform(-1, 1, (B, H, W, C)).astype(np.float32)
    col = orc.im2col(im, K, s, p)
    Ho, Wo = orc.conv_out(H, K, s, p), orc.conv_out(W, K, s, p)
    u = F.unfold(torch.from_numpy(im).permute(0, 3, 1, 2), K, padding=p, stride=s)  # [B, C*K*K, L]
    u = u.reshape(B, C, K, K, Ho * Wo).permute(0, 4, 2, 3, 1).reshape(B * Ho * Wo, K * K * C)
    assert np.array_equal(col, u.numpy())


@pytest.mark.parametrize("geom", [(2, 6, 6, 3, 3, 1, 1), (1, 7, 5, 4, 3, 2, 1), (1, 8, 8, 2, 4, 2, 1)])
def test_col2im_vs_torch_fold_on_integers(orc, rng, geom):
    """Integer-valued floats: every sum is exact, so fold and col2im agree bitwise."""
    B, H, W, C, K, s, p = geom
    Ho, Wo = orc.conv_out(H, K, s, p), orc.conv_out(W, K, s, p)
    col = rng.integers(-8, 9, (B * Ho * Wo, K * K * C)).astype(np.float32)
    got = orc.col2im(col, (B, H, W, C), K, s, p)
    c = torch.from_numpy(col).reshape(B, Ho * Wo, K, K, C).permute(0, 4, 2, 3, 1).reshape(B, C * K * K, Ho * Wo)
    ref = F.fold(c, (H, W), K, padding=p, stride=s).permute(0, 2, 3, 1).numpy()
    assert np.array_equal(got, ref)


def test_col2im_summation_order(orc, rng):
    """The defined order: for each im pixel, contributions in ascending (oh, ow)
    (stride 1: kh descending, then kw descending), added in fp32 onto the
    incoming value.  Non-integer data makes the order visible in the bits."""
    B, H, W, C, K, s, p = 1, 5, 6, 3, 3, 1, 1
    Ho, Wo = orc.conv_out(H, K, s, p), orc.conv_out(W, K, s, p)
    col = (rng.standard_normal((B * Ho * Wo, K * K * C)) * 1e3).astype(np.float32)
    init = rng.standard_normal((B, H, W, C)).astype(np.float32)
    got = orc.col2im(col, (B, H, W, C), K, s, p, init=init)
    ref = init.copy()
    colr = col.reshape(B, Ho, Wo, K, K, C)
    for ih in range(H):
        for iw in range(W):
            for kh in reversed(range(K)):
                for kw in reversed(range(K)):
                    oh, ow = ih + p - kh, iw + p - kw
                    if 0 <= oh < Ho and 0 <= ow < Wo:
                        ref[0, ih, iw] = ref[0, ih, iw] + colr[0, oh, ow, kh, kw]
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------------------
# Adam (kernels.cu:170-183 + optimizer.c:54-69) and EMA (ema.c:29-35)
# ---------------------------------------------------------------------------
def test_adam_step1_is_signed_lr(orc, rng):
    g = rng.standard_normal(1000).astype(np.float32)
    bc1, bc2 = orc.adam_bias_corrections(0.9, 0.999, 1)
    p, m, v = orc.adam_step(np.zeros(1000), np.zeros(1000), np.zeros(1000), g, 1e-3, 0.9, 0.999, 1e-8, bc1, bc2)
    np.testing.assert_allclose(-p, 1e-3 * g / (np.abs(g) + 1e-8), rtol=2e-6)
    assert np.array_equal(m, np.float32(1 - np.float32(0.9)) * g)


def test_adam_matches_torch_adam(orc, rng):
    n, steps = 512, 10
    p0 = (0.02 * rng.standard_normal(n)).astype(np.float32)
    p, m, v = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    pt = torch.nn.Parameter(torch.from_numpy(p0.copy()).double())
    opt = torch.optim.Adam([pt], lr=1e-4, betas=(0.9, 0.999), eps=1e-8)
    for t in range(1, steps + 1):
        g = (1e-3 * rng.standard_normal(n)).astype(np.float32)
        bc1, bc2 = orc.adam_bias_corrections(0.9, 0.999, t)
        p, m, v = orc.adam_step(p, m, v, g, 1e-4, 0.9, 0.999, 1e-8, bc1, bc2)
        pt.grad = torch.from_numpy(g).double()
        opt.step()
    assert np.max(np.abs(p - pt.detach().numpy())) < 1e-8


def test_ema_geometric_decay(orc, rng):
    p = rng.standard_normal(256).astype(np.float32)
    shadow = rng.standard_normal(256).astype(np.float32)
    s0 = shadow.copy()
    decay = np.float32(0.99)
    w1 = float(np.float32(1) - decay)
    for _ in range(30):
        shadow = orc.weighted_sum(shadow, p, float(decay), w1)
    ref = p.astype(np.float64) + float(decay) ** 30 * (s0.astype(np.float64) - p)
    assert np.max(np.abs(shadow - ref)) < 1e-5
    lerp = torch.lerp(torch.from_numpy(s0), torch.from_numpy(p), w1).numpy()
    one = orc.weighted_sum(s0, p, float(decay), w1)
    assert np.max(np.abs(one - lerp)) < 1e-6


# ---------------------------------------------------------------------------
# Spatial broadcasts / reductions (kernels.cu:1052-1178) and the EDM block's
# fused modulate + activation pair (cond_conv_residual.c:30-33, 46-49)
# ---------------------------------------------------------------------------
def test_spatial_add_and_modulate_are_single_ops(orc, rng):
    """One add / one multiply per element: numpy's float32 broadcast gives the
    same bits; special cond values: 0 is the identity, -1 gives zeros."""
    B, HW, C = 3, 10, 6
    x = rng.standard_normal((B, HW, C)).astype(np.float32)
    v = rng.standard_normal((B, C)).astype(np.float32)
    assert np.array_equal(orc.spatial_add(x, v), x + v[:, None, :])
    assert np.array_equal(orc.spatial_modulate(x, v), x * (v + np.float32(1.0))[:, None, :])
    assert np.array_equal(orc.spatial_modulate(x, np.zeros((B, C), np.float32)), x)
    assert not np.any(orc.spatial_modulate(x, -np.ones((B, C), np.float32)))


def test_spatial_reduce_sum_closed_forms(orc, rng):
    B, HW, C = 2, 257, 5
    x = rng.standard_normal((B, HW, C)).astype(np.float32)
    np.testing.assert_allclose(orc.spatial_reduce_sum(x), x.astype(np.float64).sum(axis=1), rtol=1e-6, atol=1e-6)
    # constant rows: HW * value exactly (small integers)
    ones = np.full((B, HW, C), 3.0, np.float32)
    assert np.array_equal(orc.spatial_reduce_sum(ones), np.full((B, C), 3.0 * HW, np.float32))
    # spatial_reduce_sum is the adjoint of spatial_add: <add(0, v), y> = <v, reduce(y)>
    v = rng.standard_normal((B, C)).astype(np.float32)
    lhs = float(np.sum(orc.spatial_add(np.zeros_like(x), v).astype(np.float64) * x))
    rhs = float(np.sum(v.astype(np.float64) * orc.spatial_reduce_sum(x)))
    assert abs(lhs - rhs) <= 1e-5 * max(1.0, abs(lhs))


def test_spatial_modulate_backward_gradcheck(orc, rng):
    B, HW, C = 2, 9, 4
    x = rng.standard_normal((B, HW, C)).astype(np.float32)
    cond = (0.5 * rng.standard_normal((B, C))).astype(np.float32)
    g = rng.standard_normal((B, HW, C)).astype(np.float32)
    gin, gc = orc.spatial_modulate_backward(g, x, cond)
    _fd_check(rng, lambda xx: float(np.sum(orc.spatial_modulate(xx, cond).astype(np.float64) * g)), x.copy(), gin,
              "grad_in")
    _fd_check(rng, lambda cc: float(np.sum(orc.spatial_modulate(x, cc).astype(np.float64) * g)), cond.copy(), gc,
              "grad_cond")


@pytest.mark.parametrize("act", [IDENT, SILU, MP_SILU, GELU, TANH])
def test_spatial_modulate_act_is_the_reference_pair(orc, rng, act):
    """The fused forms equal the reference's two-launch sequences: bits for the
    elementwise outputs, the double-accumulated sum for grad_cond; and the
    backward passes the reference's finite-difference gradcheck."""
    B, HW, C = 2, 12, 6
    x = (1.5 * rng.standard_normal((B, HW, C))).astype(np.float32)
    cond = (0.5 * rng.standard_normal((B, C))).astype(np.float32)
    g = rng.standard_normal((B, HW, C)).astype(np.float32)
    h2 = orc.spatial_modulate(x, cond)
    assert np.array_equal(orc.spatial_modulate_act_forward(x, cond, act), orc.act_forward(h2, act))
    gin, gc = orc.spatial_modulate_act_backward(g, x, cond, act)
    gin_ref, gc_ref = orc.spatial_modulate_backward(orc.act_backward(g, h2, act), x, cond)
    assert np.array_equal(gin, gin_ref)
    np.testing.assert_allclose(gc, gc_ref, rtol=1e-6, atol=1e-6)
    if act != IDENT:
        _fd_check(rng, lambda xx: float(np.sum(orc.spatial_modulate_act_forward(xx, cond, act).astype(np.float64) * g)),
                  x.copy(), gin, "grad_in")
        _fd_check(rng, lambda cc: float(np.sum(orc.spatial_modulate_act_forward(x, cc, act).astype(np.float64) * g)),
                  cond.copy(), gc, "grad_cond")
