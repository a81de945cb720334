"""Pin the CPU oracle by mathematics the reference fixes, independent of its code.

* Tokenwise recurrences == Mobius / WY chunk decompositions (two independent
  derivations, as the reference's private chunk paths were used).
* K = 1 KDN is exactly a scalar Kalman filter: the filtered mean and variance
  equal dense Gaussian conditioning of the joint state-space model.
* kappa -> 0 gives pure decay of the carried state; T = 1 closed form.
* Frontend maps at special points (softplus(0) = ln 2, alpha clamp, chunk restart).
"""
import math

import pytest
import torch

from oracle import kdn_oracle as ko



@pytest.fixture(autouse=True)
def _fp64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _inputs(seed, B, T, H, K, V, diag):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, K, generator=g)
    k = torch.randn(B, T, H, K, generator=g)
    v = torch.randn(B, T, H, V, generator=g)
    alpha = torch.sigmoid(1.5 + torch.randn(B, T, H, K, generator=g))
    omega = torch.nn.functional.softplus(torch.randn(*((B, T, H, K) if diag else (B, T, H)), generator=g))
    r = 0.01 + torch.nn.functional.softplus(torch.randn(B, T, H, generator=g))
    return q, k, v, alpha, omega, r


@pytest.mark.parametrize("T,chunk", [(37, 8), (64, 64), (50, 16), (5, 32)])
@pytest.mark.parametrize("variant", ["iso", "diag"])
def test_tokenwise_equals_chunked(variant, T, chunk):
    q, k, v, alpha, omega, r = _inputs(1, 2, T, 2, 6, 5, variant == "diag")
    g = torch.Generator().manual_seed(7)
    S0 = 0.3 * torch.randn(2, 2, 6, 5, generator=g)
    p0 = 0.5 + torch.rand(2, 2, 6, generator=g) if variant == "diag" else 0.5 + torch.rand(2, 2, generator=g)
    fn = ko.iso_recurrent if variant == "iso" else ko.diag_recurrent
    kw = dict(info_scale=2.5, scale=0.8, initial_state=S0, initial_precision=p0, output_final_state=True)
    o1, (S1, c1) = fn(q, k, v, alpha, omega, r, **kw)
    o2, (S2, c2) = fn(q, k, v, alpha, omega, r, chunked=True, chunk_size=chunk, **kw)
    torch.testing.assert_close(o1, o2, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(S1, S2, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(c1, c2, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("variant", ["iso", "diag"])
def test_segments_from_carried_state_equal_whole_sequence(variant):
    """The state-carry contract: running tokens [0, T1) and then [T1, T) from the first part's
    final memory and precision gives the outputs and final state of [0, T) run at once."""
    T, T1 = 23, 9
    q, k, v, alpha, omega, r = _inputs(3, 2, T, 2, 6, 5, variant == "diag")
    fn = ko.iso_recurrent if variant == "iso" else ko.diag_recurrent
    kw = dict(info_scale=3.0, scale=0.7, output_final_state=True)
    o, (S, c) = fn(q, k, v, alpha, omega, r, **kw)
    a = (q[:, :T1], k[:, :T1], v[:, :T1], alpha[:, :T1], omega[:, :T1], r[:, :T1])
    b = (q[:, T1:], k[:, T1:], v[:, T1:], alpha[:, T1:], omega[:, T1:], r[:, T1:])
    o1, (S1, c1) = fn(*a, **kw)
    assert c1.shape == ((2, 2, 6) if variant == "diag" else (2, 2))
    o2, (S2, c2) = fn(*b, initial_state=S1, initial_precision=c1, **kw)
    torch.testing.assert_close(torch.cat([o1, o2], 1), o, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(S2, S, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(c2, c, rtol=1e-12, atol=1e-12)
    # one more token from the carried state is the tokenwise step (the decode kernel's contract)
    o3, (S3, _) = fn(*(x[:, :1] for x in b), initial_state=S1, initial_precision=c1, **kw)
    torch.testing.assert_close(o3, o2[:, :1], rtol=1e-12, atol=1e-12)


def _kalman_by_conditioning(alpha, omega, r, k, y, x0_mean, x0_var):
    """Filtered mean/variance of x_t | y_1..t by dense Gaussian conditioning.

    x_0 ~ N(m0, v0); x_t = alpha_t x_{t-1} + w_t, w_t ~ N(0, omega_t);
    y_t = k_t x_t + e_t, e_t ~ N(0, r_t).  Scalar state, T steps.
    """
    T = alpha.shape[0]
    # x_t = (prod alpha) x_0 + sum_j (prod_{j<i<=t} alpha_i) w_j : linear map of z=(x0, w_1..w_T)
    Lmap = torch.zeros(T, T + 1)
    for t in range(T):
        Lmap[t, 0] = torch.prod(alpha[: t + 1])
        for j in range(t + 1):
            Lmap[t, j + 1] = torch.prod(alpha[j + 1: t + 1])
    Zcov = torch.diag(torch.cat([x0_var.view(1), omega]))
    Xcov = Lmap @ Zcov @ Lmap.T
    Xmean = Lmap[:, 0] * x0_mean
    Ycov = torch.diag(k) @ Xcov @ torch.diag(k) + torch.diag(r)
    means, variances = [], []
    for t in range(T):
        idx = slice(0, t + 1)
        C_xy = Xcov[t, idx] * k[idx]
        Syy = Ycov[idx, idx]
        sol = torch.linalg.solve(Syy, torch.stack([y[idx] - k[idx] * Xmean[idx], C_xy], 1))
        means.append(Xmean[t] + C_xy @ sol[:, 0])
        variances.append(Xcov[t, t] - C_xy @ sol[:, 1])
    return torch.stack(means), torch.stack(variances)


@pytest.mark.parametrize("variant", ["iso", "diag"])
def test_unit_dimension_is_scalar_kalman_filter(variant):
    T = 12
    g = torch.Generator().manual_seed(3)
    alpha = torch.sigmoid(torch.randn(T, generator=g) + 1)
    omega = torch.nn.functional.softplus(torch.randn(T, generator=g))
    r = 0.05 + torch.rand(T, generator=g)
    k = torch.randn(T, generator=g)
    y = torch.randn(T, generator=g)
    m0 = torch.tensor(0.4)
    c0 = torch.tensor(1.7)  # prior precision
    mean, var = _kalman_by_conditioning(alpha, omega, r, k, y, m0, 1 / c0)
    sh = lambda x: x.view(1, T, 1, 1)
    fn = ko.iso_recurrent if variant == "iso" else ko.diag_recurrent
    om = omega.view(1, T, 1, 1) if variant == "diag" else omega.view(1, T, 1)
    o, (S, c) = fn(sh(torch.ones(T)), sh(k), sh(y), sh(alpha), om, r.view(1, T, 1),
                   info_scale=1.0, scale=1.0, initial_state=m0.view(1, 1, 1, 1),
                   initial_precision=c0.view(1), output_final_state=True)
    torch.testing.assert_close(o.view(T), mean, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(1.0 / c.view(()), var[-1], rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("variant", ["iso", "diag"])
def test_zero_gain_is_pure_decay(variant):
    B, T, H, K, V = 1, 9, 2, 4, 3
    q, k, v, alpha, omega, r = _inputs(5, B, T, H, K, V, variant == "diag")
    omega = torch.zeros_like(omega)
    S0 = torch.randn(B, H, K, V)
    fn = ko.iso_recurrent if variant == "iso" else ko.diag_recurrent
    # Infinite prior precision with no process noise means zero covariance: no writes.
    o, (S, _) = fn(q, k, v, alpha, omega, r, initial_state=S0, initial_precision=1e300,
                   scale=1.0, output_final_state=True)
    decay = torch.cumprod(alpha, 1)
    expect_o = torch.einsum("bthk,bthk,bhkv->bthv", q, decay, S0)
    torch.testing.assert_close(o, expect_o, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(S, decay[:, -1, :, :, None] * S0, rtol=1e-12, atol=1e-12)


def test_single_token_closed_form_diag():
    B, T, H, K, V = 1, 1, 1, 5, 3
    q, k, v, alpha, omega, r = _inputs(11, B, T, H, K, V, True)
    o, _ = ko.diag_recurrent(q, k, v, alpha, omega, r, initial_precision=2.0, scale=1.0)
    ph = alpha[0, 0, 0] ** 2 / 2.0 + omega[0, 0, 0]
    kap = ph * k[0, 0, 0] / (r[0, 0, 0] + (ph * k[0, 0, 0] ** 2).sum())
    expect = (q[0, 0, 0] @ kap) * v[0, 0, 0]
    torch.testing.assert_close(o[0, 0, 0], expect, rtol=1e-12, atol=1e-12)


def test_iso_gate_frontend_special_points():
    B, T, H, K = 1, 70, 2, 4
    x = torch.rand(B, T, H, K) * 2 + 0.1
    g_raw = torch.log(torch.expm1(x))           # softplus(g_raw) == x
    orr = torch.zeros(B, T, 2 * H)
    g, gc, a, omega, r, mu = ko.iso_gate_frontend(
        g_raw, orr, torch.zeros(H), torch.zeros(H), torch.zeros(H), torch.zeros(H * K),
        torch.zeros(H), omega_min=0.25, r_min=0.01)
    torch.testing.assert_close(g, -x, rtol=1e-6, atol=1e-6)
    # chunk restart at t = 64: the prefix at the first token of a chunk is that token's gate
    torch.testing.assert_close(gc[:, 64] * math.log(2), g[:, 64], rtol=1e-6, atol=1e-6)
    torch.testing.assert_close((gc[:, 1:64] - gc[:, :63]) * math.log(2), g[:, 1:64], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(a, torch.exp(-2 * x).mean(-1), rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(omega, torch.full_like(omega, 0.25 + math.log(2)))
    torch.testing.assert_close(r, torch.full_like(r, 0.01 + math.log(2)))
    torch.testing.assert_close(mu, torch.full_like(mu, 0.1 + math.log(2)))


def test_diag_frontend_alpha_clamp_only_on_memory_path():
    B, T, H, K = 1, 3, 1, 2
    f = torch.tensor([[[[100.0, -30.0]]] * T]).view(B, T, H, K)
    A_log = torch.tensor([math.log(0.5)])
    l_mem, gc, alpha, *_ = ko.diag_frontend(f, torch.zeros(B, T, H, K), torch.zeros(B, T, H), A_log,
                                            torch.zeros(H, K), torch.zeros(H))
    assert float(alpha[0, 0, 0, 0]) == pytest.approx(math.exp(-50.0), rel=1e-5)  # unclamped
    assert float(l_mem[0, 0, 0, 0]) == pytest.approx(math.log(1e-6), rel=1e-5)    # clamped
    assert float(alpha[0, 0, 0, 1]) == pytest.approx(math.exp(-0.5 * math.log1p(math.exp(-30.0))), rel=1e-6)
