"""CPU checks of the two-pass large-batch router's error bound.

The GPU kernel approximates a router logit C (canonical fp32 order, the C
oracle's orc_canon_dot) by A = 2^-s * sum fp16(x_i) fp16(2^s w_i), with the
products exact and the sum in fp32, and treats every expert whose interval
A +- eps can reach the K-th largest lower bound as a candidate for exact
recomputation, where eps = |w| (c1 |x| + c2) with
c1 = 9/8 (2^-10 + 2^-21 + 2^-28 sqrt(H) + 2 gamma_H(2^-23)), c2 = 9/8 2^-14 sqrt(H).
Here A is emulated in numpy (fp16 rounding of both operands, float64 sums:
the fp32 accumulation error is part of the bound's own budget) and checked
against the oracle's canonical logits, including rows whose scaled values
fall into fp16's subnormal range and rows of very different magnitude."""
import numpy as np
import pytest

import oracle as O
import orome_amd


def eps_coeffs(H):
    u = 2.0 ** -23
    g = H * u / (1 - H * u)
    c1 = 1.125 * (2.0 ** -10 + 2.0 ** -21 + 2.0 ** -28 * np.sqrt(H) + 2 * g)
    c2 = 1.125 * 2.0 ** -14 * np.sqrt(H)
    return c1, c2


def approx(W, x):
    m = np.abs(W).max(axis=1)
    sh = np.where(m > 0, 15 - np.frexp(m)[1], 0)
    W16 = (W * np.ldexp(1.0, sh)[:, None]).astype(np.float16).astype(np.float64)
    return (x.astype(np.float16).astype(np.float64) @ W16.T) * np.ldexp(1.0, -sh)[None, :]


def canon(W, x):
    E, H = W.shape
    T = x.shape[0]
    L = O.lib(omp=True)
    out = np.empty((T, E + 1), np.float32)
    wsg = np.zeros(H, np.float32)
    L.orc_router_logits(W.ctypes.data, wsg.ctypes.data, x.ctypes.data, T, E, H, out.ctypes.data)
    return out[:, :E].astype(np.float64)


@pytest.mark.parametrize("kind", ["synthetic", "wide_range", "tiny_rows"])
def test_bound_holds_and_candidates_cover_winners(kind):
    E, H, T, K = 256, 2048, 64, 8
    rng = np.random.default_rng(7)
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    if kind == "wide_range":  # row magnitudes over 2^-20 .. 2^10
        W *= np.ldexp(1.0, rng.integers(-20, 11, E))[:, None].astype(np.float32)
    if kind == "tiny_rows":   # entries spanning fp16's subnormal range after scaling
        W *= (10.0 ** rng.uniform(-12, 0, (E, H))).astype(np.float32)
    x = orome_amd.synth_normal(3, 1, T * H).reshape(T, H)
    x[0, :] = 0.0
    x[1, ::7] *= 1e-6  # small activations (subnormal in fp16)
    C = canon(np.ascontiguousarray(W), np.ascontiguousarray(x))
    A = approx(W.astype(np.float64), x.astype(np.float64))
    c1, c2 = eps_coeffs(H)
    wn = np.linalg.norm(W.astype(np.float64), axis=1)
    xn = np.linalg.norm(x.astype(np.float64), axis=1)
    eps = wn[None, :] * (c1 * xn[:, None] + c2)
    ratio = np.max(np.abs(A - C) / np.maximum(eps, 1e-300))
    print("%s: max |A-C|/eps = %.4f" % (kind, ratio))
    assert ratio < 0.25  # the bound holds with a wide margin
    lo, hi = A - eps, A + eps
    L = np.sort(lo, axis=1)[:, ::-1][:, K - 1]
    cand = hi >= L[:, None]
    order = np.lexsort((np.tile(np.arange(E), (T, 1)), -C), axis=1)[:, :K]
    assert np.all(np.take_along_axis(cand, order, axis=1)), "a canonical winner is not a candidate"
    print("%s: candidates per token mean %.1f max %d" % (kind, cand.sum(1).mean(), cand.sum(1).max()))
