"""Vectorized float64 numpy evaluation of a PONNI layer chain.

An independent formulation used to pin the C++ oracle: whole-batch matrix
algebra on a running state instead of the oracle's per-sample loops over
tmp1 / tmp2 / saved buffers.  Layer math is taken from the reference layer
templates (src/layers/*.h); Matvec weights are [n_in, n_out] so a layer is
y = W^T x (ponni_Matvec.h:70-79).
"""
from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

from ponni_amd import _abi as A


def _pointwise(l, x):
    k = l.kind
    if k == A.LAYER_BIAS:
        return x + l.params[:, None]
    if k == A.LAYER_RELU:
        return np.where(x > 0, x, 0.0)
    if k == A.LAYER_LEAKY_RELU:
        return np.where(x > 0, x, l.attr[0] * x)
    if k == A.LAYER_ELU:
        return np.where(x > 0, x, l.attr[0] * np.expm1(np.minimum(x, 0)))
    if k == A.LAYER_SELU:
        alpha, scale = 1.6732632423543772848, 1.0507009873554804934
        return np.where(x > 0, scale * x, scale * alpha * np.expm1(np.minimum(x, 0)))
    if k == A.LAYER_GELU:
        if l.flags & A.FLAG_GELU_APPROXIMATE:
            return 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
        return 0.5 * x * (1 + erf(x / math.sqrt(2)))
    if k == A.LAYER_SILU:
        return x / (1 + np.exp(-x))
    if k == A.LAYER_SIGMOID:
        return 1 / (1 + np.exp(-x))
    if k == A.LAYER_TANH:
        return np.tanh(x)
    if k == A.LAYER_SOFTPLUS:
        beta = l.attr[0]
        return np.logaddexp(0.0, beta * x) / beta
    if k == A.LAYER_HARD_SIGMOID:
        return np.clip(l.attr[0] * x + l.attr[1], 0.0, 1.0)
    if k == A.LAYER_HARD_SWISH:
        return x * np.clip(x + 3, 0, 6) / 6
    if k == A.LAYER_MISH:
        return x * np.tanh(np.logaddexp(0.0, x))
    raise ValueError(k)


def evaluate(layers, x: np.ndarray) -> np.ndarray:
    """x [n_in, B] -> [n_out, B] in float64."""
    s = np.asarray(x, dtype=np.float64)
    saved = {}
    for l in layers:
        k = l.kind
        if k == A.LAYER_MATVEC:
            W = l.params.reshape(l.n_in, l.n_out)
            s = W.T @ s
        elif k == A.LAYER_LAYER_NORM:
            n = l.n_in
            g, b = l.params[:n], l.params[n:]
            mu = s.mean(axis=0)
            var = ((s - mu) ** 2).mean(axis=0)
            s = g[:, None] * (s - mu) / np.sqrt(var + l.attr[0]) + b[:, None]
        elif k == A.LAYER_SOFTMAX:
            e = np.exp(s - s.max(axis=0))
            s = e / e.sum(axis=0)
        elif k == A.LAYER_LOG_SOFTMAX:
            m = s.max(axis=0)
            s = s - (np.log(np.exp(s - m).sum(axis=0)) + m)
        elif k == A.LAYER_MIN_MAX_NORM:
            lo, hi = s.min(axis=0), s.max(axis=0)
            s = l.attr[0] + (s - lo) * (l.attr[1] - l.attr[0]) / ((hi - lo) + l.attr[2])
        elif k == A.LAYER_SAVE_STATE:
            saved[l.slot] = s.copy()
        elif k == A.LAYER_BINOP_ADD:
            s = s + saved[l.slot]
        elif k == A.LAYER_BINOP_CONCATENATE:
            sv = saved[l.slot]
            s = np.concatenate([s, sv] if l.flags & A.FLAG_CONCAT_AFTER else [sv, s], axis=0)
        elif k == A.LAYER_BINOP_PROJECTION_ADD:
            n, ns = l.n_in, l.n_aux
            W = l.params[: ns * n].reshape(ns, n)
            b = l.params[ns * n:]
            s = s + (W.T @ saved[l.slot] + b[:, None])
        else:
            s = _pointwise(l, s)
    return s
