"""The benchmark configurations of BASELINE.json as PONNI layer chains.

Synthetic data follows one counter-based definition on host and device:
u64(i) = splitmix64(key + i), key = splitmix64(seed ^ splitmix64(tag));
uniform = a + (b - a) * (top 24 bits / 2^24) as one fma in double; normal =
Box-Muller on the uniforms of indices 2i, 2i+1.  Weights are drawn on the
host and uploaded; inputs are drawn on the device (ponni_fill_synthetic).
Fan conventions follow the reference initializers: for a [n_in, n_out]
weight, Glorot-uniform limit sqrt(6/(n_in+n_out)) and He-normal std
sqrt(2/n_in) (src/initializers/ponni_initializer.h:89-107, :226-282).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, List

import numpy as np

from . import model as M

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(x):
    with np.errstate(over="ignore"):
        z = np.asarray(x, dtype=np.uint64) + _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def stream_key(seed: int, tag: int) -> np.uint64:
    return splitmix64(np.uint64(seed) ^ splitmix64(np.uint64(tag)))


def uniform(n: int, seed: int, tag: int, a: float, b: float) -> np.ndarray:
    key = stream_key(seed, tag)
    with np.errstate(over="ignore"):
        r = splitmix64(key + np.arange(n, dtype=np.uint64))
    u = (r >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)
    # The device evaluates fma(b - a, u, a); mul + add here can differ from it
    # only in a final float rounding, and only inputs ever come from the device.
    return (a + (b - a) * u).astype(np.float32)


def normal(n: int, seed: int, tag: int, mean: float, std: float) -> np.ndarray:
    key = stream_key(seed, tag)
    idx = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        r1 = splitmix64(key + np.uint64(2) * idx)
        r2 = splitmix64(key + np.uint64(2) * idx + np.uint64(1))
    u1 = ((r1 >> np.uint64(40)) + np.uint64(1)).astype(np.float64) * (1.0 / 16777216.0)
    u2 = (r2 >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)
    return (mean + std * z).astype(np.float32)


def glorot_uniform(n_in: int, n_out: int, seed: int, tag: int) -> np.ndarray:
    lim = math.sqrt(6.0 / (n_in + n_out))
    return uniform(n_in * n_out, seed, tag, -lim, lim).reshape(n_in, n_out)


def he_normal(n_in: int, n_out: int, seed: int, tag: int) -> np.ndarray:
    return normal(n_in * n_out, seed, tag, 0.0, math.sqrt(2.0 / n_in)).reshape(n_in, n_out)


@dataclass
class Config:
    name: str
    description: str
    batch: int
    n_in: int
    n_out: int
    dtype: str               # "f32" / "f16"
    layers: Callable[[bool], List[M.Layer]]   # nonzero_bias -> layer chain
    input_dist: tuple        # ("uniform", a, b) or ("normal", mean, std)
    seed: int
    bound: str               # "hbm" or "mfma"
    bytes_per_sample: int    # algorithmic HBM bytes (input + output)
    flops_per_sample: int    # 2 * MACs of the dense layers
    peak: float              # bytes/s or FLOP/s of MI355X


HBM_PEAK = 8.0e12
FP32_PEAK = 157.3e12
FP64_PEAK = 78.6e12
FP16_PEAK = 2.5e15

INPUT_TAG = 1000  # tag of the input tensor stream


def _bias(n, seed, tag, nonzero):
    if nonzero:
        return uniform(n, seed, tag, -0.1, 0.1)
    return np.zeros(n, dtype=np.float32)


def c1_layers(nonzero_bias: bool = True) -> List[M.Layer]:
    s = 0
    return [M.Matvec(uniform(6, s, 1, -0.5, 0.5).reshape(2, 3)), M.Bias(uniform(3, s, 2, -0.1, 0.1)), M.Relu(3),
            M.Matvec(uniform(3, s, 3, -0.5, 0.5).reshape(3, 1)), M.Bias(uniform(1, s, 4, -0.1, 0.1))]


def c2_layers(nonzero_bias: bool = False) -> List[M.Layer]:
    s, widths, out = 1, [16, 64, 64, 64], []
    for i in range(3):
        out += [M.Matvec(glorot_uniform(widths[i], widths[i + 1], s, 1 + 2 * i)),
                M.Bias(_bias(widths[i + 1], s, 2 + 2 * i, nonzero_bias)), M.Relu(widths[i + 1])]
    out += [M.Matvec(glorot_uniform(64, 8, s, 7)), M.Bias(_bias(8, s, 8, nonzero_bias))]
    return out


def c3_layers(nonzero_bias: bool = False) -> List[M.Layer]:
    s = 2
    out = [M.Matvec(he_normal(32, 128, s, 1))]
    for blk in range(4):
        t = 10 + 10 * blk
        out += [M.Save_State(0, 128), M.LayerNorm(128),
                M.Matvec(he_normal(128, 128, s, t)), M.Bias(_bias(128, s, t + 1, nonzero_bias)), M.Gelu(128, True),
                M.Matvec(he_normal(128, 128, s, t + 2)), M.Bias(_bias(128, s, t + 3, nonzero_bias)),
                M.Binop_Add(0, 128)]
    out += [M.Matvec(he_normal(128, 16, s, 99))]
    return out


def c4_layers(nonzero_bias: bool = False) -> List[M.Layer]:
    s, widths, out = 3, [64, 256, 256, 256], []
    for i in range(3):
        out += [M.Matvec(glorot_uniform(widths[i], widths[i + 1], s, 1 + 2 * i)),
                M.Bias(_bias(widths[i + 1], s, 2 + 2 * i, nonzero_bias)), M.Tanh(widths[i + 1])]
    out += [M.Matvec(glorot_uniform(256, 64, s, 7)), M.Bias(_bias(64, s, 8, nonzero_bias))]
    return out


def c5_graph(nonzero_bias: bool = False):
    """The generator-style branched graph of configs[4] in the canonical IR:
    Dense weights are [out, in] (Glorot over fan_in = in, fan_out = out),
    biases zero unless nonzero_bias, Concat order [branch A, branch B]."""
    from .graph import GraphBuilder

    s = 4

    def w(n_in, n_out, tag):
        return glorot_uniform(n_in, n_out, s, tag).T.copy()

    g = GraphBuilder(24)
    x = g.input
    a = g.unary("Relu", g.dense(x, w(24, 96, 1), _bias(96, s, 2, nonzero_bias), name="branch_a.fc1"))
    a = g.dense(a, w(96, 48, 3), _bias(48, s, 4, nonzero_bias), name="branch_a.fc2")
    b = g.unary("Sigmoid", g.dense(x, w(24, 48, 5), _bias(48, s, 6, nonzero_bias), name="branch_b.fc"))
    c = g.concat(a, b)
    p = g.dense(x, w(24, 96, 7), _bias(96, s, 8, nonzero_bias), name="skip.proj")
    t = g.binary("Add", c, p)
    t = g.binary("Sub", t, g.reduce("ReduceMean", t))
    out = g.softmax(g.dense(t, w(96, 10, 9), _bias(10, s, 10, nonzero_bias), name="head.fc"))
    return g.finish(out)


def c5_layers(nonzero_bias: bool = False) -> List[M.Layer]:
    """c5 linearized into the layer chain libponni_hip runs, parameters set."""
    from .graph import GeneratedModel

    gm = GeneratedModel(c5_graph(nonzero_bias))
    layers = gm.lowered.layers
    for l, v in zip(layers, gm.lowered.layer_params(gm._constants("f64"))):
        if v.size:
            l.params = v
    return layers


CONFIGS = {
    "c1": Config("c1", "Template-mode MLP 2->3->1 fp32", 1_000_000, 2, 1, "f32", c1_layers, ("uniform", -1.0, 1.0),
                 0, "hbm", 12, 18, HBM_PEAK),
    "c2": Config("c2", "Sequential fp32 MLP 16->64->64->64->8, ReLU", 4_194_304, 16, 8, "f32", c2_layers,
                 ("normal", 0.0, 1.0), 1, "mfma", 96, 19_456, FP32_PEAK),
    "c3": Config("c3", "Residual fp32 MLP 32->128, 4x[LN->128->GELU(tanh)->128 + skip], ->16", 2_097_152, 32, 16,
                 "f32", c3_layers, ("normal", 0.0, 1.0), 2, "mfma", 192, 274_432, FP32_PEAK),
    "c4": Config("c4", "fp16 MLP 64->256->256->256->64, tanh, fp32 accumulate", 8_388_608, 64, 64, "f16", c4_layers,
                 ("normal", 0.0, 1.0), 3, "mfma", 256, 327_680, FP16_PEAK),
    "c5": Config("c5", "Generated branched fp32 graph 24->[96->48 | 48]->concat 96 + proj skip, centre, ->10 softmax",
                 4_194_304, 24, 10, "f32", c5_layers, ("normal", 0.0, 1.0), 4, "mfma", 136, 22_656, FP32_PEAK),
}


def wide512_layers(nonzero_bias: bool = False) -> List[M.Layer]:
    """Supplementary wide chain: fp16 MLP 64->512->512->64 with tanh, weights
    Glorot-uniform, biases zero unless nonzero_bias."""
    s, widths, out = 5, [64, 512, 512], []
    for i in range(2):
        out += [M.Matvec(glorot_uniform(widths[i], widths[i + 1], s, 1 + 2 * i)),
                M.Bias(_bias(widths[i + 1], s, 2 + 2 * i, nonzero_bias)), M.Tanh(widths[i + 1])]
    out += [M.Matvec(glorot_uniform(512, 64, s, 5)), M.Bias(_bias(64, s, 6, nonzero_bias))]
    return out


# Workloads measured beside the BASELINE configurations (not part of BASELINE.json).
SUPPLEMENTARY = {
    "wide512": Config("wide512", "fp16 MLP 64->512->512->64, tanh, fp32 accumulate (supplementary, wider than "
                      "256 features; not a BASELINE config)", 4_194_304, 64, 64, "f16", wide512_layers,
                      ("normal", 0.0, 1.0), 5, "mfma", 256, 655_360, FP16_PEAK),
}
