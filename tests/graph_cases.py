"""Random generated-model graphs over the selection, logic, normalization and
unary-math operations of kokkos_nn (interpreter.py:15-193), arranged so the
reference optimizer (passes.py) forms each of its compound nodes:
ElementwiseChain (chains of unary / element-wise nodes), PointwiseRegion
(reconverging pointwise DAGs), DenseEpilogue (a Dense followed by
Where / Clip / PRelu / BatchNormalization / Mean ...), mapped reductions
(a reduction of a pointwise chain), CompareSelect (Where of a comparison),
ResidualAddActivation and Dense input maps (a Dense reading a Concat or a
Gather).

smooth=True keeps every output a continuous function of the input: the
comparisons only choose between branches that agree where the comparison
flips (a leaky ramp, a clamp, |x| through IsNaN(Sqrt(x))), so fp16 runs,
whose intermediate values differ from the oracle's by a rounding, cannot
land on the other side of a jump.  smooth=False adds Floor / Ceil / Round /
Sign, comparisons as values and logic; those graphs are for fp32 / fp64.
"""
from __future__ import annotations

import math

import numpy as np

from ponni_amd import graph as G

# Unary operations applied to a value squashed into (-0.9, 0.9) by tanh, so
# every inverse function stays in its domain.
_BOUNDED = ["Acos", "Asin", "Atan", "Atanh", "Sin", "Cos", "Tan", "Erf", "Asinh", "Sinh", "Cosh", "Softsign",
            "Exp", "Neg", "Abs", "Celu", "Selu", "Elu", "Relu", "Sigmoid", "HardSwish"]
_STEP = ["Floor", "Ceil", "Round", "Sign"]


def op_graph(seed: int, smooth: bool = True, dtype: str = "float32", aligned: bool = True, blocks: int = 9,
             n_in: int | None = None, narrow: bool = False) -> G.Graph:
    """aligned: every width a multiple of 16 (FUSED concatenation); narrow:
    every width at most 16 (the NARROW kernels)."""
    rng = np.random.default_rng(1000 + seed)
    widths = [3, 5, 8, 13, 16] if narrow else [16, 32, 48] if aligned else [3, 8, 13, 24]
    n_in = n_in or int(rng.choice(widths))
    g = G.GraphBuilder(n_in, dtype=dtype)
    counter = [0]

    def name(p: str) -> str:
        counter[0] += 1
        return f"{p}{counter[0]}"

    def const(values) -> int:
        return g.constant(name("k"), np.asarray(values, dtype=np.float64))

    def dense(t: int, m: int, bias: bool = True) -> int:
        n = g.size(t)
        lim = math.sqrt(6 / (n + m))
        return g.dense(t, rng.uniform(-lim, lim, (m, n)), rng.uniform(-0.2, 0.2, m) if bias else None,
                       name=name("fc"))

    def squash(t: int) -> int:
        return g.binary("Mul", g.unary("Tanh", t), const([0.9]))

    def bounded_unary(t: int) -> int:
        op = str(rng.choice(_BOUNDED))
        x = squash(t)
        if op == "Acos":  # acos - pi/2 keeps the value centred
            return g.binary("Sub", g.unary(op, x), const([math.pi / 2]))
        if op == "Exp":
            return g.binary("Sub", g.unary(op, x), const([1.0]))
        if op == "Cosh":
            return g.binary("Sub", g.unary(op, x), const([1.0]))
        return g.unary(op, x)

    pool = [dense(g.input, int(rng.choice(widths)))]
    for _ in range(blocks):
        t = pool[-1] if rng.random() < 0.6 else pool[int(rng.integers(len(pool)))]
        n = g.size(t)
        kind = int(rng.integers(14))
        if kind == 0:  # Dense + activation, or Dense + residual Add + activation
            d = dense(t, n if rng.random() < 0.5 else int(rng.choice(widths)))
            if g.size(d) == n and rng.random() < 0.5:
                d = g.binary("Add", d, t)
            out = g.unary(str(rng.choice(["Relu", "Tanh", "Sigmoid", "Gelu"])), d)
        elif kind == 1:  # element-wise chain with constants
            out = bounded_unary(t)
            out = g.binary(str(rng.choice(["Add", "Mul", "Sub"])), out, const(rng.uniform(0.5, 1.5, n)))
            out = g.unary(str(rng.choice(["Atan", "Softsign", "Erf"])), out)
        elif kind == 2:  # reconverging pointwise region
            a, b = bounded_unary(t), bounded_unary(t)
            out = g.binary(str(rng.choice(["Add", "Mul", "Max", "Min"])), a, b)
        elif kind == 3:  # leaky ramp through CompareSelect
            zero = const([0.0])
            out = g.where(g.compare("Greater", t, zero), t, g.binary("Mul", t, const([0.1])))
        elif kind == 4:  # clamp written with Where
            lo = const([-0.5])
            out = g.where(g.compare("Less", t, lo), lo, t)
        elif kind == 5:  # Clip with attribute or constant bounds
            if rng.random() < 0.5:
                out = g.clip(t, -0.6, 0.8)
            else:
                out = g.node("Clip", [t, const([-0.7]), const([0.5])], n)
        elif kind == 6:  # PRelu with a per-feature or shared slope
            out = g.node("PRelu", [t, const(rng.uniform(0.05, 0.3, n if rng.random() < 0.5 else 1))], n)
        elif kind == 7:  # BatchNormalization after a dense layer (a DenseEpilogue)
            d = dense(t, n)
            out = g.batch_norm(d, rng.uniform(0.5, 1.5, n), rng.uniform(-0.2, 0.2, n), rng.uniform(-0.2, 0.2, n),
                               rng.uniform(0.5, 1.5, n), epsilon=1e-3, name=name("bn"))
        elif kind == 8:  # n-ary Mean / Sum of equal-width tensors
            same = [u for u in pool if g.size(u) == n and u != t]
            if not same:
                continue
            xs = [t] + [same[int(rng.integers(len(same)))] for _ in range(int(rng.integers(1, 3)))]
            out = g.nary(str(rng.choice(["Mean", "Sum"])), *xs)
        elif kind == 9:  # Dense reading a Gather or a Concat (an input map)
            if rng.random() < 0.5:
                idx = rng.integers(0, n, int(rng.choice(widths)))
                src = g.gather(t, idx)
            else:
                others = [u for u in pool if u != t]
                if not others:
                    continue
                other = others[int(rng.integers(len(others)))]
                if g.size(t) + g.size(other) > (16 if narrow else 96):
                    continue
                src = g.concat(t, other)
            out = dense(src, int(rng.choice(widths)))
        elif kind == 10:  # reduction of a pointwise chain (a mapped reduction), broadcast back
            op = str(rng.choice(["ReduceSum", "ReduceMean", "ReduceL2", "ReduceSumSquare", "ReduceMax", "ReduceL1"]))
            red = g.reduce(op, bounded_unary(t))
            out = g.binary("Sub", t, g.binary("Mul", red, const([0.1])))
        elif kind == 11:  # LpNormalization
            out = g.binary("Mul", g.node("LpNormalization", [t], n, {"axis": -1, "p": int(rng.choice([1, 2]))}),
                           const([2.0]))
        elif kind == 12:  # |x| through IsNaN(Sqrt(x)) (smooth), or IsInf / logic
            if smooth or rng.random() < 0.5:
                out = g.where(g.unary("IsNaN", g.unary("Sqrt", t)), g.unary("Neg", t), t)
            else:
                big = g.binary("Div", const([1.0]), g.binary("Sub", t, t))  # 1 / 0: inf, or NaN
                inf = g.node("IsInf", [big], n, {"detect_negative": 0, "detect_positive": 1})
                pos = g.compare("Greater", t, const([0.0]))
                both = g.binary("And", inf, pos)
                out = g.binary("Add", t, g.node("Cast", [g.binary("Xor", both, g.unary("Not", pos))], n, {"to": 1},
                                                dtype=G.DType(dtype)))
        else:  # step functions (fp32 / fp64 only), else a bounded unary
            if smooth:
                out = bounded_unary(t)
            else:
                op = str(rng.choice(_STEP))
                out = g.binary("Add", g.binary("Mul", t, const([0.01])),
                               g.unary(op, g.binary("Mul", t, const([3.0]))))
        pool.append(out)
    tail = pool[-1]
    if g.size(tail) == 1:
        tail = dense(tail, int(rng.choice(widths)))
    return g.finish(dense(tail, int(rng.choice([8, 16])) if aligned and not narrow else 5))


def in_domain_input(n_in: int, batch: int, seed: int) -> np.ndarray:
    """Inputs exactly representable in fp16 (so every precision reads the same values)."""
    x = np.random.default_rng(seed).standard_normal((n_in, batch))
    return x.astype(np.float16).astype(np.float64)


def forms_graph(dtype: str = "float32") -> G.Graph:
    """A fixed graph that makes the optimizer form the compound nodes the
    random ones may miss: a reduction over a reconverging pointwise region
    (map_region_steps), a residual Add + activation with no Dense operand
    (ResidualAddActivation), a comparison feeding Where (CompareSelect), a
    Dense over a Concat and a Gather (input_map) and an ElementwiseChain."""
    rng = np.random.default_rng(77)
    g = G.GraphBuilder(16, dtype=dtype)

    def dense(t, m, name):
        n = g.size(t)
        return g.dense(t, rng.uniform(-0.5, 0.5, (m, n)), rng.uniform(-0.2, 0.2, m), name=name)

    a = g.unary("Tanh", dense(g.input, 32, "fa"))
    b = g.unary("Sigmoid", dense(g.input, 32, "fb"))
    # region: sin(a) * cos(a) + a, reduced (map_region_steps)
    s = g.unary("Sin", a)
    c = g.unary("Cos", a)
    r = g.binary("Add", g.binary("Mul", s, c), a)
    red = g.reduce("ReduceSum", r)
    # residual add + activation of two non-dense tensors
    res = g.unary("Relu", g.binary("Add", a, b))
    # CompareSelect and a chain
    sel = g.where(g.compare("GreaterOrEqual", res, g.constant("thr", [0.3])), res, b)
    ch = g.unary("Atan", g.binary("Mul", g.unary("Softsign", sel), g.constant("k", [1.5])))
    # input map over a Concat and a Gather
    cat = g.concat(ch, a)
    d1 = dense(cat, 16, "fc")
    gat = g.gather(d1, [15, 0, 3, 3, 7, 9, 1, 2, 4, 5, 6, 8, 10, 11, 12, 13])
    d2 = dense(gat, 16, "fd")
    out = g.binary("Sub", d2, red)
    return g.finish(out)
