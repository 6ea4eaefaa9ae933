"""Vectorized float64 numpy evaluation of a canonical PONNI graph.

An independent formulation of the generated model's per-sample semantics,
used to pin the oracle's graph operations and the graph linearization: it
walks the DAG itself (no slots, no chain) over whole [features, batch]
arrays, following the reference's verification interpreter
(kokkos_nn/interpreter.py:15-131 for unary / binary operations, :195-400 for
nodes) with the broadcasting restricted to one-feature or exact operands.
"""
from __future__ import annotations

import math

import numpy as np
from scipy.special import erf


def unary(op: str, v: np.ndarray, attrs: dict) -> np.ndarray:
    if op == "Relu":
        return np.maximum(v, 0)
    if op == "Sigmoid":
        return 0.5 * (1 + np.tanh(0.5 * v))  # = 1 / (1 + e^-v) without overflow
    if op == "Tanh":
        return np.tanh(v)
    if op == "LeakyRelu":
        return np.where(v >= 0, v, float(attrs.get("alpha", 0.01)) * v)
    if op == "Elu":
        return np.where(v >= 0, v, float(attrs.get("alpha", 1.0)) * np.expm1(np.minimum(v, 0)))
    if op == "Celu":
        a = float(attrs.get("alpha", 1.0))
        return np.maximum(v, 0) + np.minimum(0, a * np.expm1(np.minimum(v, 0) / a))
    if op == "Selu":
        a = float(attrs.get("alpha", 1.6732631921768188))
        g = float(attrs.get("gamma", 1.0507010221481323))
        return g * np.where(v > 0, v, a * np.expm1(np.minimum(v, 0)))
    if op == "Gelu":
        if attrs.get("approximate", "none") == "tanh":
            return 0.5 * v * (1 + np.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))
        return 0.5 * v * (1 + erf(v / math.sqrt(2)))
    if op == "Silu":
        return v * 0.5 * (1 + np.tanh(0.5 * v))
    if op == "Softplus":
        return np.logaddexp(v, 0)
    if op == "Softsign":
        return v / (1 + np.abs(v))
    if op == "ThresholdedRelu":
        return np.where(v > float(attrs.get("alpha", 1.0)), v, 0)
    if op == "HardSigmoid":
        return np.clip(float(attrs.get("alpha", 0.2)) * v + float(attrs.get("beta", 0.5)), 0, 1)
    if op == "HardSwish":
        return v * np.clip(v / 6 + 0.5, 0, 1)
    if op == "Mish":
        return v * np.tanh(np.logaddexp(v, 0))
    if op == "IsInf":
        neg = np.isneginf(v) & bool(int(attrs.get("detect_negative", 1)))
        pos = np.isposinf(v) & bool(int(attrs.get("detect_positive", 1)))
        return (neg | pos).astype(np.float64)
    if op == "Round":  # ties to even (emitter.py:1659-1667)
        return np.rint(v)
    table = {"Abs": np.abs, "Neg": np.negative, "Exp": np.exp, "Log": np.log, "Sqrt": np.sqrt,
             "Reciprocal": np.reciprocal, "Erf": erf, "Acos": np.arccos, "Acosh": np.arccosh, "Asin": np.arcsin,
             "Asinh": np.arcsinh, "Atan": np.arctan, "Atanh": np.arctanh, "Ceil": np.ceil, "Cos": np.cos,
             "Cosh": np.cosh, "Floor": np.floor, "Sin": np.sin, "Sinh": np.sinh, "Tan": np.tan, "Sign": np.sign,
             "IsNaN": lambda a: np.isnan(a).astype(np.float64), "Not": lambda a: (a == 0).astype(np.float64)}
    return table[op](v)


def binary(op: str, a: np.ndarray, b: np.ndarray, n: int) -> np.ndarray:
    for x in (a, b):
        if x.shape[0] not in (1, n):
            raise ValueError(f"unsupported {op} broadcasting")
    if op in LOGIC:  # booleans are 1 / 0; any nonzero operand is true
        return LOGIC[op](a != 0, b != 0).astype(np.float64)
    if op in COMPARE:
        return COMPARE[op](a, b).astype(np.float64)
    if op == "PRelu":
        return np.where(a >= 0, a, a * b)
    return {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide, "Min": np.minimum,
            "Max": np.maximum, "Pow": np.power}[op](a, b)


COMPARE = {"Equal": np.equal, "Greater": np.greater, "GreaterOrEqual": np.greater_equal, "Less": np.less,
           "LessOrEqual": np.less_equal}
LOGIC = {"And": np.logical_and, "Or": np.logical_or, "Xor": np.logical_xor}
BINARY = {"Add", "Sub", "Mul", "Div", "Min", "Max", "Pow", "PRelu"} | set(COMPARE) | set(LOGIC)


def pointwise(op: str, ops: list, attrs: dict, n: int, ftype=np.float64) -> np.ndarray:
    """One operation of a fused pointwise program or a plain pointwise node.
    ftype: the graph's scalar type, in which a BatchNormalization denominator
    sqrt(var + eps) is evaluated (the emitted Scalar arithmetic)."""
    if op in BINARY:
        return binary(op, ops[0], ops[1], n)
    if op == "Cast":
        return ops[0]
    if op in ("Mean", "Sum"):
        acc = ops[0]
        for o in ops[1:]:
            acc = acc + o
        return acc / len(ops) if op == "Mean" else acc
    if op == "Where":
        return np.where(ops[0] != 0, ops[1], ops[2])
    if op == "CompareSelect":
        return np.where(COMPARE[attrs["comparison"]](ops[0], ops[1]), ops[2], ops[3])
    if op == "Clip":
        lo = ops[1] if len(ops) > 1 else attrs.get("min")
        hi = ops[2] if len(ops) > 2 else attrs.get("max")
        v = ops[0]
        if lo is not None:
            v = np.where(v < lo, lo, v)
        if hi is not None:
            v = np.where(v > hi, hi, v)
        return v
    if op == "BatchNormalization":
        x, scale, bias, mean, var = ops
        den = np.sqrt(var.astype(ftype) + ftype(float(attrs.get("epsilon", 1e-5)))).astype(np.float64)
        return (x - mean) / den * scale + bias
    return unary(op, ops[0], attrs)


def chain(steps: list, prev, get, n: int, ftype=np.float64):
    cur = prev
    for st in steps:
        cur = pointwise(st["op"], [cur if v == "prev" else get(int(v)) for v in st["inputs"]],
                        st.get("attributes", {}), n, ftype)
    return cur


def run_graph(graph, x: np.ndarray) -> np.ndarray:
    """graph: ponni_amd.graph.Graph; x [n_in, B] -> [n_out, B] in float64."""
    T = graph.tensors
    vals: dict[int, np.ndarray] = {graph.inputs[0]: np.asarray(x, dtype=np.float64)}
    ftype = np.float32 if T[graph.inputs[0]].dtype.value == "float32" else np.float64

    def get(t: int) -> np.ndarray:
        if T[t].is_constant:
            return np.asarray(graph.constants[T[t].constant_name].values, dtype=np.float64).reshape(-1, 1)
        return vals[t]

    def region(steps: list, n: int) -> dict:
        local: dict = {}
        for st in steps:
            def rget(t, local=local):
                return local[t] if t in local else get(t)
            if st["op"] == "ElementwiseChain":
                v = chain(st["attributes"]["steps"], None, rget, n, ftype)
            else:
                v = pointwise(st["op"], [rget(int(t)) for t in st["inputs"]], st.get("attributes", {}), n, ftype)
            local[int(st["outputs"][0])] = v
        return local

    for n in graph.nodes:
        ins = n.inputs
        size = T[n.outputs[0]].sample_size
        op = n.op
        if op in ("Dense", "DenseBiasActivation", "DenseResidualActivation", "DenseEpilogue"):
            w = np.asarray(graph.constants[T[n.attributes["weight"]].constant_name].values, dtype=np.float64)
            if "input_map" in n.attributes:
                batch = vals[graph.inputs[0]].shape[1]
                xin = np.stack([np.broadcast_to(get(int(e["tensor"]))[int(e["index"])], (batch,))
                                for e in n.attributes["input_map"]])
            else:
                xin = get(ins[0])
            r = w.reshape(size, -1) @ xin
            if n.attributes.get("bias") is not None:
                r = r + get(n.attributes["bias"])
            aattrs = n.attributes.get("activation_attributes", {})
            if op == "DenseBiasActivation":
                r = unary(n.attributes["activation"], r, aattrs)
            elif op == "DenseResidualActivation":
                r = unary(n.attributes["activation"], r + get(int(n.attributes["residual"])), aattrs)
            elif op == "DenseEpilogue":
                r = chain(n.attributes["epilogue_steps"], r, get, size, ftype)
        elif op in BINARY:
            r = binary(op, get(ins[0]), get(ins[1]), size)
        elif op == "ResidualAddActivation":
            r = unary(n.attributes["activation"], get(ins[0]) + get(ins[1]), n.attributes.get("activation_attributes", {}))
        elif op == "ElementwiseChain":
            r = chain(n.attributes["steps"], None, get, size, ftype)
        elif op == "PointwiseRegion":
            r = region(n.attributes["steps"], size)[n.outputs[0]]
        elif op == "Gather":
            r = get(ins[0])[[int(i) for i in n.attributes["indices"]]]
        elif op == "LpNormalization":
            v = get(ins[0])
            norm = np.abs(v).sum(axis=0) if int(n.attributes.get("p", 2)) == 1 else np.sqrt((v * v).sum(axis=0))
            with np.errstate(invalid="ignore", divide="ignore"):
                r = np.where(norm == 0, 0.0, v / np.where(norm == 0, 1.0, norm))
        elif op == "Concat":
            r = np.concatenate([get(t) for t in ins], axis=0)
        elif op in ("Identity", "Flatten", "Reshape", "Squeeze", "Unsqueeze"):
            r = get(ins[0])
        elif op in ("Softmax", "LogSoftmax"):
            v = get(ins[0])
            sh = v - v.max(axis=0, keepdims=True)
            lse = np.log(np.exp(sh).sum(axis=0, keepdims=True))
            r = sh - lse if op == "LogSoftmax" else np.exp(sh - lse)
        elif op == "LayerNormalization":
            v = get(ins[0])
            mean = v.mean(axis=0, keepdims=True)
            r = (v - mean) / np.sqrt(((v - mean) ** 2).mean(axis=0, keepdims=True) + float(n.attributes.get("epsilon", 1e-5)))
            r = r * get(ins[1])
            if len(ins) == 3:
                r = r + get(ins[2])
        elif op.startswith("Reduce"):
            if "map_steps" in n.attributes:
                v = chain(n.attributes["map_steps"], None, get, int(n.attributes["map_size"]), ftype)
            elif "map_region_steps" in n.attributes:
                v = region(n.attributes["map_region_steps"], int(n.attributes["map_size"]))[
                    int(n.attributes["map_output"])]
            else:
                v = get(ins[0])
            if op == "ReduceSum":
                r = v.sum(axis=0)
            elif op == "ReduceMean":
                r = v.mean(axis=0)
            elif op == "ReduceMax":
                r = v.max(axis=0)
            elif op == "ReduceMin":
                r = v.min(axis=0)
            elif op == "ReduceL1":
                r = np.abs(v).sum(axis=0)
            elif op == "ReduceL2":
                r = np.sqrt((v ** 2).sum(axis=0))
            elif op == "ReduceSumSquare":
                r = (v ** 2).sum(axis=0)
            elif op == "ReduceLogSum":
                r = np.log(v.sum(axis=0))
            elif op == "ReduceLogSumExp":
                m = v.max(axis=0)
                r = m + np.log(np.exp(v - m).sum(axis=0))
            elif op == "ReduceProd":
                r = v.prod(axis=0)
            else:
                raise ValueError(op)
            r = r.reshape(1, -1)
        else:
            r = pointwise(op, [get(t) for t in ins], n.attributes, size, ftype)
        if r.shape[0] != size:
            r = np.broadcast_to(r, (size, r.shape[1])).copy()
        vals[n.outputs[0]] = r
    return vals[graph.outputs[0]]
