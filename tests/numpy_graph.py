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
    table = {"Abs": np.abs, "Neg": np.negative, "Exp": np.exp, "Log": np.log, "Sqrt": np.sqrt,
             "Reciprocal": np.reciprocal, "Erf": erf}
    return table[op](v)


def binary(op: str, a: np.ndarray, b: np.ndarray, n: int) -> np.ndarray:
    for x in (a, b):
        if x.shape[0] not in (1, n):
            raise ValueError(f"unsupported {op} broadcasting")
    return {"Add": np.add, "Sub": np.subtract, "Mul": np.multiply, "Div": np.divide, "Min": np.minimum,
            "Max": np.maximum, "Pow": np.power}[op](a, b)


def run_graph(graph, x: np.ndarray) -> np.ndarray:
    """graph: ponni_amd.graph.Graph; x [n_in, B] -> [n_out, B] in float64."""
    T = graph.tensors
    vals: dict[int, np.ndarray] = {graph.inputs[0]: np.asarray(x, dtype=np.float64)}

    def get(t: int) -> np.ndarray:
        if T[t].is_constant:
            return np.asarray(graph.constants[T[t].constant_name].values, dtype=np.float64).reshape(-1, 1)
        return vals[t]

    for n in graph.nodes:
        ins = n.inputs
        size = T[n.outputs[0]].sample_size
        op = n.op
        if op == "Dense":
            w = np.asarray(graph.constants[T[n.attributes["weight"]].constant_name].values, dtype=np.float64)
            r = w.reshape(size, -1) @ get(ins[0])
            if n.attributes.get("bias") is not None:
                r = r + get(n.attributes["bias"])
        elif op in ("Add", "Sub", "Mul", "Div", "Min", "Max", "Pow"):
            r = binary(op, get(ins[0]), get(ins[1]), size)
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
            r = unary(op, get(ins[0]), n.attributes)
        if r.shape[0] != size:
            r = np.broadcast_to(r, (size, r.shape[1])).copy()
        vals[n.outputs[0]] = r
    return vals[graph.outputs[0]]
