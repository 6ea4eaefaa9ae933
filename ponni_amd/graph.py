"""Generated-model path: PONNI's canonical graph IR, its lowering onto
libponni_hip, and the generated model class API.

The reference's generator (kokkos_nn) imports ONNX into a small canonical IR
(kokkos_nn/ir.py), optimizes it, and emits a C++ header whose infer_batch runs
one thread per sample over the emitted node bodies (kokkos_nn/emitter.py:
1537-1573, 1903-1953).  Here the same IR is the input, and instead of
emitting per-sample code the graph is *linearized* into a PONNI layer chain
with saved-state slots -- the template path's own vocabulary plus the graph
operations of include/ponni_hip.h (Dense, Load_State, Binary, Reduce, Unary,
Const_Binary) -- so every kernel family of libponni_hip, and in particular the
FUSED generator (one MFMA kernel per graph, compiled by hipRTC), runs it.

    g = GraphBuilder(24)
    a = g.dense(g.input, wa, ba); a = g.unary("Relu", a)
    ...
    model = GeneratedModel(g.finish(out))
    model.infer_batch(x, y)          # x [24, B], y [n_out, B] on the GPU

The IR classes keep ir.py's field names and to_dict() layout, so
graph_fingerprint (kokkos_nn/weights.py:85-92) is computed over the same
JSON.  ONNX import is out of scope (onnx is not installed); graphs are built
directly.
"""
from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass, field
from enum import Enum
from typing import Any, Callable

import numpy as np

from . import _abi as A
from .model import Inference, Layer


class GraphError(ValueError):
    """A graph the lowering cannot express (kokkos_nn.errors.CompilerError)."""


# ---- canonical IR (kokkos_nn/ir.py) -------------------------------------------

class DType(str, Enum):
    BOOL = "bool"
    FLOAT32 = "float32"
    FLOAT64 = "float64"
    INT32 = "int32"
    INT64 = "int64"


@dataclass(frozen=True)
class Symbol:
    """A symbolic dimension: only the batch axis (ir.py:27-30)."""
    name: str


@dataclass
class ConstantTensor:
    name: str
    shape: tuple
    dtype: DType
    values: np.ndarray = field(repr=False)
    canonical_layout: str = "onnx"
    learned: bool = False

    def to_dict(self) -> dict[str, Any]:
        return {"name": self.name, "shape": list(self.shape), "dtype": self.dtype.value,
                "canonical_layout": self.canonical_layout, "learned": self.learned}


@dataclass
class TensorValue:
    id: int
    name: str
    shape: tuple
    dtype: DType
    producer: int | None = None
    consumers: list = field(default_factory=list)
    is_input: bool = False
    is_output: bool = False
    is_constant: bool = False
    constant_name: str | None = None

    @property
    def sample_shape(self) -> tuple:
        return tuple(d for d in self.shape if isinstance(d, int))

    @property
    def sample_size(self) -> int:
        n = 1
        for d in self.sample_shape:
            n *= d
        return n

    def to_dict(self) -> dict[str, Any]:
        return {"id": self.id, "name": self.name,
                "shape": [d.name if isinstance(d, Symbol) else d for d in self.shape],
                "dtype": self.dtype.value, "producer": self.producer, "consumers": list(self.consumers),
                "is_input": self.is_input, "is_output": self.is_output, "is_constant": self.is_constant,
                "constant_name": self.constant_name}


@dataclass
class Node:
    id: int
    op: str
    inputs: list
    outputs: list
    attributes: dict = field(default_factory=dict)
    source_name: str = ""

    def to_dict(self) -> dict[str, Any]:
        return {"id": self.id, "op": self.op, "inputs": list(self.inputs), "outputs": list(self.outputs),
                "attributes": json.loads(json.dumps(self.attributes)), "source_name": self.source_name}


@dataclass
class Graph:
    inputs: list
    outputs: list
    tensors: dict
    nodes: list
    constants: dict
    metadata: dict = field(default_factory=dict)

    def rebuild_links(self) -> None:
        for t in self.tensors.values():
            t.producer = None
            t.consumers = []
        for n in self.nodes:
            for t in n.inputs:
                self.tensors[t].consumers.append(n.id)
            for t in n.outputs:
                self.tensors[t].producer = n.id

    def to_dict(self) -> dict[str, Any]:
        return {"inputs": self.inputs, "outputs": self.outputs,
                "tensors": {str(k): v.to_dict() for k, v in sorted(self.tensors.items())},
                "nodes": [n.to_dict() for n in self.nodes],
                "constants": {k: v.to_dict() for k, v in sorted(self.constants.items())},
                "metadata": self.metadata}

    def to_json(self) -> str:
        return json.dumps(self.to_dict(), indent=2, sort_keys=True)

    def size(self, tensor_id: int) -> int:
        return self.tensors[tensor_id].sample_size


def fnv1a64(data: bytes) -> int:
    """FNV-1a-64 (kokkos_nn/weights.py:50-56)."""
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def graph_fingerprint(graph: Graph) -> str:
    """Fingerprint of the graph schema without weight values (weights.py:85-92)."""
    data = graph.to_dict()
    data["metadata"] = {}
    canonical = json.dumps(data, sort_keys=True, separators=(",", ":"))
    text = "ponni-generated-model-v1\n" + canonical
    return f"fnv1a64:{fnv1a64(text.encode('utf-8')):016x}"


def graph_from_dict(data: dict) -> Graph:
    """A Graph from its to_dict() form, the canonical_ir.json the reference
    compiler writes next to every generated header (kokkos_nn/compiler.py:316,
    ir.py:137-148).  The JSON holds no constant values: every constant starts
    at zero in its declared shape and is filled by load_weights."""
    tensors: dict[int, TensorValue] = {}
    for key, t in data["tensors"].items():
        shape = tuple(Symbol(d) if isinstance(d, str) else int(d) for d in t["shape"])
        tensors[int(key)] = TensorValue(int(t["id"]), t["name"], shape, DType(t["dtype"]), t.get("producer"),
                                        list(t.get("consumers", [])), bool(t.get("is_input", False)),
                                        bool(t.get("is_output", False)), bool(t.get("is_constant", False)),
                                        t.get("constant_name"))
    nodes = [Node(int(n["id"]), n["op"], [int(i) for i in n["inputs"]], [int(o) for o in n["outputs"]],
                  dict(n.get("attributes", {})), n.get("source_name", "")) for n in data["nodes"]]
    constants = {}
    for name, c in data["constants"].items():
        dtype = DType(c["dtype"])
        npt = {DType.FLOAT32: np.float32, DType.FLOAT64: np.float64, DType.INT32: np.int32,
               DType.INT64: np.int64, DType.BOOL: np.bool_}[dtype]
        shape = tuple(int(d) for d in c["shape"])
        constants[name] = ConstantTensor(c["name"], shape, dtype, np.zeros(shape, dtype=npt),
                                         c.get("canonical_layout", "onnx"), bool(c.get("learned", False)))
    g = Graph([int(i) for i in data["inputs"]], [int(o) for o in data["outputs"]], tensors, nodes, constants,
              dict(data.get("metadata", {})))
    g.rebuild_links()
    return g


def load_canonical_ir(path) -> Graph:
    """Read a canonical_ir.json file (graph_from_dict)."""
    with open(path, encoding="utf-8") as f:
        return graph_from_dict(json.load(f))


# ---- building graphs ------------------------------------------------------------

class GraphBuilder:
    """Builds a canonical graph directly (the importer's output form): Dense
    nodes carry [out, in] weights ("output_input", passes.py:341-346) and an
    optional bias as constant inputs."""

    def __init__(self, num_inputs: int, dtype: str = "float32", input_name: str = "input"):
        self.dtype = DType(dtype)
        self.tensors: dict[int, TensorValue] = {}
        self.nodes: list[Node] = []
        self.constants: dict[str, ConstantTensor] = {}
        self.batch = Symbol("batch")
        self.input = self._tensor(input_name, num_inputs)
        self.tensors[self.input].is_input = True

    def _tensor(self, name: str, size: int) -> int:
        tid = len(self.tensors)
        self.tensors[tid] = TensorValue(tid, name, (self.batch, int(size)), self.dtype)
        return tid

    def constant(self, name: str, values, layout: str = "onnx", learned: bool = True) -> int:
        npt = np.float32 if self.dtype == DType.FLOAT32 else np.float64
        v = np.asarray(values, dtype=npt)
        if name in self.constants:
            raise GraphError(f"duplicate constant {name!r}")
        self.constants[name] = ConstantTensor(name, tuple(int(d) for d in v.shape), self.dtype, v, layout, learned)
        tid = len(self.tensors)
        self.tensors[tid] = TensorValue(tid, name, tuple(int(d) for d in v.shape), self.dtype, is_constant=True,
                                        constant_name=name)
        return tid

    def node(self, op: str, inputs: list, size: int, attributes: dict | None = None, name: str = "",
             dtype: DType | None = None) -> int:
        """A node with one output of `size` features; the output is boolean
        for comparisons, logic and predicates, else the graph's type."""
        nid = len(self.nodes)
        out = self._tensor(name or f"{op.lower()}_{nid}", size)
        if dtype is None and op in _BOOL_OPS:
            dtype = DType.BOOL
        if dtype is not None:
            self.tensors[out].dtype = DType(dtype)
        self.nodes.append(Node(nid, op, list(inputs), [out], dict(attributes or {}), name))
        return out

    def dense(self, x: int, weight, bias=None, name: str = "") -> int:
        w = np.asarray(weight)
        if w.ndim != 2 or w.shape[1] != self.size(x):
            raise GraphError(f"dense weight shape {w.shape} does not take {self.size(x)} inputs")
        name = name or f"dense_{len(self.nodes)}"
        wid = self.constant(f"{name}.weight", w, "output_input")
        inputs, bid = [x, wid], None
        if bias is not None:
            bid = self.constant(f"{name}.bias", np.asarray(bias).reshape(-1), "output")
            inputs.append(bid)
        return self.node("Dense", inputs, w.shape[0], {"weight": wid, "bias": bid}, name)

    def unary(self, op: str, x: int, **attributes) -> int:
        return self.node(op, [x], self.size(x), attributes)

    def binary(self, op: str, a: int, b: int) -> int:
        return self.node(op, [a, b], max(self.size(a), self.size(b)))

    def concat(self, *xs: int) -> int:
        return self.node("Concat", list(xs), sum(self.size(x) for x in xs), {"axis": 1})

    def reduce(self, op: str, x: int) -> int:
        return self.node(op, [x], 1, {"keepdims": 1})

    def softmax(self, x: int, log: bool = False) -> int:
        return self.node("LogSoftmax" if log else "Softmax", [x], self.size(x), {"axis": -1})

    def compare(self, op: str, a: int, b: int) -> int:
        """Equal / Greater / GreaterOrEqual / Less / LessOrEqual (boolean output)."""
        return self.node(op, [a, b], max(self.size(a), self.size(b)))

    def where(self, cond: int, a: int, b: int) -> int:
        return self.node("Where", [cond, a, b], max(self.size(cond), self.size(a), self.size(b)))

    def nary(self, op: str, *xs: int) -> int:
        """Mean or Sum of tensors of one or the same number of features."""
        return self.node(op, list(xs), max(self.size(x) for x in xs))

    def clip(self, x: int, lo: float | None = None, hi: float | None = None) -> int:
        """Clip with attribute bounds (either may be absent)."""
        attrs = {}
        if lo is not None:
            attrs["min"] = float(lo)
        if hi is not None:
            attrs["max"] = float(hi)
        return self.node("Clip", [x], self.size(x), attrs)

    def gather(self, x: int, indices) -> int:
        idx = [int(i) for i in indices]
        return self.node("Gather", [x], len(idx), {"axis": 1, "indices": idx})

    def batch_norm(self, x: int, scale, bias, mean, var, epsilon: float = 1e-5, name: str = "") -> int:
        name = name or f"batch_norm_{len(self.nodes)}"
        ins = [x] + [self.constant(f"{name}.{k}", np.asarray(v).reshape(-1), "output", learned=k in ("scale", "bias"))
                     for k, v in (("scale", scale), ("bias", bias), ("mean", mean), ("var", var))]
        return self.node("BatchNormalization", ins, self.size(x), {"epsilon": float(epsilon)}, name)

    def layer_norm(self, x: int, scale, bias=None, epsilon: float = 1e-5, name: str = "") -> int:
        name = name or f"layer_norm_{len(self.nodes)}"
        ins = [x, self.constant(f"{name}.scale", np.asarray(scale).reshape(-1))]
        if bias is not None:
            ins.append(self.constant(f"{name}.bias", np.asarray(bias).reshape(-1)))
        return self.node("LayerNormalization", ins, self.size(x), {"epsilon": float(epsilon)}, name)

    def size(self, tid: int) -> int:
        return self.tensors[tid].sample_size

    def finish(self, output: int) -> Graph:
        self.tensors[output].is_output = True
        g = Graph([self.input], [output], self.tensors, self.nodes, self.constants, {"builder": "ponni_amd"})
        g.rebuild_links()
        return g


# ---- lowering: graph -> layer chain ----------------------------------------------

_ALIASES = {"Identity", "Flatten", "Reshape", "Squeeze", "Unsqueeze"}
_TEMPLATE_ACTIVATIONS = {"Relu", "Sigmoid", "Tanh", "LeakyRelu", "Elu", "Gelu", "Silu", "Softplus", "HardSigmoid",
                         "HardSwish", "Mish"}
_DENSE_OPS = {"Dense", "DenseBiasActivation", "DenseResidualActivation", "DenseEpilogue"}


def _unary_layer(op: str, n: int, attrs: dict) -> Layer:
    """A unary node as a pointwise layer; formulas of emitter.py:218-258."""
    if op == "Relu":
        return Layer(A.LAYER_RELU, n, n, label="ReLU")
    if op == "Sigmoid":
        return Layer(A.LAYER_SIGMOID, n, n, label="Sigmoid")
    if op == "Tanh":
        return Layer(A.LAYER_TANH, n, n, label="Tanh")
    if op == "LeakyRelu":
        return Layer(A.LAYER_LEAKY_RELU, n, n, attr=(float(attrs.get("alpha", 0.01)), 0, 0, 0), label="LeakyReLU")
    if op == "Elu":
        return Layer(A.LAYER_ELU, n, n, attr=(float(attrs.get("alpha", 1.0)), 0, 0, 0), label="ELU")
    if op == "Gelu":
        approx = str(attrs.get("approximate", "none")) == "tanh"
        return Layer(A.LAYER_GELU, n, n, flags=A.FLAG_GELU_APPROXIMATE if approx else 0, label="GELU")
    if op == "Silu":
        return Layer(A.LAYER_SILU, n, n, label="SiLU")
    if op == "Softplus":
        return Layer(A.LAYER_SOFTPLUS, n, n, attr=(1.0, 0, 0, 0), label="Softplus")
    if op == "HardSigmoid":
        return Layer(A.LAYER_HARD_SIGMOID, n, n,
                     attr=(float(attrs.get("alpha", 0.2)), float(attrs.get("beta", 0.5)), 0, 0), label="HardSigmoid")
    if op == "HardSwish":
        return Layer(A.LAYER_HARD_SWISH, n, n, label="HardSwish")
    if op == "Mish":
        return Layer(A.LAYER_MISH, n, n, label="Mish")
    if op == "IsInf":
        return Layer(A.LAYER_UNARY, n, n, attr=(A.UNARY_OPS[op], float(int(attrs.get("detect_negative", 1))),
                                               float(int(attrs.get("detect_positive", 1))), 0), label=op)
    if op in A.UNARY_OPS:
        alpha = float(attrs.get("alpha", 1.6732631921768188 if op == "Selu" else 1.0))
        gamma = float(attrs.get("gamma", 1.0507010221481323))
        return Layer(A.LAYER_UNARY, n, n, attr=(A.UNARY_OPS[op], alpha, gamma, 0), label=op)
    raise GraphError(f"no lowering for unary operation {op}")


@dataclass
class _Param:
    """How a layer's parameter vector is built from the graph constants."""
    build: Callable[[dict], np.ndarray]


class LoweredGraph:
    """A graph as a layer chain (`layers`) plus, per layer, the function that
    rebuilds its parameters from a {constant name: array} mapping.  `derived`
    holds the constants the expansion introduced (a Mean's divisor, a
    BatchNormalization denominator ...) as functions of that mapping."""

    def __init__(self, layers: list[Layer], params: list[_Param | None], notes: list[str],
                 derived: dict[str, Callable[[dict], np.ndarray]] | None = None):
        self.layers = layers
        self.params = params
        self.notes = notes
        self.derived = derived or {}

    def layer_params(self, constants: dict) -> list[np.ndarray]:
        c = dict(constants)
        for name, f in self.derived.items():
            c[name] = f(c)
        return [p.build(c) if p is not None else np.zeros(0) for p in self.params]


# Operations the layer chain takes as they are after expansion.
_ELEM_BINARY = set(A.BINARY_OPS)
_ELEM_UNARY = _TEMPLATE_ACTIVATIONS | set(A.UNARY_OPS)
_COMPARISONS = {"Equal", "Greater", "GreaterOrEqual", "Less", "LessOrEqual"}
_BOOL_OPS = _COMPARISONS | {"And", "Or", "Xor", "Not", "IsNaN", "IsInf"}


@dataclass
class _Expanded:
    nodes: list
    alias: dict
    tensors: dict
    derived: dict


def _expand(graph: Graph) -> _Expanded:
    """Rewrite the graph into the operations the layer chain takes.

    Aliases resolve away (and Cast, which keeps the value: interpreter.py:
    157-159, a boolean being 1 / 0); the optimizer's compound forms split into
    their elementary steps in evaluation order: the fused Dense variants
    (interpreter.py:353-381), ResidualAddActivation, ElementwiseChain,
    PointwiseRegion and the mapped reductions (interpreter.py:206-237, :389-
    425), CompareSelect, Clip, PRelu, n-ary Mean / Sum, BatchNormalization,
    LpNormalization (interpreter.py:136-193, :344-351).  A Dense input_map
    becomes a Dense over the concatenation of the tensors it reads, its
    weight columns summed per source element (and constant entries folded
    into the bias); a lone Gather becomes a Dense with one-hot rows.  Both
    read unselected elements with weight 0, so a non-finite unselected
    element (0 * inf) spoils the output where the reference skips it.

    The graph itself is not modified: new tensors go into a copy of its
    tensor table."""
    alias: dict[int, int] = {}
    tensors = dict(graph.tensors)
    derived: dict[str, Callable[[dict], np.ndarray]] = {}
    nodes: list[Node] = []
    fdtype = graph.tensors[graph.inputs[0]].dtype
    npt = np.float32 if fdtype == DType.FLOAT32 else np.float64
    next_tensor = max(tensors) + 1

    def r(t: int) -> int:
        while t in alias:
            t = alias[t]
        return t

    def size(t: int) -> int:
        return tensors[t].sample_size

    def new_tensor(n: int, name: str, dtype: DType | None = None) -> int:
        nonlocal next_tensor
        tid = next_tensor
        next_tensor += 1
        tensors[tid] = TensorValue(tid, name, (Symbol("batch"), int(n)), dtype or fdtype)
        return tid

    def derived_constant(n: int, name: str, f: Callable[[dict], np.ndarray]) -> int:
        """A constant tensor of n values computed from the graph constants."""
        nonlocal next_tensor
        tid = next_tensor
        next_tensor += 1
        cname = f"__ponni_derived_{tid}"
        tensors[tid] = TensorValue(tid, name, (int(n),), fdtype, is_constant=True, constant_name=cname)
        derived[cname] = f
        return tid

    def literal(values, name: str) -> int:
        v = np.asarray(values, dtype=np.float64).reshape(-1)
        return derived_constant(v.size, name, lambda c, v=v: v)

    def cvalues(c: dict, t: int) -> np.ndarray:
        return np.asarray(c[tensors[t].constant_name], dtype=np.float64).reshape(-1)

    def add(op: str, ins: list, out: int, attrs: dict | None = None, src: Node | None = None) -> None:
        nodes.append(Node(src.id if src else -1, op, list(ins), [out], dict(attrs or {}),
                          src.source_name if src else ""))

    def out_for(op: str, ins: list, out: int | None, label: str) -> int:
        if out is not None:
            return out
        n = max(size(t) for t in ins)
        return new_tensor(n, f"{label}.{op}", DType.BOOL if op in _BOOL_OPS else None)

    def pointwise(op: str, ins: list, attrs: dict, out: int | None, label: str, src: Node | None) -> int:
        """Emit one pointwise operation (interpreter.py _pointwise_step); returns its tensor."""
        ins = [r(t) for t in ins]
        if op == "Cast":
            if out is None:
                return ins[0]
            alias[out] = ins[0]
            return ins[0]
        if op in _ELEM_BINARY and len(ins) == 2:
            out = out_for(op, ins, out, label)
            add(op, ins, out, {}, src)
            return out
        if op == "IsInf":
            out = out_for(op, ins, out, label)
            add(op, ins, out, {"detect_negative": int(attrs.get("detect_negative", 1)),
                               "detect_positive": int(attrs.get("detect_positive", 1))}, src)
            return out
        if op in _ELEM_UNARY and len(ins) == 1:
            out = out_for(op, ins, out, label)
            add(op, ins, out, attrs, src)
            return out
        if op in ("Mean", "Sum"):
            acc = ins[0]
            for k, t in enumerate(ins[1:]):
                last = op == "Sum" and k == len(ins) - 2
                acc = pointwise("Add", [acc, t], {}, out if last else None, label, src)
            if op == "Mean":
                acc = pointwise("Div", [acc, literal([len(ins)], f"{label}.count")], {}, out, label, src)
            elif len(ins) == 1 and out is not None:
                alias[out] = acc
            return acc
        if op == "Where":
            out = out_for(op, ins, out, label)
            add("Where", ins, out, {}, src)
            return out
        if op == "CompareSelect":
            cond = pointwise(str(attrs["comparison"]), ins[:2], {}, None, label, src)
            return pointwise("Where", [cond, ins[2], ins[3]], {}, out, label, src)
        if op == "Clip":
            # value < lo ? lo : value, then value > hi ? hi : value: the
            # constant on the left keeps a NaN (emitter.py:823-835, np.clip).
            lo = ins[1] if len(ins) > 1 else (literal([attrs["min"]], f"{label}.min") if "min" in attrs else None)
            hi = ins[2] if len(ins) > 2 else (literal([attrs["max"]], f"{label}.max") if "max" in attrs else None)
            v = ins[0]
            if lo is None and hi is None:
                if out is not None:
                    alias[out] = v
                return v
            if lo is not None:
                v = pointwise("Max", [lo, v], {}, out if hi is None else None, label, src)
            if hi is not None:
                v = pointwise("Min", [hi, v], {}, out, label, src)
            return v
        if op == "BatchNormalization":
            # (x - mean) / sqrt(var + eps) * scale + bias (emitter.py:890-900)
            x, scale, bias, mean, var = ins
            eps = float(attrs.get("epsilon", 1e-5))
            if tensors[var].is_constant:
                def denom(c, var=var, eps=eps):
                    v = cvalues(c, var).astype(npt)
                    return np.sqrt(v + npt(eps)).astype(np.float64)
                den = derived_constant(size(var), f"{label}.denominator", denom)
            else:
                den = pointwise("Sqrt", [pointwise("Add", [var, literal([eps], f"{label}.eps")], {}, None, label,
                                                   src)], {}, None, label, src)
            v = pointwise("Sub", [x, mean], {}, None, label, src)
            v = pointwise("Div", [v, den], {}, None, label, src)
            v = pointwise("Mul", [v, scale], {}, None, label, src)
            return pointwise("Add", [v, bias], {}, out, label, src)
        if op == "ElementwiseChain":
            return chain(attrs["steps"], None, out, label, src)
        raise GraphError(f"no lowering for pointwise operation {op}")

    def chain(steps: list, prev: int | None, out: int | None, label: str, src: Node | None,
              local: dict | None = None) -> int:
        """Ordered steps whose operand "prev" is the previous step's value;
        `local` maps a region's own tensor ids to the emitted ones."""
        local = local or {}
        cur = prev
        for k, st in enumerate(steps):
            ins = [cur if v == "prev" else local.get(int(v), int(v)) for v in st["inputs"]]
            cur = pointwise(st["op"], ins, dict(st.get("attributes", {})), out if k == len(steps) - 1 else None,
                            label, src)
        return cur

    def region(steps: list, label: str, src: Node | None, final: int | None = None) -> dict:
        """A PointwiseRegion's steps (each naming its output tensor); the
        intermediate tensors of the region are made anew.  Returns the map
        from the region's tensor ids to the ones emitted."""
        local: dict[int, int] = {}
        for st in steps:
            ins = [local.get(int(v), int(v)) for v in st["inputs"]]
            target = int(st["outputs"][0])
            out = final if target == final else None
            if st["op"] == "ElementwiseChain":
                res = chain(st["attributes"]["steps"], None, out, label, src, local)
            else:
                res = pointwise(st["op"], ins, dict(st.get("attributes", {})), out, label, src)
            local[target] = res
        return local

    def dense_input(n: Node, ins: list) -> tuple[int, dict]:
        """The Dense's input tensor and the weight transformation its input_map needs."""
        if "input_map" not in n.attributes:
            return r(ins[0]), {}
        entries = [(r(int(e["tensor"])), int(e["index"])) for e in n.attributes["input_map"]]
        sources: list[int] = []
        for t, _ in entries:
            if not tensors[t].is_constant and t not in sources:
                sources.append(t)
        if not sources:
            raise GraphError(f"Dense {n.source_name!r} reads constants only")
        offset, width = {}, 0
        for t in sources:
            offset[t] = width
            width += size(t)
        columns: list[list[int]] = [[] for _ in range(width)]
        const_columns: list[tuple[int, int, int]] = []
        for k, (t, i) in enumerate(entries):
            if tensors[t].is_constant:
                const_columns.append((k, t, i))
            else:
                columns[offset[t] + i].append(k)
        if len(sources) == 1:
            x = sources[0]
        else:
            x = new_tensor(width, f"{n.source_name or 'dense'}.inputs")
            add("Concat", sources, x, {"axis": 1}, n)
        if len(entries) == width and not const_columns and all(c == [k] for k, c in enumerate(columns)):
            return x, {}
        return x, {"columns": columns, "const_columns": const_columns, "map_width": len(entries)}

    for n in graph.nodes:
        ins = [r(t) for t in n.inputs]
        out = n.outputs[0]
        label = n.source_name or f"{n.op.lower()}_{n.id}"
        if n.op in _ALIASES or (n.op == "Concat" and len(ins) == 1):
            alias[out] = ins[0]
            continue
        if n.op in _DENSE_OPS:
            x, fold = dense_input(n, ins)
            attrs = {"weight": n.attributes["weight"], "bias": n.attributes.get("bias"), **fold}
            if n.op == "Dense":
                add("Dense", [x], out, attrs, n)
                continue
            pre = new_tensor(size(out), f"{label}.dense")
            add("Dense", [x], pre, attrs, n)
            if n.op == "DenseBiasActivation":
                pointwise(n.attributes["activation"], [pre], dict(n.attributes.get("activation_attributes", {})),
                          out, label, n)
            elif n.op == "DenseResidualActivation":
                mid = pointwise("Add", [pre, int(n.attributes["residual"])], {}, None, label, n)
                pointwise(n.attributes["activation"], [mid], dict(n.attributes.get("activation_attributes", {})),
                          out, label, n)
            else:
                steps = n.attributes.get("epilogue_steps", [])
                if steps:
                    chain(steps, pre, out, label, n)
                else:
                    alias[out] = pre
            continue
        if n.op == "ResidualAddActivation":
            mid = pointwise("Add", ins[:2], {}, None, label, n)
            pointwise(n.attributes["activation"], [mid], dict(n.attributes.get("activation_attributes", {})),
                      out, label, n)
            continue
        if n.op == "PointwiseRegion":
            region(n.attributes["steps"], label, n, final=out)
            continue
        if n.op == "Gather":
            idx = [int(i) % size(ins[0]) for i in n.attributes["indices"]]
            add("Dense", [ins[0]], out, {"weight": None, "bias": None, "onehot": idx}, n)
            continue
        if n.op == "LpNormalization":
            # norm == 0 ? 0 : x / norm (emitter.py:903-919)
            p = int(n.attributes.get("p", 2))
            norm = new_tensor(1, f"{label}.norm")
            add("ReduceL1" if p == 1 else "ReduceL2", [ins[0]], norm, {"keepdims": 1}, n)
            zero = pointwise("Equal", [norm, literal([0.0], f"{label}.zero")], {}, None, label, n)
            q = pointwise("Div", [ins[0], norm], {}, None, label, n)
            pointwise("Where", [zero, literal(np.zeros(size(out)), f"{label}.zeros"), q], {}, out, label, n)
            continue
        if n.op.startswith("Reduce") and ("map_steps" in n.attributes or "map_region_steps" in n.attributes):
            # The reduction reads the value of its fused map (passes.py:984-1020).
            if "map_steps" in n.attributes:
                m = chain(n.attributes["map_steps"], None, None, label, n)
            else:
                local = region(n.attributes["map_region_steps"], label, n)
                m = local[int(n.attributes["map_output"])]
            attrs = {k: v for k, v in n.attributes.items() if k not in ("map_steps", "map_region_steps",
                                                                        "map_output", "map_size")}
            add(n.op, [m], out, attrs, n)
            continue
        if n.op in ("Concat", "Softmax", "LogSoftmax", "LayerNormalization") or n.op.startswith("Reduce"):
            add(n.op, ins, out, n.attributes, n)
            continue
        pointwise(n.op, ins, dict(n.attributes), out, label, n)
    return _Expanded(nodes, alias, tensors, derived)


def _weight_column(c: dict, wname: str, nout: int, nmap: int, k: int) -> np.ndarray:
    """Column k of a Dense weight [nout, nmap]."""
    return np.asarray(c[wname], dtype=np.float64).reshape(nout, nmap)[:, k]


def lower_graph(graph: Graph, max_slots: int = A.MAX_SLOTS) -> LoweredGraph:
    """Linearize `graph` into a layer chain over one state and saved slots.

    Each node's operands must be in the state or in a slot; a tensor that is
    still needed when the state moves on is saved first, and a slot is freed
    after its tensor's last use.  Add(T, Dense(X)) whose Dense has no other
    consumer becomes Binop_Projection_Add, the template's projection skip
    (same arithmetic: T + (b + W X), bias first).
    """
    if len(graph.inputs) != 1 or len(graph.outputs) != 1:
        raise GraphError("generated models have one input and one output")
    ex = _expand(graph)
    nodes, alias, T = ex.nodes, ex.alias, ex.tensors
    output = graph.outputs[0]
    while output in alias:
        output = alias[output]
    # Nodes the output does not depend on are dropped.
    live, want = [], {output}
    for n in reversed(nodes):
        if n.outputs[0] in want:
            live.append(n)
            want.update(n.inputs)
    nodes = live[::-1]

    def size(t: int) -> int:
        return T[t].sample_size

    def is_const(t: int) -> bool:
        return T[t].is_constant

    def const_of(t: int) -> str:
        return T[t].constant_name

    producer = {n.outputs[0]: n for n in nodes}
    uses: dict[int, int] = {}
    for n in nodes:
        for t in (n.inputs if n.op != "Dense" else n.inputs[:1]):
            if not is_const(t):
                uses[t] = uses.get(t, 0) + 1
    uses[output] = uses.get(output, 0) + 1

    # Projection skip: Add(T, Dense(X)) with a single-use Dense.
    proj: dict[int, Node] = {}  # Add node id -> the Dense it absorbs
    skip: set[int] = set()
    for n in nodes:
        if n.op != "Add" or len(n.inputs) != 2 or any(is_const(t) for t in n.inputs):
            continue
        for k in (1, 0):
            d = producer.get(n.inputs[k])
            other = n.inputs[1 - k]
            if (d is not None and d.op == "Dense" and id(d) not in skip and uses.get(d.outputs[0], 0) == 1
                    and "columns" not in d.attributes and "onehot" not in d.attributes
                    and size(other) == size(n.outputs[0]) and size(d.outputs[0]) == size(other)):
                # The Dense's use of X moves to the Add; its output disappears.
                proj[id(n)] = d
                skip.add(id(d))
                uses[d.outputs[0]] = 0
                break

    layers: list[Layer] = []
    params: list[_Param | None] = []
    notes: list[str] = []
    state = graph.inputs[0]
    slots: dict[int, int] = {}  # tensor -> slot
    free = list(range(max_slots))

    def emit(layer: Layer, param: _Param | None = None) -> None:
        layers.append(layer)
        params.append(param)

    def save(t: int) -> None:
        if t in slots:
            return
        if not free:
            raise GraphError(f"graph needs more than {max_slots} live saved tensors")
        s = free.pop(0)
        slots[t] = s
        emit(Layer(A.LAYER_SAVE_STATE, size(t), size(t), slot=s, label="Save_State"))

    def release(t: int) -> None:
        if uses.get(t, 0) == 0 and t in slots:
            free.append(slots.pop(t))
            free.sort()

    def make_state(t: int, keep_after: int) -> None:
        """Bring t into the state; the current state is saved if it is needed
        later, and t is saved if it is needed after `keep_after` more uses."""
        nonlocal state
        if state != t:
            if uses.get(state, 0) > 0:
                save(state)
            if t not in slots:
                raise GraphError(f"tensor {T[t].name!r} is neither the state nor saved")
            emit(Layer(A.LAYER_LOAD_STATE, size(state), size(t), slot=slots[t], label="Load_State"))
            state = t
        if uses.get(t, 0) > keep_after:
            save(t)

    def consume(*ts: int) -> None:
        for t in ts:
            if not is_const(t):
                uses[t] -= 1
        for t in ts:
            release(t)

    def vec(name: str, n: int) -> Callable[[dict], np.ndarray]:
        def f(c: dict) -> np.ndarray:
            v = np.asarray(c[name], dtype=np.float64).reshape(-1)
            if v.size == 1:
                v = np.full(n, v[0])
            if v.size != n:
                raise GraphError(f"constant {name!r} has {v.size} values; expected 1 or {n}")
            return v
        return f

    for n in nodes:
        if id(n) in skip:
            continue
        out = n.outputs[0]
        nout = size(out)
        op = n.op
        if op == "Add" and id(n) in proj:
            d = proj[id(n)]
            x = d.inputs[0]
            other = n.inputs[1] if n.inputs[0] == d.outputs[0] else n.inputs[0]
            wname = const_of(d.attributes["weight"])
            bid = d.attributes.get("bias")
            bname = const_of(bid) if bid is not None else None
            nx = size(x)
            if x == state and x != other:
                # The saved operand must sit in a slot: park X, then load T.
                save(x)
            make_state(other, 1)
            if x not in slots:
                raise GraphError(f"projection input {T[x].name!r} is not saved")

            def build(c, wname=wname, bname=bname, nx=nx, nout=nout):
                w = np.asarray(c[wname], dtype=np.float64).reshape(nout, nx)
                b = np.zeros(nout) if bname is None else np.asarray(c[bname], dtype=np.float64).reshape(-1)
                return np.concatenate([w.T.reshape(-1), b])
            emit(Layer(A.LAYER_BINOP_PROJECTION_ADD, nout, nout, slot=slots[x], n_aux=nx,
                       label="Binop_Projection_Add"), _Param(build))
            notes.append(f"Add({T[other].name}, Dense({T[x].name})) -> Binop_Projection_Add")
            consume(other, x)
            state = out
            continue
        if op == "Dense":
            x = n.inputs[0]
            make_state(x, 1)
            nin = size(x)
            if "onehot" in n.attributes:
                # Gather: row f of W picks element idx[f] (emitter.py:931-934).
                idx = list(n.attributes["onehot"])

                def build(c, idx=idx, nin=nin):
                    w = np.zeros((len(idx), nin))
                    w[np.arange(len(idx)), idx] = 1.0
                    return w.reshape(-1)
                emit(Layer(A.LAYER_DENSE, nin, nout, label="Gather"), _Param(build))
                consume(x)
                state = out
                continue
            wname = const_of(n.attributes["weight"])
            bid = n.attributes.get("bias")
            bname = const_of(bid) if bid is not None else None
            fold = n.attributes.get("columns")
            nmap = int(n.attributes.get("map_width", nin))
            if T[n.attributes["weight"]].sample_size != nmap * nout:
                raise GraphError(f"Dense {n.source_name!r}: weight size does not match {nout}x{nmap}")
            const_cols = [(k, const_of(t), i) for k, t, i in n.attributes.get("const_columns", [])]
            has_bias = bname is not None or bool(const_cols)

            def build(c, wname=wname, bname=bname, nin=nin, nout=nout, fold=fold, nmap=nmap, const_cols=const_cols):
                w = np.asarray(c[wname], dtype=np.float64).reshape(nout, nmap)
                if fold is not None:
                    # input_map: column j of the folded weight is the sum of
                    # the map columns that read source element j; constant
                    # entries are folded into the bias.
                    wf = np.zeros((nout, nin))
                    for j, ks in enumerate(fold):
                        for k in ks:
                            wf[:, j] += w[:, k]
                    w = wf
                if bname is None and not const_cols:
                    return w.reshape(-1)
                b = vec(bname, nout)(c) if bname is not None else np.zeros(nout)
                for k, cn, i in const_cols:
                    b = b + _weight_column(c, wname, nout, nmap, k) * np.asarray(c[cn], dtype=np.float64).reshape(-1)[i]
                return np.concatenate([w.reshape(-1), b])
            emit(Layer(A.LAYER_DENSE, nin, nout, flags=A.FLAG_DENSE_BIAS if has_bias else 0, label="Dense"),
                 _Param(build))
            consume(x)
            state = out
            continue
        if op == "Where":
            # interpreter.py:181-185: cond != 0 ? a : b.  One tensor operand
            # is the state, the others saved slots or constant vectors.
            ops3 = list(n.inputs)
            if is_const(ops3[0]):
                raise GraphError("Where with a constant condition should be folded before lowering")
            tens = [t for t in ops3 if not is_const(t)]
            st = state if state in tens else tens[0]
            count = ops3.count(st)
            for t in tens:
                if t != st and t not in slots:
                    raise GraphError(f"Where: operand {T[t].name!r} is not saved")
            make_state(st, count)
            if count > 1:
                save(st)
            flags, slot_ids, const_names = 0, [], []
            used_state = False
            for k, t in enumerate(ops3):
                if is_const(t):
                    code = A.SELECT_CONST
                    const_names.append(const_of(t))
                elif t == st and not used_state:
                    code = A.SELECT_STATE
                    used_state = True
                else:
                    code = A.SELECT_SLOT
                    slot_ids.append(slots[t])
                flags |= code << (2 * k)
                if not is_const(t):
                    if size(t) not in (1, nout):
                        raise GraphError(f"unsupported Where broadcasting: operand sizes "
                                         f"{[size(u) for u in ops3]}, output size {nout}")
                    if size(t) == 1 and nout > 1:
                        flags |= (A.SELECT_COND_SCALAR, A.SELECT_A_SCALAR, A.SELECT_B_SCALAR)[k]

            def build(c, names=tuple(const_names), nout=nout):
                return np.concatenate([vec(cn, nout)(c) for cn in names]) if names else np.zeros(0)
            emit(Layer(A.LAYER_SELECT, size(st), nout, slot=slot_ids[0] if slot_ids else 0, flags=flags,
                       attr=(0, slot_ids[1] if len(slot_ids) > 1 else 0, 0, 0), label="Where"),
                 _Param(build) if const_names else None)
            consume(*ops3)
            state = out
            continue
        if op in A.BINARY_OPS:
            a, b = n.inputs
            ca, cb = is_const(a), is_const(b)
            if ca and cb:
                raise GraphError(f"{op} of two constants should be folded before lowering")
            if ca or cb:
                t, c = (b, a) if ca else (a, b)
                make_state(t, 1)
                emit(Layer(A.LAYER_CONST_BINARY, nout, nout, flags=A.FLAG_CONST_LEFT if ca else 0,
                           attr=(A.BINARY_OPS[op], 0, 0, 0), label=op), _Param(vec(const_of(c), nout)))
                if size(t) != nout:
                    raise GraphError(f"{op}: broadcasting a one-feature tensor against a constant is not supported")
                consume(t)
                state = out
                continue
            # Tensor-tensor: one operand is the state, the other a saved slot
            # (every tensor still needed is one or the other).
            if a == b:
                make_state(a, 2)
                save(a)
                st, other = a, a
            else:
                st, other = (b, a) if state == b else (a, b)
                make_state(st, 1)
            if other not in slots:
                raise GraphError(f"{op}: operand {T[other].name!r} is not saved")
            saved_left = other == a and a != b
            for t in (a, b):
                if size(t) not in (1, nout):
                    raise GraphError(f"unsupported {op} broadcasting: operand sizes {size(a)} and {size(b)}, "
                                     f"output size {nout}")
            emit(Layer(A.LAYER_BINARY, size(st), nout, slot=slots[other], n_aux=size(other),
                       flags=A.FLAG_SAVED_LEFT if saved_left else 0, attr=(A.BINARY_OPS[op], 0, 0, 0), label=op))
            consume(a, b)
            state = out
            continue
        if op == "Concat":
            xs = list(n.inputs)
            # [x1; ...; xk]: grow from the state at one end with
            # Binop_Concatenate (after=True appends, after=False prepends).
            if state == xs[-1] and xs.count(state) == 1:
                order, after = list(reversed(xs[:-1])), False
                first = xs[-1]
            else:
                if state in xs and uses.get(state, 0) > 0:
                    save(state)
                order, after = xs[1:], True
                first = xs[0]
            for t in order:
                if t not in slots:
                    if t == state:
                        save(t)
                    else:
                        raise GraphError(f"Concat operand {T[t].name!r} is not saved")
            make_state(first, xs.count(first))
            width = size(first)
            for t in order:
                emit(Layer(A.LAYER_BINOP_CONCATENATE, width, width + size(t), slot=slots[t],
                           flags=A.FLAG_CONCAT_AFTER if after else 0, label="Binop_Concatenate"))
                width += size(t)
            consume(*xs)
            state = out
            continue
        if op.startswith("Reduce"):
            if op not in A.REDUCE_OPS:
                raise GraphError(f"no lowering for {op}")
            if "map_steps" in n.attributes or "map_region_steps" in n.attributes:
                raise GraphError(f"{op} with a fused map is not supported; pass the canonical graph")
            x = n.inputs[0]
            make_state(x, 1)
            emit(Layer(A.LAYER_REDUCE, size(x), 1, attr=(A.REDUCE_OPS[op], 0, 0, 0), label=op))
            consume(x)
            state = out
            continue
        if op in ("Softmax", "LogSoftmax"):
            x = n.inputs[0]
            make_state(x, 1)
            emit(Layer(A.LAYER_SOFTMAX if op == "Softmax" else A.LAYER_LOG_SOFTMAX, nout, nout, label=op))
            consume(x)
            state = out
            continue
        if op == "LayerNormalization":
            x = n.inputs[0]
            make_state(x, 1)
            sname = const_of(n.inputs[1])
            bname = const_of(n.inputs[2]) if len(n.inputs) > 2 else None

            def build(c, sname=sname, bname=bname, nout=nout):
                g = vec(sname, nout)(c)
                b = np.zeros(nout) if bname is None else vec(bname, nout)(c)
                return np.concatenate([g, b])
            emit(Layer(A.LAYER_LAYER_NORM, nout, nout, attr=(float(n.attributes.get("epsilon", 1e-5)), 0, 0, 0),
                       label="LayerNorm"), _Param(build))
            consume(x)
            state = out
            continue
        if len(n.inputs) == 1 and (op in _TEMPLATE_ACTIVATIONS or op in A.UNARY_OPS):
            x = n.inputs[0]
            make_state(x, 1)
            emit(_unary_layer(op, nout, n.attributes))
            consume(x)
            state = out
            continue
        raise GraphError(f"no lowering for operation {op}")

    if state != output:
        if output not in slots:
            raise GraphError("graph output is neither the final state nor saved")
        emit(Layer(A.LAYER_LOAD_STATE, size(state), size(output), slot=slots[output], label="Load_State"))
    if not layers:
        raise GraphError("an empty graph has no kernel")
    return LoweredGraph(layers, params, notes, ex.derived)


# ---- the generated model -----------------------------------------------------------

@dataclass
class WeightSpec:
    """One entry of weight_specs() (emitter.py:1438-1447)."""
    name: str
    dtype: str
    shape: tuple
    offset: int

    @property
    def size(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


class GeneratedModel:
    """The generated model class API (emitter.py:1589-1953) over libponni_hip.

    Parameters live in one flat host storage vector in weights.ponni order
    (constants sorted by tensor name, weights.py:299-306); every change is
    pushed to the device plans.  infer_batch runs the Scalar plan (fp32 or
    fp64), infer_batch_half2 an fp16 plan (fp16 operands, fp32 accumulation)
    fed from the same storage.
    """

    def __init__(self, graph: Graph, path: str = "auto"):
        self.graph = graph
        self.lowered = lower_graph(graph)
        self.path_request = path
        self.scalar = "f64" if graph.tensors[graph.inputs[0]].dtype == DType.FLOAT64 else "f32"
        self.stored_scalar_code = 2 if self.scalar == "f64" else 1
        consts = sorted((t for t in graph.tensors.values() if t.is_constant), key=lambda t: t.name)
        off = 0
        self._specs: list[WeightSpec] = []
        for t in consts:
            shape = tuple(int(d) for d in graph.constants[t.constant_name].values.shape)
            self._specs.append(WeightSpec(t.name, "F64" if self.scalar == "f64" else "F32", shape, off))
            off += int(np.prod(shape, dtype=np.int64)) if shape else 1
        self.storage_parameter_elements = off
        self._offset = {s.name: s.offset for s in self._specs}
        learned = [t for _, t in sorted(graph.tensors.items())
                   if t.is_constant and graph.constants[t.constant_name].learned]
        self._learned_ranges = []
        lo = 0
        for t in learned:
            self._learned_ranges.append((lo, self._offset[t.name], t.sample_size))
            lo += t.sample_size
        self.learned_parameter_elements = lo
        self.storage = np.zeros(off)
        for t in consts:
            s = self._offset[t.name]
            v = np.asarray(graph.constants[t.constant_name].values, dtype=np.float64).reshape(-1)
            self.storage[s:s + v.size] = v
        self._name_of_constant = {t.constant_name: t.name for t in consts}
        self._plans: dict[str, Inference] = {}
        self._weights_loaded = True

    # -- schema -------------------------------------------------------------------
    @property
    def num_inputs(self) -> int:
        return self.graph.size(self.graph.inputs[0])

    @property
    def num_outputs(self) -> int:
        return self.graph.size(self.graph.outputs[0])

    def weight_specs(self) -> list[WeightSpec]:
        return list(self._specs)

    def model_fingerprint(self) -> str:
        return graph_fingerprint(self.graph)

    def parameter_storage_index(self, index: int) -> int:
        """Learned-parameter index -> storage index (emitter.py:1454-1465)."""
        for begin, storage_begin, size in self._learned_ranges:
            if index < begin + size:
                return storage_begin + index - begin
        raise IndexError("GeneratedModel learned parameter index is out of range")

    def get_num_parameters(self) -> int:
        return self.learned_parameter_elements

    def weights_loaded(self) -> bool:
        return self._weights_loaded

    # -- parameters -----------------------------------------------------------------
    def _constants(self, dtype: str) -> dict:
        c = {}
        for cname, tname in self._name_of_constant.items():
            s = self._offset[tname]
            shape = self.graph.constants[cname].values.shape
            n = int(np.prod(shape, dtype=np.int64)) if shape else 1
            v = self.storage[s:s + n]
            if dtype == "f32":
                v = v.astype(np.float32).astype(np.float64)
            c[cname] = v.reshape(shape) if shape else v
        return c

    def _push(self, plan: Inference, dtype: str) -> None:
        for i, v in enumerate(self.lowered.layer_params(self._constants(dtype))):
            if v.size:
                plan.set_layer_params(i, v)

    def plan(self, dtype: str | None = None) -> Inference:
        """The device plan for `dtype` ("f32", "f64" or "f16"), created on first use."""
        dtype = dtype or self.scalar
        p = self._plans.get(dtype)
        if p is None:
            p = Inference(self.lowered.layers, dtype=dtype, path=self.path_request)
            self._push(p, dtype)
            self._plans[dtype] = p
        return p

    def _refresh(self) -> None:
        for dt, p in self._plans.items():
            self._push(p, dt)

    def get_parameters(self) -> np.ndarray:
        idx = [self.parameter_storage_index(i) for i in range(self.learned_parameter_elements)]
        return self.storage[idx].copy()

    def set_parameters(self, values) -> None:
        v = np.asarray(values, dtype=np.float64).reshape(-1)
        if v.size != self.learned_parameter_elements:
            raise ValueError("GeneratedModel::set_parameters source extent is incorrect")
        for i in range(v.size):
            self.storage[self.parameter_storage_index(i)] = v[i]
        self._refresh()

    def refresh_half_parameters(self) -> None:
        if "f16" in self._plans:
            self._push(self._plans["f16"], "f16")

    def parameters_are_finite(self) -> bool:
        return bool(np.all(np.isfinite(self.get_parameters())))

    # -- weights files --------------------------------------------------------------
    def _cspecs(self):
        arr = (A.TensorSpec * len(self._specs))()
        keep = []
        for i, s in enumerate(self._specs):
            name = s.name.encode()
            keep.append(name)
            arr[i].name = name
            arr[i].rank = len(s.shape)
            for k, d in enumerate(s.shape):
                arr[i].shape[k] = d
            arr[i].offset = s.offset
        return arr, keep

    def save_parameters(self, path: str) -> None:
        arr, keep = self._cspecs()
        st = np.ascontiguousarray(self.storage, dtype=np.float64)
        A.check(A.lib().ponni_file_write_tensors(str(path).encode(), self.model_fingerprint().encode(), arr,
                                                 len(self._specs), st.ctypes.data, 8 if self.scalar == "f64" else 4,
                                                 b"ponni", b"generated"))

    def load_weights(self, path: str) -> None:
        arr, keep = self._cspecs()
        st = np.zeros(self.storage_parameter_elements, dtype=np.float64)
        A.check(A.lib().ponni_file_read_tensors(str(path).encode(), self.model_fingerprint().encode(), arr,
                                                len(self._specs), st.ctypes.data, 8 if self.scalar == "f64" else 4))
        self.storage = st
        self._weights_loaded = True
        self._refresh()

    # -- inference ------------------------------------------------------------------
    def kernel_source(self, dtype: str | None = None) -> str:
        return self.plan(dtype).kernel_source()

    def infer_batch(self, x, y) -> None:
        """x [num_inputs, B], y [num_outputs, B]: GPU tensors of the model's Scalar."""
        self._check(x, y)
        self.plan().forward_batch_parallel(x, y)

    def infer_batch_half2(self, x, y) -> None:
        """fp16 arithmetic (fp16 operands, fp32 accumulation) on Scalar views."""
        import torch

        self._check(x, y)
        xh = x.to(torch.float16)
        yh = torch.empty((self.num_outputs, x.shape[1]), dtype=torch.float16, device=x.device)
        self.plan("f16").forward_batch_parallel(xh, yh)
        y.copy_(yh.to(y.dtype))

    def _check(self, x, y) -> None:
        if x.dim() != 2 or y.dim() != 2:
            raise ValueError("GeneratedModel input and output must be rank two")
        if x.shape[0] != self.num_inputs:
            raise ValueError("GeneratedModel input feature extent is incorrect")
        if y.shape[0] != self.num_outputs:
            raise ValueError("GeneratedModel output feature extent is incorrect")
        if x.shape[1] != y.shape[1]:
            raise ValueError("GeneratedModel batch extents differ")
        if x.shape[1] == 0:
            raise ValueError("GeneratedModel::infer_batch requires a nonzero batch size")
