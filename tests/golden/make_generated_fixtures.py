"""Golden vectors for the generated-model formats, written by the reference
generator's own Python: the two functions no closed form pins.

- graph_fingerprint (kokkos_nn/weights.py:85-92) of graphs built with
  ponni_amd.graph, rebuilt as reference IR objects (kokkos_nn/ir.py:19-152)
  field by field, with the reference recomputing producer/consumer links;
- write_weights / write_ponni_file (weights.py:95-168, :276-323): the bytes
  of a reference-written weights file for a tiny graph.

Run in the development container only (the reference is not shipped):
    python tests/golden/make_generated_fixtures.py /root/reference
Writes tests/golden/generated_fingerprints.json and tests/golden/tiny_generated.ponni.
"""
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from ponni_amd import configs as C  # noqa: E402
from ponni_amd import graph as G  # noqa: E402


def tiny_graph() -> G.Graph:
    """3 -> Dense(4) + Relu -> Dense(2) + Sigmoid, fixed values."""
    g = G.GraphBuilder(3)
    w1 = np.arange(12, dtype=np.float64).reshape(4, 3) / 8 - 0.7
    h = g.unary("Relu", g.dense(g.input, w1, [0.1, -0.2, 0.3, -0.4], name="fc1"))
    w2 = np.array([[0.5, -0.25, 1.0, 0.125], [-1.5, 0.75, 0.0, 2.0]])
    return g.finish(g.unary("Sigmoid", g.dense(h, w2, [0.05, -0.05], name="fc2")))


def graphs() -> dict:
    from tests.test_graph import random_graph

    out = {"c5": C.c5_graph(True), "tiny": tiny_graph()}
    for seed in range(6):
        out[f"random_{seed}"] = random_graph(seed, aligned=seed % 2 == 0)
    out["random_f64"] = random_graph(11, dtype="float64")
    return out


def to_reference(g: G.Graph, ir):
    tensors = {}
    for tid, t in g.tensors.items():
        shape = tuple(ir.Symbol(d.name) if isinstance(d, G.Symbol) else int(d) for d in t.shape)
        tensors[tid] = ir.TensorValue(t.id, t.name, shape, ir.DType(t.dtype.value), is_input=t.is_input,
                                      is_output=t.is_output, is_constant=t.is_constant,
                                      constant_name=t.constant_name)
    nodes = [ir.Node(n.id, n.op, list(n.inputs), list(n.outputs), dict(n.attributes), n.source_name)
             for n in g.nodes]
    consts = {k: ir.ConstantTensor(c.name, tuple(c.shape), ir.DType(c.dtype.value), np.asarray(c.values),
                                   c.canonical_layout, c.learned) for k, c in g.constants.items()}
    rg = ir.Graph(list(g.inputs), list(g.outputs), tensors, nodes, consts, dict(g.metadata))
    rg.rebuild_links()
    return rg


def main(reference: str) -> None:
    sys.path.insert(0, os.path.join(reference, "src", "generator"))
    from kokkos_nn import ir, weights

    fps = {}
    for name, g in graphs().items():
        fps[name] = weights.graph_fingerprint(to_reference(g, ir))
    with open(os.path.join(HERE, "generated_fingerprints.json"), "w") as f:
        json.dump(fps, f, indent=1, sort_keys=True)
        f.write("\n")
    with tempfile.TemporaryDirectory() as d:
        from pathlib import Path

        weights.write_weights(to_reference(tiny_graph(), ir), Path(d))
        with open(os.path.join(d, "weights.ponni"), "rb") as src:
            data = src.read()
    with open(os.path.join(HERE, "tiny_generated.ponni"), "wb") as f:
        f.write(data)
    print(f"{len(fps)} fingerprints, tiny_generated.ponni {len(data)} bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
