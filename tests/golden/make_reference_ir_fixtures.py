"""Golden models as the reference generator writes them: canonical_ir.json
(the optimized IR, kokkos_nn/compiler.py:316), weights.ponni
(weights.py:276-323) and the reference interpreter's outputs.

For each graph built here (c5, random DAGs of tests/test_graph.py, random
selection / normalization / unary-math graphs of tests/graph_cases.py) the
script rebuilds it as reference IR objects, runs the reference optimizer
(passes.optimize), and records for a fixed fp16-exact float64 input
- y: interpreter.run_graph on the optimized graph (interpreter.py:430-440),
- y_source: interpreter.run_graph on the graph before optimization,
- the optimized graph's fingerprint (weights.py:85-92)
and which compound operations the optimizer formed.

Run in the development container only (the reference is not shipped):
    python tests/golden/make_reference_ir_fixtures.py /root/reference
Writes tests/golden/reference_ir/<case>/{canonical_ir.json, weights.ponni, io.npz}
and tests/golden/reference_ir/cases.json.
"""
import json
import os
import shutil
import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from ponni_amd import configs as C  # noqa: E402
from tests import graph_cases as GC  # noqa: E402
from tests.golden.make_generated_fixtures import to_reference  # noqa: E402

OUT = os.path.join(HERE, "reference_ir")
BATCH = 23


def cases() -> dict:
    from tests.test_graph import random_graph

    out = {"c5": (C.c5_graph(True), "float32")}
    for seed in range(6):
        out[f"random_{seed}"] = (random_graph(seed, aligned=True), "float32")
    for seed in range(6):
        out[f"ops_{seed}"] = (GC.op_graph(seed, smooth=True), "float32")
    for seed in (6, 7):
        out[f"ops_steps_{seed}"] = (GC.op_graph(seed, smooth=False), "float32")
    out["ops_f64"] = (GC.op_graph(8, smooth=False, dtype="float64", aligned=False), "float64")
    out["forms"] = (GC.forms_graph(), "float32")
    return out


def compound_forms(graph) -> list:
    forms = set()
    for n in graph.nodes:
        if n.op in ("ElementwiseChain", "PointwiseRegion", "DenseEpilogue", "DenseBiasActivation",
                    "DenseResidualActivation", "ResidualAddActivation", "CompareSelect"):
            forms.add(n.op)
        for key in ("input_map", "map_steps", "map_region_steps"):
            if key in n.attributes:
                forms.add(key)
    return sorted(forms)


def main(reference: str) -> None:
    sys.path.insert(0, os.path.join(reference, "src", "generator"))
    from kokkos_nn import interpreter, ir, passes, weights

    if os.path.isdir(OUT):
        shutil.rmtree(OUT)
    os.makedirs(OUT)
    summary = {}
    for name, (g, dtype) in cases().items():
        src = to_reference(g, ir)
        opt, _ = passes.optimize(src)
        n_in = src.tensors[src.inputs[0]].sample_size
        x = GC.in_domain_input(n_in, BATCH, 7 + len(summary))
        y = interpreter.run_graph(opt, x)
        y_source = interpreter.run_graph(src, x)
        d = os.path.join(OUT, name)
        os.makedirs(d)
        with open(os.path.join(d, "canonical_ir.json"), "w") as f:
            f.write(opt.to_json() + "\n")
        with tempfile.TemporaryDirectory() as tmp:
            weights.write_weights(opt, Path(tmp))
            shutil.copy(os.path.join(tmp, "weights.ponni"), os.path.join(d, "weights.ponni"))
        np.savez(os.path.join(d, "io.npz"), x=x, y=y, y_source=y_source)
        summary[name] = {"dtype": dtype, "fingerprint": weights.graph_fingerprint(opt),
                         "nodes_source": len(src.nodes), "nodes_optimized": len(opt.nodes),
                         "forms": compound_forms(opt), "ops": sorted({n.op for n in opt.nodes})}
        print(name, summary[name]["forms"])
    with open(os.path.join(OUT, "cases.json"), "w") as f:
        json.dump(summary, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
