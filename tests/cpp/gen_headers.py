"""Writes the generated-model headers the C++ tests compile
(tests/cpp/gen/*.h): the c5 graph with nonzero biases as class C5Model
(FUSED kernels), the tiny 3 -> 4 -> 2 graph of tests/golden as class
TinyModel (generated NARROW kernels) and a double-precision narrow graph as
class F64Model (F64 NARROW kernels)."""


def f64_graph():
    from tests.test_graph import random_graph

    return random_graph(402, narrow=True, dtype="float64")
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def main() -> None:
    from ponni_amd import configs as C
    from ponni_amd.emitter import emit_cpp_header
    from tests.golden.make_generated_fixtures import tiny_graph

    os.makedirs(os.path.join(HERE, "gen"), exist_ok=True)
    for name, graph, cls in [("c5_model.h", C.c5_graph(True), "C5Model"), ("tiny_model.h", tiny_graph(), "TinyModel"),
                             ("f64_model.h", f64_graph(), "F64Model")]:
        out = os.path.join(HERE, "gen", name)
        tmp = out + ".tmp"
        emit_cpp_header(graph, tmp, namespace="ponni::generated", class_name=cls)
        os.replace(tmp, out)


if __name__ == "__main__":
    main()
