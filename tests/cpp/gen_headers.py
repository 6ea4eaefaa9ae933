"""Writes the generated-model headers the C++ tests compile
(tests/cpp/gen/*.h): the c5 graph with nonzero biases as class C5Model."""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def main() -> None:
    from ponni_amd import configs as C
    from ponni_amd.emitter import emit_cpp_header

    os.makedirs(os.path.join(HERE, "gen"), exist_ok=True)
    out = os.path.join(HERE, "gen", "c5_model.h")
    tmp = out + ".tmp"
    emit_cpp_header(C.c5_graph(True), tmp, namespace="ponni::generated", class_name="C5Model")
    os.replace(tmp, out)


if __name__ == "__main__":
    main()
