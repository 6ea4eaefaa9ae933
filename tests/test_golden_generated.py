"""Generated-model formats against vectors the reference generator's own
Python wrote (tests/golden/make_generated_fixtures.py): graph_fingerprint
(kokkos_nn/weights.py:85-92) and the bytes of a reference-written weights file
(weights.py:95-168, :276-323).  Runs on the CPU."""
import json
import os

import numpy as np
import pytest

from ponni_amd import _abi as A
from ponni_amd import graph as G
from tests.golden.make_generated_fixtures import graphs, tiny_graph

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    return os.path.join(GOLDEN, name)


@pytest.mark.parametrize("name", sorted(json.load(open(_golden("generated_fingerprints.json")))))
def test_graph_fingerprint_matches_reference(name):
    want = json.load(open(_golden("generated_fingerprints.json")))[name]
    assert G.graph_fingerprint(graphs()[name]) == want


def test_fingerprint_catches_a_changed_graph():
    g = tiny_graph()
    g.nodes[1].op = "Tanh"  # a different activation: a different kernel ABI
    want = json.load(open(_golden("generated_fingerprints.json")))["tiny"]
    assert G.graph_fingerprint(g) != want


def test_reference_written_weights_load():
    gm = G.GeneratedModel(tiny_graph())
    want = gm.storage.copy()
    gm.storage[:] = 0
    gm.load_weights(_golden("tiny_generated.ponni"))
    np.testing.assert_array_equal(gm.storage, want.astype(np.float32).astype(np.float64))
    assert gm.get_parameters().size == gm.learned_parameter_elements == 12 + 4 + 8 + 2


def test_our_writer_reproduces_reference_bytes(tmp_path):
    # write_weights names the source framework "onnx" and the target "generated".
    gm = G.GeneratedModel(tiny_graph())
    arr, keep = gm._cspecs()
    st = np.ascontiguousarray(gm.storage, dtype=np.float64)
    path = tmp_path / "w.ponni"
    A.check(A.lib().ponni_file_write_tensors(str(path).encode(), gm.model_fingerprint().encode(), arr, len(keep),
                                             st.ctypes.data, 4, b"onnx", b"generated"))
    assert path.read_bytes() == open(_golden("tiny_generated.ponni"), "rb").read()


def test_tampered_reference_file_is_rejected(tmp_path):
    data = bytearray(open(_golden("tiny_generated.ponni"), "rb").read())
    data[-3] ^= 0x40  # payload byte: the checksum no longer matches
    path = tmp_path / "bad.ponni"
    path.write_bytes(bytes(data))
    with pytest.raises(A.PonniError):
        G.GeneratedModel(tiny_graph()).load_weights(str(path))
