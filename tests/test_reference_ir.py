"""Models as the reference generator writes them: canonical_ir.json +
weights.ponni (tests/golden/reference_ir, made by the reference's own
optimizer, weight writer and interpreter -- make_reference_ir_fixtures.py).

CPU: the reader reproduces each optimized graph's fingerprint, the weights
load through it, and the oracle (on the linearized chain) and the numpy DAG
evaluator both reproduce the reference interpreter's outputs.  GPU: every
case runs on FUSED (and GENERIC) against those outputs.

Bars: float64 oracle vs the interpreter, relative 1e-10 of max(1, |y|);
fp32 GPU runs, relative L2 <= 1e-5 and max-abs <= 1e-4 of max(1, |y|)
(check_f32); fp64 GPU runs, 1e-10; fp16 operand runs (infer_batch_half2),
relative L2 <= 2e-3 against the oracle's fp16-operand mode.
"""
import json
import os
import warnings

import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import graph as G
from tests import numpy_graph as NG

HERE = os.path.dirname(os.path.abspath(__file__))
DIR = os.path.join(HERE, "golden", "reference_ir")
with open(os.path.join(DIR, "cases.json")) as _f:
    CASES = json.load(_f)
NAMES = sorted(CASES)
FORMS = {"ElementwiseChain", "PointwiseRegion", "DenseEpilogue", "DenseBiasActivation", "DenseResidualActivation",
         "ResidualAddActivation", "CompareSelect", "input_map", "map_steps", "map_region_steps"}


@pytest.fixture(scope="module", autouse=True)
def _oracle_built():
    oracle.build()


def load(name: str, path: str = "auto") -> tuple:
    d = os.path.join(DIR, name)
    graph = G.load_canonical_ir(os.path.join(d, "canonical_ir.json"))
    gm = G.GeneratedModel(graph, path=path)
    gm.load_weights(os.path.join(d, "weights.ponni"))
    io = np.load(os.path.join(d, "io.npz"))
    return gm, io["x"], io["y"], io["y_source"]


def oracle_run(gm, x, mode=oracle.MODE_F64):
    layers = gm.lowered.layers
    for l, v in zip(layers, gm.lowered.layer_params(gm._constants("f64" if mode == oracle.MODE_F64 else "f32"))):
        if v.size:
            l.params = v
    return oracle.forward(layers, x, mode)


def graph_with_values(gm) -> G.Graph:
    """The loaded graph with its constants filled from the loaded weights."""
    g = gm.graph
    for cname, v in gm._constants("f64").items():
        g.constants[cname].values = np.asarray(v).reshape(g.constants[cname].values.shape)
    return g


def test_every_compound_form_is_covered():
    seen = set()
    for c in CASES.values():
        seen.update(c["forms"])
    assert FORMS <= seen, FORMS - seen


@pytest.mark.parametrize("name", NAMES)
def test_reader_fingerprint_and_weights(name):
    gm, x, y, y_source = load(name)
    assert G.graph_fingerprint(gm.graph) == CASES[name]["fingerprint"]
    assert gm.model_fingerprint() == CASES[name]["fingerprint"]
    assert gm.weights_loaded()
    # The reference optimizer preserved the source graph's values.
    assert np.allclose(y, y_source, rtol=1e-9, atol=1e-12)
    # Round trip: the reader's graph serializes to the same JSON.
    with open(os.path.join(DIR, name, "canonical_ir.json")) as f:
        assert json.loads(gm.graph.to_json()) == json.load(f)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_matches_reference_interpreter(name):
    gm, x, y, _ = load(name)
    got = oracle_run(gm, x)
    tol = 1e-10 * max(1.0, float(np.abs(y).max()))
    assert np.allclose(got, y, rtol=1e-10, atol=tol), np.abs(got - y).max()


@pytest.mark.parametrize("name", NAMES)
def test_numpy_evaluator_matches_reference_interpreter(name):
    gm, x, y, _ = load(name)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        got = NG.run_graph(graph_with_values(gm), x)
    tol = 1e-10 * max(1.0, float(np.abs(y).max()))
    assert np.allclose(got, y, rtol=1e-10, atol=tol), np.abs(got - y).max()


def test_missing_weights_file_is_rejected(tmp_path):
    gm, *_ = load("c5")
    with pytest.raises(P.PonniError):
        gm.load_weights(str(tmp_path / "absent.ponni"))
    other = os.path.join(DIR, "random_0", "weights.ponni")
    with pytest.raises(P.PonniError, match="fingerprint"):
        gm.load_weights(other)


# ---- GPU ------------------------------------------------------------------------

def run(gm, x, half=False):
    import torch

    dt = torch.float64 if gm.scalar == "f64" else torch.float32
    xt = torch.from_numpy(np.asarray(x)).to(dt).cuda()
    yt = torch.full((gm.num_outputs, x.shape[1]), float("nan"), dtype=dt, device="cuda:0")
    (gm.infer_batch_half2 if half else gm.infer_batch)(xt, yt)
    torch.cuda.synchronize()
    return yt.double().cpu().numpy()


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["fused", "generic"])
@pytest.mark.parametrize("name", NAMES)
def test_reference_models_on_gpu(cuda, name, path):
    from tests.test_gpu_parity import check_f32

    gm, x, y, _ = load(name, path)
    assert gm.plan().path == path, gm.plan().path
    print(f"{name} on {path} ({gm.scalar}), B={x.shape[1]}", flush=True)
    got = run(gm, x)
    if gm.scalar == "f64":
        tol = 1e-10 * max(1.0, float(np.abs(y).max()))
        assert np.allclose(got, y, rtol=1e-10, atol=tol), np.abs(got - y).max()
    else:
        check_f32(got, y)


@pytest.mark.gpu
@pytest.mark.parametrize("name", [n for n in NAMES if n.startswith(("ops_", "forms", "c5")) and "steps" not in n
                                  and CASES[n]["dtype"] == "float32"])
def test_reference_models_half2(cuda, name):
    """fp16 operands, fp32 accumulation (FUSED) vs the oracle's same-semantics
    mode, on the graphs whose outputs are continuous in their inputs."""
    from tests.test_gpu_parity import check_half

    gm, x, _, _ = load(name, "fused")
    xb = np.concatenate([x] * 40, axis=1)  # 920 columns
    got = run(gm, xb, half=True)
    check_half(got, oracle_run(gm, xb, oracle.MODE_F16_OPERANDS))
