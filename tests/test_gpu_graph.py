"""GPU parity of the generated-model path: graphs linearized onto
libponni_hip against the CPU oracle (which runs the same chain per sample and
is itself pinned against a float64 DAG evaluation in tests/test_graph.py).

fp32 bar: relative L2 <= 1e-5 and max-abs <= 1e-4 (unscaled);
fp16 (infer_batch_half2) bar: relative L2 <= 2e-3 against the oracle's
fp16-operand / fp32-accumulate mode.
"""
import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import configs as C
from ponni_amd import graph as G
from tests.test_gpu_parity import check_f32, check_half
from tests.test_graph import lowered_with_params, random_graph

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _oracle_built():
    oracle.build()


def run_model(gm, x_np, half=False):
    import torch

    x = torch.from_numpy(np.asarray(x_np, dtype=np.float32)).cuda()
    y = torch.full((gm.num_outputs, x.shape[1]), float("nan"), dtype=torch.float32, device="cuda:0")
    if half:
        gm.infer_batch_half2(x, y)
    else:
        gm.infer_batch(x, y)
    torch.cuda.synchronize()
    return y.double().cpu().numpy(), x.double().cpu().numpy()


@pytest.mark.parametrize("path", ["generic", "fused"])
@pytest.mark.parametrize("seed", range(12))
def test_random_graphs(cuda, seed, path):
    gr = random_graph(seed, aligned=seed % 3 == 0)
    gm = G.GeneratedModel(gr, path=path)
    try:
        gm.plan()
    except P.PonniError as e:
        if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
            pytest.skip(e.message)
        raise
    B = [1, 63, 129, 1000, 4097, 300][seed % 6]
    x = np.random.default_rng(100 + seed).standard_normal((gr.size(gr.inputs[0]), B))
    got, xg = run_model(gm, x)
    check_f32(got, oracle.forward(lowered_with_params(gr), xg))


@pytest.mark.parametrize("path", ["auto", "generic", "fused"])
def test_c5_generated_model(cuda, path):
    gm = G.GeneratedModel(C.c5_graph(True), path=path)
    x = C.normal(24 * 5000, 4, C.INPUT_TAG, 0.0, 1.0).reshape(24, 5000)
    got, xg = run_model(gm, x)
    check_f32(got, oracle.forward(lowered_with_params(gm.graph), xg))
    assert np.allclose(got.sum(axis=0), 1.0, atol=1e-5)  # softmax rows


def test_c5_half2(cuda):
    gm = G.GeneratedModel(C.c5_graph(True))
    x = C.normal(24 * 3000, 4, C.INPUT_TAG, 0.0, 1.0).reshape(24, 3000)
    got, xg = run_model(gm, x, half=True)
    xh = xg.astype(np.float16).astype(np.float64)
    check_half(got, oracle.forward(lowered_with_params(gm.graph), xh, oracle.MODE_F16_OPERANDS))


def test_weights_reload_changes_outputs(cuda, tmp_path):
    src = G.GeneratedModel(C.c5_graph(True))
    path = tmp_path / "w.ponni"
    src.save_parameters(str(path))
    dst = G.GeneratedModel(C.c5_graph(False))
    x = np.random.default_rng(3).standard_normal((24, 700))
    before, _ = run_model(dst, x)
    dst.load_weights(str(path))
    after, xg = run_model(dst, x)
    want, _ = run_model(src, x)
    assert not np.allclose(before, after)
    check_f32(after, want)


@pytest.mark.parametrize("seed", range(4))
def test_random_graphs_half(cuda, seed):
    gr = random_graph(40 + seed, aligned=True)
    gm = G.GeneratedModel(gr, path="fused")
    x = np.random.default_rng(seed).standard_normal((gr.size(gr.inputs[0]), 999))
    got, xg = run_model(gm, x, half=True)
    xh = xg.astype(np.float16).astype(np.float64)
    check_half(got, oracle.forward(lowered_with_params(gr), xh, oracle.MODE_F16_OPERANDS))


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("seed", range(12))
def test_random_narrow_graphs(cuda, seed, dtype):
    """Generated graphs of width <= 16 on generated NARROW kernels (graph
    operations inline, one lane per sample group) against the oracle."""
    gr = random_graph(200 + seed, narrow=True)
    gm = G.GeneratedModel(gr, path="narrow")
    try:
        plan = gm.plan(dtype)
    except P.PonniError as e:
        if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
            pytest.skip(e.message)
        raise
    assert plan.path == "narrow"
    B = [1, 63, 1025, 4096, 4099, 777][seed % 6]
    x = np.random.default_rng(300 + seed).standard_normal((gr.size(gr.inputs[0]), B))
    got, xg = run_model(gm, x, half=dtype == "f16")
    if dtype == "f32":
        check_f32(got, oracle.forward(lowered_with_params(gr), xg))
    else:
        xh = xg.astype(np.float16).astype(np.float64)
        check_half(got, oracle.forward(lowered_with_params(gr), xh, oracle.MODE_F16_OPERANDS))


@pytest.mark.parametrize("seed", range(6))
def test_random_narrow_graphs_f64(cuda, seed):
    """F64 generated graphs of width <= 16 on generated NARROW kernels (double
    state) against the oracle's fp64 mode."""
    import torch

    gr = random_graph(400 + seed, narrow=True, dtype="float64")
    gm = G.GeneratedModel(gr, path="narrow")
    assert gm.plan().path == "narrow"
    B = [1, 63, 1025, 4096, 4099, 777][seed]
    x = np.random.default_rng(500 + seed).standard_normal((gr.size(gr.inputs[0]), B))
    xt = torch.from_numpy(x).cuda()
    y = torch.full((gm.num_outputs, B), float("nan"), dtype=torch.float64, device="cuda:0")
    gm.infer_batch(xt, y)
    torch.cuda.synchronize()
    want = oracle.forward(lowered_with_params(gr), x, oracle.MODE_F64)
    got = y.cpu().numpy()
    assert np.allclose(got, want, rtol=1e-11, atol=1e-11 * max(1.0, np.abs(want).max())), np.abs(got - want).max()


@pytest.mark.parametrize("case", ["c5", "g0", "g1", "g2"])
def test_generated_graphs_f64_fused(cuda, case):
    """F64 generated graphs on the FUSED kernel (fp64 tiles) against the
    oracle's fp64 mode."""
    import torch

    gr = C.c5_graph(True) if case == "c5" else random_graph(600 + int(case[1:]), aligned=True, dtype="float64")
    if case == "c5":
        gm = G.GeneratedModel(gr, path="fused")
        plan = gm.plan("f64")
    else:
        gm = G.GeneratedModel(gr, path="fused")
        plan = gm.plan()
    assert plan.path == "fused"
    n_in = gr.size(gr.inputs[0])
    x = np.random.default_rng(7).standard_normal((n_in, 2049))
    xt = torch.from_numpy(x).cuda()
    y = torch.full((gm.num_outputs, 2049), float("nan"), dtype=torch.float64, device="cuda:0")
    plan.forward_batch_parallel(xt, y)
    torch.cuda.synchronize()
    layers = gm.lowered.layers
    for l, v in zip(layers, gm.lowered.layer_params(gm._constants("f64"))):
        if v.size:
            l.params = v
    want = oracle.forward(layers, x, oracle.MODE_F64)
    got = y.cpu().numpy()
    assert np.allclose(got, want, rtol=1e-11, atol=1e-11 * max(1.0, np.abs(want).max())), np.abs(got - want).max()
