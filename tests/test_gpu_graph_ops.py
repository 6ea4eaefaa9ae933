"""Graph operations that need a restricted input domain -- Exp, Log, Sqrt,
Reciprocal, Pow (constant and state exponents), ReduceL1, ReduceSumSquare,
ReduceLogSum and ReduceProd (kokkos_nn/emitter.py:218-262, :475-547;
kokkos_nn/interpreter.py:15-131) -- on the GENERIC, generated NARROW and
FUSED kernels, in fp32 and fp16, against the CPU oracle.

Each graph feeds the operation from a dense layer through Abs + 0.5 (or
Sigmoid + 0.5 for products), so logs, roots, reciprocals and powers stay in
their real domain.  The oracle's restatement of each operation is pinned
first against the float64 numpy evaluation of the graph itself
(tests/numpy_graph.py), on the CPU.

fp32 bar: relative L2 <= 1e-5 and max-abs <= 1e-4 (unscaled);
fp16 bar: relative L2 <= 2e-3 against the oracle's fp16-operand /
fp32-accumulate mode on the same fp16-rounded inputs.
"""
import math

import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import graph as G
from tests import numpy_graph as NG
from tests.test_graph import lowered_with_params

OPS = ["Exp", "Log", "Sqrt", "Reciprocal", "Pow", "PowState", "ReduceL1", "ReduceSumSquare", "ReduceLogSum",
       "ReduceProd"]


@pytest.fixture(scope="module", autouse=True)
def _oracle_built():
    oracle.build()


def op_graph(op: str, seed: int = 0, n_in: int = 8, w: int = 16):
    rng = np.random.default_rng(1000 + seed)
    g = G.GraphBuilder(n_in)
    lim = math.sqrt(6 / (n_in + w))
    d = g.dense(g.input, rng.uniform(-lim, lim, (w, n_in)), rng.uniform(-0.2, 0.2, w), name="fc")
    pos = g.binary("Add", g.unary("Abs", d), g.constant("shift", np.full(w, 0.5)))
    if op == "Exp":
        out = g.unary("Exp", d)
    elif op in ("Log", "Sqrt", "Reciprocal"):
        out = g.unary(op, pos)
    elif op == "Pow":
        out = g.binary("Pow", pos, g.constant("expo", rng.uniform(0.5, 2.0, w)))
    elif op == "PowState":
        out = g.binary("Pow", pos, g.unary("Sigmoid", d))
    else:
        if op == "ReduceProd":
            src = g.binary("Add", g.unary("Sigmoid", d), g.constant("half", np.full(w, 0.5)))
        elif op == "ReduceLogSum":
            src = pos
        else:
            src = d
        out = g.binary("Add", d, g.reduce(op, src))
    return g.finish(out)


def inputs(n_in, B, seed):
    return np.random.default_rng(seed).standard_normal((n_in, B))


@pytest.mark.parametrize("op", OPS)
def test_oracle_matches_numpy_graph(op):
    gr = op_graph(op)
    x = inputs(8, 257, 7)
    want = NG.run_graph(gr, x)
    got = oracle.forward(lowered_with_params(gr), x, oracle.MODE_F64)
    assert np.isfinite(want).all()
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12 * max(1.0, np.abs(want).max())), np.abs(got - want).max()
    got32 = oracle.forward(lowered_with_params(gr), x, oracle.MODE_F32)
    assert np.linalg.norm(got32 - want) / np.linalg.norm(want) < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("path", ["generic", "narrow", "fused", "layered"])
@pytest.mark.parametrize("op", OPS)
def test_domain_ops_on_gpu(cuda, op, path, dtype):
    import torch

    from tests.test_gpu_parity import check_f32, check_half

    gr = op_graph(op, seed=OPS.index(op))
    gm = G.GeneratedModel(gr, path=path)
    plan = gm.plan(dtype)
    assert plan.path == path
    B = 4099
    x = inputs(8, B, 11 + OPS.index(op))
    print(f"graph op {op}: path={path} dtype={dtype} B={B}", flush=True)
    xt = torch.from_numpy(x.astype(np.float32)).cuda()
    y = torch.full((gm.num_outputs, B), float("nan"), dtype=torch.float32, device="cuda:0")
    if dtype == "f16":
        gm.infer_batch_half2(xt, y)
    else:
        gm.infer_batch(xt, y)
    torch.cuda.synchronize()
    got = y.double().cpu().numpy()
    xg = xt.double().cpu().numpy()
    layers = lowered_with_params(gr)
    if dtype == "f32":
        check_f32(got, oracle.forward(layers, xg))
    else:
        xh = xg.astype(np.float16).astype(np.float64)
        check_half(got, oracle.forward(layers, xh, oracle.MODE_F16_OPERANDS))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("path", ["generic", "narrow", "fused", "layered"])
@pytest.mark.parametrize("seed", range(6))
def test_op_graphs_on_gpu(cuda, seed, path, dtype):
    """Random graphs over Where / comparisons / logic / Clip / PRelu /
    BatchNormalization / Mean / Sum / Gather / LpNormalization / IsNaN /
    IsInf and the unary math (tests/graph_cases.py) on every kernel family.
    fp16 runs and most fp32 runs use graphs continuous in their input; seeds
    0 and 3 add the step functions in fp32."""
    import torch

    from tests import graph_cases as GC
    from tests.test_gpu_parity import check_f32, check_half

    smooth = dtype == "f16" or seed % 3 != 0
    gr = GC.op_graph(seed, smooth=smooth, aligned=path == "fused", narrow=path == "narrow")
    gm = G.GeneratedModel(gr, path=path)
    try:
        plan = gm.plan(dtype)
    except P.PonniError as e:
        if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
            pytest.skip(e.message)
        raise
    assert plan.path == path
    B = [4099, 1000, 257][seed % 3]
    x = GC.in_domain_input(gr.size(gr.inputs[0]), B, 50 + seed)
    print(f"op graph seed={seed} smooth={smooth}: path={path} dtype={dtype} B={B} "
          f"layers={len(gm.lowered.layers)}", flush=True)
    xt = torch.from_numpy(x.astype(np.float32)).cuda()
    y = torch.full((gm.num_outputs, B), float("nan"), dtype=torch.float32, device="cuda:0")
    if dtype == "f16":
        gm.infer_batch_half2(xt, y)
    else:
        gm.infer_batch(xt, y)
    torch.cuda.synchronize()
    got = y.double().cpu().numpy()
    layers = lowered_with_params(gr)
    if dtype == "f32":
        check_f32(got, oracle.forward(layers, x))
    else:
        check_half(got, oracle.forward(layers, x, oracle.MODE_F16_OPERANDS))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("path", ["generic", "narrow", "fused", "layered"])
@pytest.mark.parametrize("n", [12, 16])
def test_reductions_of_non_finite_inputs(cuda, n, path, dtype):
    """ReduceMax / ReduceMin / ReduceLogSumExp (kokkos_nn/emitter.py:502-526)
    straight on inputs holding NaN, infinities, values that overflow fp16
    and signed zeros: the running maximum or minimum starts from feature 0,
    so a NaN there makes it NaN and a NaN elsewhere is passed over, on every
    kernel family as in the oracle."""
    import torch

    from tests.test_gpu_parity import check_non_finite, non_finite_input

    g = G.GraphBuilder(n)
    x = g.input
    gr = g.finish(g.concat(g.reduce("ReduceMax", x), g.reduce("ReduceMin", x), g.reduce("ReduceLogSumExp", x)))
    gm = G.GeneratedModel(gr, path=path)
    try:
        plan = gm.plan(dtype)
    except P.PonniError as e:
        if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
            pytest.skip(e.message)
        raise
    assert plan.path == path
    B = 4099
    xin = non_finite_input(n, B, np.random.default_rng(90 + n))
    print(f"non-finite reductions: n={n} path={path} dtype={dtype} B={B}", flush=True)
    xt = torch.from_numpy(xin.astype(np.float32)).cuda()
    y = torch.full((gm.num_outputs, B), 7.0, dtype=torch.float32, device="cuda:0")
    (gm.infer_batch_half2 if dtype == "f16" else gm.infer_batch)(xt, y)
    torch.cuda.synchronize()
    xg = xt.double().cpu().numpy()
    if dtype == "f16":
        with np.errstate(over="ignore"):  # 1e30 rounds to inf in fp16, as on the GPU
            xh = xg.astype(np.float16).astype(np.float64)
        want = oracle.forward(lowered_with_params(gr), xh, oracle.MODE_F16_OPERANDS)
    else:
        want = oracle.forward(lowered_with_params(gr), xg)
    check_non_finite(y.double().cpu().numpy(), want, dtype)
