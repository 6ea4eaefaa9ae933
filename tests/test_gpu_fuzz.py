"""Randomized parity: fixed seeds over random layer chains (fp32, fp16/bf16,
fp64) and random generated graphs (wide and NARROW, fp32 and half2), each on a
path drawn from every kernel family, against the CPU oracle.

Pass rule, per case:
- within the fixed bar of its precision against the oracle in the same
  precision (fp32: relL2 <= 1e-5 and max-abs <= 1e-4;
  fp64: 1e-10; fp16 / bf16: relL2 <= 2e-3); or
- for fp32 graphs only: no further from the fp64 result than the oracle's
  own fp32 evaluation is, with a factor of 3 (an ill-conditioned graph, e.g.
  a LayerNorm over nearly equal features, amplifies the last-bit
  differences of any two fp32 evaluation orders).  Columns whose exact
  (fp64) output moves by more than half the GPU's deviation under a
  relative input perturbation of 1e-7 (about two fp32 ulps) are left out
  of both comparisons: their answer is not determined at fp32 precision
  (a ThresholdedRelu or comparison flipping at a discontinuity, or extreme
  conditioning).
"""
import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import graph as G
from tests import test_oracle as K
from tests.test_graph import lowered_with_params, random_graph

BATCHES = [1, 17, 64, 255, 1000, 4097, 20011]
CASES_PER_GROUP = 15
GROUPS = 10


@pytest.fixture(scope="module", autouse=True)
def _oracle_built():
    oracle.build()


def _rel(a, b):
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def _fp32_ok(got, want):
    return bool(np.isfinite(got).all() and _rel(got, want) <= 1e-5 and np.abs(got - want).max() <= 1e-4)


def _discontinuous_columns(layers, x, got, exact):
    """Columns whose fp64 output jumps under a 1e-7 relative input perturbation
    by more than half the GPU's deviation there."""
    dev = np.abs(got - exact).max(axis=0)
    cols = np.nonzero(dev > 1e-4 * max(1.0, np.abs(exact).max()))[0]
    rng = np.random.default_rng(0)
    out = []
    for c in cols[:16]:
        xc = x[:, c:c + 1]
        ys = np.stack([oracle.forward(layers, xc * (1 + 1e-7 * rng.standard_normal(xc.shape)), oracle.MODE_F64)[:, 0]
                       for _ in range(12)])
        if np.abs(ys - exact[:, c][None, :]).max() > 0.5 * dev[c]:
            out.append(c)
    return np.array(out, dtype=np.int64)


def _graph_fp32_ok(layers, x, got):
    want = oracle.forward(layers, x)
    if _fp32_ok(got, want):
        return True, f"relL2={_rel(got, want):.2e}"
    exact = oracle.forward(layers, x, oracle.MODE_F64)
    keep = np.setdiff1d(np.arange(x.shape[1]), _discontinuous_columns(layers, x, got, exact))
    g, w, e = got[:, keep], want[:, keep], exact[:, keep]
    if keep.size and _fp32_ok(g, w):
        return True, f"{x.shape[1] - keep.size} discontinuous columns"
    own = _rel(w, e)
    ok = bool(np.isfinite(g).all() and _rel(g, e) <= 3 * own + 1e-7)
    return ok, f"relL2 vs oracle {_rel(g, w):.2e}, GPU vs fp64 {_rel(g, e):.2e}, oracle fp32 vs fp64 {own:.2e}"


def _run_chain(layers, x, dtype, path, pad):
    import torch

    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f64": torch.float64}[dtype]
    try:
        m = P.create_inference_model(*layers, dtype=dtype, path=path)
    except P.PonniError as e:
        if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
            return None
        raise
    n_in, B = x.shape
    xs = torch.zeros((n_in, B + pad), dtype=tdt, device="cuda:0")
    xs[:, :B] = torch.from_numpy(x).to(tdt)
    ys = torch.full((m.get_num_outputs(), B + pad), float("nan"), dtype=tdt, device="cuda:0")
    m.forward_batch_parallel(xs[:, :B], ys[:, :B])
    torch.cuda.synchronize()
    assert torch.isnan(ys[:, B:].float()).all(), "kernel wrote past the batch"
    return ys[:, :B].double().cpu().numpy(), xs[:, :B].double().cpu().numpy()


def _run_graph(gr, x, path, half):
    import torch

    gm = G.GeneratedModel(gr, path=path)
    try:
        gm.plan("f16" if half else "f32")
    except P.PonniError as e:
        if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
            return None
        raise
    xt = torch.from_numpy(np.asarray(x, dtype=np.float32)).cuda()
    y = torch.full((gm.num_outputs, x.shape[1]), float("nan"), dtype=torch.float32, device="cuda:0")
    (gm.infer_batch_half2 if half else gm.infer_batch)(xt, y)
    torch.cuda.synchronize()
    return y.double().cpu().numpy(), xt.double().cpu().numpy()


def _case(seed):
    """One random case; returns (description, passed, detail) or None if the
    drawn path does not take it."""
    rng = np.random.default_rng(seed)
    B = int(rng.choice(BATCHES))
    kind = seed % 5
    if kind == 0:
        width = int(rng.choice([3, 8, 13, 16, 24, 40, 64, 100, 128, 200, 256]))
        layers = K.random_chain(rng, width, 2 + int(rng.integers(3)))
        x = rng.standard_normal((width, B))
        path = ["auto", "fused", "narrow", "mfma", "generic"][int(rng.integers(5))]
        desc = f"chain fp32 width={width} path={path} B={B}"
        print(desc, flush=True)
        r = _run_chain(layers, x, "f32", path, int(rng.integers(4)))
        if r is None:
            return None
        got, xg = r
        want = oracle.forward(layers, xg)
        return desc, _fp32_ok(got, want), f"relL2={_rel(got, want):.2e}"
    if kind == 1:
        width = int(rng.choice([16, 24, 32, 40, 64, 96, 128]))
        layers = K.random_chain(rng, width, 2)
        x = rng.standard_normal((width, B))
        dtype = ["f16", "bf16"][int(rng.integers(2))]
        path = ["fused", "auto"][int(rng.integers(2))]
        desc = f"chain {dtype} width={width} path={path} B={B}"
        print(desc, flush=True)
        r = _run_chain(layers, x, dtype, path, int(rng.integers(8)))
        if r is None:
            return None
        got, xg = r
        mode = oracle.MODE_F16_OPERANDS if dtype == "f16" else oracle.MODE_BF16_OPERANDS
        rel = _rel(got, oracle.forward(layers, xg, mode))
        return desc, bool(np.isfinite(got).all() and rel <= 2e-3), f"relL2={rel:.2e}"
    if kind in (2, 3):
        narrow = kind == 3
        gr = random_graph(seed, narrow=True) if narrow else random_graph(seed, aligned=bool(rng.integers(2)))
        x = rng.standard_normal((gr.size(gr.inputs[0]), B))
        path = "narrow" if narrow else ["auto", "fused", "generic"][int(rng.integers(3))]
        half = narrow and bool(rng.integers(2))
        desc = f"graph {'narrow ' if narrow else ''}{'half2' if half else 'fp32'} path={path} B={B}"
        print(desc, flush=True)
        r = _run_graph(gr, x, path, half)
        if r is None:
            return None
        got, xg = r
        layers = lowered_with_params(gr)
        if half:
            rel = _rel(got, oracle.forward(layers, xg.astype(np.float16).astype(np.float64), oracle.MODE_F16_OPERANDS))
            return desc, bool(np.isfinite(got).all() and rel <= 2e-3), f"relL2={rel:.2e}"
        ok, detail = _graph_fp32_ok(layers, xg, got)
        return desc, ok, detail
    width = int(rng.choice([3, 8, 16, 24, 64]))
    layers = K.random_chain(rng, width, 2)
    x = rng.standard_normal((width, B))
    path = ["auto", "fused", "narrow"][int(rng.integers(3))]
    desc = f"chain fp64 width={width} path={path} B={B}"
    print(desc, flush=True)
    r = _run_chain(layers, x, "f64", path, int(rng.integers(3)))
    if r is None:
        return None
    got, xg = r
    want = oracle.forward(layers, xg, oracle.MODE_F64)
    lim = 1e-10 * max(1.0, np.abs(want).max())
    rel = _rel(got, want)
    return desc, bool(np.isfinite(got).all() and rel <= 1e-10 and np.abs(got - want).max() <= lim), f"relL2={rel:.2e}"


def _graph_case_inputs(seed, B):
    rng = np.random.default_rng(seed)
    rng.choice(BATCHES)
    gr = random_graph(seed, aligned=bool(rng.integers(2)))
    return lowered_with_params(gr), rng.standard_normal((gr.size(gr.inputs[0]), B)).astype(np.float32).astype(np.float64)


def test_graph_rule_rejects_planted_errors():
    """The fp32 graph rule on the CPU: the oracle's own output passes; one
    column off by 1e-2, or every output scaled by 1 + 1e-4, fails; a column
    flipped the way an fp32 evaluation can flip it at a discontinuity (seed
    8747: the exact output of column 5136 jumps under a 1e-7 input
    perturbation) passes."""
    layers, x = _graph_case_inputs(7002, 1000)
    want = oracle.forward(layers, x)
    assert _graph_fp32_ok(layers, x, want)[0]
    bad = want.copy()
    bad[:, 17] += 1e-2
    assert not _graph_fp32_ok(layers, x, bad)[0]
    assert not _graph_fp32_ok(layers, x, want * (1 + 1e-4))[0]

    layers, x = _graph_case_inputs(8747, 20011)
    want = oracle.forward(layers, x)
    c = 5136
    rng = np.random.default_rng(3)
    flips = [oracle.forward(layers, x[:, c:c + 1] * (1 + 1e-7 * rng.standard_normal((x.shape[0], 1))),
                            oracle.MODE_F64)[:, 0] for _ in range(12)]
    flipped = max(flips, key=lambda y: np.abs(y - want[:, c]).max())
    assert np.abs(flipped - want[:, c]).max() > 1e-2
    got = want.copy()
    got[:, c] = flipped
    ok, detail = _graph_fp32_ok(layers, x, got)
    assert ok and "discontinuous" in detail, detail
    got[:, 100] += 1e-2
    assert not _graph_fp32_ok(layers, x, got)[0]


@pytest.mark.gpu
@pytest.mark.parametrize("group", range(GROUPS))
def test_random_cases(cuda, group):
    failed = []
    for seed in range(7000 + group * CASES_PER_GROUP, 7000 + (group + 1) * CASES_PER_GROUP):
        print(f"seed {seed}: ", end="", flush=True)
        r = _case(seed)
        if r is not None and not r[1]:
            failed.append(f"seed {seed}: {r[0]}: {r[2]}")
    assert not failed, "\n".join(failed)


def _wide_case(seed):
    """A random chain wider than 256 features (fp32, fp16 or bf16) on a path
    drawn from those that take it: AUTO, FUSED (16-bit up to 1024, fp32 up
    to 512), LAYERED (any width) or GENERIC; fixed bars."""
    rng = np.random.default_rng(seed)
    B = int(rng.choice([1, 255, 1000, 4097]))
    width = int(rng.choice([272, 320, 384, 512, 700, 1024]))
    dtype = ["f32", "f16", "bf16"][int(rng.integers(3))]
    layers = K.random_chain(rng, width, 2)
    x = rng.standard_normal((width, B))
    path = ["auto", "fused", "layered", "generic"][int(rng.integers(4))]
    desc = f"wide chain {dtype} width={width} path={path} B={B}"
    print(desc, flush=True)
    r = _run_chain(layers, x, dtype, path, int(rng.integers(4)))
    if r is None:
        return None
    got, xg = r
    if dtype == "f32":
        want = oracle.forward(layers, xg)
        return desc, _fp32_ok(got, want), f"relL2={_rel(got, want):.2e}"
    mode = oracle.MODE_F16_OPERANDS if dtype == "f16" else oracle.MODE_BF16_OPERANDS
    rel = _rel(got, oracle.forward(layers, xg, mode))
    return desc, bool(np.isfinite(got).all() and rel <= 2e-3), f"relL2={rel:.2e}"


@pytest.mark.gpu
@pytest.mark.parametrize("group", range(2))
def test_random_wide_cases(cuda, group):
    failed = []
    for seed in range(9000 + group * 12, 9000 + (group + 1) * 12):
        print(f"seed {seed}: ", end="", flush=True)
        r = _wide_case(seed)
        if r is not None and not r[1]:
            failed.append(f"seed {seed}: {r[0]}: {r[2]}")
    assert not failed, "\n".join(failed)


_SPECIAL = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0])


def _non_finite_chain(rng, w):
    """Save, then 1-4 of: an activation, LayerNorm, MinMaxNorm, Softmax /
    LogSoftmax, a residual Tanh, a concatenation, a dense block."""
    acts = [P.Relu, P.Elu, P.Selu, P.Silu, P.Sigmoid, P.Tanh, P.HardSwish, P.Mish, lambda n: P.Gelu(n, True)]
    n, layers = w, [P.Save_State(0, w)]
    for _ in range(int(rng.integers(1, 5))):
        c = int(rng.integers(8))
        if c <= 1:
            layers.append(acts[int(rng.integers(len(acts)))](n))
        elif c == 2:
            layers.append(P.LayerNorm(rng.uniform(0.5, 1.5, n), rng.uniform(-0.2, 0.2, n), 1e-5))
        elif c == 3:
            layers.append(P.MinMaxNorm(n, -1.0, 2.0))
        elif c == 4:
            layers.append([P.Softmax, P.LogSoftmax][int(rng.integers(2))](n))
        elif c == 5:
            layers += [P.Save_State(1, n), P.Tanh(n), P.Binop_Add(1, n)]
        elif c == 6 and n + w <= 48:
            layers.append(P.Binop_Concatenate(0, n, n + w, bool(rng.integers(2))))
            n += w
        else:
            m = int(rng.integers(max(2, n // 2), n + 1))
            layers += [P.Matvec(rng.standard_normal((n, m)) / np.sqrt(n)), P.Bias(rng.uniform(-0.2, 0.2, m))]
            n = m
    return layers


@pytest.mark.gpu
@pytest.mark.parametrize("group", range(2))
def test_random_non_finite_cases(cuda, group):
    """Random chains (above) and generated graphs on inputs holding NaN, +-inf
    and signed zeros, on a path and dtype drawn per case: the oracle's NaNs
    and infinities exactly, its finite values within the dtype's bar."""
    import torch

    from tests.test_gpu_parity import ORACLE_MODE, PATHS, TORCH_DT, check_non_finite, make_model

    failed = []
    for seed in range(11000 + 30 * group, 11000 + 30 * (group + 1)):
        rng = np.random.default_rng(seed)
        graph = seed % 3 == 0
        if graph:
            gr = random_graph(seed, aligned=bool(rng.integers(2)))
            n = gr.size(gr.inputs[0])
        else:
            n = int(rng.choice([2, 5, 12, 16, 24]))
            layers = _non_finite_chain(rng, n)
        B = int(rng.choice([17, 1000, 4099]))
        x = rng.standard_normal((n, B))
        for j in range(min(B, 256)):
            k = int(rng.integers(1, 3))
            x[rng.choice(n, k, replace=False), j] = _SPECIAL[rng.integers(5, size=k)]
        if graph:
            path = ["auto", "fused", "generic", "layered"][int(rng.integers(4))]
            dtype = ["f32", "f16"][int(rng.integers(2))]
            print(f"seed {seed}: graph path={path} dtype={dtype} B={B}", flush=True)
            gm = G.GeneratedModel(gr, path=path)
            try:
                gm.plan(dtype)
            except P.PonniError as e:
                if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
                    continue
                raise
            xt = torch.from_numpy(x.astype(np.float32)).cuda()
            y = torch.full((gm.num_outputs, B), 7.0, dtype=torch.float32, device="cuda:0")
            (gm.infer_batch_half2 if dtype == "f16" else gm.infer_batch)(xt, y)
            torch.cuda.synchronize()
            got, xg, layers = y.double().cpu().numpy(), xt.double().cpu().numpy(), lowered_with_params(gr)
            if dtype == "f16":
                with np.errstate(over="ignore"):
                    xg = xg.astype(np.float16).astype(np.float64)
        else:
            path = PATHS[int(rng.integers(len(PATHS)))]
            dtype = ["f32", "f16", "bf16", "f64"][int(rng.integers(4))]
            print(f"seed {seed}: chain width={n} path={path} dtype={dtype} B={B}", flush=True)
            try:
                m = make_model(layers, dtype, path)
            except P.PonniError as e:
                if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
                    continue
                raise
            xs = torch.from_numpy(x).to(getattr(torch, TORCH_DT[dtype])).cuda()
            y = m.forward_batch_parallel(xs)
            torch.cuda.synchronize()
            got, xg = y.double().cpu().numpy(), xs.double().cpu().numpy()
        want = oracle.forward(layers, xg, ORACLE_MODE[dtype])
        try:
            check_non_finite(got, want, dtype)
        except AssertionError as e:
            failed.append(f"seed {seed} ({path}, {dtype}): {e}")
    assert not failed, "\n".join(failed)
