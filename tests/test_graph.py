"""Generated-model path on the CPU: graph linearization, the oracle's graph
operations, the generated model API and weights files.

Pinning: the oracle runs the *linearized chain* per sample; tests/numpy_graph.py
evaluates the *graph* itself (DAG walk, whole-batch float64 numpy, following
kokkos_nn/interpreter.py).  Agreement on random DAGs pins both the
linearization (slot allocation, loads, projection-skip rewrite, concat order)
and the oracle's Dense / Binary / Reduce / Unary / Const_Binary restatements.
Hand-computed closed forms pin the numpy evaluator in turn.
"""
import math

import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import _abi as A
from ponni_amd import configs as C
from ponni_amd import graph as G
from tests import numpy_graph as NG


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


def lowered_with_params(graph):
    gm = G.GeneratedModel(graph)
    layers = gm.lowered.layers
    for l, v in zip(layers, gm.lowered.layer_params(gm._constants("f64"))):
        if v.size:
            l.params = v
    return layers


def run_oracle(graph, x, mode=oracle.MODE_F64):
    return oracle.forward(lowered_with_params(graph), x, mode)


# ---- closed forms --------------------------------------------------------------

def tiny_graph():
    g = G.GraphBuilder(2)
    x = g.input
    d = g.dense(x, [[1.0, 2.0], [3.0, 4.0], [0.5, -1.0]], [1.0, 1.0, -0.5], name="fc")  # bias first
    m = g.reduce("ReduceMean", d)
    c = g.binary("Sub", d, m)
    s = g.softmax(c)
    return g.finish(s)


def test_tiny_graph_closed_form():
    x = np.array([[1.0, 0.0], [1.0, 2.0]])
    for b in range(2):
        x0, x1 = x[:, b]
        d = [1 + 1 * x0 + 2 * x1, 1 + 3 * x0 + 4 * x1, -0.5 + 0.5 * x0 - 1.0 * x1]
        mean = sum(d) / 3
        c = [v - mean for v in d]
        mx = max(c)
        e = [math.exp(v - mx) for v in c]
        want = [v / sum(e) for v in e]
        got_np = NG.run_graph(tiny_graph(), x)[:, b]
        got_or = run_oracle(tiny_graph(), x)[:, b]
        assert np.allclose(got_np, want, rtol=1e-14, atol=1e-15)
        assert np.allclose(got_or, want, rtol=1e-14, atol=1e-15)


def test_binary_operand_order_and_broadcast():
    # (m - x) with the one-feature operand on the left, x / 4 with a constant,
    # 2^x with a constant base: operand order is kept in every form.
    g = G.GraphBuilder(3)
    x = g.input
    m = g.reduce("ReduceMax", x)
    a = g.binary("Sub", m, x)                     # saved one-feature left operand
    b = g.binary("Div", a, g.constant("four", [4.0]))
    c = g.binary("Pow", g.constant("two", [2.0]), b)
    d = g.binary("Max", c, g.constant("floor", [1.25, 1.0, 1.0]))
    gr = g.finish(d)
    x = np.array([[1.0, -2.0], [3.0, 0.0], [2.0, 1.0]])
    mx = x.max(axis=0)
    want = np.maximum(2.0 ** ((mx - x) / 4.0), np.array([[1.25], [1.0], [1.0]]))
    assert np.allclose(NG.run_graph(gr, x), want, rtol=1e-14)
    assert np.allclose(run_oracle(gr, x), want, rtol=1e-14)


def test_reductions_closed_form():
    x = np.array([[1.0, -2.0], [3.0, 0.5], [2.0, 4.0]])
    want = {
        "ReduceSum": x.sum(0), "ReduceMean": x.mean(0), "ReduceMax": x.max(0), "ReduceMin": x.min(0),
        "ReduceL1": np.abs(x).sum(0), "ReduceL2": np.sqrt((x * x).sum(0)), "ReduceSumSquare": (x * x).sum(0),
        "ReduceLogSumExp": np.log(np.exp(x).sum(0)), "ReduceProd": x.prod(0),
    }
    for op, w in want.items():
        g = G.GraphBuilder(3)
        gr = g.finish(g.reduce(op, g.unary("Relu", g.input) if op == "ReduceLogSum" else g.input))
        assert np.allclose(run_oracle(gr, x)[0], w, rtol=1e-13), op
        assert np.allclose(NG.run_graph(gr, x)[0], w, rtol=1e-13), op
    g = G.GraphBuilder(3)
    gr = g.finish(g.reduce("ReduceLogSum", g.unary("Abs", g.input)))
    assert np.allclose(run_oracle(gr, x)[0], np.log(np.abs(x).sum(0)), rtol=1e-13)


def test_unary_graph_ops_closed_form():
    v = np.array([[-2.0, -0.5, 0.0, 0.7, 3.0]])
    cases = {
        "Abs": np.abs(v), "Neg": -v, "Exp": np.exp(v), "Softsign": v / (1 + np.abs(v)),
        "Erf": np.array([[math.erf(t) for t in v[0]]]),
        "ThresholdedRelu": np.where(v > 1.0, v, 0.0),
        "Celu": np.where(v > 0, v, 1.0 * (np.exp(v / 1.0) - 1)),
        "Selu": 1.0507010221481323 * np.where(v > 0, v, 1.6732631921768188 * (np.exp(v) - 1)),
    }
    for op, want in cases.items():
        g = G.GraphBuilder(1)
        gr = g.finish(g.unary(op, g.input))
        assert np.allclose(run_oracle(gr, v), want, rtol=1e-13, atol=1e-15), op
        assert np.allclose(NG.run_graph(gr, v), want, rtol=1e-13, atol=1e-15), op
    g = G.GraphBuilder(1)
    w = np.abs(v) + 0.5
    gr = g.finish(g.unary("Reciprocal", g.unary("Sqrt", g.unary("Log", g.binary("Add", g.unary("Abs", g.input),
                                                                                 g.constant("c", [1.5]))))))
    want = 1 / np.sqrt(np.log(np.abs(v) + 1.5))
    assert np.allclose(run_oracle(gr, v), want, rtol=1e-13)
    del w


# ---- linearization ---------------------------------------------------------------

def test_c5_linearization():
    layers = C.CONFIGS["c5"].layers(False)
    assert [l.label for l in layers] == [
        "Save_State", "Dense", "ReLU", "Dense", "Save_State", "Load_State", "Dense", "Sigmoid",
        "Binop_Concatenate", "Binop_Projection_Add", "Save_State", "ReduceMean", "Sub", "Dense", "Softmax"]
    concat = layers[8]
    assert concat.flags == 0 and concat.n_in == 48 and concat.n_out == 96  # [branch A; branch B]
    proj = layers[9]
    assert proj.n_aux == 24 and proj.slot == layers[0].slot  # reads the saved input
    sub = layers[12]
    assert sub.n_in == 1 and sub.n_aux == 96 and sub.flags == P._abi.FLAG_SAVED_LEFT


def test_c5_oracle_matches_graph_evaluation():
    gr = C.c5_graph(True)
    x = C.normal(24 * 257, 4, C.INPUT_TAG, 0.0, 1.0).reshape(24, 257).astype(np.float64)
    want = NG.run_graph(gr, x)
    got = run_oracle(gr, x)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-15)
    got32 = oracle.forward(lowered_with_params(gr), x, oracle.MODE_F32)
    assert np.linalg.norm(got32 - want) / np.linalg.norm(want) < 1e-6


ELEMENTWISE = ["Relu", "Sigmoid", "Tanh", "LeakyRelu", "Elu", "Gelu", "Silu", "Softplus", "HardSigmoid",
               "HardSwish", "Mish", "Abs", "Neg", "Softsign", "Celu", "Erf", "Selu", "ThresholdedRelu"]


def random_graph(seed: int, aligned: bool = False, n_in: int | None = None, nodes: int = 14, dtype="float32",
                 narrow: bool = False):
    """A random DAG over the supported operations.  aligned: every width a
    multiple of 16 (what the FUSED concatenation needs); narrow: every width
    at most 16 (what the NARROW kernels take)."""
    rng = np.random.default_rng(seed)
    widths = [16, 32, 48] if aligned else [1, 3, 5, 8, 12, 16] if narrow else [1, 3, 5, 8, 13, 16, 24, 33]
    n_in = n_in or int(rng.choice(widths[1:] if aligned else widths[2:]))
    g = G.GraphBuilder(n_in, dtype=dtype)
    pool = [g.input]
    for k in range(nodes):
        t = pool[-1] if rng.random() < 0.5 else pool[int(rng.integers(len(pool)))]
        n = g.size(t)
        r = rng.random()
        if r < 0.3 or n == 1:
            m = int(rng.choice(widths))
            lim = math.sqrt(6 / (n + m))
            bias = rng.uniform(-0.2, 0.2, m) if rng.random() < 0.7 else None
            out = g.dense(t, rng.uniform(-lim, lim, (m, n)), bias, name=f"d{k}")
        elif r < 0.5:
            op = str(rng.choice(ELEMENTWISE))
            attrs = {}
            if op == "Gelu":
                attrs["approximate"] = "tanh" if rng.random() < 0.5 else "none"
            if op == "ThresholdedRelu":
                attrs["alpha"] = 0.25
            out = g.unary(op, t, **attrs)
        elif r < 0.62:
            same = [u for u in pool if g.size(u) in (n, 1) and u != t]
            if not same:
                continue
            u = same[int(rng.integers(len(same)))]
            op = str(rng.choice(["Add", "Sub", "Mul", "Max", "Min"]))
            out = g.binary(op, t, u) if rng.random() < 0.5 else g.binary(op, u, t)
        elif r < 0.7:
            op = str(rng.choice(["Add", "Sub", "Mul", "Div", "Max", "Min"]))
            cv = rng.uniform(0.5, 1.5, n if rng.random() < 0.6 else 1)
            c = g.constant(f"c{k}", cv)
            out = g.binary(op, t, c) if rng.random() < 0.5 else g.binary(op, c, t) if op != "Div" else g.binary(op, t, c)
        elif r < 0.8:
            others = [u for u in pool if u != t]
            if not others:
                continue
            parts = [t, others[int(rng.integers(len(others)))]]
            if rng.random() < 0.5:
                parts.reverse()
            if sum(g.size(p) for p in parts) > (256 if aligned else 16 if narrow else 96):
                continue
            out = g.concat(*parts)
        elif r < 0.87:
            op = str(rng.choice(["ReduceMean", "ReduceSum", "ReduceMax", "ReduceMin", "ReduceL2", "ReduceLogSumExp"]))
            red = g.reduce(op, t)
            out = g.binary("Sub", t, red) if rng.random() < 0.7 else red
        elif r < 0.93:
            out = g.softmax(t, log=rng.random() < 0.3)
        else:
            out = g.layer_norm(t, rng.uniform(0.5, 1.5, n), rng.uniform(-0.2, 0.2, n) if rng.random() < 0.5 else None,
                               name=f"ln{k}")
        pool.append(out)
    if g.size(pool[-1]) == 1 and len(pool) > 1:
        pool.append(g.dense(pool[-1], rng.uniform(-1, 1, (int(rng.choice(widths[1:])), 1)), None, name="tail"))
    return g.finish(pool[-1])


@pytest.mark.parametrize("seed", range(24))
def test_random_graphs_oracle_vs_numpy(seed):
    gr = random_graph(seed, aligned=seed % 3 == 0)
    B = 64
    n_in = gr.size(gr.inputs[0])
    x = np.random.default_rng(100 + seed).standard_normal((n_in, B))
    want = NG.run_graph(gr, x)
    got = run_oracle(gr, x)
    assert np.isfinite(want).all()
    tol = 1e-9 * max(1.0, np.abs(want).max())
    assert np.allclose(got, want, rtol=1e-9, atol=tol), np.abs(got - want).max()


def test_slot_reuse_and_limit():
    # 9 tensors live at once take at least eight saved slots: fine by
    # default, too many for a linearization capped below what it uses.
    g = G.GraphBuilder(4)
    xs = [g.unary("Relu", g.dense(g.input, np.eye(4), None, name=f"b{i}")) for i in range(9)]
    acc = xs[0]
    for t in xs[1:]:
        acc = g.binary("Add", acc, t)
    gr = g.finish(acc)
    used = len({l.slot for l in G.lower_graph(gr).layers if l.kind == A.LAYER_SAVE_STATE})
    assert used >= 8
    with pytest.raises(G.GraphError, match="live saved tensors"):
        G.lower_graph(gr, max_slots=used - 1)
    # A chain reuses slot 0 after each tensor's last use.
    g = G.GraphBuilder(4)
    t = g.input
    for i in range(10):
        u = g.unary("Tanh", t)
        t = g.binary("Add", t, u)
    lw = G.lower_graph(g.finish(t))
    assert max(l.slot for l in lw.layers) == 0


def test_unsupported_broadcast_rejected():
    g = G.GraphBuilder(4)
    a = g.dense(g.input, np.ones((3, 4)), None, name="a")
    b = g.dense(g.input, np.ones((2, 4)), None, name="b")
    with pytest.raises(G.GraphError, match="broadcasting"):
        G.lower_graph(g.finish(g.binary("Add", a, b)))


def test_fused_variants_expand():
    # DenseBiasActivation / DenseResidualActivation / DenseEpilogue nodes of an
    # optimized graph (interpreter.py:353-381) lower to the same arithmetic.
    g = G.GraphBuilder(3)
    x = g.input
    w1 = g.constant("w1", np.arange(12.0).reshape(4, 3) / 10, "output_input")
    b1 = g.constant("b1", [0.1, -0.2, 0.3, 0.0], "output")
    h = g.node("DenseBiasActivation", [x, w1, b1], 4, {"weight": w1, "bias": b1, "activation": "Tanh"})
    w2 = g.constant("w2", np.ones((4, 4)) / 4, "output_input")
    r = g.node("DenseResidualActivation", [h, w2], 4, {"weight": w2, "bias": None, "residual": h,
                                                       "activation": "Relu"})
    w3 = g.constant("w3", np.ones((2, 4)), "output_input")
    s = g.constant("s", [2.0, 3.0])
    e = g.node("DenseEpilogue", [r, w3], 2, {"weight": w3, "bias": None, "epilogue_steps": [
        {"op": "Mul", "inputs": ["prev", s]}, {"op": "Sigmoid", "inputs": ["prev"]}]})
    gr = g.finish(e)
    x = np.array([[1.0, -1.0], [0.5, 2.0], [-0.3, 0.0]])
    W1 = np.arange(12.0).reshape(4, 3) / 10
    hh = np.tanh(W1 @ x + np.array([[0.1], [-0.2], [0.3], [0.0]]))
    rr = np.maximum(np.ones((4, 4)) / 4 @ hh + hh, 0)
    ee = 1 / (1 + np.exp(-(np.ones((2, 4)) @ rr * np.array([[2.0], [3.0]]))))
    assert np.allclose(run_oracle(gr, x), ee, rtol=1e-13)


# ---- generated model API ------------------------------------------------------------

def test_weight_specs_and_storage_index():
    gm = G.GeneratedModel(C.c5_graph(True))
    specs = gm.weight_specs()
    names = [s.name for s in specs]
    assert names == sorted(names)  # weights.ponni order (weights.py:299-306)
    off = 0
    for s in specs:
        assert s.offset == off and s.dtype == "F32"
        off += s.size
    assert off == gm.storage_parameter_elements == 2304 + 96 + 4608 + 48 + 1152 + 48 + 2304 + 96 + 960 + 10
    # learned order is tensor-id order (emitter.py:1449-1465)
    learned = [t for _, t in sorted(gm.graph.tensors.items()) if t.is_constant]
    idx = 0
    for t in learned:
        spec = next(s for s in specs if s.name == t.name)
        assert gm.parameter_storage_index(idx) == spec.offset
        idx += t.sample_size
    assert gm.get_num_parameters() == idx
    with pytest.raises(IndexError):
        gm.parameter_storage_index(idx)


def test_set_get_parameters_roundtrip():
    gm = G.GeneratedModel(C.c5_graph(False))
    v = np.random.default_rng(0).standard_normal(gm.get_num_parameters())
    gm.set_parameters(v)
    assert np.array_equal(gm.get_parameters(), v)
    with pytest.raises(ValueError):
        gm.set_parameters(v[:-1])


def test_weights_file_roundtrip_and_rejections(tmp_path):
    gm = G.GeneratedModel(C.c5_graph(True))
    path = tmp_path / "weights.ponni"
    gm.save_parameters(str(path))
    blob = path.read_bytes()
    hlen = int.from_bytes(blob[:8], "little")
    import json
    header = json.loads(blob[8:8 + hlen])
    assert header["__metadata__"]["ponni.model_fingerprint"] == gm.model_fingerprint()
    assert header["__metadata__"]["ponni.target"] == "generated"
    assert hlen % 8 == 0
    offsets = [header[s.name]["data_offsets"] for s in gm.weight_specs()]
    assert offsets[0][0] == 0 and all(a[1] == b[0] for a, b in zip(offsets, offsets[1:]))
    other = G.GeneratedModel(C.c5_graph(False))
    assert not np.array_equal(other.storage, gm.storage)
    other.load_weights(str(path))
    assert np.array_equal(other.storage, gm.storage.astype(np.float32).astype(np.float64))
    # a graph with another structure has another fingerprint: rejected
    g = G.GraphBuilder(24)
    small = G.GeneratedModel(g.finish(g.dense(g.input, np.ones((10, 24)), None, name="x")))
    with pytest.raises(P.PonniError, match="fingerprint"):
        small.load_weights(str(path))
    bad = bytearray(blob)
    bad[-1] ^= 1
    (tmp_path / "bad.ponni").write_bytes(bytes(bad))
    with pytest.raises(P.PonniError, match="checksum"):
        other.load_weights(str(tmp_path / "bad.ponni"))


def test_fingerprint_tracks_structure_not_values():
    a = G.graph_fingerprint(C.c5_graph(False))
    b = G.graph_fingerprint(C.c5_graph(True))
    assert a == b and a.startswith("fnv1a64:") and len(a) == 8 + 16
    g = G.GraphBuilder(24)
    assert G.graph_fingerprint(g.finish(g.dense(g.input, np.ones((10, 24)), None))) != a
    assert G.fnv1a64(b"") == 0xCBF29CE484222325 and G.fnv1a64(b"a") == 0xAF63DC4C8601EC8C


def test_c5_plan_is_fused_and_compiles():
    gm = G.GeneratedModel(C.c5_graph(False))
    plan = gm.plan()
    assert plan.path == "fused"
    src = plan.kernel_source()
    # four Dense ops and the projection skip, epilogues pinned among their
    # MFMAs; the skip's bias seeds its accumulators and the Add with the
    # concatenation runs in its epilogue
    assert src.count("dense_ep_il<16, ") == 5 and src.count("dense_ep<") == 0
    assert "bias_rows<6>(P + 12480, L)" in src and "add_rows<" not in src
    assert src.count("tile_add_state(t, ") == 1 and "    add(" not in src
    assert "reduce<1, 96, false>" in src and "binary<96, false, true>" in src
    assert "concat<3, 3>" in src and "softmax<10, false>" in src
    plan.compile()
    half = gm.plan("f16")
    assert half.path == "fused" and half.kernel_source().count("dense_hs<") == 4
    half.compile()


@pytest.mark.parametrize("form", ["dense_right", "dense_left", "same_input", "dense_has_other_use"])
def test_projection_skip_forms(form):
    rng = np.random.default_rng(7)
    g = G.GraphBuilder(6)
    x = g.input
    t = g.unary("Tanh", g.dense(x, rng.standard_normal((5, 6)), rng.standard_normal(5), name="main"))
    src = x if form != "same_input" else t
    n_src = g.size(src)
    p = g.dense(src, rng.standard_normal((5, n_src)), rng.standard_normal(5), name="proj")
    s = g.binary("Add", p, t) if form == "dense_left" else g.binary("Add", t, p)
    if form == "dense_has_other_use":
        s = g.binary("Mul", s, p)
    gr = g.finish(s)
    lw = G.lower_graph(gr)
    labels = [l.label for l in lw.layers]
    assert ("Binop_Projection_Add" in labels) == (form != "dense_has_other_use")
    xin = rng.standard_normal((6, 9))
    assert np.allclose(run_oracle(gr, xin), NG.run_graph(gr, xin), rtol=1e-12, atol=1e-12)


def test_dead_nodes_dropped():
    g = G.GraphBuilder(4)
    y = g.unary("Relu", g.input)
    g.dense(g.input, np.ones((7, 4)), None, name="unused")
    lw = G.lower_graph(g.finish(y))
    assert [l.label for l in lw.layers] == ["ReLU"]


def test_narrow_generated_graphs_take_the_narrow_path():
    """Generated graphs of width <= 16 run generated NARROW kernels (one lane
    per sample group, graph operations inline); wider ones stay FUSED."""
    from tests.golden.make_generated_fixtures import tiny_graph

    src = G.GeneratedModel(tiny_graph()).plan("f32").kernel_source()
    assert "ponni_narrow_3x4x2" in src and src.count("dense_bias<") == 2
    seen = set()
    for seed in range(12):
        gm = G.GeneratedModel(random_graph(seed, narrow=True))
        plan = gm.plan("f32")
        assert plan.path in ("narrow", "fused"), plan.path
        if plan.path == "narrow":
            text = plan.kernel_source()
            seen.update(op for op in ("binary<", "reduce<", "copy<", "softmax<", "layer_norm<", "concat<")
                        if op in text)
    assert {"binary<", "reduce<"} <= seen, seen
    assert G.GeneratedModel(C.c5_graph(False)).plan("f32").path == "fused"


# ---- selection, logic, normalization and unary math -----------------------------

def _one_node(op, ins_values, attrs=None, size=None, bool_out=False):
    """y = op(x, constants...) on a 1-row input; returns the oracle's float64 answer per column."""
    x = np.asarray(ins_values[0], dtype=np.float64)
    n = x.shape[0]
    g = G.GraphBuilder(n, dtype="float64")
    args = [g.input] + [g.constant(f"c{k}", v) for k, v in enumerate(ins_values[1:])]
    out = g.node(op, args, size or n, attrs or {})
    gr = g.finish(out)
    return run_oracle(gr, x.reshape(n, -1)), NG.run_graph(gr, x.reshape(n, -1))


def test_new_ops_closed_forms():
    nan, inf = float("nan"), float("inf")
    x = np.array([[-2.5], [-0.5], [0.5], [1.5], [2.5], [0.0]])
    # Round: ties to even (emitter.py:1659-1667); Sign keeps NaN
    got, ref = _one_node("Round", [x])
    assert got.ravel().tolist() == [-2.0, -0.0, 0.0, 2.0, 2.0, 0.0]
    got, _ = _one_node("Sign", [np.array([[-3.0], [0.0], [2.0], [nan]])])
    assert got.ravel()[:3].tolist() == [-1.0, 0.0, 1.0] and np.isnan(got.ravel()[3])
    # IsInf with detect_negative = 0
    v = np.array([[-inf], [inf], [1.0], [nan]])
    got, _ = _one_node("IsInf", [v], {"detect_negative": 0, "detect_positive": 1})
    assert got.ravel().tolist() == [0.0, 1.0, 0.0, 0.0]
    got, _ = _one_node("IsInf", [v])
    assert got.ravel().tolist() == [1.0, 1.0, 0.0, 0.0]
    got, _ = _one_node("IsNaN", [v])
    assert got.ravel().tolist() == [0.0, 0.0, 0.0, 1.0]
    # PRelu: x >= 0 ? x : x * slope
    got, _ = _one_node("PRelu", [np.array([[-2.0], [0.0], [3.0]]), [0.25]])
    assert got.ravel().tolist() == [-0.5, 0.0, 3.0]
    # Clip keeps a NaN (the constant bound on the left of the comparison)
    got, _ = _one_node("Clip", [np.array([[-5.0], [0.3], [5.0], [nan]])], {"min": -1.0, "max": 2.0})
    assert got.ravel()[:3].tolist() == [-1.0, 0.3, 2.0] and np.isnan(got.ravel()[3])
    # comparisons and logic give 1 / 0; any nonzero is true
    a = np.array([[1.0], [2.0], [3.0]])
    for op, want in (("Equal", [0, 1, 0]), ("Greater", [0, 0, 1]), ("GreaterOrEqual", [0, 1, 1]),
                     ("Less", [1, 0, 0]), ("LessOrEqual", [1, 1, 0])):
        got, _ = _one_node(op, [a, [2.0]])
        assert got.ravel().tolist() == want, op
    b = np.array([[0.0], [0.5], [-2.0], [0.0]])
    for op, want in (("And", [0, 1, 0, 0]), ("Or", [1, 1, 1, 0]), ("Xor", [1, 0, 1, 0])):
        got, _ = _one_node(op, [b, [1.0, 1.0, 0.0, 0.0]])
        assert got.ravel().tolist() == want, op
    got, _ = _one_node("Not", [b])
    assert got.ravel().tolist() == [1.0, 0.0, 0.0, 1.0]
    # LpNormalization: a zero vector stays zero; p = 1 and p = 2
    got, _ = _one_node("LpNormalization", [np.array([[0.0, 3.0], [0.0, -4.0]])], {"p": 2})
    assert got.tolist() == [[0.0, 0.6], [0.0, -0.8]]
    got, _ = _one_node("LpNormalization", [np.array([[3.0], [-1.0]])], {"p": 1})
    assert got.ravel().tolist() == [0.75, -0.25]
    # BatchNormalization: (x - mean) / sqrt(var + eps) * scale + bias
    got, _ = _one_node("BatchNormalization", [np.array([[3.0], [1.0]]), [2.0, 1.0], [0.5, -1.0], [1.0, 1.0],
                                              [4.0 - 1e-5, 0.25 - 1e-5]], {"epsilon": 1e-5})
    assert np.allclose(got.ravel(), [2.5, -1.0], rtol=1e-12)
    # n-ary Mean / Sum
    g = G.GraphBuilder(2, dtype="float64")
    u = g.unary("Neg", g.input)
    m = g.nary("Mean", g.input, u, g.binary("Mul", g.input, g.constant("k", [4.0])))
    got = run_oracle(g.finish(m), np.array([[3.0], [-6.0]]))
    assert got.ravel().tolist() == [4.0, -8.0]
    # Gather reorders and repeats
    g = G.GraphBuilder(3, dtype="float64")
    got = run_oracle(g.finish(g.gather(g.input, [2, 0, 0, -1])), np.array([[1.0], [2.0], [3.0]]))
    assert got.ravel().tolist() == [3.0, 1.0, 1.0, 3.0]


def test_unary_math_against_numpy():
    x = np.linspace(-0.95, 0.95, 41).reshape(41, 1)
    for op, f in (("Acos", np.arccos), ("Asin", np.arcsin), ("Atan", np.arctan), ("Atanh", np.arctanh),
                  ("Asinh", np.arcsinh), ("Sin", np.sin), ("Cos", np.cos), ("Tan", np.tan), ("Sinh", np.sinh),
                  ("Cosh", np.cosh), ("Floor", np.floor), ("Ceil", np.ceil)):
        got, _ = _one_node(op, [x])
        assert np.allclose(got, f(x), rtol=1e-15, atol=1e-15), op
    got, _ = _one_node("Acosh", [1.0 + np.abs(x)])
    assert np.allclose(got, np.arccosh(1.0 + np.abs(x)), rtol=1e-15)


def test_where_operand_sources():
    """Where takes the state, one or two saved slots and constants in every
    position; a one-feature operand broadcasts."""
    rng = np.random.default_rng(3)
    g = G.GraphBuilder(4, dtype="float64")
    a = g.dense(g.input, rng.standard_normal((6, 4)), None, name="a")
    b = g.dense(g.input, rng.standard_normal((6, 4)), None, name="b")
    c = g.compare("Greater", a, b)
    s = g.reduce("ReduceSum", b)
    w1 = g.where(c, a, b)                     # cond state, two slots
    w2 = g.where(c, g.constant("k", rng.standard_normal(6)), w1)
    w3 = g.where(g.compare("Less", s, g.constant("z", [0.0])), w2, g.constant("k2", [0.5]))  # scalar cond
    w4 = g.where(c, s, w3)                    # scalar a from a slot
    gr = g.finish(g.binary("Add", w4, a))
    lw = G.lower_graph(gr)
    assert sum(l.label == "Where" for l in lw.layers) == 4
    x = rng.standard_normal((4, 50))
    assert np.allclose(run_oracle(gr, x), NG.run_graph(gr, x), rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("smooth", [True, False])
@pytest.mark.parametrize("seed", range(16))
def test_op_graphs_oracle_vs_numpy(seed, smooth):
    from tests import graph_cases as GC

    gr = GC.op_graph(seed, smooth=smooth, aligned=seed % 2 == 0, dtype="float64" if seed % 4 == 3 else "float32")
    x = GC.in_domain_input(gr.size(gr.inputs[0]), 48, seed)
    with np.errstate(all="ignore"):
        want = NG.run_graph(gr, x)
    got = run_oracle(gr, x)
    assert np.isfinite(want).all()
    tol = 1e-12 * max(1.0, np.abs(want).max())
    assert np.allclose(got, want, rtol=1e-11, atol=tol), np.abs(got - want).max()
