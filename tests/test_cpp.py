"""Runs the C++ facade tests (tests/cpp/test_facade.cpp) built by
__graft_entry__.build() (make -C tests/cpp)."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "test_facade")


def _run(args):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: build with `python -c 'import __graft_entry__ as g; g.build()'`")
    r = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failures" in r.stdout


def test_facade_host_only():
    _run(["--cpu"])


@pytest.mark.gpu
def test_facade_on_gpu(cuda):
    _run([])


# ---- generated-model header (ponni_amd/emitter.py) ---------------------------------

GEN_BIN = os.path.join(os.path.dirname(BIN), "test_generated")


def _apply_gather(table, literals, storage):
    import numpy as np

    return np.array([storage[g] if g >= 0 else literals[-g - 1] for g in table], dtype=np.float64)


@pytest.mark.parametrize("which", ["c5"] + [f"random{k}" for k in range(16)] + [f"narrow{k}" for k in range(8)])
def test_emitted_gather_tables_rebuild_layer_params(which):
    """The header's per-layer gather tables, applied to the weights storage,
    give exactly the parameter vectors the Python model pushes to its plans
    (the tables are found by tracing the builders on index-valued constants)."""
    import numpy as np

    from ponni_amd import configs as C
    from ponni_amd import emitter as E
    from ponni_amd import graph as G
    from tests.test_graph import random_graph

    if which == "c5":
        gr = C.c5_graph(True)
    elif which.startswith("narrow"):
        gr = random_graph(200 + int(which[6:]), narrow=True)
    else:
        k = int(which[6:])
        gr = random_graph(k, aligned=k % 2 == 0)
    gm = G.GeneratedModel(gr)
    gm.storage = np.random.default_rng(7).standard_normal(gm.storage.size)
    tables, literals = E._gather_tables(gm)
    want = gm.lowered.layer_params(gm._constants("f64"))
    assert len(tables) == len(want)
    for t, v in zip(tables, want):
        v = np.asarray(v, dtype=np.float64).reshape(-1)
        assert len(t) == v.size
        np.testing.assert_array_equal(_apply_gather(t, literals, gm.storage), v)


def test_emitted_header_text(tmp_path):
    from ponni_amd import configs as C
    from ponni_amd import emitter as E
    from ponni_amd import graph as G

    gm = G.GeneratedModel(C.c5_graph(True))
    text = E.emit_cpp_header(C.c5_graph(True), str(tmp_path / "m.h"), class_name="M5")
    assert "class M5 {" in text and "namespace ponni { namespace generated {" in text
    assert f'return "{gm.model_fingerprint()}"' in text
    assert "static constexpr int num_inputs = 24;" in text and "static constexpr int num_outputs = 10;" in text
    for dt in ("f32", "f16"):
        gm.plan(dt).kernel_config()  # settles the occupancy the source carries
        src = gm.plan(dt).kernel_source()
        name = E._kernel_name(src)
        assert f"M5_kernels::k_{dt}::{name}" in text  # infer_batch / infer_batch_half2 launch it
        assert E._kernel_text(src) in text  # the library's own kernel text, compiled ahead of time
    assert "#include" not in text.split("namespace M5_kernels")[1]


def _generated_case(tmp_path, model):
    """(graph factory, weights file, x, batch, output reader, oracle layer builder,
    oracle mode, check) of one emitted-header case: c5 and f64 on weights the
    Python model saved, tiny on the file the reference generator wrote."""
    import numpy as np

    import oracle
    from ponni_amd import configs as C
    from ponni_amd import graph as G
    from tests.cpp.gen_headers import f64_graph
    from tests.golden.make_generated_fixtures import tiny_graph
    from tests.test_gpu_parity import check_f32

    if not os.path.exists(GEN_BIN):
        pytest.fail(f"{GEN_BIN} is missing: build with `python -c 'import __graft_entry__ as g; g.build()'`")
    oracle.build()
    make_graph = {"c5": lambda: C.c5_graph(True), "tiny": tiny_graph, "f64": f64_graph}[model]
    if model == "tiny":
        weights = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_generated.ponni")
    else:
        gm = G.GeneratedModel(make_graph())
        gm.storage = gm.storage * 0.5 + np.random.default_rng(11).uniform(-0.05, 0.05, gm.storage.size)
        weights = tmp_path / "w.ponni"
        gm.save_parameters(str(weights))
    ref = G.GeneratedModel(make_graph())
    ref.load_weights(str(weights))  # the values the file holds
    dt = np.float64 if ref.scalar == "f64" else np.float32
    n_in, n_out = ref.num_inputs, ref.num_outputs
    B = 4099
    x = np.random.default_rng(12).standard_normal((n_in, B)).astype(dt)
    x.tofile(tmp_path / "x.bin")

    def out(name):
        return np.fromfile(tmp_path / name, dtype=dt).reshape(n_out, B).astype(np.float64)

    def oracle_layers(m):
        layers = m.lowered.layers
        for l, v in zip(layers, m.lowered.layer_params(m._constants("f64"))):
            if v.size:
                l.params = v
        return layers

    def check(got, want):
        if dt == np.float64:
            assert np.allclose(got, want, rtol=1e-11, atol=1e-11 * max(1.0, np.abs(want).max()))
        else:
            check_f32(got, want)

    mode = oracle.MODE_F64 if dt == np.float64 else oracle.MODE_F32
    return make_graph, weights, ref, x, B, dt, out, oracle_layers, mode, check


@pytest.mark.parametrize("model", ["c5", "tiny", "f64"])
def test_generated_header_infer_one_on_host(tmp_path, model):
    """The emitted header's infer_one on the host (no GPU): the model's
    per-sample program compiled into the header (ponni_plan_program_source,
    ponni::forward_one_program), run by a copy of the model taken before its
    weights were loaded, against the CPU oracle; again after halving the
    parameters.  fp32: relative L2 <= 1e-5, max-abs <= 1e-4; fp64: 1e-11."""
    import oracle

    _, weights, ref, x, B, dt, out, oracle_layers, mode, check = _generated_case(tmp_path, model)
    r = subprocess.run([GEN_BIN, model, str(weights), str(tmp_path / "x.bin"), str(B), str(tmp_path), "--host"],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    check(out("y_host.bin"), oracle.forward(oracle_layers(ref), x.astype("float64"), mode))
    ref.set_parameters(ref.get_parameters() * 0.5)
    check(out("y_host_scaled.bin"), oracle.forward(oracle_layers(ref), x.astype("float64"), mode))


def test_program_source_is_the_generic_lowering():
    """ponni_plan_program_source is the plan's GENERIC lowering whatever path
    the plan runs on (same text, the plan's scratch widths), keeps doubles
    exact, and refuses 16-bit plans."""
    import numpy as np

    import ponni_amd as P
    from ponni_amd import configs as C

    for layers in (C.c2_layers(True), C.c3_layers(True)):
        m = P.create_inference_model(*layers, dtype="f32")
        g = P.create_inference_model(*layers, dtype="f32", path="generic")
        src = m.program_source()
        assert src == g.program_source()
        body = src.split("ops[")[1].split("};")[0]
        n_ops = int(src.split("num_ops = ")[1].split(";")[0])
        assert n_ops >= len(layers) // 3 and body.count("\n      {") == n_ops
        inf = g.info()
        assert f"tmp_features[2] = {{{inf.tmp1_features}, {inf.tmp2_features}}};" in src
        assert "static constexpr int dtype = 1;" in src
    ln = P.create_inference_model(P.LayerNorm(np.ones(3), np.zeros(3), 1.0 / 3.0), dtype="f64")
    assert repr(1.0 / 3.0) in ln.program_source() or "0.33333333333333331" in ln.program_source()
    with pytest.raises(P.PonniError):
        P.create_inference_model(*C.c4_layers(), dtype="f16").program_source()


@pytest.mark.gpu
@pytest.mark.parametrize("model", ["c5", "tiny", "f64"])
def test_generated_header_on_gpu(cuda, tmp_path, model):
    """tests/cpp/test_generated.cpp over an emitted header: infer_batch
    (the ahead-of-time kernel), infer_batch_half2 and infer_one (an
    application kernel over device(), a kernel lambda holding a copy of the
    model taken before its weights were loaded -- bit-identical to the
    device() kernel -- and the host) against the CPU oracle, on a weights
    file saved by the Python model (c5, f64) or written by the reference
    generator (tiny, tests/golden/tiny_generated.ponni); then the parameter
    API (get, set from a device view, save) against the Python model.  fp32
    bar: relative L2 <= 1e-5 and max-abs <= 1e-4; fp64: 1e-11; fp16: relative
    L2 <= 2e-3 against fp16 operands."""
    import numpy as np

    import oracle
    from ponni_amd import graph as G
    from tests.test_gpu_parity import check_half

    make_graph, weights, ref, x, B, dt, out, oracle_layers, mode, check = _generated_case(tmp_path, model)
    r = subprocess.run([GEN_BIN, model, str(weights), str(tmp_path / "x.bin"), str(B), str(tmp_path)],
                       capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr

    want = oracle.forward(oracle_layers(ref), x.astype(np.float64), mode)
    check(out("y_batch.bin"), want)
    check(out("y_one.bin"), want)
    # The model captured by value runs the device() handle's code on the same description.
    np.testing.assert_array_equal(out("y_copy.bin"), out("y_one.bin"))
    check(out("y_host.bin"), want)
    if model != "f64":  # (the random F64 graph's Exp / Div leave the fp16 range)
        xh = x.astype(np.float16).astype(np.float64)
        check_half(out("y_half.bin"), oracle.forward(oracle_layers(ref), xh, oracle.MODE_F16_OPERANDS))

    learned = ref.get_parameters()
    np.testing.assert_array_equal(np.fromfile(tmp_path / "params.bin", dtype=dt), learned.astype(dt))
    ref.set_parameters(learned * 0.5)
    want = oracle.forward(oracle_layers(ref), x.astype(np.float64), mode)
    check(out("y_batch_scaled.bin"), want)
    check(out("y_one_scaled.bin"), want)
    np.testing.assert_array_equal(out("y_copy_scaled.bin"), out("y_one_scaled.bin"))
    check(out("y_host_scaled.bin"), want)
    saved = G.GeneratedModel(make_graph())
    saved.load_weights(str(tmp_path / "saved.ponni"))
    np.testing.assert_array_equal(saved.storage, ref.storage)
