"""GPU parity: every kernel path of libponni_hip.so against the CPU oracle.

fp32 bar: relative L2 <= 1e-5 and max-abs <= 1e-4,
unscaled, in every test.  fp16 / bf16 bar: relative L2 <= 2e-3 against the
oracle's fp16-operand / fp32-accumulate mode on the same inputs.
"""
import math

import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import configs as C
from tests import test_oracle as K

pytestmark = pytest.mark.gpu

# "narrow-aot" is the interpreted NARROW kernel (run-time compilation off);
# "narrow" is the generated NARROW kernel.
# "layered" runs the GENERIC op list with each dense block as an MFMA
# contraction over the batch.
PATHS = ["generic", "narrow", "narrow-aot", "mfma", "fused", "layered"]
TORCH_DT = {"f32": "float32", "f16": "float16", "bf16": "bfloat16", "f64": "float64"}
ORACLE_MODE = {"f32": oracle.MODE_F32, "f64": oracle.MODE_F64, "f16": oracle.MODE_F16_OPERANDS,
               "bf16": oracle.MODE_BF16_OPERANDS}


@pytest.fixture(scope="module", autouse=True)
def _oracle_built():
    oracle.build()


def make_model(layers, dtype, path):
    """Plan for `path`; "narrow-aot" disables run-time compilation (PONNI_JIT=0)."""
    import os

    if path != "narrow-aot":
        return P.create_inference_model(*layers, dtype=dtype, path=path)
    old = os.environ.get("PONNI_JIT")
    os.environ["PONNI_JIT"] = "0"
    try:
        return P.create_inference_model(*layers, dtype=dtype, path="narrow")
    finally:
        if old is None:
            del os.environ["PONNI_JIT"]
        else:
            os.environ["PONNI_JIT"] = old


def gpu_run(layers, x_np, dtype="f32", path="auto", pad=0, dev="cuda:0"):
    import torch

    tdt = getattr(torch, TORCH_DT[dtype])
    try:
        m = make_model(layers, dtype, path)
    except P.PonniError as e:
        if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
            pytest.skip(f"{path} does not support this chain: {e.message}")
        raise
    n_in, B = x_np.shape
    xs = torch.zeros((n_in, B + pad), dtype=tdt, device=dev)
    xs[:, :B] = torch.from_numpy(np.asarray(x_np, dtype=np.float64)).to(tdt)
    x = xs[:, :B]
    ys = torch.full((m.get_num_outputs(), B + pad), float("nan"), dtype=tdt, device=dev)
    y = ys[:, :B]
    m.forward_batch_parallel(x, y)
    torch.cuda.synchronize()
    if pad:
        assert torch.isnan(ys[:, B:].float()).all(), "kernel wrote past the batch"
    return y.double().cpu().numpy(), xs[:, :B].double().cpu().numpy(), m


def check_f32(got, want):
    """The north star's fp32 bar: relative L2 <= 1e-5 and max-abs <= 1e-4."""
    err = np.abs(got - want)
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert np.isfinite(got).all()
    assert rel <= 1e-5 and err.max() <= 1e-4, f"relL2={rel:.3e} maxabs={err.max():.3e}"


def check_half(got, want, tol=2e-3):
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    print(f"16-bit parity: relL2={rel:.3e} (bar {tol:.1e})", flush=True)
    assert np.isfinite(got).all() and rel <= tol, f"relL2={rel:.3e}"


KNOWN = {
    "first_model": ([P.Matvec(np.ones((2, 2))), P.Bias(np.ones(2)), P.LeakyRelu(2, 0.1)], [[1.0], [2.0]],
                    [[4.0], [4.0]]),
    "layout_36_42": ([P.Matvec(np.arange(10.0, 16.0).reshape(2, 3))], [[1.0], [2.0]], [[36.0], [39.0], [42.0]]),
    "leading_save": ([P.Save_State(0, 2), P.Relu(2), P.Binop_Add(0, 2)], [[-2.0], [3.0]], [[-2.0], [6.0]]),
    "multi_save": ([P.Save_State(0, 2), P.Relu(2), P.Binop_Concatenate(0, 2, 4, True), P.Save_State(1, 4),
                    P.Relu(4), P.Binop_Add(1, 4), P.Binop_Concatenate(0, 4, 6, True)], [[-2.0], [3.0]],
                   [[0.0], [6.0], [-2.0], [6.0], [-2.0], [3.0]]),
    "projection": ([P.Save_State(0, 2), P.Matvec(np.array([[0.25, 0.0, 0.0], [0.0, 0.4, 0.6]])),
                    P.Binop_Projection_Add(0, np.array([[1.0, 0.0, 0.5], [0.0, 1.0, 0.5]]), [0.1, 0.2, 0.3])],
                   [[4.0], [5.0]], [[5.1], [7.2], [7.8]]),
    "softmax_barrier": ([P.Matvec(np.ones((2, 3))), P.Bias([0.0, 1.0, 2.0]), P.Relu(3), P.Softmax(3),
                         P.Matvec(np.ones((3, 2))), P.Bias([0.0, -1.0]), P.Tanh(2)], [[0.5], [0.5]],
                        [[math.tanh(1.0)], [0.0]]),
}


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("name", sorted(KNOWN))
def test_known_answers(cuda, name, path):
    layers, x, want = KNOWN[name]
    x = np.tile(np.asarray(x), (1, 70))  # several waves, ragged last wave
    got, _, _ = gpu_run(layers, x, path=path)
    assert np.allclose(got, np.tile(np.asarray(want), (1, 70)), atol=1e-5), got[:, :3]


@pytest.mark.parametrize("path", PATHS)
def test_four_block_closed_form(cuda, path):
    layers = [P.Matvec(np.ones((2, 5))), P.Bias(np.full(5, 0.5)), P.Relu(5), P.Tanh(5),
              P.Matvec(np.ones((5, 3))), P.Bias(np.full(3, -0.25)), P.Sigmoid(3),
              P.Matvec(np.ones((3, 7))), P.Bias(np.full(7, 0.1)), P.LeakyRelu(7, 0.2),
              P.Matvec(np.ones((7, 2))), P.Bias(np.full(2, -0.2)), P.HardSwish(2)]
    x = np.random.default_rng(0).uniform(-2, 2, (2, 1000))
    got, xg, _ = gpu_run(layers, x, path=path)
    check_f32(got, oracle.forward(layers, xg))


def test_performance_benchmark_closed_form(cuda):
    # unit/performance_benchmark: 8-wide, ones, LeakyRelu(0.1), x = 0.1 -> mean 15.4
    layers = [P.Matvec(np.ones((8, 8))), P.Bias(np.ones(8)), P.LeakyRelu(8, 0.1),
              P.Matvec(np.ones((8, 8))), P.Bias(np.ones(8)), P.LeakyRelu(8, 0.1)]
    for path in PATHS:
        got, _, _ = gpu_run(layers, np.full((8, 1 << 16), 0.1), path=path)
        assert abs(got.mean() - 15.4) <= 1e-3 and np.allclose(got, 15.4, atol=1e-4)


@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("seed", range(10))
def test_random_chains(cuda, seed, path):
    rng = np.random.default_rng(500 + seed)
    width = [3, 8, 13, 16, 24, 40, 64, 100, 128, 7][seed]
    layers = K.random_chain(rng, width, 2 + seed % 4)
    B = [1, 31, 33, 255, 257, 1000, 4097, 64, 129, 2049][seed]
    x = rng.standard_normal((width, B))
    got, xg, _ = gpu_run(layers, x, path=path, pad=3)
    check_f32(got, oracle.forward(layers, xg))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("path", PATHS)
def test_reduced_precision_paths(cuda, dtype, path):
    rng = np.random.default_rng(11)
    layers = [P.Matvec(rng.standard_normal((12, 16)) * 0.3), P.Bias(rng.uniform(-0.1, 0.1, 16)), P.Tanh(16),
              P.Save_State(0, 16), P.LayerNorm(16), P.Matvec(rng.standard_normal((16, 16)) * 0.25),
              P.Gelu(16, True), P.Binop_Add(0, 16), P.Matvec(rng.standard_normal((16, 6)) * 0.3), P.Softmax(6)]
    x = rng.standard_normal((12, 3000))
    got, xg, _ = gpu_run(layers, x, dtype=dtype, path=path)
    check_half(got, oracle.forward(layers, xg, ORACLE_MODE[dtype]), 2e-3)


@pytest.mark.parametrize("seed,width,blocks", [(12, 20, 3), (502, 13, 4), (507, 64, 3)])
def test_f64_generic(cuda, seed, width, blocks):
    # Layer attributes (slopes, epsilons, ranges) stay exact in F64 plans.
    rng = np.random.default_rng(seed)
    layers = K.random_chain(rng, width, blocks)
    x = rng.standard_normal((width, 500))
    got, xg, _ = gpu_run(layers, x, dtype="f64", path="generic")
    want = oracle.forward(layers, xg, oracle.MODE_F64)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seed", range(8))
def test_f64_narrow(cuda, seed):
    """F64 chains of width <= 16 on the generated NARROW kernel (double state,
    exact attributes) against the oracle's fp64 mode."""
    rng = np.random.default_rng(700 + seed)
    width = [3, 8, 13, 16, 5, 7, 12, 16][seed]
    layers = K.random_chain(rng, width, 2 + seed % 3)
    try:
        m = P.create_inference_model(*layers, dtype="f64", path="narrow")
    except P.PonniError as e:
        if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
            pytest.skip(e.message)
        raise
    assert m.path == "narrow"
    B = [1, 257, 4099, 1000, 64, 3001, 4096, 77][seed]
    got, xg, _ = gpu_run(layers, rng.standard_normal((width, B)), dtype="f64", path="narrow", pad=seed % 2)
    want = oracle.forward(layers, xg, oracle.MODE_F64)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12 * max(1.0, np.abs(want).max())), np.abs(got - want).max()


@pytest.mark.parametrize("case", ["c2", "c3", "chain0", "chain1", "chain2", "chain3"])
def test_f64_fused(cuda, case):
    """F64 models on the FUSED kernel (fp64 tiles, v_mfma_f64_16x16x4f64,
    exact attributes, libm activations) against the oracle's fp64 mode; the
    MFMA summation order is the only difference, hence 1e-12."""
    rng = np.random.default_rng(800 + len(case))
    if case.startswith("chain"):
        k = int(case[5:])
        width = [32, 64, 96, 128][k]
        layers = K.random_chain(rng, width, 2 + k % 3)
        x = rng.standard_normal((width, 3001))
    else:
        layers = C.CONFIGS[case].layers(True)
        x = rng.standard_normal((layers[0].n_in, 3001))
    got, xg, m = gpu_run(layers, x, dtype="f64", path="fused", pad=2)
    assert m.path == "fused"
    want = oracle.forward(layers, xg, oracle.MODE_F64)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12 * max(1.0, np.abs(want).max())), np.abs(got - want).max()


def config_input(cfg, B, dev="cuda:0"):
    import torch

    tdt = torch.float16 if cfg.dtype == "f16" else torch.float32
    x = torch.empty((cfg.n_in, B), dtype=tdt, device=dev)
    kind, a, b = cfg.input_dist
    P.fill_synthetic(x, cfg.seed, C.INPUT_TAG, kind, a, b)
    return x


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
@pytest.mark.parametrize("path", ["auto", "mfma", "generic"])
def test_configs_small_batch(cuda, name, path):
    """Each BASELINE config (with nonzero biases) vs the oracle."""
    import torch

    cfg = C.CONFIGS[name]
    layers = cfg.layers(True)
    B = 20_000 + 13
    x = config_input(cfg, B)
    try:
        m = P.create_inference_model(*layers, dtype=cfg.dtype, path=path)
    except P.PonniError as e:
        pytest.skip(e.message)
    y = m.forward_batch_parallel(x)
    torch.cuda.synchronize()
    xg = x.double().cpu().numpy()
    got = y.double().cpu().numpy()
    if cfg.dtype == "f32":
        check_f32(got, oracle.forward(layers, xg))
    else:
        check_half(got, oracle.forward(layers, xg, oracle.MODE_F16_OPERANDS))


def _full_tensor_distance(got_cols, want_cols, B, chunk, label):
    """relL2 and max-abs of got against want over all B columns, chunk by chunk
    (got_cols / want_cols: (c0, c1) -> float64 arrays of those columns)."""
    sq_err = sq_ref = max_err = 0.0
    for c0 in range(0, B, chunk):
        c1 = min(c0 + chunk, B)
        got, want = got_cols(c0, c1), want_cols(c0, c1)
        sq_err += float(((got - want) ** 2).sum())
        sq_ref += float((want ** 2).sum())
        max_err = max(max_err, float(np.abs(got - want).max()))
        print(f"{label}: columns {c0}..{c1 - 1} of {B} compared", flush=True)
    return math.sqrt(sq_err / max(sq_ref, 1e-300)), max_err


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c5"])
def test_configs_full_size(cuda, name):
    """Full BASELINE batch against the CPU baseline -- the oracle in fp32 --
    over the whole output tensor, in column chunks of 2^20: relative L2 <=
    1e-5 and max-abs <= 1e-4.  Beside it, the fp64 oracle on a strided subset
    of columns gives both sides' distance to exact arithmetic (which side
    drifts)."""
    import torch

    cfg = C.CONFIGS[name]
    layers = cfg.layers(False)
    x = config_input(cfg, cfg.batch)
    m = P.create_inference_model(*layers, dtype=cfg.dtype)
    y = m.forward_batch_parallel(x)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    rel, max_err = _full_tensor_distance(
        lambda c0, c1: y[:, c0:c1].double().cpu().numpy(),
        lambda c0, c1: oracle.forward(layers, x[:, c0:c1].cpu().numpy(), oracle.MODE_F32).astype(np.float64),
        cfg.batch, 1 << 20, name)
    print(f"{name} full tensor vs CPU baseline: relL2={rel:.3e} maxabs={max_err:.3e}", flush=True)
    assert rel <= 1e-5 and max_err <= 1e-4, f"relL2={rel:.3e} maxabs={max_err:.3e}"
    cols = torch.arange(0, cfg.batch, 4099, device=x.device)
    xg = x[:, cols].double().cpu().numpy()
    exact = oracle.forward(layers, xg, oracle.MODE_F64)

    def dist(v):
        return np.linalg.norm(v - exact) / max(np.linalg.norm(exact), 1e-300)

    print(f"{name} strided subset vs fp64: GPU relL2={dist(y[:, cols].double().cpu().numpy()):.3e}, "
          f"CPU baseline relL2={dist(oracle.forward(layers, xg, oracle.MODE_F32)):.3e}", flush=True)


def test_c4_full_size(cuda):
    """c4 at its full batch (8,388,608 columns, fp16 operands, fp32
    accumulation).  The CPU baseline needs minutes for the whole tensor, so:
    the whole output tensor against a float32 torch evaluation of the same
    semantics on the GPU (fp16-rounded weights and inputs, fp32 products and
    sums, bias and tanh in fp32, every state rounded to fp16), relative L2 <=
    2e-3; that evaluation and the kernel against the CPU baseline (the
    oracle's fp16-operand mode) on the first 2^18 columns and a strided
    subset, relative L2 <= 2e-3; and every side's distance to the fp64 oracle
    on the subset."""
    import torch

    cfg = C.CONFIGS["c4"]
    layers = cfg.layers(False)
    x = config_input(cfg, cfg.batch)
    m = P.create_inference_model(*layers, dtype=cfg.dtype)
    y = m.forward_batch_parallel(x)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    dense = []  # (W [out, in] fp16-rounded, bias fp32, tanh after?)
    for i, l in enumerate(layers):
        if l.label == "Matvec":
            w = torch.from_numpy(l.params.reshape(l.n_in, l.n_out).T.copy()).to("cuda:0").half().float()
            dense.append([w, torch.zeros(l.n_out, device="cuda:0"), False])
        elif l.label == "Bias":  # (per-feature vectors stay fp32)
            dense[-1][1] = torch.from_numpy(l.params).to("cuda:0").float()
        elif l.label == "Tanh":
            dense[-1][2] = True
    assert torch.backends.cuda.matmul.allow_tf32 is False

    def torch_ref(xs):
        h = xs.float()
        for w, b, act in dense:
            z = torch.matmul(w, h) + b[:, None]
            h = (torch.tanh(z) if act else z).half().float()
        return h

    rel, _ = _full_tensor_distance(lambda c0, c1: y[:, c0:c1].double().cpu().numpy(),
                                   lambda c0, c1: torch_ref(x[:, c0:c1]).double().cpu().numpy(),
                                   cfg.batch, 1 << 21, "c4")
    print(f"c4 full tensor vs torch fp32 evaluation: relL2={rel:.3e}", flush=True)
    assert rel <= 2e-3, f"relL2={rel:.3e}"
    # The CPU baseline on a contiguous block and a strided subset.
    cols = torch.cat([torch.arange(0, 1 << 18, device=x.device),
                      torch.arange(1 << 18, cfg.batch, 4099, device=x.device)])
    xg = x[:, cols].double().cpu().numpy()
    base = oracle.forward(layers, xg, oracle.MODE_F16_OPERANDS).astype(np.float64)
    exact = oracle.forward(layers, xg, oracle.MODE_F64)
    got = y[:, cols].double().cpu().numpy()
    ref = torch_ref(x[:, cols]).double().cpu().numpy()

    def dist(a, b):
        return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300)

    d_kernel, d_torch = dist(got, base), dist(ref, base)
    print(f"c4 vs CPU baseline on {cols.numel()} columns: kernel relL2={d_kernel:.3e}, torch evaluation "
          f"relL2={d_torch:.3e}; vs fp64: kernel {dist(got, exact):.3e}, torch evaluation {dist(ref, exact):.3e}, "
          f"CPU baseline {dist(base, exact):.3e}", flush=True)
    assert d_kernel <= 2e-3 and d_torch <= 2e-3


@pytest.mark.parametrize("name,B", [("c1", 1_100_000_004), ("c2", 140_000_003), ("c4", 34_000_001)])
def test_more_than_2_31_elements(cuda, name, B):
    """Tensors of more than 2^31 elements (the batch stays below INT_MAX, as
    the reference requires): every kernel offset must be 64-bit.  Columns at
    both ends and spread over the batch are checked against the oracle."""
    import torch

    cfg = C.CONFIGS[name]
    layers = cfg.layers(True)
    assert max(cfg.n_in, cfg.n_out) * B > 2**31
    x = config_input(cfg, B)
    m = P.create_inference_model(*layers, dtype=cfg.dtype)
    y = m.forward_batch_parallel(x)
    torch.cuda.synchronize()
    cols = torch.cat([torch.arange(0, 700), torch.arange(B // 2 - 300, B // 2 + 300), torch.arange(B - 700, B),
                      torch.from_numpy(np.random.default_rng(1).integers(0, B, 500))]).to(x.device)
    xg = x.index_select(1, cols).double().cpu().numpy()
    got = y.index_select(1, cols).double().cpu().numpy()
    del x, y
    torch.cuda.empty_cache()
    if cfg.dtype == "f32":
        check_f32(got, oracle.forward(layers, xg))
    else:
        check_half(got, oracle.forward(layers, xg, oracle.MODE_F16_OPERANDS))


@pytest.mark.parametrize("path", ["narrow", "fused", "generic", "mfma"])
def test_hip_graph_capture_and_replay(cuda, path):
    """After its first call for a batch size, a forward pass is one kernel
    launch with no allocation, copy or memset, so callers can capture it in a
    HIP graph.  Every replay, with new inputs written between replays, must
    equal the eager result on the same inputs."""
    import torch

    rng = np.random.default_rng(21)
    layers = C.c2_layers(True) if path != "narrow" else [P.Matvec(rng.uniform(-1, 1, (16, 12))),
                                                         P.Bias(rng.uniform(-0.1, 0.1, 12)), P.Tanh(12),
                                                         P.Matvec(rng.uniform(-1, 1, (12, 8)))]
    m = make_model(layers, "f32", path)
    B = 5003
    x = torch.empty((16, B), device="cuda:0")
    y = torch.empty((m.get_num_outputs(), B), device="cuda:0")
    x.copy_(torch.from_numpy(rng.standard_normal((16, B))).float())
    m.forward_batch_parallel(x, y)  # warm-up: upload, compile, scratch
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        m.forward_batch_parallel(x, y)
    for r in range(3):
        x.copy_(torch.from_numpy(rng.standard_normal((16, B))).float())
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = y.clone()
        y.zero_()
        m.forward_batch_parallel(x, y)
        torch.cuda.synchronize()
        assert torch.equal(got, y), f"replay {r} differs from the eager pass"
    check_f32(got.double().cpu().numpy(), oracle.forward(layers, x.double().cpu().numpy()))


@pytest.mark.parametrize("path", PATHS)
def test_state_rounded_before_min_max_norm(cuda, path):
    """Each layer's state is rounded before the next layer reads it, so
    MinMaxNorm's x - min is exactly 0 for the minimum.  In this random chain
    (the random sweep's seed 175) one sample's two MinMaxNorm inputs differ by
    17 fp32 ulps, which scales any sub-ulp difference by 1 / (max - min)."""
    rng = np.random.default_rng(10_175)
    width = int(rng.choice([1, 2, 3, 5, 8, 11, 16, 17, 24, 32, 40, 64, 96, 128, 200, 256]))
    layers = K.random_chain(rng, width, int(rng.integers(1, 6)))
    B = int(rng.choice([1, 7, 64, 255, 1000, 4097, 20011]))
    x = rng.standard_normal((width, B))
    assert [l.label for l in layers[3:5]] == ["Mish", "MinMaxNorm"] and B == 20011
    for k in (5, 6, len(layers)):
        got, xg, m = gpu_run(layers[:k], x, "f32", path)
        assert m.path == path.replace("-aot", "")
        check_f32(got, oracle.forward(layers[:k], xg, oracle.MODE_F32))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_half_fused_chain_without_dense_layers(cuda, dtype):
    """16-bit FUSED kernels stream each tile's input rows into LDS ahead of
    use; a chain with no dense layer issues no other memory operation, so
    this pins the explicit wait for those rows (several runs, ragged and
    multi-tile batches)."""
    rng = np.random.default_rng(46)
    layers = [P.Elu(48, 1.0), P.Save_State(0, 48), P.LayerNorm(48), P.Softmax(48), P.Binop_Add(0, 48)]
    for B in (999, 20011, 257):
        x = rng.standard_normal((48, B))
        want = None
        for _ in range(3):
            got, xg, m = gpu_run(layers, x, dtype=dtype, path="fused")
            assert m.path == "fused"
            if want is None:
                want = oracle.forward(layers, xg, ORACLE_MODE[dtype])
            check_half(got, want, 2e-3)


HALF_IO_CHAINS = {
    # one dense layer: next tile's rows requested at the top of the tile;
    # transposed output of 24 features (a partial feature tile)
    "one_dense": lambda r: [P.Matvec(r.uniform(-0.3, 0.3, (40, 24))), P.Bias(r.uniform(-0.1, 0.1, 24)),
                            P.Sigmoid(24)],
    # two dense layers: the request rides on the last (transposed) layer's chunk
    "two_dense": lambda r: [P.Matvec(r.uniform(-0.2, 0.2, (64, 48))), P.Bias(r.uniform(-0.1, 0.1, 48)),
                            P.Tanh(48), P.Matvec(r.uniform(-0.2, 0.2, (48, 10))), P.Bias(r.uniform(-0.1, 0.1, 10))],
    # three dense layers, c4's shape at small widths
    "three_dense": lambda r: [P.Matvec(r.uniform(-0.2, 0.2, (32, 64))), P.Bias(r.uniform(-0.1, 0.1, 64)),
                              P.Tanh(64), P.Matvec(r.uniform(-0.15, 0.15, (64, 64))),
                              P.Bias(r.uniform(-0.1, 0.1, 64)), P.Tanh(64),
                              P.Matvec(r.uniform(-0.15, 0.15, (64, 16))), P.Bias(r.uniform(-0.1, 0.1, 16))],
    # last op not a dense layer: the untransposed store
    "dense_then_norm": lambda r: [P.Matvec(r.uniform(-0.2, 0.2, (24, 40))), P.Bias(r.uniform(-0.1, 0.1, 40)),
                                  P.Tanh(40), P.Matvec(r.uniform(-0.2, 0.2, (40, 40))), P.LayerNorm(40)],
}


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("chain", sorted(HALF_IO_CHAINS))
def test_half_fused_input_output_paths(cuda, chain, dtype):
    """16-bit FUSED input and output paths: whole tiles of an aligned x
    (row stride a multiple of 8) stream through LDS with 16-byte requests,
    the last tile and misaligned strides load directly; a last dense layer
    runs transposed and writes 8-byte runs of output rows when y's stride
    allows, element by element otherwise.  Batches with a partial last tile,
    aligned and misaligned strides; nothing is written past the batch."""
    rng = np.random.default_rng(77)
    layers = HALF_IO_CHAINS[chain](rng)
    n_in = layers[0].n_in
    # 200,003 columns: every workgroup of the persistent grid loops over
    # several tiles, so the next tile's rows are requested during this one.
    for B in (4099, 20013, 200_003):
        x = rng.standard_normal((n_in, B))
        for pad in ((-B) % 8 + 8, (-B) % 8 + 3):
            print(f"half io: chain={chain} dtype={dtype} B={B} ld={B + pad}", flush=True)
            got, xg, m = gpu_run(layers, x, dtype=dtype, path="fused", pad=pad)
            assert m.path == "fused"
            check_half(got, oracle.forward(layers, xg, ORACLE_MODE[dtype]), 2e-3)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_half_fused_vectors_in_global_memory(cuda, dtype):
    """A 16-bit FUSED plan whose per-feature vectors do not fit in LDS next
    to the A-fragment staging and the input rows reads them from global
    memory (tests/test_abi.py deep_half_chain)."""
    from tests.test_abi import deep_half_chain

    layers = deep_half_chain()
    x = np.random.default_rng(62).standard_normal((96, 2049))
    got, xg, m = gpu_run(layers, x, dtype=dtype, path="fused", pad=7)
    assert m.path == "fused"
    check_half(got, oracle.forward(layers, xg, ORACLE_MODE[dtype]), 2e-3)


OFFSET_CHAINS = {
    # every layer at most 16 wide: the NARROW paths take it too
    "narrow12": lambda r: [P.Matvec(r.uniform(-0.5, 0.5, (12, 16))), P.Bias(r.uniform(-0.1, 0.1, 16)),
                           P.Tanh(16), P.Matvec(r.uniform(-0.5, 0.5, (16, 10))), P.Bias(r.uniform(-0.1, 0.1, 10))],
    # several feature tiles, a LayerNorm and a partial last tile
    "wide40": lambda r: [P.Matvec(r.uniform(-0.2, 0.2, (40, 64))), P.Bias(r.uniform(-0.1, 0.1, 64)),
                         P.Tanh(64), P.LayerNorm(64), P.Matvec(r.uniform(-0.2, 0.2, (64, 24))),
                         P.Bias(r.uniform(-0.1, 0.1, 24))],
}


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16", "f64"])
@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("chain", sorted(OFFSET_CHAINS))
def test_column_subviews_at_any_offset(cuda, chain, path, dtype):
    """x and y as column subviews of wider LayoutRight arrays that begin
    inside a row (a Kokkos subview over a column range): base pointers at
    every alignment to 16 bytes, row strides that are and are not multiples
    of the vector width.  Vector loads and stores, and the 16-bit path's LDS
    requests, are taken only where the pointer and stride allow; the result
    matches the oracle, and nothing left or right of y's columns is
    written."""
    import torch

    rng = np.random.default_rng(404)
    layers = OFFSET_CHAINS[chain](rng)
    try:
        m = make_model(layers, dtype, path)
    except P.PonniError as e:
        if e.status == P._abi.PONNI_ERR_UNSUPPORTED:
            pytest.skip(f"{path} does not support this chain in {dtype}: {e.message}")
        raise
    tdt = getattr(torch, TORCH_DT[dtype])
    n_in, n_out, B = layers[0].n_in, m.get_num_outputs(), 4099
    x = rng.standard_normal((n_in, B))
    want = None
    for ox, oy, extra in ((1, 3, 0), (3, 0, 5), (0, 5, 2), (8, 8, 16), (5, 1, 11)):
        ldx, ldy = B + ox + extra, B + oy + 2 * extra + 1
        print(f"offsets: chain={chain} path={path} dtype={dtype} x col {ox} ld {ldx}, y col {oy} ld {ldy}", flush=True)
        xs = torch.zeros((n_in, ldx), dtype=tdt, device="cuda:0")
        xs[:, ox:ox + B] = torch.from_numpy(x).to(tdt)
        ys = torch.full((n_out, ldy), float("nan"), dtype=tdt, device="cuda:0")
        m.forward_batch_parallel(xs[:, ox:ox + B], ys[:, oy:oy + B])
        torch.cuda.synchronize()
        assert torch.isnan(ys[:, :oy].float()).all() and torch.isnan(ys[:, oy + B:].float()).all(), \
            "kernel wrote outside y's columns"
        got = ys[:, oy:oy + B].double().cpu().numpy()
        if want is None:
            want = oracle.forward(layers, xs[:, ox:ox + B].double().cpu().numpy(), ORACLE_MODE[dtype])
        if dtype == "f32":
            check_f32(got, want)
        elif dtype == "f64":
            rel = np.linalg.norm(got - want) / np.linalg.norm(want)
            assert rel <= 1e-10 and np.abs(got - want).max() <= 1e-10, f"relL2={rel:.3e}"
        else:
            check_half(got, want)


NONFINITE_CHAINS = {
    "MinMaxNorm16": (lambda: [P.MinMaxNorm(16, -1.0, 2.0)], True),
    "MinMaxNorm12": (lambda: [P.MinMaxNorm(12)], True),
    "Softmax12": (lambda: [P.Softmax(12)], True),
    "LogSoftmax16": (lambda: [P.LogSoftmax(16)], True),
    "LayerNorm12": (lambda: [P.LayerNorm(12)], True),
    "Tanh12": (lambda: [P.Tanh(12)], False),
    "Sigmoid12": (lambda: [P.Sigmoid(12)], False),
    "Silu12": (lambda: [P.Silu(12)], False),
    "GeluTanh12": (lambda: [P.Gelu(12, True)], False),
    "Relu12": (lambda: [P.Relu(12)], False),
}


def non_finite_input(n, B, rng):
    """Normal samples with NaN, +-inf, +-1e30 and signed zeros planted:
    feature 0 of columns 0-63, a later feature of columns 64-127, two
    features of columns 128-191 and one feature of every tenth column after."""
    special = np.array([np.nan, np.inf, -np.inf, 1e30, -1e30, 0.0, -0.0])
    x = rng.standard_normal((n, B))
    for j in range(64):
        x[0, j] = special[j % 7]
        x[1 + j % (n - 1), 64 + j] = special[(j + 3) % 7]
        x[rng.choice(n, 2, replace=False), 128 + j] = special[rng.integers(7, size=2)]
    for j in range(192, B, 10):
        x[rng.integers(n), j] = special[rng.integers(7)]
    return x


def check_non_finite(got, want, dtype):
    """NaN where the oracle has NaN, the same infinities, and the finite
    outputs within the dtype's bar (fp32 per element: 1e-4 + 1e-5 |ref|)."""
    bad = np.isnan(got) != np.isnan(want)
    assert not bad.any(), f"NaN mismatch at (feature, column) {np.argwhere(bad)[:5].tolist()}"
    inf = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf) and np.array_equal(got[inf], want[inf]), "infinities differ"
    fin = np.isfinite(want)
    g, w = got[fin], want[fin]
    if dtype == "f32":
        err = np.abs(g - w) - (1e-4 + 1e-5 * np.abs(w))
        assert err.max() <= 0, f"finite outputs off by {np.abs(g - w)[err.argmax()]:.3e}"
    elif dtype == "f64":
        assert np.all(np.abs(g - w) <= 1e-10 * np.maximum(1.0, np.abs(w)))
    else:
        check_half(g, w)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16", "f64"])
@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("chain", sorted(NONFINITE_CHAINS))
def test_non_finite_inputs(cuda, chain, path, dtype):
    """NaN, infinities, values that overflow fp16 and signed zeros fed
    straight into each barrier layer and into the activations the generated
    kernels evaluate on the hardware transcendentals: every path gives the
    oracle's NaNs and infinities (the reference's loops: a NaN in feature 0
    of a MinMaxNorm makes the whole column NaN, elsewhere only its own
    output; tanh(+-inf) = +-1) and its finite values."""
    import torch

    make, barrier = NONFINITE_CHAINS[chain]
    if not barrier and dtype in ("bf16", "f64"):
        pytest.skip("pointwise layers: fp32 and fp16 cover the generated forms")
    layers = make()
    rng = np.random.default_rng(int.from_bytes(chain.encode()[:4], "little"))
    x = non_finite_input(layers[0].n_in, 4099, rng)
    print(f"non-finite: chain={chain} path={path} dtype={dtype}", flush=True)
    got, xg, _ = gpu_run(layers, x, dtype=dtype, path=path, pad=5)
    want = oracle.forward(layers, xg, ORACLE_MODE[dtype])
    check_non_finite(got, want, dtype)


PADDED_DENSE_CHAINS = {
    # infinities out of the first dense layer, finite again after the
    # activation; the next dense layer must not see the padding rows
    "narrow": lambda r: [P.Matvec(r.uniform(-1, 1, (5, 7))), P.Bias(r.uniform(-0.1, 0.1, 7)), P.Tanh(7),
                         P.Matvec(r.uniform(-1, 1, (7, 3))), P.Bias(r.uniform(-0.1, 0.1, 3))],
    "tiles": lambda r: [P.Matvec(r.uniform(-1, 1, (20, 23))), P.Bias(r.uniform(-0.1, 0.1, 23)), P.Sigmoid(23),
                        P.Matvec(r.uniform(-1, 1, (23, 9))), P.Bias(r.uniform(-0.1, 0.1, 9)), P.Selu(9),
                        P.Matvec(r.uniform(-1, 1, (9, 18)))],
    # the projection of a saved state holding the infinity
    "projection": lambda r: [P.Save_State(0, 5), P.Matvec(r.uniform(-1, 1, (5, 7))), P.Tanh(7),
                             P.Binop_Projection_Add(0, r.uniform(-1, 1, (5, 7)), r.uniform(-0.1, 0.1, 7)),
                             P.Tanh(7), P.Matvec(r.uniform(-1, 1, (7, 3)))],
}


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16", "f64"])
@pytest.mark.parametrize("path", PATHS)
@pytest.mark.parametrize("chain", sorted(PADDED_DENSE_CHAINS))
def test_infinities_through_padded_dense_layers(cuda, chain, path, dtype):
    """An infinite input makes every output of the next dense layer infinite
    and a Tanh / Sigmoid / Selu after it finite again.  Kernels that pad a
    layer to whole tiles must keep the padding rows at zero: a zero weight
    times an infinity is NaN, and a NaN padding row read by the next
    contraction would turn the finite outputs into NaN."""
    rng = np.random.default_rng(606)
    layers = PADDED_DENSE_CHAINS[chain](rng)
    n_in, B = layers[0].n_in, 4099
    x = rng.standard_normal((n_in, B))
    x[rng.integers(n_in, size=300), np.arange(0, 600, 2)] = np.where(np.arange(300) % 2, np.inf, -np.inf)
    print(f"padded dense: chain={chain} path={path} dtype={dtype}", flush=True)
    got, xg, _ = gpu_run(layers, x, dtype=dtype, path=path, pad=3)
    want = oracle.forward(layers, xg, ORACLE_MODE[dtype])
    assert np.isfinite(want[:, 0:600:2]).mean() > 0.5  # the case this test is about
    check_non_finite(got, want, dtype)


def test_strided_views_and_stream(cuda):
    """ld > batch (a column subview of a wider LayoutRight array) on a side stream."""
    import torch

    rng = np.random.default_rng(5)
    layers = C.c2_layers(True)
    x = rng.standard_normal((16, 777))
    got, xg, _ = gpu_run(layers, x, pad=50)
    check_f32(got, oracle.forward(layers, xg))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        got2, _, _ = gpu_run(layers, x, pad=0)
    s.synchronize()
    assert np.array_equal(got, got2)


def test_parameter_update_is_seen(cuda):
    rng = np.random.default_rng(9)
    layers = C.c2_layers(True)
    x = rng.standard_normal((16, 300))
    got, xg, m = gpu_run(layers, x)
    import torch

    w = rng.standard_normal((16, 64)) * 0.1
    m.set_layer_params(0, w)
    layers[0].params = w.reshape(-1)
    xt = torch.from_numpy(xg).float().cuda()
    y = m.forward_batch_parallel(xt)
    torch.cuda.synchronize()
    check_f32(y.double().cpu().numpy(), oracle.forward(layers, xg))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("seed", range(4))
def test_random_chains_reduced_precision_fused(cuda, dtype, seed):
    rng = np.random.default_rng(900 + seed)
    width = [24, 40, 64, 96][seed]
    layers = K.random_chain(rng, width, 2 + seed % 3)
    x = rng.standard_normal((width, 777))
    for pad in (2, 7):  # row strides 779 (direct input loads) and 784 (input through LDS)
        got, xg, _ = gpu_run(layers, x, dtype=dtype, path="fused", pad=pad)
        check_half(got, oracle.forward(layers, xg, ORACLE_MODE[dtype]), 2e-3)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("B", [4096, 4099, 37])
def test_narrow_vector_rows(cuda, dtype, B):
    """Generated NARROW kernel: rows move as aligned vectors (ld a multiple of
    8), with a partial last vector when B is not; every width class."""
    rng = np.random.default_rng(B)
    for w in (3, 6, 12):
        layers = [P.Matvec(rng.uniform(-0.5, 0.5, (5, w))), P.Bias(rng.uniform(-0.1, 0.1, w)), P.Tanh(w),
                  P.Save_State(0, w), P.Relu(w), P.Binop_Add(0, w), P.Matvec(rng.uniform(-0.5, 0.5, (w, 2))),
                  P.Bias(rng.uniform(-0.1, 0.1, 2))]
        x = rng.normal(size=(5, B))
        got, xg, m = gpu_run(layers, x, dtype=dtype, path="narrow", pad=(-B) % 8 + 8)
        assert m.path == "narrow"
        if dtype == "f32":
            check_f32(got, oracle.forward(layers, xg))
        else:
            check_half(got, oracle.forward(layers, xg, oracle.MODE_F16_OPERANDS))


@pytest.mark.parametrize("dtype", ["f32", "f16", "f64"])
@pytest.mark.parametrize("after", [True, False])
def test_concatenation_any_lead_width_fused(cuda, after, dtype):
    """Binop_Concatenate whose leading block is not a whole number of 16-row
    tiles (the FUSED tile library moves the other block by lane-group
    shuffles): lead widths 1..40, mid-chain, so the result feeds a dense layer,
    on FUSED against the oracle."""
    rng = np.random.default_rng(5)
    for lead in (1, 3, 4, 5, 8, 12, 13, 16, 17, 20, 28, 40):
        other = int(rng.choice([3, 7, 16, 24]))
        n_state, n_saved = (lead, other) if after else (other, lead)
        layers = [P.Save_State(0, 6), P.Matvec(rng.uniform(-0.5, 0.5, (6, n_saved))), P.Tanh(n_saved),
                  P.Save_State(1, n_saved), P.Matvec(rng.uniform(-0.5, 0.5, (n_saved, n_state))), P.Relu(n_state),
                  P.Binop_Concatenate(1, n_state, n_state + n_saved, after),
                  P.Matvec(rng.uniform(-0.5, 0.5, (n_state + n_saved, 5))), P.Sigmoid(5)]
        # (slot 0 is never read: it checks that an unused save changes nothing)
        x = rng.standard_normal((6, 1000))
        print(f"concat lead={lead} other={other} after={after} dtype={dtype}", flush=True)
        got, xg, m = gpu_run(layers, x, dtype, "fused")
        assert m.path == "fused"
        if dtype == "f64":
            want = oracle.forward(layers, xg, oracle.MODE_F64)
            assert np.allclose(got, want, rtol=1e-12, atol=1e-12), np.abs(got - want).max()
        elif dtype == "f16":
            check_half(got, oracle.forward(layers, xg, oracle.MODE_F16_OPERANDS))
        else:
            check_f32(got, oracle.forward(layers, xg))
