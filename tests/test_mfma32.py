"""16-bit FUSED plans on 32x32x16 MFMA tiles, and A-fragment chunks staged by
LDS DMA (both opt-in; the defaults, 16x16x32 tiles with chunks staged through
registers, measured faster on c4).

With PONNI_MFMA32=1, a FUSED fp16 / bf16 plan made only of dense layers and
pointwise steps, with every width a multiple of 32, runs on
v_mfma_f32_32x32x16 (fused_f16.h H32, dense_hs32), its weights packed for that
fragment layout; every other 16-bit plan, and every plan by default, keeps the
16x16x32 tiles.  CPU tests pin which plans take which layout and that the
kernels compile; GPU tests check parity with the oracle's fp16-operand /
fp32-accumulate mode (relative L2 <= 2e-3 for fp16 and bf16) and with
the same plan on the default 16x16 tiles.
"""
import math

import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import graph as G
from tests.test_graph import lowered_with_params

TOL = {"f16": 2e-3, "bf16": 2e-3}
MODE = {"f16": oracle.MODE_F16_OPERANDS, "bf16": oracle.MODE_BF16_OPERANDS}


def mlp(rng, widths, acts, bias=True):
    """Matvec (+ Bias) per step, acts[i % len(acts)] after every hidden layer."""
    layers = []
    for i in range(len(widths) - 1):
        a, b = widths[i], widths[i + 1]
        lim = math.sqrt(6.0 / (a + b))
        layers.append(P.Matvec(rng.uniform(-lim, lim, (a, b))))
        if bias:
            layers.append(P.Bias(rng.uniform(-0.2, 0.2, b)))
        if i < len(widths) - 2:
            layers.append(acts[i % len(acts)](b))
    return layers


CHAINS = {
    "c4_shape": ([64, 256, 256, 256, 64], [P.Tanh]),
    "mixed": ([128, 64, 160, 32], [P.Relu, lambda n: P.Gelu(n, approximate=True)]),
    "narrow_k": ([32, 96, 32], [P.Sigmoid]),
    "wide_out": ([32, 256], [P.Relu]),
}


def leading_pointwise(rng):
    return [P.Bias(rng.uniform(-0.5, 0.5, 64)), P.Tanh(64)] + mlp(rng, [64, 32, 64], [P.Silu])


def const_graph(rng):
    """Dense -> Mul by a constant vector -> Relu -> Dense -> Add a constant."""
    g = G.GraphBuilder(64)
    d = g.dense(g.input, rng.uniform(-0.3, 0.3, (96, 64)), rng.uniform(-0.2, 0.2, 96), name="d0")
    m = g.binary("Mul", d, g.constant("scale", rng.uniform(0.5, 1.5, 96)))
    r = g.unary("Relu", m)
    d1 = g.dense(r, rng.uniform(-0.3, 0.3, (32, 96)), None, name="d1")
    return g.finish(g.binary("Add", d1, g.constant("shift", rng.uniform(-0.5, 0.5, 32))))


def _create(layers, dtype, monkeypatch, m32=True):
    """FUSED plan with 32x32 tiles requested (PONNI_MFMA32=1) or left at the
    default 16x16 tiles."""
    if m32:
        monkeypatch.setenv("PONNI_MFMA32", "1")
    else:
        monkeypatch.delenv("PONNI_MFMA32", raising=False)
    return P.create_inference_model(*layers, dtype=dtype, path="fused")


# ---- CPU: which plans take the 32x32 layout, and their kernels compile ----------

@pytest.mark.parametrize("name", sorted(CHAINS))
def test_aligned_chains_take_32x32_tiles(name, monkeypatch):
    widths, acts = CHAINS[name]
    m = _create(mlp(np.random.default_rng(1), widths, acts), "f16", monkeypatch)
    src = m.kernel_source()
    assert src.count("dense_hs32<") == len(widths) - 1 and "dense_hs<" not in src
    assert "store_rows_h32<" in src
    m16 = _create(mlp(np.random.default_rng(1), widths, acts), "f16", monkeypatch, m32=False)
    assert "dense_hs32<" not in m16.kernel_source()


def test_other_chains_keep_16x16_tiles(monkeypatch):
    rng = np.random.default_rng(2)
    unaligned = mlp(rng, [64, 48, 32], [P.Relu])  # a width of 48
    barrier = mlp(rng, [64, 64], [P.Relu]) + [P.LayerNorm(64)] + mlp(rng, [64, 32], [P.Relu])
    residual = [P.Save_State(0, 64)] + mlp(rng, [64, 64], [P.Relu]) + [P.Binop_Add(0, 64)]
    for layers in (unaligned, barrier, residual):
        for dt in ("f16", "bf16"):
            src = _create(layers, dt, monkeypatch).kernel_source()
            assert "dense_hs32<" not in src and "dense_hs<" in src
    # without the request, aligned chains keep 16x16 tiles too
    monkeypatch.delenv("PONNI_MFMA32")
    widths, acts = CHAINS["c4_shape"]
    assert "dense_hs32<" not in P.create_inference_model(*mlp(rng, widths, acts), dtype="f16",
                                                          path="fused").kernel_source()
    # fp32 plans never use the 16-bit tiles
    f32 = P.create_inference_model(*mlp(rng, [64, 64, 32], [P.Relu]), dtype="f32", path="fused")
    assert "dense_hs" not in f32.kernel_source()


def test_leading_pointwise_and_const_steps_take_32x32_tiles(monkeypatch):
    rng = np.random.default_rng(3)
    src = _create(leading_pointwise(rng), "bf16", monkeypatch).kernel_source()
    assert "for_tiles32(" in src and "t32_add_rows(" in src and src.count("dense_hs32<") == 2
    plan = G.GeneratedModel(const_graph(rng)).plan("f16")  # PONNI_MFMA32=1 still set
    assert plan.path == "fused"
    gsrc = plan.kernel_source()
    assert gsrc.count("dense_hs32<") == 2 and "t32_const(" in gsrc


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_32x32_kernels_compile_on_the_host(dtype, tmp_path, monkeypatch):
    monkeypatch.setenv("PONNI_JIT_CACHE", str(tmp_path))
    widths, acts = CHAINS["c4_shape"]
    m = _create(mlp(np.random.default_rng(4), widths, acts), dtype, monkeypatch)
    m.compile()
    assert any(f.suffix == ".co" for f in tmp_path.iterdir())


# ---- GPU parity ----------------------------------------------------------------

def _run(m, x, dtype):
    import torch

    tdt = {"f16": torch.float16, "bf16": torch.bfloat16}[dtype]
    xt = torch.from_numpy(x).to(tdt).cuda()
    B = x.shape[1]
    ys = torch.full((m.get_num_outputs(), B + 5), float("nan"), dtype=tdt, device="cuda")
    m.forward_batch_parallel(xt, ys[:, :B])
    torch.cuda.synchronize()
    assert torch.isnan(ys[:, B:].float()).all(), "kernel wrote past the batch"
    return ys[:, :B].double().cpu().numpy(), xt.double().cpu().numpy()


def _check(got, want, tol):
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert np.isfinite(got).all() and rel <= tol, f"relL2={rel:.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("name", sorted(CHAINS))
def test_32x32_chains_match_oracle(name, dtype, monkeypatch):
    oracle.build()
    widths, acts = CHAINS[name]
    rng = np.random.default_rng(10)
    layers = mlp(rng, widths, acts)
    m = _create(layers, dtype, monkeypatch)
    m16 = _create(layers, dtype, monkeypatch, m32=False)
    assert "dense_hs32<" in m.kernel_source() and "dense_hs32<" not in m16.kernel_source()
    for B in (1, 31, 33, 257, 4099, 70001):
        x = rng.standard_normal((widths[0], B))
        got, xg = _run(m, x, dtype)
        want = oracle.forward(layers, xg, MODE[dtype])
        _check(got, want, TOL[dtype])
        got16, _ = _run(m16, x, dtype)
        _check(got, got16, 2 * TOL[dtype])


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_32x32_leading_pointwise_and_const_graph(dtype, monkeypatch):
    oracle.build()
    rng = np.random.default_rng(11)
    layers = leading_pointwise(rng)
    m = _create(layers, dtype, monkeypatch)
    assert "for_tiles32(" in m.kernel_source()
    x = rng.standard_normal((64, 5003))
    got, xg = _run(m, x, dtype)
    _check(got, oracle.forward(layers, xg, MODE[dtype]), TOL[dtype])

    gr = const_graph(rng)
    plan = G.GeneratedModel(gr).plan(dtype)
    assert "t32_const(" in plan.kernel_source()
    x = rng.standard_normal((64, 3001))
    got, xg = _run(plan, x, dtype)
    _check(got, oracle.forward(lowered_with_params(gr), xg, MODE[dtype]), TOL[dtype])


@pytest.mark.gpu
def test_32x32_c4_full_size_matches_16x16(monkeypatch):
    """c4 at its full batch: the 32x32 plan against the 16x16 plan of the same
    weights (both fp32-accumulated; the oracle checks them at smaller sizes)."""
    import torch
    from ponni_amd import configs as C

    cfg = C.CONFIGS["c4"]
    layers = cfg.layers(False)
    m = _create(layers, "f16", monkeypatch)
    m16 = _create(layers, "f16", monkeypatch, m32=False)
    assert "dense_hs32<" in m.kernel_source() and "dense_hs32<" not in m16.kernel_source()
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn((64, cfg.batch), generator=g, device="cuda", dtype=torch.float32).half()
    y = m.forward_batch_parallel(x)
    y16 = m16.forward_batch_parallel(x)
    torch.cuda.synchronize()
    d = (y.float() - y16.float())
    rel = (d.norm() / y16.float().norm()).item()
    assert torch.isfinite(y.float()).all().item() and rel <= 2e-3, rel


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_dma_chunk_staging_matches_oracle(dtype, monkeypatch):
    """PONNI_CHUNK_DMA=1: the 16x16 kernel stages its A-fragment chunks with
    16-byte LDS-DMA loads (fused_f16.h chunk_dma)."""
    oracle.build()
    monkeypatch.setenv("PONNI_CHUNK_DMA", "1")
    rng = np.random.default_rng(12)
    widths, acts = CHAINS["c4_shape"]
    for layers in (mlp(rng, widths, acts), mlp(rng, [48, 80, 16], [P.Relu])):
        m = _create(layers, dtype, monkeypatch, m32=False)
        src = m.kernel_source()
        assert "#define PONNI_CHUNK_DMA 1" in src and "dense_hs<" in src
        for B in (33, 20011):
            x = rng.standard_normal((layers[0].n_in, B))
            got, xg = _run(m, x, dtype)
            _check(got, oracle.forward(layers, xg, MODE[dtype]), TOL[dtype])
