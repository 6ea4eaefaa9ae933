"""Chains wider than 256 features.

The reference runs any width through the same forward_batch_parallel: the
widths come from the layers' View extents (src/layers/ponni_Matvec.h:62-65)
and one launch covers the chain (src/ponni_Inference.h:384-388).  Here FUSED
keeps the states of 16-bit chains up to 1024 features and of fp32 chains up
to 512 in registers (one 16-column tile per wave beyond 256 features; the
contraction runs over 32-feature steps of any count); wider fp32 and fp64
chains take LAYERED (the GENERIC op list with every dense block run over
the whole batch as an MFMA contraction, states in HBM).

CPU: the path each width takes, that every FUSED kernel compiles (hipRTC,
no device), and the occupancy 16-bit plans settle on (two waves per SIMD
with fragments read two steps ahead, spilled registers or not).  GPU: chains of 320, 512 and 1024 features with a
residual and a LayerNorm at full width, on the default path, on GENERIC
and on LAYERED, against the oracle at the fixed bars."""
import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import _abi as A


def wide_chain(width, n_in=40, n_out=24, seed=0):
    rng = np.random.default_rng(seed + width)

    def W(a, b):
        return rng.uniform(-1, 1, (a, b)) * np.sqrt(3.0 / a)

    return [P.Matvec(W(n_in, width)), P.Bias(rng.uniform(-0.1, 0.1, width)), P.Tanh(width),
            P.Save_State(0, width), P.Matvec(W(width, width)), P.Bias(rng.uniform(-0.1, 0.1, width)),
            P.Gelu(width, True), P.LayerNorm(rng.uniform(0.5, 1.5, width), rng.uniform(-0.2, 0.2, width)),
            P.Binop_Add(0, width), P.Matvec(W(width, width)), P.Bias(rng.uniform(-0.1, 0.1, width)), P.Relu(width),
            P.Matvec(W(width, n_out)), P.Bias(rng.uniform(-0.1, 0.1, n_out))]


EXPECTED = {("f32", 320): "fused", ("f32", 512): "fused", ("f32", 1024): "layered",
            ("f16", 320): "fused", ("f16", 512): "fused", ("f16", 1024): "fused",
            ("bf16", 512): "fused", ("f64", 320): "layered"}


@pytest.mark.parametrize("dtype,width", sorted(EXPECTED))
def test_wide_path_choice_and_compile(dtype, width, tmp_path, monkeypatch):
    monkeypatch.setenv("PONNI_JIT_CACHE", str(tmp_path))
    m = P.create_inference_model(*wide_chain(width), dtype=dtype)
    assert m.path == EXPECTED[(dtype, width)]
    if m.path == "fused":
        m.compile()
        src = m.kernel_source()
        assert "#define PONNI_NT 1" in src
        threads, _, _ = m.kernel_config()
        if dtype in ("f16", "bf16"):
            # one column tile per wave: two waves per SIMD (eight-wave
            # workgroups) whatever the compile spills, fragments read two
            # steps ahead
            assert threads == 512 and "#define PONNI_PIPE 2" in src
    else:
        with pytest.raises(P.PonniError) as e:
            P.create_inference_model(*wide_chain(width), dtype=dtype, path="fused")
        assert e.value.status == A.PONNI_ERR_UNSUPPORTED


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_wide_mlp_runs_two_waves_per_simd(dtype, tmp_path, monkeypatch):
    """A 16-bit 64 -> 512 -> 512 -> 64 tanh MLP (the supplementary bench
    chain) runs two waves per SIMD (its compile spills 19-20 registers)."""
    monkeypatch.setenv("PONNI_JIT_CACHE", str(tmp_path))
    m = P.create_inference_model(*P.configs.SUPPLEMENTARY["wide512"].layers(False), dtype=dtype)
    m.compile()
    assert m.kernel_config()[0] == 512 and "#define PONNI_PIPE 2" in m.kernel_source()


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["auto", "generic", "layered"])
@pytest.mark.parametrize("dtype,width", sorted(EXPECTED))
def test_wide_chain_on_gpu(cuda, dtype, width, path):
    from tests.test_gpu_parity import ORACLE_MODE, check_f32, check_half, gpu_run

    layers = wide_chain(width)
    x = np.random.default_rng(width).standard_normal((40, 3001))
    print(f"wide chain: width={width} dtype={dtype} path={path} B=3001", flush=True)
    got, xg, m = gpu_run(layers, x, dtype=dtype, path=path, pad=5)
    assert m.path == (EXPECTED[(dtype, width)] if path == "auto" else path)
    want = oracle.forward(layers, xg, ORACLE_MODE[dtype])
    if dtype == "f64":
        assert np.allclose(got, want, rtol=1e-12, atol=1e-12 * np.abs(want).max())
    elif dtype == "f32":
        check_f32(got, want)
    else:
        check_half(got, want)
