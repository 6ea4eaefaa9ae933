"""ponni_forward_no_alloc: the allocation-free forward pass against
ponni_forward through the C ABI -- bit-identical outputs (same kernels, same
arithmetic) on two calls in a row, the second with a smaller batch, on the
GENERIC path (state buffers carved from the fixed per-GPU scratch) and on
FUSED and NARROW (no scratch); its two refusals (plan not on the device yet,
batch beyond the fixed scratch)."""
import numpy as np
import pytest

import ponni_amd as P
from ponni_amd import _abi as A
from ponni_amd import configs as C


def residual_chain(width=24):
    """Saved slots, tmp1 and tmp2 all in use on the GENERIC path."""
    rng = np.random.default_rng(77)
    return [P.Matvec(rng.standard_normal((12, width)) * 0.3), P.Bias(rng.uniform(-0.1, 0.1, width)), P.Tanh(width),
            P.Save_State(0, width), P.LayerNorm(width), P.Matvec(rng.standard_normal((width, width)) * 0.2),
            P.Gelu(width, True), P.Binop_Add(0, width), P.Save_State(1, width), P.Softmax(width),
            P.Binop_Concatenate(1, width, 2 * width, True), P.Matvec(rng.standard_normal((2 * width, 5)) * 0.3)]


def call(fn, m, x, y, B, stream):
    return fn(m._plan, x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0), B, stream)


@pytest.mark.gpu
@pytest.mark.parametrize("path,layers", [("generic", residual_chain()), ("fused", residual_chain(32)),
                                         ("narrow", C.c1_layers())])
def test_no_alloc_matches_forward(cuda, path, layers):
    import torch

    L = A.lib()
    m = P.create_inference_model(*layers, path=path)
    assert m.path == path
    n_in, n_out = m.get_num_inputs(), m.get_num_outputs()
    stream = torch.cuda.current_stream().cuda_stream
    for B in (20_011, 3_001):  # the second call is smaller
        print(f"no-alloc forward: path={path} B={B}", flush=True)
        x = torch.empty((n_in, B), dtype=torch.float32, device=cuda)
        P.fill_synthetic(x, B, C.INPUT_TAG, "normal", 0.0, 1.0)
        want = torch.full((n_out, B), float("nan"), device=cuda)
        got = torch.full((n_out, B), float("nan"), device=cuda)
        A.check(call(L.ponni_forward, m, x, want, B, stream))
        A.check(call(L.ponni_forward_no_alloc, m, x, got, B, stream))
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got, want)


@pytest.mark.gpu
def test_no_alloc_rejects_a_batch_beyond_the_fixed_scratch(cuda):
    import torch

    L = A.lib()
    m = P.create_inference_model(*residual_chain(128), path="generic")
    x = torch.zeros((12, 64), device=cuda)
    y = torch.zeros((5, 64), device=cuda)
    A.check(call(L.ponni_forward, m, x, y, 64, 0))  # puts the plan on the device
    torch.cuda.synchronize()
    # tmp1, tmp2 and two saved slots of up to 256 features: far beyond 64 MiB
    # at this batch.  The refusal comes before any launch, so x and y need
    # not be that large.
    B = 200_000
    st = L.ponni_forward_no_alloc(m._plan, x.data_ptr(), B, y.data_ptr(), B, B, 0)
    assert st == A.PONNI_ERR_SHAPE
    assert "fixed scratch" in L.ponni_last_error().decode()


def test_no_alloc_refuses_a_plan_not_on_the_device():
    """A fresh plan has never been uploaded; the call fails before touching
    any device (so this runs without a GPU)."""
    L = A.lib()
    m = P.create_inference_model(*C.c1_layers())
    st = L.ponni_forward_no_alloc(m._plan, 16, 8, 32, 8, 8, None)
    assert st == A.PONNI_ERR_INVALID_ARGUMENT
    assert "not on the device" in L.ponni_last_error().decode()
