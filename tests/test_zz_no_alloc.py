"""ponni_forward_no_alloc: the allocation-free forward pass against
ponni_forward through the C ABI -- bit-identical outputs (same kernels, same
arithmetic) on two calls in a row, the second with a smaller batch, on the
GENERIC path (state buffers carved from the fixed per-GPU scratch) and on
FUSED and NARROW (no scratch); its refusals (plan not on the device yet, a
host-shared array changed, batch beyond the fixed scratch); no change of the
device's free memory across the calls; a captured graph of it, replayed."""
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
                                         ("narrow", C.c1_layers()), ("layered", residual_chain(80))])
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
    # tmp1, tmp2 and two saved slots of up to 256 features: far beyond 64 MiB
    # at this batch.  x and y are of the full size all the same (13 MB), so
    # that no regression of the size check can reach past them.
    B = 200_000
    x = torch.zeros((12, B), device=cuda)
    y = torch.zeros((5, B), device=cuda)
    A.check(call(L.ponni_forward, m, x, y, 64, 0))  # puts the plan on the device
    torch.cuda.synchronize()
    st = call(L.ponni_forward_no_alloc, m, x, y, B, 0)
    assert st == A.PONNI_ERR_SHAPE
    assert "fixed scratch" in L.ponni_last_error().decode()


@pytest.mark.gpu
def test_no_alloc_allocates_nothing(cuda):
    """The device's free memory is the same before and after the first
    allocation-free call on a GENERIC plan (whose fixed scratch is looked up
    when the plan is put on the device) and after a second one."""
    import torch

    L = A.lib()
    m = P.create_inference_model(*residual_chain(), path="generic")
    B = 20_011
    x = torch.empty((12, B), device=cuda)
    P.fill_synthetic(x, 5, C.INPUT_TAG, "normal", 0.0, 1.0)
    want = torch.empty((5, B), device=cuda)
    got = torch.empty((5, B), device=cuda)
    A.check(call(L.ponni_forward, m, x, want, B, 0))
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for i in range(2):
        print(f"no-alloc forward {i}: free memory before {free0}", flush=True)
        A.check(call(L.ponni_forward_no_alloc, m, x, got, B, 0))
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        assert free1 == free0
    assert torch.equal(got, want)


@pytest.mark.gpu
def test_no_alloc_captured_in_a_graph(cuda):
    """A GENERIC allocation-free forward captured in a HIP graph (through
    torch.cuda.graph) and replayed several times, with new inputs written and
    the program's own eager work and synchronizations between the replays:
    every replay equals ponni_forward on the same input."""
    import torch

    L = A.lib()
    m = P.create_inference_model(*residual_chain(), path="generic")
    B = 8_191
    x = torch.empty((12, B), device=cuda)
    y = torch.full((5, B), float("nan"), device=cuda)
    want = torch.empty((5, B), device=cuda)
    P.fill_synthetic(x, 1, C.INPUT_TAG, "normal", 0.0, 1.0)
    A.check(call(L.ponni_forward, m, x, want, B, 0))  # puts the plan on the device
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = call(L.ponni_forward_no_alloc, m, x, y, B, torch.cuda.current_stream().cuda_stream)
    A.check(st)
    torch.cuda.synchronize()
    for seed in (2, 3, 4):
        print(f"graph replay: seed {seed}", flush=True)
        P.fill_synthetic(x, seed, C.INPUT_TAG, "normal", 0.0, 1.0)
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        A.check(call(L.ponni_forward, m, x, want, B, 0))
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(y, want)


def test_no_alloc_refuses_a_plan_not_on_the_device():
    """A fresh plan has never been uploaded; the call fails before touching
    any device (so this runs without a GPU)."""
    L = A.lib()
    m = P.create_inference_model(*C.c1_layers())
    st = L.ponni_forward_no_alloc(m._plan, 16, 8, 32, 8, 8, None)
    assert st == A.PONNI_ERR_INVALID_ARGUMENT
    assert "not on the device" in L.ponni_last_error().decode()


@pytest.mark.gpu
def test_no_alloc_names_a_changed_host_shared_array(cuda):
    """A host array shared with the plan changed after the last upload: the
    allocation-free call refuses with a message naming that cause, and one
    ponni_forward brings the plan back."""
    import torch

    L = A.lib()
    layers = C.c1_layers()
    m = P.create_inference_model(*layers, path="generic")
    w = np.ascontiguousarray(np.asarray(layers[0].params, dtype=np.float32).reshape(2, 3))
    m.share_layer_params(0, 0, w)
    B = 1_000
    x = torch.empty((2, B), device=cuda)
    P.fill_synthetic(x, 3, C.INPUT_TAG, "uniform", -1.0, 1.0)
    y = torch.empty((1, B), device=cuda)
    A.check(call(L.ponni_forward, m, x, y, B, 0))
    A.check(call(L.ponni_forward_no_alloc, m, x, y, B, 0))
    torch.cuda.synchronize()
    w *= 0.5
    st = call(L.ponni_forward_no_alloc, m, x, y, B, 0)
    assert st == A.PONNI_ERR_INVALID_ARGUMENT
    assert "host array shared" in L.ponni_last_error().decode()
    A.check(call(L.ponni_forward, m, x, y, B, 0))
    got = torch.empty_like(y)
    A.check(call(L.ponni_forward_no_alloc, m, x, got, B, 0))
    torch.cuda.synchronize()
    assert torch.equal(got, y)
