"""Layer parameters shared with caller-owned arrays (ponni_plan_share_layer_params):
the rebind rule of src/ponni_create_model.h:10-18, where a layer whose Views
live in the model's memory space is shared with the model, not copied, so a
write through the caller's View reaches the next forward pass
(unit/core/test_core_unit.cpp:516-546: Matvec W [2, 3] = 10..15 and x = (1, 2)
give 36, 39, 42).

Host arrays are exercised with host execution-space plans (ponni_forward_host,
no GPU); device arrays with torch tensors on every GPU kernel family, the
tensor rewritten in place between forward passes on the same stream.
"""
import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import configs as C

W_KNOWN = np.arange(10.0, 16.0).reshape(2, 3)  # test_core_unit.cpp:516-546 layout case
X_KNOWN = np.array([[1.0], [2.0]])


def test_host_array_is_shared_with_a_host_plan():
    w = np.arange(1.0, 7.0, dtype=np.float32).reshape(2, 3)
    m = P.Inference([P.Matvec(np.zeros((2, 3)))])
    m.share_layer_params(0, 0, w)
    assert np.array_equal(m.get_layer_params(0), w.reshape(-1))
    assert np.allclose(m.forward_host(X_KNOWN)[:, 0], [9.0, 12.0, 15.0])
    w[:] = W_KNOWN  # a write through the caller's array
    assert np.allclose(m.forward_host(X_KNOWN)[:, 0], [36.0, 39.0, 42.0])
    assert np.array_equal(m.get_layer_params(0), W_KNOWN.reshape(-1))
    m.set_layer_params(0, np.full(6, 0.5))  # writes into the shared array
    assert np.all(w == 0.5)
    m.share_layer_params(0, 0, None)  # the plan keeps the last contents
    w[:] = 7.0
    assert np.allclose(m.forward_host(X_KNOWN)[:, 0], [1.5, 1.5, 1.5])


def test_strided_and_converted_host_arrays():
    big = np.zeros((2, 8), dtype=np.float64)
    big[:, 2:5] = W_KNOWN
    m = P.Inference([P.Matvec(np.zeros((2, 3))), P.Bias(np.zeros(3))], dtype="f64")
    m.share_layer_params(0, 0, big[:, 2:5])  # row stride 8, three columns
    b16 = np.array([0.5, -1.0, 2.0], dtype=np.float16)
    m.share_layer_params(1, 0, b16)
    assert np.allclose(m.forward_host(X_KNOWN)[:, 0], [36.5, 38.0, 44.0])


def test_two_segment_layers():
    gamma = np.array([2.0, 1.0, 0.5, -1.0], dtype=np.float32)
    beta = np.array([0.5, 0.0, -0.5, 1.0], dtype=np.float32)
    m = P.Inference([P.LayerNorm(4)])
    m.share_layer_params(0, 0, gamma)
    m.share_layer_params(0, 1, beta)
    x = np.array([[1.0], [2.0], [3.0], [4.0]])
    xhat = (x[:, 0] - 2.5) / np.sqrt(1.25 + 1e-5)
    assert np.allclose(m.forward_host(x)[:, 0], gamma * xhat + beta, atol=1e-6)
    beta[:] = 0.0
    assert np.allclose(m.forward_host(x)[:, 0], gamma * xhat, atol=1e-6)
    # Projection_Add: W [NSAVE, n_in] then bias (test_core_unit.cpp:814-872)
    w = np.array([[1.0, 0.0, 0.5], [0.0, 1.0, 0.5]], dtype=np.float32)
    b = np.array([0.1, 0.2, 0.3], dtype=np.float32)
    layers = [P.Save_State(0, 2), P.Matvec(np.array([[0.25, 0.0, 0.0], [0.0, 0.4, 0.6]])),
              P.Binop_Projection_Add(0, np.zeros((2, 3)), np.zeros(3))]
    m = P.Inference(layers)
    m.share_layer_params(2, 0, w)
    m.share_layer_params(2, 1, b)
    assert np.allclose(m.forward_host(np.array([[4.0], [5.0]]))[:, 0], [5.1, 7.2, 7.8], atol=1e-5)


def test_share_rejections():
    m = P.Inference([P.Matvec(np.zeros((2, 3))), P.Relu(3)])
    with pytest.raises(P.PonniError) as e:
        m.share_layer_params(0, 0, np.zeros((3, 3), dtype=np.float32))
    assert e.value.status == P._abi.PONNI_ERR_SHAPE
    with pytest.raises(P.PonniError) as e:
        m.share_layer_params(0, 1, np.zeros(3, dtype=np.float32))  # Matvec has one segment
    assert e.value.status == P._abi.PONNI_ERR_INVALID_ARGUMENT
    with pytest.raises(P.PonniError) as e:
        m.share_layer_params(1, 0, np.zeros(3, dtype=np.float32))  # Relu has none
    assert e.value.status == P._abi.PONNI_ERR_INVALID_ARGUMENT


CASES = [("generic", "f32", "c2"), ("narrow", "f32", "c1"), ("mfma", "f32", "c2"), ("fused", "f32", "c2"),
         ("fused", "f16", "c2"), ("fused", "bf16", "c2"), ("fused", "f64", "c2"), ("generic", "f16", "c2")]
TORCH_DT = {"f32": "float32", "f16": "float16", "bf16": "bfloat16", "f64": "float64"}
MODE = {"f32": oracle.MODE_F32, "f64": oracle.MODE_F64, "f16": oracle.MODE_F16_OPERANDS,
        "bf16": oracle.MODE_BF16_OPERANDS}


@pytest.mark.gpu
@pytest.mark.parametrize("path,dtype,cfg", CASES)
def test_device_arrays_are_read_at_every_forward(cuda, path, dtype, cfg):
    """Every parameter segment of the chain lives in a device tensor (fp32
    storage); the tensors are rewritten in place between forward passes with
    no host synchronization, and each pass must see the values written
    before it on the stream."""
    import torch

    oracle.build()
    c = C.CONFIGS[cfg]
    layers = c.layers(True)
    m = P.create_inference_model(*layers, dtype=dtype, path=path)
    assert m.path == path
    arrays = []
    for i, l in enumerate(layers):
        if l.params.size:
            shape = (l.n_in, l.n_out) if l.kind == P._abi.LAYER_MATVEC else (l.params.size,)
            t = torch.from_numpy(l.params.reshape(shape).astype(np.float32)).cuda()
            m.share_layer_params(i, 0, t)
            arrays.append((i, t))
    B = 5003
    x = torch.empty((c.n_in, B), dtype=getattr(torch, TORCH_DT[dtype]), device=cuda)
    P.fill_synthetic(x, 9, C.INPUT_TAG, "normal", 0.0, 1.0)
    xg = x.double().cpu().numpy()
    outs = []
    for step in range(3):
        print(f"shared parameters: path={path} dtype={dtype} cfg={cfg} step={step}", flush=True)
        if step:
            for _, t in arrays:
                t.mul_(0.5 if step == 1 else -1.5)  # queued on the same stream, no sync
        y = m.forward_batch_parallel(x)
        outs.append((y, [t.clone() for _, t in arrays]))
    torch.cuda.synchronize()
    for y, values in outs:
        for (i, _), v in zip(arrays, values):
            layers[i].params = v.double().cpu().numpy().reshape(-1)
        want = oracle.forward(layers, xg, MODE[dtype])
        got = y.double().cpu().numpy()
        if dtype in ("f32", "f64"):
            tol = 1e-9 if dtype == "f64" else 1e-5
            assert np.linalg.norm(got - want) <= tol * np.linalg.norm(want)
        else:
            assert np.linalg.norm(got - want) <= 2e-3 * np.linalg.norm(want)
    assert not np.allclose(outs[0][0].double().cpu().numpy(), outs[1][0].double().cpu().numpy())


@pytest.mark.gpu
def test_reference_layout_case_through_a_shared_device_view(cuda):
    """test_core_unit.cpp:516-546: W = 1..6 shared, rewritten to 10..15 on the
    device; the next forward gives 36, 39, 42; get_layer_params reads it and
    set_layer_params writes into it."""
    import torch

    w = torch.arange(1.0, 7.0, device=cuda).reshape(2, 3)
    m = P.create_inference_model(P.Matvec(np.zeros((2, 3))))
    m.share_layer_params(0, 0, w)
    x = torch.tensor([[1.0], [2.0]], device=cuda)
    assert torch.allclose(m.forward_batch_parallel(x)[:, 0].cpu(), torch.tensor([9.0, 12.0, 15.0]))
    w.copy_(torch.from_numpy(W_KNOWN).float())
    assert torch.equal(m.forward_batch_parallel(x)[:, 0].cpu(), torch.tensor([36.0, 39.0, 42.0]))
    torch.cuda.synchronize()
    assert np.array_equal(m.get_layer_params(0), W_KNOWN.reshape(-1))
    m.set_layer_params(0, np.full(6, 0.25))
    assert torch.all(w == 0.25)
