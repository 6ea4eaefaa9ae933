"""Framework integration: models built and run in PyTorch (CPU, fp32),
exported to .ponni files (weights in the reference's [in, out] Matvec order
plus test.input / test.output), rebuilt from the file in template mode by
tests/cpp/test_frameworks.cpp and checked against PyTorch's outputs within
1e-5, as the reference's unit/pytorch_resnet and unit/projection_skip tests
do with their own generated fixtures.  PyTorch is the independent
implementation here; the host execution space runs on the CPU, the HIP one
on the GPU."""
import os
import subprocess

import numpy as np
import pytest

from ponni_amd import _abi as A

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin", "test_frameworks")


def _write(path, tensors):
    """tensors: name -> float32 array, written in name order as F32."""
    names = sorted(tensors)
    specs = (A.TensorSpec * len(names))()
    keep, storage, off = [], [], 0
    for i, n in enumerate(names):
        a = np.asarray(tensors[n], dtype=np.float32)
        keep.append(n.encode())
        specs[i].name = keep[-1]
        specs[i].rank = a.ndim
        for k, d in enumerate(a.shape):
            specs[i].shape[k] = d
        specs[i].offset = off
        storage.append(a.reshape(-1).astype(np.float64))
        off += a.size
    st = np.ascontiguousarray(np.concatenate(storage))
    A.check(A.lib().ponni_file_write_tensors(str(path).encode(), b"pytorch-export", specs, len(names), st.ctypes.data, 4,
                                             b"pytorch", b"test-fixture"))


def _resnet(path, batch):
    import torch
    import torch.nn.functional as F

    g = torch.Generator().manual_seed(4321)
    dims = [(12, 5), (5, 5), (5, 5), (5, 5), (5, 4)]
    layers = [torch.nn.Linear(a, b) for a, b in dims]
    with torch.no_grad():
        for l in layers:
            l.weight.uniform_(-0.2, 0.2, generator=g)
            l.bias.uniform_(-0.2, 0.2, generator=g)
        x = torch.randn(batch, 12, generator=g)
        h = F.silu(layers[0](x))
        for l in layers[1:4]:
            h = F.silu(l(h)) + h
        y = layers[4](h)
    tensors = {"test.input": x.numpy().T, "test.output": y.numpy().T}
    for k, l in enumerate(layers, 1):
        tensors[f"fc{k}.weight"] = l.weight.detach().numpy().T  # torch [out, in] -> Matvec [in, out]
        tensors[f"fc{k}.bias"] = l.bias.detach().numpy()
    _write(path, tensors)


def _projection(path, batch):
    import torch

    g = torch.Generator().manual_seed(8765)
    main, skip = torch.nn.Linear(2, 3), torch.nn.Linear(2, 3)
    with torch.no_grad():
        for l in (main, skip):
            l.weight.uniform_(-1.0, 1.0, generator=g)
            l.bias.uniform_(-0.5, 0.5, generator=g)
        x = torch.rand(batch, 2, generator=g) + 0.1  # positive: the rebuilt model leads with Relu
        y = main(x) + skip(x)
    _write(path, {"w_main": main.weight.detach().numpy().T, "b_main": main.bias.detach().numpy(), "w_skip": skip.weight.detach().numpy().T,
                  "b_skip": skip.bias.detach().numpy(), "test.input": x.numpy().T, "test.output": y.numpy().T})


def _run(model, path, host):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is missing: build with `python -c 'import __graft_entry__ as g; g.build()'`")
    r = subprocess.run([BIN, model, str(path)] + (["--host"] if host else []), capture_output=True, text=True,
                       timeout=300)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr


@pytest.mark.parametrize("model,batch", [("resnet", 1), ("resnet", 777), ("projection", 1), ("projection", 300)])
def test_pytorch_models_on_host(tmp_path, model, batch):
    path = tmp_path / f"{model}.ponni"
    (_resnet if model == "resnet" else _projection)(path, batch)
    _run(model, path, host=True)


@pytest.mark.gpu
@pytest.mark.parametrize("model,batch", [("resnet", 1), ("resnet", 4099), ("projection", 1), ("projection", 300)])
def test_pytorch_models_on_gpu(cuda, tmp_path, model, batch):
    path = tmp_path / f"{model}.ponni"
    (_resnet if model == "resnet" else _projection)(path, batch)
    _run(model, path, host=False)
