"""c4 (fp16 64->256->256->256->64, tanh) against three CPU semantics on the
same fp16 inputs and weights:

  - fp16 operands with fp32 accumulation (oracle MODE_F16_OPERANDS): the
    build's own arithmetic and the parity bar, relative L2 <= 2e-3;
  - the reference's fp16 chains, which accumulate in fp16: the generated
    half2 model (MODE_F16_HALF2, one rounded fma per step,
    ponni_TwoHalf.h:97-105) and the template half_t model (MODE_F16_CHAIN,
    product and sum rounded separately);
  - float64 (MODE_F64), to show which side drifts.

The distances to the fp16 chains are reported, not graded: fp16 accumulation
over 256 terms is less accurate than the build's fp32 accumulation, and the
test checks exactly that (the build is nearer the float64 result).
"""
import numpy as np
import pytest

import oracle
import ponni_amd as P
from ponni_amd import configs as C

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def test_c4_distances(cuda):
    import torch

    oracle.build()
    cfg = C.CONFIGS["c4"]
    layers = cfg.layers(False)
    m = P.create_inference_model(*layers, dtype="f16")
    B = 4099
    x = torch.empty((cfg.n_in, B), dtype=torch.float16, device=cuda)
    P.fill_synthetic(x, cfg.seed, C.INPUT_TAG, "normal", 0.0, 1.0)
    y = m.forward_batch_parallel(x)
    torch.cuda.synchronize()
    got = y.double().cpu().numpy()
    xh = x.double().cpu().numpy()
    ref = {name: oracle.forward(layers, xh, mode) for name, mode in [
        ("fp16 operands, fp32 accumulation", oracle.MODE_F16_OPERANDS),
        ("fp16 half2 chain", oracle.MODE_F16_HALF2),
        ("fp16 half_t chain", oracle.MODE_F16_CHAIN),
        ("float64", oracle.MODE_F64)]}
    for name, want in ref.items():
        print(f"c4 B={B}: relL2 to {name} = {rel(got, want):.3e}; that semantics to float64 = "
              f"{rel(want, ref['float64']):.3e}", flush=True)
    assert rel(got, ref["fp16 operands, fp32 accumulation"]) <= 2e-3
    assert rel(got, ref["float64"]) < rel(ref["fp16 half2 chain"], ref["float64"])
    assert rel(got, ref["float64"]) < rel(ref["fp16 half_t chain"], ref["float64"])
