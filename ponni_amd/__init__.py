"""MI355X-native PONNI batched forward pass.

The product is the C ABI library libponni_hip.so (include/ponni_hip.h) and the
header-only C++ facade in ponni_amd/include/ponni.h.  This Python package is a
thin ctypes mirror used by the tests and bench.py.
"""
from . import _abi
from ._abi import PonniError
from . import configs  # noqa: F401
from .model import (  # noqa: F401
    Bias, Binop_Add, Binop_Concatenate, Binop_Projection_Add, Elu, Gelu, GELU, HardSigmoid, HardSwish,
    Inference, Layer, LayerNorm, LeakyRelu, LeakyReLU, LogSoftmax, Matvec, MinMaxNorm, Mish, Relu, ReLU,
    Save_State, Selu, Sigmoid, Silu, Softmax, Softplus, Tanh, concat_params, create_inference_model, descs,
    fill_synthetic,
)

__all__ = [n for n in dir() if not n.startswith("_")] + ["_abi"]
