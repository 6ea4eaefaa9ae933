"""Python mirror of PONNI's template API over libponni_hip.

    model = create_inference_model(Matvec(W), Bias(b), Relu(3), Matvec(W2), Bias(b2))
    y = model.forward_batch_parallel(x)          # x: [n_in, B] on the GPU

Layer classes carry the same constructor arguments as the reference's layer
templates (src/layers/*.h) and the model exposes the Inference methods
(src/ponni_Inference.h).  Parameters are float64 host arrays in each layer's
own layout; the C library owns the device copy.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from . import _abi as A

_DTYPES = {"f32": A.F32, "f64": A.F64, "f16": A.F16, "bf16": A.BF16}
_PATHS = {"auto": A.PATH_AUTO, "generic": A.PATH_GENERIC, "narrow": A.PATH_NARROW, "mfma": A.PATH_MFMA,
          "fused": A.PATH_FUSED, "layered": A.PATH_LAYERED}


@dataclass
class Layer:
    kind: int
    n_in: int
    n_out: int
    slot: int = 0
    n_aux: int = 0
    flags: int = 0
    attr: tuple = (0.0, 0.0, 0.0, 0.0)
    params: np.ndarray = field(default_factory=lambda: np.zeros(0))
    trainable: bool = True
    label: str = ""

    def desc(self) -> A.LayerDesc:
        d = A.LayerDesc()
        d.kind, d.n_in, d.n_out, d.slot, d.n_aux, d.flags = (
            self.kind, self.n_in, self.n_out, self.slot, self.n_aux, self.flags)
        for i, v in enumerate(self.attr):
            d.attr[i] = float(v)
        return d

    def get_num_inputs(self) -> int:
        return self.n_in

    def get_num_outputs(self) -> int:
        return self.n_out

    def get_label(self) -> str:
        return self.label

    def get_num_trainable_parameters(self) -> int:
        return int(self.params.size) if self.trainable else 0


def Matvec(weights, trainable: bool = True) -> Layer:
    """ponni_Matvec.h: weights [n_in, n_out]."""
    w = np.asarray(weights, dtype=np.float64)
    assert w.ndim == 2
    return Layer(A.LAYER_MATVEC, w.shape[0], w.shape[1], params=w.reshape(-1).copy(), trainable=trainable,
                 label="Matvec")


def Bias(weights, trainable: bool = True) -> Layer:
    b = np.asarray(weights, dtype=np.float64).reshape(-1)
    return Layer(A.LAYER_BIAS, b.size, b.size, params=b.copy(), trainable=trainable, label="Bias")


def _act(kind, label, n, attr=(0.0, 0.0, 0.0, 0.0), flags=0) -> Layer:
    return Layer(kind, n, n, attr=attr, flags=flags, label=label)


def Relu(n): return _act(A.LAYER_RELU, "ReLU", n)
def LeakyRelu(n, negative_slope=0.01): return _act(A.LAYER_LEAKY_RELU, "LeakyReLU", n, (negative_slope, 0, 0, 0))
def Elu(n, alpha=1.0): return _act(A.LAYER_ELU, "ELU", n, (alpha, 0, 0, 0))
def Selu(n): return _act(A.LAYER_SELU, "SELU", n)
def Gelu(n, approximate=False): return _act(A.LAYER_GELU, "GELU", n, flags=A.FLAG_GELU_APPROXIMATE if approximate else 0)
def Silu(n): return _act(A.LAYER_SILU, "SiLU", n)
def Sigmoid(n): return _act(A.LAYER_SIGMOID, "Sigmoid", n)
def Tanh(n): return _act(A.LAYER_TANH, "Tanh", n)
def Softplus(n, beta=1.0): return _act(A.LAYER_SOFTPLUS, "Softplus", n, (beta, 0, 0, 0))
def HardSigmoid(n, alpha=0.2, beta=0.5): return _act(A.LAYER_HARD_SIGMOID, "HardSigmoid", n, (alpha, beta, 0, 0))
def HardSwish(n): return _act(A.LAYER_HARD_SWISH, "HardSwish", n)
def Mish(n): return _act(A.LAYER_MISH, "Mish", n)
def Softmax(n): return _act(A.LAYER_SOFTMAX, "Softmax", n)
def LogSoftmax(n): return _act(A.LAYER_LOG_SOFTMAX, "LogSoftmax", n)
def MinMaxNorm(n, out_min=0.0, out_max=1.0, epsilon=1e-12):
    return _act(A.LAYER_MIN_MAX_NORM, "MinMaxNorm", n, (out_min, out_max, epsilon, 0))


ReLU, LeakyReLU, GELU = Relu, LeakyRelu, Gelu


def LayerNorm(n_or_gamma, beta=None, epsilon=1e-5, trainable=True) -> Layer:
    """ponni_LayerNorm.h: LayerNorm(n) has gamma = 1, beta = 0."""
    if beta is None:
        n = int(n_or_gamma)
        gamma, beta = np.ones(n), np.zeros(n)
    else:
        gamma = np.asarray(n_or_gamma, dtype=np.float64).reshape(-1)
        beta = np.asarray(beta, dtype=np.float64).reshape(-1)
        n = gamma.size
    return Layer(A.LAYER_LAYER_NORM, n, n, attr=(epsilon, 0, 0, 0), params=np.concatenate([gamma, beta]),
                 trainable=trainable, label="LayerNorm")


def Save_State(slot: int, n: int) -> Layer:
    return Layer(A.LAYER_SAVE_STATE, n, n, slot=slot, label="Save_State")


def Binop_Add(slot: int, n: int) -> Layer:
    return Layer(A.LAYER_BINOP_ADD, n, n, slot=slot, label="Binop_Add")


def Binop_Concatenate(slot: int, num_inputs: int, num_outputs: int, after: bool = True) -> Layer:
    return Layer(A.LAYER_BINOP_CONCATENATE, num_inputs, num_outputs, slot=slot,
                 flags=A.FLAG_CONCAT_AFTER if after else 0, label="Binop_Concatenate")


def Binop_Projection_Add(slot: int, weights, bias, trainable: bool = True) -> Layer:
    """weights [NSAVE, n_in], bias [n_in]; out = in + (bias + W^T saved)."""
    w = np.asarray(weights, dtype=np.float64)
    b = np.asarray(bias, dtype=np.float64).reshape(-1)
    return Layer(A.LAYER_BINOP_PROJECTION_ADD, w.shape[1], w.shape[1], slot=slot, n_aux=w.shape[0],
                 params=np.concatenate([w.reshape(-1), b]), trainable=trainable, label="Binop_Projection_Add")


def descs(layers: Sequence[Layer]):
    arr = (A.LayerDesc * len(layers))()
    for i, l in enumerate(layers):
        arr[i] = l.desc()
    return arr


def concat_params(layers: Sequence[Layer]) -> np.ndarray:
    parts = [np.asarray(l.params, dtype=np.float64).reshape(-1) for l in layers]
    return np.concatenate(parts) if parts else np.zeros(0)


class Inference:
    """A compiled plan for a layer chain (src/ponni_Inference.h:13-742)."""

    def __init__(self, layers: Sequence[Layer], dtype: str = "f32", path: str = "auto"):
        self.layers = list(layers)
        self.dtype = dtype
        self._shared = {}  # arrays shared with the plan, kept alive here
        L = A.lib()
        self._plan = ctypes.c_void_p()
        A.check(L.ponni_plan_create(descs(self.layers), len(self.layers), _DTYPES[dtype], _PATHS[path],
                                    ctypes.byref(self._plan)))
        for i, l in enumerate(self.layers):
            if l.params.size:
                self.set_layer_params(i, l.params)

    def __del__(self):
        plan = getattr(self, "_plan", None)
        if plan is not None and plan.value:
            try:
                A.lib().ponni_plan_destroy(plan)
            except (AttributeError, TypeError):  # interpreter shutdown: the module is gone
                pass
            self._plan = None

    # -- parameters -----------------------------------------------------------
    def _param_ctype(self):
        return (np.float64, 8) if self.dtype == "f64" else (np.float32, 4)

    def set_layer_params(self, i: int, values) -> None:
        npt, _ = self._param_ctype()
        v = np.ascontiguousarray(np.asarray(values, dtype=np.float64).reshape(-1), dtype=npt)
        A.check(A.lib().ponni_plan_set_layer_params(self._plan, i, v.ctypes.data, v.size))
        self.layers[i].params = np.asarray(values, dtype=np.float64).reshape(-1).copy()

    def share_layer_params(self, i: int, segment: int, array) -> None:
        """Share parameter segment `segment` of layer i with `array` (a 1-D or
        2-D torch tensor on the GPU or numpy array on the host, with unit
        column stride; it must outlive the sharing), as the reference shares a
        layer's Views with a model in the same memory space
        (ponni_plan_share_layer_params).  None ends the sharing."""
        if array is None:
            A.check(A.lib().ponni_plan_share_layer_params(self._plan, i, segment, None, 0, 0, 0, 0, 0))
            self._shared.pop((i, segment), None)
            return
        if hasattr(array, "data_ptr"):  # torch tensor
            names = {"torch.float32": A.F32, "torch.float64": A.F64, "torch.float16": A.F16,
                     "torch.bfloat16": A.BF16}
            dt, ptr, on_device = names[str(array.dtype)], array.data_ptr(), int(array.is_cuda)
            shape, strides = tuple(array.shape), tuple(array.stride())
        else:
            names = {"float32": A.F32, "float64": A.F64, "float16": A.F16}
            dt, ptr, on_device = names[str(array.dtype)], array.ctypes.data, 0
            shape, strides = array.shape, tuple(s // array.itemsize for s in array.strides)
        rows, cols = (1, shape[0]) if len(shape) == 1 else shape
        ld = cols if len(shape) == 1 else strides[0]
        if strides[-1] != 1:
            raise ValueError("shared arrays need unit column stride")
        A.check(A.lib().ponni_plan_share_layer_params(self._plan, i, segment, ptr, dt, rows, cols, ld, on_device))
        self._shared[(i, segment)] = array

    def get_layer_params(self, i: int) -> np.ndarray:
        npt, _ = self._param_ctype()
        n = A.lib().ponni_plan_layer_param_count(self._plan, i)
        out = np.zeros(n, dtype=npt)
        A.check(A.lib().ponni_plan_get_layer_params(self._plan, i, out.ctypes.data, n))
        return out.astype(np.float64)

    def get_num_trainable_parameters(self) -> int:
        return sum(l.get_num_trainable_parameters() for l in self.layers)

    def get_trainable_parameters(self) -> np.ndarray:
        parts = [self.get_layer_params(i) for i, l in enumerate(self.layers) if l.trainable and l.params.size]
        return np.concatenate(parts) if parts else np.zeros(0)

    def set_trainable_parameters(self, values) -> None:
        """Each trainable layer consumes its prefix, in tuple order (ponni_Inference.h:688-699)."""
        v = np.asarray(values, dtype=np.float64).reshape(-1)
        off = 0
        for i, l in enumerate(self.layers):
            n = l.get_num_trainable_parameters()
            if n:
                if v.size - off < n:
                    raise ValueError(f"{l.label} trainable input too small")
                self.set_layer_params(i, v[off:off + n])
                off += n

    # -- generated kernel ---------------------------------------------------------
    def kernel_source(self) -> str:
        n = A.lib().ponni_plan_kernel_source(self._plan, None, 0)
        if n < 0:
            A.check(A.PONNI_ERR_UNSUPPORTED)
        buf = ctypes.create_string_buffer(n)
        A.lib().ponni_plan_kernel_source(self._plan, buf, n)
        return buf.value.decode()

    def program_source(self) -> str:
        """constexpr C++ members of the plan's per-sample program (F32 / F64 plans),
        for ponni::forward_one_program (ponni_plan_program_source)."""
        n = A.lib().ponni_plan_program_source(self._plan, None, 0)
        if n < 0:
            A.check(A.PONNI_ERR_UNSUPPORTED)
        buf = ctypes.create_string_buffer(n)
        A.lib().ponni_plan_program_source(self._plan, buf, n)
        return buf.value.decode()

    def kernel_config(self) -> tuple[int, int, bool]:
        """(threads per workgroup, batch columns per workgroup, persistent grid) of the
        generated kernel (FUSED or generated NARROW plans)."""
        t, c, p = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        A.check(A.lib().ponni_plan_kernel_config(self._plan, ctypes.byref(t), ctypes.byref(c), ctypes.byref(p)))
        return t.value, c.value, bool(p.value)

    def compile(self) -> None:
        A.check(A.lib().ponni_plan_compile(self._plan))

    # -- info -------------------------------------------------------------------
    def info(self) -> A.PlanInfo:
        inf = A.PlanInfo()
        A.check(A.lib().ponni_plan_get_info(self._plan, ctypes.byref(inf)))
        return inf

    @property
    def path(self) -> str:
        return A.PATH_NAMES[self.info().path]

    def get_num_inputs(self) -> int:
        return self.layers[0].n_in

    def get_num_outputs(self) -> int:
        return self.layers[-1].n_out

    def internal_state_capacity(self) -> int:
        return int(self.info().internal_state_capacity)

    def reallocate_internal_state(self, batch: int) -> None:
        A.check(A.lib().ponni_plan_reallocate_internal_state(self._plan, batch))

    def weight_schema_fingerprint(self) -> str:
        n = len(self.layers)
        labels = (ctypes.c_char_p * n)(*[l.label.encode() for l in self.layers])
        nin = (ctypes.c_int32 * n)(*[l.n_in for l in self.layers])
        nout = (ctypes.c_int32 * n)(*[l.n_out for l in self.layers])
        ntr = (ctypes.c_int64 * n)(*[l.get_num_trainable_parameters() for l in self.layers])
        buf = ctypes.create_string_buffer(64)
        A.check(A.lib().ponni_template_fingerprint(n, labels, nin, nout, ntr, buf, 64))
        return buf.value.decode()

    # -- weights files ------------------------------------------------------------
    def save_weights(self, path: str) -> None:
        count = self.get_num_trainable_parameters()
        if count == 0:
            raise A.PonniError(A.PONNI_ERR_IO, "cannot save weights from a model with no trainable parameters")
        p = self.get_trainable_parameters()
        npt, es = (np.float64, 8) if self.dtype == "f64" else (np.float32, 4)
        v = np.ascontiguousarray(p, dtype=npt)
        A.check(A.lib().ponni_file_write_parameters(path.encode(), self.weight_schema_fingerprint().encode(),
                                                    v.ctypes.data, count, es, b"template"))

    def load_weights(self, path: str) -> None:
        count = self.get_num_trainable_parameters()
        if count == 0:
            raise A.PonniError(A.PONNI_ERR_IO, "cannot load weights into a model with no trainable parameters")
        npt, es = (np.float64, 8) if self.dtype == "f64" else (np.float32, 4)
        v = np.zeros(count, dtype=npt)
        A.check(A.lib().ponni_file_read_parameters(path.encode(), self.weight_schema_fingerprint().encode(),
                                                   v.ctypes.data, count, es))
        self.set_trainable_parameters(v.astype(np.float64))

    # -- forward ------------------------------------------------------------------
    def forward_raw(self, x_ptr: int, ld_in: int, y_ptr: int, ld_out: int, batch: int, stream: int = 0) -> None:
        A.check(A.lib().ponni_forward(self._plan, x_ptr, ld_in, y_ptr, ld_out, batch, stream))

    def forward_raw_no_alloc(self, x_ptr: int, ld_in: int, y_ptr: int, ld_out: int, batch: int,
                             stream: int = 0) -> None:
        """forward_raw with no device allocation: GENERIC state buffers come
        from the library's fixed per-GPU scratch (ponni_forward_no_alloc)."""
        A.check(A.lib().ponni_forward_no_alloc(self._plan, x_ptr, ld_in, y_ptr, ld_out, batch, stream))

    def forward_raw_timed(self, x_ptr: int, ld_in: int, y_ptr: int, ld_out: int, batch: int, stream: int,
                          start_event: int, stop_event: int) -> None:
        """forward_raw whose kernel dispatch stamps two caller-created HIP events
        with its own start and end (ponni_forward_timed)."""
        A.check(A.lib().ponni_forward_timed(self._plan, x_ptr, ld_in, y_ptr, ld_out, batch, stream, start_event,
                                            stop_event))

    def forward_host(self, x, threads: int = 0):
        """Host execution space: x a numpy array [n_in, B] of the plan's dtype
        (F32 or F64 plans), evaluated on the host by the GENERIC op list
        (ponni_forward_host).  Returns y [n_out, B]."""
        import numpy as np

        want = {"f32": np.float32, "f64": np.float64}.get(self.dtype)
        if want is None:
            raise ValueError("host execution runs f32 and f64 models")
        x = np.ascontiguousarray(x, dtype=want)
        if x.ndim != 2:
            raise ValueError("input must be rank two [features, batch]")
        y = np.empty((self.get_num_outputs(), x.shape[1]), dtype=want)
        A.check(A.lib().ponni_forward_host(self._plan, x.ctypes.data, x.shape[1], y.ctypes.data, y.shape[1],
                                           x.shape[1], threads))
        return y

    def forward_batch_parallel(self, x, y=None):
        """x: torch tensor [n_in, B] on the GPU (row-contiguous).  Returns y [n_out, B]."""
        import torch

        assert x.dim() == 2 and x.is_cuda and x.stride(1) == 1
        B = x.shape[1]
        if y is None:
            y = torch.empty((self.get_num_outputs(), B), dtype=x.dtype, device=x.device)
        stream = torch.cuda.current_stream(x.device).cuda_stream
        self.forward_raw(x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0), B, stream)
        return y


def create_inference_model(*layers: Layer, dtype: str = "f32", path: str = "auto") -> Inference:
    return Inference(layers, dtype=dtype, path=path)


def fill_synthetic(t, seed: int, tag: int, dist: str, a: float, b: float) -> None:
    """Fill a GPU tensor with the counter-based synthetic stream (see include/ponni_hip.h)."""
    import torch

    dt = {torch.float32: A.F32, torch.float64: A.F64, torch.float16: A.F16, torch.bfloat16: A.BF16}[t.dtype]
    stream = torch.cuda.current_stream(t.device).cuda_stream
    A.check(A.lib().ponni_fill_synthetic(t.data_ptr(), dt, t.numel(), seed, tag,
                                         0 if dist == "uniform" else 1, a, b, stream))
