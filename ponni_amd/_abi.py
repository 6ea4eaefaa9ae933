"""ctypes binding of libponni_hip.so (declarations in include/ponni_hip.h)."""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libponni_hip.so"

PONNI_OK = 0
PONNI_ERR_INVALID_ARGUMENT = 1
PONNI_ERR_INVALID_MODEL = 2
PONNI_ERR_SHAPE = 3
PONNI_ERR_UNSUPPORTED = 4
PONNI_ERR_DEVICE = 5
PONNI_ERR_IO = 6

F32, F64, F16, BF16 = 1, 2, 3, 4
PATH_AUTO, PATH_GENERIC, PATH_NARROW, PATH_MFMA, PATH_FUSED, PATH_LAYERED = 0, 1, 2, 3, 4, 5
PATH_NAMES = {PATH_AUTO: "auto", PATH_GENERIC: "generic", PATH_NARROW: "narrow", PATH_MFMA: "mfma",
              PATH_FUSED: "fused", PATH_LAYERED: "layered"}

LAYER_MATVEC = 1
LAYER_BIAS = 2
LAYER_RELU = 3
LAYER_LEAKY_RELU = 4
LAYER_ELU = 5
LAYER_SELU = 6
LAYER_GELU = 7
LAYER_SILU = 8
LAYER_SIGMOID = 9
LAYER_TANH = 10
LAYER_SOFTPLUS = 11
LAYER_HARD_SIGMOID = 12
LAYER_HARD_SWISH = 13
LAYER_MISH = 14
LAYER_SOFTMAX = 20
LAYER_LOG_SOFTMAX = 21
LAYER_LAYER_NORM = 22
LAYER_MIN_MAX_NORM = 23
LAYER_SAVE_STATE = 30
LAYER_BINOP_ADD = 31
LAYER_BINOP_CONCATENATE = 32
LAYER_BINOP_PROJECTION_ADD = 33

LAYER_DENSE = 40
LAYER_LOAD_STATE = 41
LAYER_BINARY = 42
LAYER_REDUCE = 43
LAYER_UNARY = 44
LAYER_CONST_BINARY = 45

LAYER_SELECT = 46
BINARY_OPS = {"Add": 0, "Sub": 1, "Mul": 2, "Div": 3, "Min": 4, "Max": 5, "Pow": 6, "Equal": 7, "Greater": 8,
              "GreaterOrEqual": 9, "Less": 10, "LessOrEqual": 11, "And": 12, "Or": 13, "Xor": 14, "PRelu": 15}
SELECT_STATE, SELECT_SLOT, SELECT_CONST = 0, 1, 2
SELECT_COND_SCALAR, SELECT_A_SCALAR, SELECT_B_SCALAR = 64, 128, 256
REDUCE_OPS = {"ReduceSum": 0, "ReduceMean": 1, "ReduceMax": 2, "ReduceMin": 3, "ReduceL1": 4, "ReduceL2": 5,
              "ReduceSumSquare": 6, "ReduceLogSum": 7, "ReduceLogSumExp": 8, "ReduceProd": 9}
UNARY_OPS = {"Abs": 0, "Neg": 1, "Exp": 2, "Log": 3, "Sqrt": 4, "Reciprocal": 5, "Softsign": 6, "Celu": 7,
             "ThresholdedRelu": 8, "Erf": 9, "Selu": 10, "Acos": 11, "Acosh": 12, "Asin": 13, "Asinh": 14,
             "Atan": 15, "Atanh": 16, "Ceil": 17, "Cos": 18, "Cosh": 19, "Floor": 20, "Sin": 21, "Sinh": 22,
             "Tan": 23, "Round": 24, "Sign": 25, "IsNaN": 26, "IsInf": 27, "Not": 28, "NonZero": 29}

FLAG_GELU_APPROXIMATE = 1
FLAG_CONCAT_AFTER = 1
FLAG_DENSE_BIAS = 1
FLAG_SAVED_LEFT = 1
FLAG_CONST_LEFT = 1


class LayerDesc(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("n_in", ctypes.c_int32),
        ("n_out", ctypes.c_int32),
        ("slot", ctypes.c_int32),
        ("n_aux", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("attr", ctypes.c_double * 4),
    ]


class TensorSpec(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("rank", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 8),
        ("offset", ctypes.c_int64),
    ]


class Peaks(ctypes.Structure):
    _fields_ = [("hbm_copy_gbps", ctypes.c_double), ("mfma_f16_tflops", ctypes.c_double),
                ("mfma_f32_tflops", ctypes.c_double), ("hbm_read_gbps", ctypes.c_double),
                ("hbm_copy_12mb_gbps", ctypes.c_double), ("copy_12mb_us", ctypes.c_double)]


# Saved-state slot indices a plan may use: 0 .. MAX_SLOTS - 1 (program.h kMaxSlots).
MAX_SLOTS = 4096


class PlanInfo(ctypes.Structure):
    _fields_ = [
        ("path", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("num_inputs", ctypes.c_int32),
        ("num_outputs", ctypes.c_int32),
        ("num_fused_dense_blocks", ctypes.c_int32),
        ("num_saved_states", ctypes.c_int32),
        ("tmp1_features", ctypes.c_int32),
        ("tmp2_features", ctypes.c_int32),
        ("saved_features", ctypes.c_int32 * 8),
        ("num_parameters", ctypes.c_int64),
        ("internal_state_capacity", ctypes.c_int64),
        ("max_width", ctypes.c_int32),
        ("width_class", ctypes.c_int32),
    ]


_lib = None


class PonniError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"ponni status {status}: {message}")
        self.status = status
        self.message = message


class DeviceModel(ctypes.Structure):
    """ponni_device_model (include/ponni_hip.h)."""
    _fields_ = [("ops", ctypes.c_void_p), ("steps", ctypes.c_void_p), ("params", ctypes.c_void_p),
                ("num_ops", ctypes.c_int32), ("dtype", ctypes.c_int32), ("num_inputs", ctypes.c_int32),
                ("num_outputs", ctypes.c_int32), ("max_width", ctypes.c_int32),
                ("tmp_features", ctypes.c_int32 * 2), ("num_slots", ctypes.c_int32), ("saved_total", ctypes.c_int32),
                ("slot_rows", ctypes.c_void_p)]


def lib() -> ctypes.CDLL:
    """Load the in-tree libponni_hip.so; fail loudly when it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    L = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    vp, i32, i64, u64, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64, ctypes.c_size_t
    L.ponni_last_error.restype = ctypes.c_char_p
    L.ponni_last_error.argtypes = []
    L.ponni_abi_version.restype = ctypes.c_int
    L.ponni_plan_create.restype = ctypes.c_int
    L.ponni_plan_create.argtypes = [ctypes.POINTER(LayerDesc), i32, i32, i32, ctypes.POINTER(vp)]
    L.ponni_plan_destroy.restype = None
    L.ponni_plan_destroy.argtypes = [vp]
    L.ponni_plan_get_info.restype = ctypes.c_int
    L.ponni_plan_get_info.argtypes = [vp, ctypes.POINTER(PlanInfo)]
    L.ponni_plan_layer_param_count.restype = i64
    L.ponni_plan_layer_param_count.argtypes = [vp, i32]
    L.ponni_plan_saved_state_size.restype = i32
    L.ponni_plan_saved_state_size.argtypes = [vp, i32]
    L.ponni_plan_set_layer_params.restype = ctypes.c_int
    L.ponni_plan_set_layer_params.argtypes = [vp, i32, vp, i64]
    L.ponni_plan_share_layer_params.restype = ctypes.c_int
    L.ponni_plan_share_layer_params.argtypes = [vp, i32, i32, vp, i32, i64, i64, i64, i32]
    L.ponni_plan_get_layer_params.restype = ctypes.c_int
    L.ponni_plan_get_layer_params.argtypes = [vp, i32, vp, i64]
    L.ponni_plan_reallocate_internal_state.restype = ctypes.c_int
    L.ponni_plan_reallocate_internal_state.argtypes = [vp, i64]
    L.ponni_forward.restype = ctypes.c_int
    L.ponni_forward.argtypes = [vp, vp, i64, vp, i64, i64, vp]
    L.ponni_forward_no_alloc.restype = ctypes.c_int
    L.ponni_forward_no_alloc.argtypes = [vp, vp, i64, vp, i64, i64, vp]
    L.ponni_forward_timed.restype = ctypes.c_int
    L.ponni_forward_timed.argtypes = [vp, vp, i64, vp, i64, i64, vp, vp, vp]
    L.ponni_forward_steps.restype = ctypes.c_int
    L.ponni_forward_steps.argtypes = [vp, vp, i64, vp, i64, i64, i32, i32, vp, ctypes.POINTER(ctypes.c_double)]
    L.ponni_plan_kernel_source.restype = i64
    L.ponni_plan_kernel_source.argtypes = [vp, ctypes.c_char_p, i64]
    L.ponni_plan_program_source.restype = i64
    L.ponni_plan_program_source.argtypes = [vp, ctypes.c_char_p, i64]
    L.ponni_plan_compile.restype = ctypes.c_int
    L.ponni_plan_compile.argtypes = [vp]
    L.ponni_plan_kernel_config.restype = ctypes.c_int
    L.ponni_plan_kernel_config.argtypes = [vp, ctypes.POINTER(i32), ctypes.POINTER(i32), ctypes.POINTER(i32)]
    L.ponni_plan_device_params.restype = ctypes.c_int
    L.ponni_plan_device_params.argtypes = [vp, ctypes.POINTER(vp)]
    L.ponni_plan_device_model.restype = ctypes.c_int
    L.ponni_plan_device_model.argtypes = [vp, ctypes.POINTER(DeviceModel)]
    L.ponni_plan_host_model.restype = ctypes.c_int
    L.ponni_plan_host_model.argtypes = [vp, ctypes.POINTER(DeviceModel)]
    L.ponni_forward_host.restype = ctypes.c_int
    L.ponni_forward_host.argtypes = [vp, vp, i64, vp, i64, i64, ctypes.c_int32]
    L.ponni_fill_synthetic.restype = ctypes.c_int
    L.ponni_fill_synthetic.argtypes = [vp, i32, i64, u64, u64, i32, ctypes.c_double, ctypes.c_double, vp]
    L.ponni_measure_peaks.restype = ctypes.c_int
    L.ponni_measure_peaks.argtypes = [ctypes.POINTER(Peaks), vp]
    L.ponni_fnv1a64.restype = u64
    L.ponni_fnv1a64.argtypes = [vp, sz]
    L.ponni_template_fingerprint.restype = ctypes.c_int
    L.ponni_template_fingerprint.argtypes = [
        i32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(i32), ctypes.POINTER(i32),
        ctypes.POINTER(i64), ctypes.c_char_p, sz,
    ]
    L.ponni_file_write_parameters.restype = ctypes.c_int
    L.ponni_file_write_parameters.argtypes = [ctypes.c_char_p, ctypes.c_char_p, vp, i64, i32, ctypes.c_char_p]
    L.ponni_file_read_parameters.restype = ctypes.c_int
    L.ponni_file_read_parameters.argtypes = [ctypes.c_char_p, ctypes.c_char_p, vp, i64, i32]
    L.ponni_file_write_tensors.restype = ctypes.c_int
    L.ponni_file_write_tensors.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(TensorSpec), i32, vp, i32,
                                           ctypes.c_char_p, ctypes.c_char_p]
    L.ponni_file_read_tensors.restype = ctypes.c_int
    L.ponni_file_read_tensors.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(TensorSpec), i32, vp, i32]
    _lib = L
    return L


def check(status: int) -> None:
    if status != PONNI_OK:
        msg = lib().ponni_last_error().decode(errors="replace")
        raise PonniError(status, msg)
