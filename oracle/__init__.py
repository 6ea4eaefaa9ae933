"""TEST INFRASTRUCTURE ONLY: ctypes loader of the CPU oracle (libponni_oracle.so).

The oracle restates the reference's per-sample forward pass on the CPU
(see ponni_oracle.cpp).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module, and only to check or to time the
CPU baseline -- never as the product path.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libponni_oracle.so"

MODE_F32, MODE_F64, MODE_F16_OPERANDS, MODE_BF16_OPERANDS, MODE_F16_CHAIN, MODE_F16_HALF2 = 0, 1, 2, 3, 4, 5
# Modes 2 / 3 with every dense dot product summed in 32-feature blocks: a
# second fp32 order, for measuring a chain's sensitivity to summation order.
MODE_F16_OPERANDS_BLOCKED, MODE_BF16_OPERANDS_BLOCKED = 6, 7

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(LIB_PATH))
        vp = ctypes.c_void_p
        L.oracle_forward.restype = ctypes.c_int
        L.oracle_forward.argtypes = [vp, ctypes.c_int32, vp, ctypes.c_int32, vp, ctypes.c_int64, vp,
                                     ctypes.c_int64, ctypes.c_int64, ctypes.c_int32]
        L.oracle_plan_widths.restype = ctypes.c_int32
        L.oracle_plan_widths.argtypes = [vp, ctypes.c_int32, vp, vp, ctypes.c_int32]
        L.oracle_round_half.restype = ctypes.c_float
        L.oracle_round_half.argtypes = [ctypes.c_float]
        L.oracle_round_bf16.restype = ctypes.c_float
        L.oracle_round_bf16.argtypes = [ctypes.c_float]
        L.oracle_fma_half.restype = ctypes.c_float
        L.oracle_fma_half.argtypes = [ctypes.c_float] * 3
        L.oracle_add_half.restype = ctypes.c_float
        L.oracle_add_half.argtypes = [ctypes.c_float] * 2
        _lib = L
    return _lib


def forward(layers, x: np.ndarray, mode: int = MODE_F32, threads: int = 0) -> np.ndarray:
    """Run the oracle on host array x [n_in, B]; returns [n_out, B]."""
    from ponni_amd.model import concat_params, descs

    io = np.float64 if mode == MODE_F64 else np.float32
    x = np.ascontiguousarray(x, dtype=io)
    B = x.shape[1]
    y = np.zeros((layers[-1].n_out, B), dtype=io)
    p = np.ascontiguousarray(concat_params(layers), dtype=np.float64)
    if p.size == 0:
        p = np.zeros(1)
    d = descs(layers)
    rc = lib().oracle_forward(ctypes.addressof(d), len(layers), p.ctypes.data, mode, x.ctypes.data, B,
                              y.ctypes.data, B, B, threads)
    if rc != 0:
        raise RuntimeError(f"oracle_forward failed with {rc}")
    return y


def plan_widths(layers):
    """([tmp1, tmp2] widths, [saved width of each slot 0 .. num_saved_states - 1])."""
    from ponni_amd.model import descs

    d = descs(layers)
    tmp = (ctypes.c_int32 * 2)()
    cap = max([L.slot + 1 for L in layers if hasattr(L, "slot")] + [1])
    saved = (ctypes.c_int32 * cap)()
    n = lib().oracle_plan_widths(ctypes.addressof(d), len(layers), ctypes.addressof(tmp), ctypes.addressof(saved), cap)
    return list(tmp), list(saved)[:n]


def round_half(v: float) -> float:
    return lib().oracle_round_half(v)


def round_bf16(v: float) -> float:
    return lib().oracle_round_bf16(v)


def fma_half(a: float, b: float, c: float) -> float:
    return lib().oracle_fma_half(a, b, c)


def add_half(a: float, b: float) -> float:
    return lib().oracle_add_half(a, b)


def num_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
