"""ctypes wrapper around the CPU oracle (liboracle.so). Test infrastructure: imported only
by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg."""
from __future__ import annotations

import ctypes
import json
import os
import subprocess
from typing import Dict, Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'liboracle.so')
_lib = None


def build() -> None:
    subprocess.run(['make', '-s', '-C', HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_create.restype = ctypes.c_void_p
        L.orc_create.argtypes = [ctypes.c_char_p]
        L.orc_destroy.argtypes = [ctypes.c_void_p]
        L.orc_last_error.restype = ctypes.c_char_p
        L.orc_set_home.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int64]
        L.orc_get_home.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int64]
        arr = [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_void_p),
               ctypes.POINTER(ctypes.c_int64)]
        L.orc_step.argtypes = arr + [ctypes.POINTER(ctypes.c_double)]
        L.orc_run.argtypes = arr
        L.orc_get_tensor.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64]
        L.orc_retain_all.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.orc_output_tid.argtypes = [ctypes.c_void_p]
        L.orc_set_lr.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
        L.orc_reset_optimizer.argtypes = [ctypes.c_void_p]
        L.orc_set_threads.argtypes = [ctypes.c_int]
        L.orc_set_matmul_f32.argtypes = [ctypes.c_int]
        L.orc_set_sum_f64.argtypes = [ctypes.c_int]
        L.orc_pcg_f64.restype = ctypes.c_uint32
        L.orc_pcg_f64.argtypes = [ctypes.c_uint32] * 3
        L.orc_pcg_imul2.argtypes = [ctypes.c_uint32] * 3 + [ctypes.POINTER(ctypes.c_uint32)] * 2
        L.orc_salt_const.restype = ctypes.c_uint32
        L.orc_salt_const.argtypes = [ctypes.c_int64]
        L.orc_resolve_lr.restype = ctypes.c_double
        L.orc_resolve_lr.argtypes = [ctypes.c_char_p, ctypes.c_double]
        _lib = L
    return _lib


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


def set_matmul_f32(on: bool) -> None:
    """Matmuls accumulate in f32 (the parity fixtures' f32 twin); off by default."""
    lib().orc_set_matmul_f32(1 if on else 0)


def set_sum_f64(on: bool) -> None:
    """sum_to_shape accumulates in f64 (the parity fixtures' f64-sum twin); off by default."""
    lib().orc_set_sum_f64(1 if on else 0)


def _pack_inputs(inputs: Dict[str, np.ndarray]):
    names = list(inputs.keys())
    arrs = [np.ascontiguousarray(inputs[n]) for n in names]
    for a in arrs:
        assert a.dtype.itemsize == 4, a.dtype
    c_names = (ctypes.c_char_p * len(names))(*[n.encode() for n in names])
    c_data = (ctypes.c_void_p * len(names))(*[a.ctypes.data for a in arrs])
    c_sizes = (ctypes.c_int64 * len(names))(*[a.nbytes for a in arrs])
    return len(names), c_names, c_data, c_sizes, arrs


class OracleRuntime:
    """A training (or forward) graph evaluated by the CPU oracle, with the reference
    worker's step semantics: t/seed counters, lrt/decayShrink injection, writebacks."""

    def __init__(self, wire: dict):
        L = lib()
        self._h = L.orc_create(json.dumps(wire, allow_nan=False).encode())
        if not self._h:
            raise RuntimeError(L.orc_last_error().decode())
        self.wire = wire
        self.tensors = wire['graph']['tensors']

    def __del__(self):
        h = getattr(self, '_h', None)
        if h:
            lib().orc_destroy(h)
            self._h = None

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(lib().orc_last_error().decode())

    def set_home(self, name: str, data: np.ndarray) -> None:
        a = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        self._check(lib().orc_set_home(self._h, name.encode(), a.ctypes.data, a.size))

    def get_home(self, name: str, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        self._check(lib().orc_get_home(self._h, name.encode(), out.ctypes.data, n))
        return out

    def upload_params(self, params: Dict[str, np.ndarray]) -> None:
        for k, v in params.items():
            self.set_home(k, v)

    def step(self, inputs: Dict[str, np.ndarray]) -> float:
        n, names, data, sizes, keep = _pack_inputs(inputs)
        loss = ctypes.c_double()
        self._check(lib().orc_step(self._h, n, names, data, sizes, ctypes.byref(loss)))
        return loss.value

    def run(self, inputs: Dict[str, np.ndarray]) -> None:
        n, names, data, sizes, keep = _pack_inputs(inputs)
        self._check(lib().orc_run(self._h, n, names, data, sizes))

    def retain_all(self, on: bool = True) -> None:
        lib().orc_retain_all(self._h, 1 if on else 0)

    def tensor(self, tid: int) -> np.ndarray:
        t = self.tensors[tid]
        dt = np.float32 if t['dtype'] == 'f32' else np.int32
        n = int(np.prod(t['shape'])) if t['shape'] else 1
        out = np.empty(n, dt)
        self._check(lib().orc_get_tensor(self._h, tid, out.ctypes.data, out.nbytes))
        return out.reshape(t['shape'])

    def output(self) -> np.ndarray:
        return self.tensor(lib().orc_output_tid(self._h))

    def set_lr(self, lr) -> None:
        self._check(lib().orc_set_lr(self._h, json.dumps(lr).encode()))

    def reset_optimizer(self) -> None:
        lib().orc_reset_optimizer(self._h)


def pcg_f64(seed: int, salt_const: int, idx: int) -> int:
    return lib().orc_pcg_f64(seed, salt_const, idx)


def pcg_imul2(seed: int, salt_const: int, idx: int):
    h1, h2 = ctypes.c_uint32(), ctypes.c_uint32()
    lib().orc_pcg_imul2(seed, salt_const, idx, ctypes.byref(h1), ctypes.byref(h2))
    return h1.value, h2.value


def salt_const(salt: int) -> int:
    return lib().orc_salt_const(salt)


def resolve_lr(lr, step: float) -> float:
    return lib().orc_resolve_lr(json.dumps(lr).encode(), step)
