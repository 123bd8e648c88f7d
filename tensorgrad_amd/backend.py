"""ctypes binding of the C ABI (include/tg.h) exposed by libtg.so.

The library is built in-tree (`tensorgrad_amd/libtg.so`) by `build()`; loading fails
loudly if it is missing — there is no CPU fallback on the product path.
"""
from __future__ import annotations

import ctypes
import json
import os
import subprocess
from typing import Dict, List, Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'libtg.so')
CSRC = os.path.join(HERE, 'csrc')

TG_OK, TG_ABORTED, TG_INVALID_ARGUMENT, TG_DEVICE_ERROR, TG_INTERNAL = range(5)

# Every symbol include/tg.h declares (checked by the CPU test suite).
EXPORTED = (
    'tg_last_error', 'tg_device_count', 'tg_runtime_create', 'tg_runtime_create_sibling', 'tg_destroy',
    'tg_param_count', 'tg_param_name', 'tg_param_numel', 'tg_upload_params', 'tg_download_params', 'tg_step',
    'tg_step_device', 'tg_stage_batch', 'tg_step_staged', 'tg_run', 'tg_capture_count', 'tg_capture_name', 'tg_get_capture', 'tg_reset_optimizer',
    'tg_set_lr', 'tg_describe', 'tg_plan', 'tg_profile_nodes', 'tg_profile_kernels', 'tg_time_replays', 'tg_time_kinds',
    'tg_state_count', 'tg_state_name', 'tg_state_numel', 'tg_download_state', 'tg_upload_state',
    'tg_save_checkpoint', 'tg_load_checkpoint', 'tg_check_checkpoint', 'tg_safetensors_index', 'tg_step_noalloc',
)


class AbortError(RuntimeError):
    """The graph was destroyed or replaced while the call was in flight (the reference's
    `AbortError`, src/worker.ts:262-266)."""


class BackendError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def build(jobs: int = 8) -> str:
    """Compile libtg.so for gfx950 with hipcc (works without a GPU)."""
    subprocess.run(['make', '-s', '-C', CSRC, f'-j{jobs}'], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f'tensorgrad_amd: {LIB_PATH} is not built; run __graft_entry__.build() first')
    L = ctypes.CDLL(LIB_PATH)
    c_char_pp = ctypes.POINTER(ctypes.c_char_p)
    vp, i64p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64)
    L.tg_last_error.restype = ctypes.c_char_p
    L.tg_device_count.restype = ctypes.c_int
    L.tg_runtime_create.argtypes = [ctypes.c_char_p, ctypes.POINTER(vp)]
    L.tg_runtime_create_sibling.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(vp)]
    L.tg_destroy.argtypes = [vp]
    L.tg_destroy.restype = None
    L.tg_param_count.argtypes = [vp]
    L.tg_param_name.argtypes = [vp, ctypes.c_int]
    L.tg_param_name.restype = ctypes.c_char_p
    L.tg_param_numel.argtypes = [vp, ctypes.c_int]
    L.tg_param_numel.restype = ctypes.c_int64
    L.tg_upload_params.argtypes = [vp, ctypes.c_int, c_char_pp, ctypes.POINTER(vp), i64p]
    L.tg_download_params.argtypes = [vp, ctypes.c_int, c_char_pp, ctypes.POINTER(vp), i64p]
    L.tg_step.argtypes = [vp, ctypes.c_int, c_char_pp, ctypes.POINTER(vp), i64p, ctypes.POINTER(ctypes.c_float)]
    L.tg_step_device.argtypes = L.tg_step.argtypes
    L.tg_step_noalloc.argtypes = L.tg_step.argtypes
    L.tg_run.argtypes = [vp, ctypes.c_int, c_char_pp, ctypes.POINTER(vp), i64p, vp, ctypes.c_int64]
    L.tg_stage_batch.argtypes = [vp, ctypes.c_int, ctypes.c_int, c_char_pp, ctypes.POINTER(vp), i64p]
    L.tg_step_staged.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_float)]
    L.tg_capture_count.argtypes = [vp]
    L.tg_capture_name.argtypes = [vp, ctypes.c_int]
    L.tg_capture_name.restype = ctypes.c_char_p
    L.tg_get_capture.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_int64]
    L.tg_reset_optimizer.argtypes = [vp]
    L.tg_set_lr.argtypes = [vp, ctypes.c_char_p]
    L.tg_describe.argtypes = [vp, ctypes.c_char_p, ctypes.c_int64]
    L.tg_plan.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int64]
    L.tg_profile_nodes.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_double), ctypes.c_int64]
    L.tg_profile_kernels.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_double), ctypes.c_int64]
    L.tg_time_replays.argtypes = [vp, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    L.tg_time_kinds.argtypes = [vp, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                ctypes.POINTER(ctypes.c_int)]
    L.tg_state_count.argtypes = [vp]
    L.tg_state_name.argtypes = [vp, ctypes.c_int]
    L.tg_state_name.restype = ctypes.c_char_p
    L.tg_state_numel.argtypes = [vp, ctypes.c_int]
    L.tg_state_numel.restype = ctypes.c_int64
    L.tg_download_state.argtypes = [vp, ctypes.c_int, c_char_pp, ctypes.POINTER(vp), i64p, i64p, i64p]
    L.tg_upload_state.argtypes = [vp, ctypes.c_int, c_char_pp, ctypes.POINTER(vp), i64p, ctypes.c_int64,
                                  ctypes.c_int64]
    L.tg_save_checkpoint.argtypes = [vp, ctypes.c_char_p]
    L.tg_load_checkpoint.argtypes = [vp, ctypes.c_char_p]
    L.tg_safetensors_index.argtypes = [ctypes.c_char_p, ctypes.c_int64, ctypes.c_char_p, ctypes.c_int64]
    L.tg_check_checkpoint.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int64]
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc == TG_OK:
        return
    msg = lib().tg_last_error().decode()
    if rc == TG_ABORTED:
        raise AbortError(msg)
    raise BackendError(rc, msg)


def device_count() -> int:
    return lib().tg_device_count()


def plan(ir_json: str) -> dict:
    """Lower an IR document on the host only; returns the launch schedule."""
    buf = ctypes.create_string_buffer(1 << 24)
    _check(lib().tg_plan(ir_json.encode(), buf, len(buf)))
    return json.loads(buf.value.decode())


def check_checkpoint(ir_json: str, path: str) -> dict:
    """The checks a checkpoint load into the graph `ir_json` would make, on the host only
    (tg_check_checkpoint)."""
    out = ctypes.create_string_buffer(4096)
    _check(lib().tg_check_checkpoint(ir_json.encode(), str(path).encode(), out, len(out)))
    return json.loads(out.value.decode())


def safetensors_index(buf: bytes) -> dict:
    """Index a safetensors container on the host (tg_safetensors_index)."""
    hlen = int.from_bytes(buf[:8], 'little') if len(buf) >= 8 else 0
    out = ctypes.create_string_buffer(4096 + 8 * min(hlen, len(buf)))
    _check(lib().tg_safetensors_index(buf, len(buf), out, len(out)))
    return json.loads(out.value.decode())


def _names(names: Sequence[str]):
    return (ctypes.c_char_p * len(names))(*[n.encode() for n in names])


def _inputs(inputs: Dict[str, np.ndarray]):
    names = list(inputs.keys())
    arrs = []
    for n in names:
        a = inputs[n]
        if isinstance(a, np.ndarray):
            a = np.ascontiguousarray(a)
            if a.dtype not in (np.float32, np.int32):
                raise TypeError(f"input '{n}': expected float32 or int32, got {a.dtype}")
        arrs.append(a)
    ptrs = (ctypes.c_void_p * len(names))(*[a.ctypes.data for a in arrs])
    sizes = (ctypes.c_int64 * len(names))(*[a.nbytes for a in arrs])
    return len(names), _names(names), ptrs, sizes, arrs


class NativeRuntime:
    """One runtime handle (training graph or forward sibling)."""

    def __init__(self, ir_json: str, parent: Optional['NativeRuntime'] = None):
        h = ctypes.c_void_p()
        if parent is None:
            _check(lib().tg_runtime_create(ir_json.encode(), ctypes.byref(h)))
        else:
            _check(lib().tg_runtime_create_sibling(parent._h, ir_json.encode(), ctypes.byref(h)))
        self._h = h
        self.parent = parent
        n = lib().tg_param_count(h)
        self.param_names: List[str] = [lib().tg_param_name(h, i).decode() for i in range(n)]
        self.param_numel: Dict[str, int] = {self.param_names[i]: lib().tg_param_numel(h, i) for i in range(n)}
        self.capture_names = [lib().tg_capture_name(h, i).decode() for i in range(lib().tg_capture_count(h))]

    @property
    def alive(self) -> bool:
        return bool(self._h)

    def destroy(self) -> None:
        if self._h:
            lib().tg_destroy(self._h)
            self._h = ctypes.c_void_p()

    def upload_params(self, params: Dict[str, np.ndarray]) -> None:
        names = list(params.keys())
        arrs = [np.ascontiguousarray(params[n], dtype=np.float32).reshape(-1) for n in names]
        ptrs = (ctypes.c_void_p * len(names))(*[a.ctypes.data for a in arrs])
        sizes = (ctypes.c_int64 * len(names))(*[a.size for a in arrs])
        _check(lib().tg_upload_params(self._h, len(names), _names(names), ptrs, sizes))

    def download_params(self) -> Dict[str, np.ndarray]:
        names = self.param_names
        arrs = [np.empty(self.param_numel[n], np.float32) for n in names]
        ptrs = (ctypes.c_void_p * len(names))(*[a.ctypes.data for a in arrs])
        sizes = (ctypes.c_int64 * len(names))(*[a.size for a in arrs])
        _check(lib().tg_download_params(self._h, len(names), _names(names), ptrs, sizes))
        return dict(zip(names, arrs))

    def step(self, inputs: Dict[str, np.ndarray]) -> float:
        n, names, ptrs, sizes, keep = _inputs(inputs)
        loss = ctypes.c_float()
        _check(lib().tg_step(self._h, n, names, ptrs, sizes, ctypes.byref(loss)))
        return float(loss.value)

    def step_device(self, names: Sequence[str], dev_ptrs: Sequence[int], nbytes: Sequence[int]) -> float:
        loss = ctypes.c_float()
        ptrs = (ctypes.c_void_p * len(names))(*dev_ptrs)
        sizes = (ctypes.c_int64 * len(names))(*nbytes)
        _check(lib().tg_step_device(self._h, len(names), _names(names), ptrs, sizes, ctypes.byref(loss)))
        return float(loss.value)

    def step_noalloc(self, names: Sequence[str], dev_ptrs: Sequence[int], nbytes: Sequence[int]) -> float:
        """tg_step_noalloc: tg_step_device with the step's scratch in the static device array."""
        loss = ctypes.c_float()
        ptrs = (ctypes.c_void_p * len(names))(*dev_ptrs)
        sizes = (ctypes.c_int64 * len(names))(*nbytes)
        _check(lib().tg_step_noalloc(self._h, len(names), _names(names), ptrs, sizes, ctypes.byref(loss)))
        return float(loss.value)

    def stage_batch(self, slot: int, inputs: Dict[str, np.ndarray]) -> None:
        n, names, ptrs, sizes, keep = _inputs(inputs)
        _check(lib().tg_stage_batch(self._h, slot, n, names, ptrs, sizes))

    def step_staged(self, slot: int) -> float:
        loss = ctypes.c_float()
        _check(lib().tg_step_staged(self._h, slot, ctypes.byref(loss)))
        return float(loss.value)

    def run(self, inputs: Dict[str, np.ndarray], out_shape, out_dtype) -> np.ndarray:
        n, names, ptrs, sizes, keep = _inputs(inputs)
        out = np.empty(out_shape, out_dtype)
        _check(lib().tg_run(self._h, n, names, ptrs, sizes, out.ctypes.data, out.nbytes))
        return out

    def state_names(self) -> List[str]:
        L = lib()
        return [L.tg_state_name(self._h, i).decode() for i in range(L.tg_state_count(self._h))]

    def download_state(self):
        """({state name: values}, optimizer step t, PRNG seed counter)."""
        L = lib()
        names = self.state_names()
        arrs = [np.empty(L.tg_state_numel(self._h, i), np.float32) for i in range(len(names))]
        ptrs = (ctypes.c_void_p * len(names))(*[a.ctypes.data for a in arrs])
        sizes = (ctypes.c_int64 * len(names))(*[a.size for a in arrs])
        t, c = ctypes.c_int64(), ctypes.c_int64()
        _check(L.tg_download_state(self._h, len(names), _names(names), ptrs, sizes, ctypes.byref(t), ctypes.byref(c)))
        return dict(zip(names, arrs)), t.value, c.value

    def upload_state(self, state: Dict[str, np.ndarray], t: int, prng_counter: int) -> None:
        names = list(state.keys())
        arrs = [np.ascontiguousarray(state[n], dtype=np.float32).reshape(-1) for n in names]
        ptrs = (ctypes.c_void_p * len(names))(*[a.ctypes.data for a in arrs])
        sizes = (ctypes.c_int64 * len(names))(*[a.size for a in arrs])
        _check(lib().tg_upload_state(self._h, len(names), _names(names), ptrs, sizes, t, prng_counter))

    def save_checkpoint(self, path: str) -> None:
        _check(lib().tg_save_checkpoint(self._h, os.fsencode(path)))

    def load_checkpoint(self, path: str) -> None:
        _check(lib().tg_load_checkpoint(self._h, os.fsencode(path)))

    def capture(self, name: str, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        _check(lib().tg_get_capture(self._h, name.encode(), out.ctypes.data, out.nbytes))
        return out

    def reset_optimizer(self) -> None:
        _check(lib().tg_reset_optimizer(self._h))

    def set_lr(self, lr) -> None:
        _check(lib().tg_set_lr(self._h, json.dumps(lr).encode()))

    def describe(self) -> dict:
        buf = ctypes.create_string_buffer(1 << 24)
        _check(lib().tg_describe(self._h, buf, len(buf)))
        return json.loads(buf.value.decode())

    def profile_nodes(self, iters: int) -> List[float]:
        n = len(self.describe()['nodes'])
        out = (ctypes.c_double * n)()
        _check(lib().tg_profile_nodes(self._h, iters, out, n))
        return list(out)

    def profile_kernels(self, iters: int) -> List[float]:
        """Mean kernel time (ms) of each launch node over `iters` eager steps: the kernels'
        own start-to-end durations, without the gaps between launches."""
        n = len(self.describe()['nodes'])
        out = (ctypes.c_double * n)()
        _check(lib().tg_profile_kernels(self._h, iters, out, n))
        return list(out)

    def time_replays(self, steps: int) -> float:
        ms = ctypes.c_double()
        _check(lib().tg_time_replays(self._h, steps, ctypes.byref(ms)))
        return ms.value

    def time_kinds(self, kinds: str, iters: int):
        """(milliseconds per pass, launches per pass) over the nodes of the listed kinds."""
        ms, n = ctypes.c_double(), ctypes.c_int()
        _check(lib().tg_time_kinds(self._h, kinds.encode(), iters, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value
