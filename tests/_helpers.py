"""Shared test helpers: trace small graphs, evaluate them on the CPU oracle, run the
reference's finite-difference harness (test/_fdgrad.ts) against the oracle."""
from __future__ import annotations

import numpy as np

import pyoracle
from tensorgrad_amd import ir as IR
from tensorgrad_amd.grad import append_grad
from tensorgrad_amd.module import Mulberry32
from tensorgrad_amd.trace import param_input, trace_fn


def rel_err(got, want, what: str = 'value') -> float:
    """Relative error ||got - want|| / ||want|| (L2 over all elements; plain relative error
    for scalars). Raises on any NaN or infinity on either side, so a non-finite GPU result
    can never pass a tolerance check by comparing false."""
    g = np.asarray(got, np.float64).reshape(-1)
    w = np.asarray(want, np.float64).reshape(-1)
    if g.shape != w.shape:
        raise AssertionError(f'{what}: {g.size} elements against {w.size}')
    if not (np.all(np.isfinite(g)) and np.all(np.isfinite(w))):
        raise AssertionError(f'{what}: non-finite values (got {g[~np.isfinite(g)][:4]}, want {w[~np.isfinite(w)][:4]})')
    return float(np.linalg.norm(g - w) / max(np.linalg.norm(w), 1e-30))


def sign_ambiguous(diff, lr: float, steps: int, upd=None) -> np.ndarray:
    """Parameter elements whose difference is that of Adam updates gone opposite ways.

    Adam's first updates are lr * g / (|g| + eps), about lr * sign(g): a gradient entry
    inside the f32 rounding noise of its GEMM can move either way by lr. Such an element
    differs by at least lr/4 (ordinary differences are ~1e-7) and by at most 2.5 * lr *
    steps (two opposite updates of size lr per step, plus slack); a larger difference is
    never excused. Later updates are lrt * m / (sqrt(v) + eps), smaller than lr where the
    element's gradient is mostly noise (m near zero) and the bias correction lrt / lr is
    below 1: given the elements' update sizes `upd` (from the oracle's optimizer state,
    stored in the fixture, never from the runtime under test), the floor is half the
    element's update, kept within [lr/16, lr/4] (lr/16 is still two orders of magnitude
    above rounding-sized differences at every benchmark lr)."""
    a = np.abs(np.asarray(diff, np.float64))
    floor = lr / 4 if upd is None else np.clip(np.asarray(upd, np.float64) / 2, lr / 16, lr / 4)
    return (a >= floor) & (a <= 2.5 * lr * steps)


class HipBuffers:
    """Device copies of host arrays, made through the HIP runtime libtg.so itself links
    (torch ships its own HIP runtime; device pointers are only exchanged within one)."""

    def __init__(self, arrays):
        import ctypes
        from tensorgrad_amd import backend
        backend.lib()                                   # loads /opt/rocm's libamdhip64 first
        self._hip = ctypes.CDLL('libamdhip64.so.7')
        self._hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self._hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self._hip.hipFree.argtypes = [ctypes.c_void_p]
        self.names, self.ptrs, self.nbytes = [], [], []
        for name, a in arrays.items():
            a = np.ascontiguousarray(a)
            p = ctypes.c_void_p()
            if self._hip.hipMalloc(ctypes.byref(p), max(a.nbytes, 4)) != 0:
                raise RuntimeError('hipMalloc failed')
            if self._hip.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) != 0:      # hipMemcpyHostToDevice
                raise RuntimeError('hipMemcpy failed')
            self.names.append(name)
            self.ptrs.append(p.value)
            self.nbytes.append(a.nbytes)

    def free(self):
        for p in self.ptrs:
            self._hip.hipFree(p)
        self.ptrs = []


def make_range(shape) -> np.ndarray:
    """The reference tests' fixture: sin(0.1 i) * 0.5 (test/grad.ts:254-259)."""
    n = int(np.prod(shape)) if len(shape) else 1
    return (np.sin(np.arange(n, dtype=np.float64) * 0.1) * 0.5).astype(np.float32)


def random_buf(n: int, seed: int = 12345) -> np.ndarray:
    """mulberry32 uniform in [-0.5, 0.5) (test/_fdgrad.ts:116-127)."""
    return (Mulberry32(seed).take(n) - 0.5).astype(np.float32)


def wire(graph, param_grads=None, writebacks=None, optimizer=None) -> dict:
    return {'graph': IR.graph_to_wire(graph), 'paramGrads': {k: v.id for k, v in (param_grads or {}).items()},
            'writebacks': writebacks or [], 'optimizer': optimizer}


def oracle_eval(graph, params=None, inputs=None, param_grads=None):
    """Evaluate every op of `graph` on the oracle; returns {tensor id: value}."""
    o = pyoracle.OracleRuntime(wire(graph, param_grads))
    for k, v in (params or {}).items():
        o.set_home(k, v)
    o.retain_all(True)
    o.run(inputs or {})
    out = {}
    for t in graph.tensors:
        try:
            out[t.id] = o.tensor(t.id)
        except RuntimeError:
            pass
    return out


def fd_check(name, shape, build, eps=1e-3, atol=5e-3, rtol=5e-3, extra=None, init=None):
    """assertGradMatchesFD (test/_fdgrad.ts:43-106) on the oracle."""
    extra = extra or {}
    size = int(np.prod(shape))
    p0 = random_buf(size) if init is None else np.array(init, np.float32).reshape(-1)
    g = trace_fn(lambda: build(param_input('w', list(shape))))
    gr = append_grad(g)
    vals = oracle_eval(g, {'w': p0}, extra, gr.param_grads)
    auto = vals[gr.param_grads['w'].id].reshape(-1).astype(np.float64)
    fg = trace_fn(lambda: build(param_input('w', list(shape))))
    o = pyoracle.OracleRuntime(wire(fg))
    fd = np.zeros(size)
    for i in range(size):
        p = p0.copy()
        p[i] = np.float32(p0[i] + eps)
        o.set_home('w', p)
        o.run(extra)
        lp = float(o.output().reshape(-1)[0])
        p[i] = np.float32(p0[i] - eps)
        o.set_home('w', p)
        o.run(extra)
        lm = float(o.output().reshape(-1)[0])
        fd[i] = (lp - lm) / (2 * eps)
    err = np.abs(auto - fd)
    rel = err / np.maximum(np.abs(fd), 1e-6)
    worst = int(np.argmax(err))
    assert not (err[worst] > atol and rel.max() > rtol), \
        f'{name}: autograd={auto[worst]} fd={fd[worst]} |d|={err[worst]:.2e} rel={rel.max():.2e}'
    return float(err.max())
