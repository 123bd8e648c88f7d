"""Static shape inference (reference `src/shape.ts`). Trailing-suffix broadcasting only
(shape.ts:44-58); one rule per op kind; `ShapeError` names the op that raised it."""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

Shape = Tuple[int, ...]


class ShapeError(ValueError):
    """Raised when an op's shape constraints are violated (shape.ts:13-19)."""

    def __init__(self, message: str, site: Optional[str] = None):
        super().__init__(f'{message}\n  at [{site}]' if site else message)
        self.site = site


def fail(message: str, site: Optional[str]):
    raise ShapeError(message, site)


def shapes_equal(a: Sequence[int], b: Sequence[int]) -> bool:
    return tuple(a) == tuple(b)


def shape_size(shape: Sequence[int]) -> int:
    n = 1
    for d in shape:
        n *= d
    return n


def show(shape: Sequence[int]) -> str:
    return '[' + ', '.join(str(d) for d in shape) + ']'


def broadcast_trailing(a: Sequence[int], b: Sequence[int]) -> Optional[Shape]:
    rank = max(len(a), len(b))
    out = []
    for i in range(rank):
        ai = i - (rank - len(a))
        bi = i - (rank - len(b))
        av = 1 if ai < 0 else a[ai]
        bv = 1 if bi < 0 else b[bi]
        if av == bv:
            out.append(av)
        elif av == 1:
            out.append(bv)
        elif bv == 1:
            out.append(av)
        else:
            return None
    return tuple(out)


def infer_elementwise_binop(name, a, b, site) -> Shape:
    r = broadcast_trailing(a, b)
    if r is None:
        fail(f'{name}: incompatible shapes {show(a)} and {show(b)}. Trailing-suffix broadcasting only '
             f'— the smaller shape must be a suffix of the larger, with size-1 axes broadcasting to any size.',
             site)
    return r


def infer_mean_last(name, a, site) -> Shape:
    if len(a) == 0:
        fail(f'{name}: cannot reduce a 0-d tensor', site)
    return tuple(a[:-1]) + (1,)


def infer_sum_last(name, a, site) -> Shape:
    if len(a) == 0:
        fail(f'{name}: cannot reduce a 0-d tensor', site)
    return tuple(a[:-1])


def infer_reshape(name, a, new_shape, site) -> Shape:
    infer_idx = -1
    known = 1
    for i, d in enumerate(new_shape):
        if d == -1:
            if infer_idx != -1:
                fail(f'{name}: at most one -1 dim allowed in newShape {show(new_shape)}', site)
            infer_idx = i
        elif d <= 0:
            fail(f'{name}: invalid dim {d} in newShape {show(new_shape)}', site)
        else:
            known *= d
    total = shape_size(a)
    out = list(new_shape)
    if infer_idx != -1:
        if total % known != 0:
            fail(f'{name}: cannot reshape {show(a)} (size {total}) to {show(new_shape)} — known dims multiply to {known}', site)
        out[infer_idx] = total // known
    elif known != total:
        fail(f'{name}: size mismatch — input {show(a)} has {total} elements but newShape {show(new_shape)} has {known}', site)
    return tuple(out)


def infer_permute(name, a, perm, site) -> Shape:
    if len(perm) != len(a):
        fail(f'{name}: perm length {len(perm)} must equal input rank {len(a)}', site)
    seen = set()
    for p in perm:
        if p < 0 or p >= len(a):
            fail(f'{name}: perm index {p} out of range for rank {len(a)}', site)
        if p in seen:
            fail(f'{name}: perm has duplicate index {p}', site)
        seen.add(p)
    return tuple(a[p] for p in perm)


def infer_matmul(name, a, b, site) -> Shape:
    if len(a) < 2:
        fail(f'{name}: lhs must have rank >= 2, got {show(a)}', site)
    if len(b) != 2:
        fail(f'{name}: internal: inferMatmul expects rank-2 rhs, got {show(b)}', site)
    M, Ka, Kb, N = a[-2], a[-1], b[0], b[1]
    if Ka != Kb:
        fail(f"{name}: inner dims don't match — {show(a)} · {show(b)} (last axis of lhs = {Ka}, first axis of rhs = {Kb})", site)
    return tuple(a[:-2]) + (M, N)


def infer_matmul_batched(name, a, b, site) -> Shape:
    if len(a) < 2 or len(b) < 2:
        fail(f'{name}: both inputs must have rank >= 2, got {show(a)} and {show(b)}', site)
    if len(a) != len(b):
        fail(f'{name}: ranks must match (got {len(a)} vs {len(b)}). Reshape if you need different batch dims.', site)
    if tuple(a[:-2]) != tuple(b[:-2]):
        fail(f'{name}: batch dims must match — {show(a)} vs {show(b)}', site)
    if a[-1] != b[-2]:
        fail(f"{name}: inner dims don't match — last axis of lhs = {a[-1]}, second-to-last of rhs = {b[-2]}", site)
    return tuple(a[:-2]) + (a[-2], b[-1])


def infer_one_hot(name, idx, depth, site) -> Shape:
    if depth <= 0:
        fail(f'{name}: depth must be positive, got {depth}', site)
    return tuple(idx) + (depth,)


def infer_where_causal(name, a, site) -> Shape:
    if len(a) < 2:
        fail(f'{name}: requires rank >= 2, got {show(a)}', site)
    if a[-2] != a[-1]:
        fail(f'{name}: last two axes must be equal (square mask), got {show(a)}', site)
    return tuple(a)


def infer_slice_range(name, a, axis, start, end, site) -> Shape:
    if len(a) == 0:
        fail(f'{name}: cannot slice 0-d tensor', site)
    if axis < 0 or axis >= len(a):
        fail(f'{name}: axis {axis} out of range for shape {show(a)}', site)
    dim = a[axis]
    if start < 0 or end > dim or start >= end:
        fail(f'{name}: invalid range [{start}, {end}) for axis {axis} of size {dim}', site)
    out = list(a)
    out[axis] = end - start
    return tuple(out)


def infer_scatter_axis(name, a, out_shape, axis, start, end, site) -> Shape:
    if len(out_shape) == 0:
        fail(f'{name}: cannot scatter into 0-d tensor', site)
    if axis < 0 or axis >= len(out_shape):
        fail(f'{name}: axis {axis} out of range for output shape {show(out_shape)}', site)
    dim = out_shape[axis]
    if start < 0 or end > dim or start >= end:
        fail(f'{name}: invalid range [{start}, {end}) for axis {axis} of size {dim}', site)
    if len(a) != len(out_shape):
        fail(f'{name}: input rank {len(a)} must equal output rank {len(out_shape)}', site)
    for i in range(len(out_shape)):
        expected = end - start if i == axis else out_shape[i]
        if a[i] != expected:
            fail(f"{name}: input {show(a)} doesn't match output {show(out_shape)} at axis {i} (expected {expected})", site)
    return tuple(out_shape)


def infer_concat(name, shapes, axis, site) -> Shape:
    if len(shapes) == 0:
        fail(f'{name}: needs at least one input', site)
    first = shapes[0]
    if axis < 0 or axis >= len(first):
        fail(f'{name}: axis {axis} out of range for shape {show(first)}', site)
    total = first[axis]
    for i in range(1, len(shapes)):
        s = shapes[i]
        if len(s) != len(first):
            fail(f'{name}: input {i} has rank {len(s)}, expected {len(first)}', site)
        for d in range(len(first)):
            if d != axis and s[d] != first[d]:
                fail(f'{name}: input {i} has shape {show(s)}, must match {show(first)} except along axis {axis}', site)
        total += s[axis]
    out = list(first)
    out[axis] = total
    return tuple(out)


def infer_broadcast_to(name, a, target, site) -> Shape:
    if len(a) > len(target):
        fail(f'{name}: source rank {len(a)} > target rank {len(target)}', site)
    off = len(target) - len(a)
    for i, av in enumerate(a):
        tv = target[off + i]
        if av != tv and av != 1:
            fail(f"{name}: cannot broadcast {show(a)} to {show(target)} — axis {i} (size {av}) doesn't match "
                 f"target axis {off + i} (size {tv}) and isn't 1", site)
    return tuple(target)


def infer_sum_to_shape(name, a, target, site) -> Shape:
    if len(target) > len(a):
        fail(f'{name}: target rank {len(target)} > source rank {len(a)}', site)
    off = len(a) - len(target)
    for i, tv in enumerate(target):
        av = a[off + i]
        if av != tv and tv != 1:
            fail(f'{name}: cannot sum-reduce {show(a)} to {show(target)} — target axis {i} (size {tv}) must be 1 or match source', site)
    return tuple(target)


def infer_where(name, c, a, b, site) -> Shape:
    ab = broadcast_trailing(a, b)
    if ab is None:
        fail(f'{name}: a/b incompatible: {show(a)} vs {show(b)}', site)
    r = broadcast_trailing(c, ab)
    if r is None:
        fail(f'{name}: cond {show(c)} incompatible with broadcast(a, b) {show(ab)}', site)
    return r


def infer_relu_grad(name, x, dy, site) -> Shape:
    if tuple(x) != tuple(dy):
        fail(f'{name}: x and dy must have matching shapes, got {show(x)} and {show(dy)}', site)
    return tuple(x)


def conv_out(name, in_size, kernel, stride, pad, axis_name, site) -> int:
    """PyTorch convention `floor((in + 2*pad - kernel) / stride) + 1` (shape.ts:306-317)."""
    if kernel < 1:
        fail(f'{name}: {axis_name} kernel must be >= 1, got {kernel}', site)
    if stride < 1:
        fail(f'{name}: {axis_name} stride must be >= 1, got {stride}', site)
    if pad < 0:
        fail(f'{name}: {axis_name} padding must be >= 0, got {pad}', site)
    out = (in_size + 2 * pad - kernel) // stride + 1
    if out < 1:
        fail(f'{name}: {axis_name} output size would be {out} (in={in_size}, kernel={kernel}, stride={stride}, pad={pad})', site)
    return out


def infer_conv2d(name, x, w, sH, sW, pH, pW, groups, site) -> Shape:
    if len(x) != 4:
        fail(f'{name}: input must be rank-4 [B, C_in, H, W], got {show(x)}', site)
    if len(w) != 4:
        fail(f'{name}: weight must be rank-4 [C_out, C_in/groups, K_h, K_w], got {show(w)}', site)
    if not isinstance(groups, int) or groups < 1:
        fail(f'{name}: groups must be a positive integer, got {groups}', site)
    B, cIn, H, W = x
    cOut, wInC, kH, kW = w
    if cIn % groups != 0:
        fail(f'{name}: input C_in={cIn} is not divisible by groups={groups}', site)
    if cOut % groups != 0:
        fail(f'{name}: weight C_out={cOut} is not divisible by groups={groups}', site)
    if wInC * groups != cIn:
        fail(f"{name}: weight's C_in/groups={wInC} (x groups={groups} = {wInC * groups}) doesn't match input C_in={cIn}", site)
    hOut = conv_out(name, H, kH, sH, pH, 'H', site)
    wOut = conv_out(name, W, kW, sW, pW, 'W', site)
    return (B, cOut, hOut, wOut)


def infer_max_pool2d(name, x, kH, kW, sH, sW, pH, pW, site) -> Shape:
    if len(x) != 4:
        fail(f'{name}: input must be rank-4 [B, C, H, W], got {show(x)}', site)
    B, C, H, W = x
    return (B, C, conv_out(name, H, kH, sH, pH, 'H', site), conv_out(name, W, kW, sW, pW, 'W', site))
