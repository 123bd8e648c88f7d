"""safetensors I/O for parameters: `load_safetensors` with the reference loader's
semantics (src/safetensors.ts:49-103) and a writer.

The container is indexed by the native library (`tg_safetensors_index`, host-only, no
device needed), which applies the reference's checks: F32 tensors load, integer / bool
tensors (e.g. BatchNorm's `num_batches_tracked`) are skipped and reported, other float
dtypes are refused, and truncated buffers, out-of-range offsets and byte lengths that
disagree with the shape are errors. Runtime checkpoints (params + optimizer state) are
written and read natively: `CompiledTraining.save_checkpoint` / `load_checkpoint`.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from . import backend


@dataclass
class SafetensorsData:
    tensors: Dict[str, np.ndarray] = field(default_factory=dict)   # F32 name -> flat values
    shapes: Dict[str, List[int]] = field(default_factory=dict)     # every tensor, skipped ones too
    skipped: Dict[str, str] = field(default_factory=dict)          # name -> integer / bool dtype
    metadata: Dict[str, str] = field(default_factory=dict)


def load_safetensors(buf) -> SafetensorsData:
    """Parse a safetensors container into flat float32 arrays ready for `upload_params`.
    Raises `backend.BackendError` on a malformed container or a non-F32 float tensor."""
    data = bytes(buf)
    ix = backend.safetensors_index(data)
    out = SafetensorsData(metadata=dict(ix['metadata']))
    start = ix['dataStart']
    for e in ix['tensors']:
        out.shapes[e['name']] = list(e['shape'])
        # a copy: the blob need not be 4-byte aligned, and the result must not alias `buf`
        out.tensors[e['name']] = np.frombuffer(data[start + e['begin']:start + e['end']], dtype='<f4').copy()
    for e in ix['skipped']:
        out.shapes[e['name']] = list(e['shape'])
        out.skipped[e['name']] = e['dtype']
    return out


def save_safetensors(tensors: Dict[str, np.ndarray], metadata: Optional[Dict[str, str]] = None,
                     shapes: Optional[Dict[str, List[int]]] = None) -> bytes:
    """Write float32 tensors (in the given order) as a safetensors container. `shapes`
    overrides the arrays' own shapes (e.g. for flat arrays from `download_params`)."""
    header = {}
    if metadata:
        header['__metadata__'] = {str(k): str(v) for k, v in metadata.items()}
    blobs, off = [], 0
    for name, a in tensors.items():
        arr = np.ascontiguousarray(a, dtype='<f4')
        shape = list(shapes[name]) if shapes and name in shapes else list(arr.shape)
        if int(np.prod(shape)) != arr.size:
            raise ValueError(f"save_safetensors: '{name}' has {arr.size} elements, shape {shape}")
        header[name] = {'dtype': 'F32', 'shape': shape, 'data_offsets': [off, off + arr.nbytes]}
        blobs.append(arr.tobytes())
        off += arr.nbytes
    h = json.dumps(header, separators=(',', ':')).encode()
    h += b' ' * ((-(8 + len(h))) % 8)
    return len(h).to_bytes(8, 'little') + h + b''.join(blobs)
