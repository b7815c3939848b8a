"""npu_memref descriptors built from torch tensors (device memory plumbing only)."""
from __future__ import annotations

import ctypes as C

from ._lib import NpuMemref

F32, BF16, I8, I32 = 0, 1, 2, 3

_DTYPE_CODES = None


def _codes():
    global _DTYPE_CODES
    if _DTYPE_CODES is None:
        import torch
        _DTYPE_CODES = {torch.float32: F32, torch.bfloat16: BF16, torch.int8: I8,
                        torch.int32: I32}
    return _DTYPE_CODES


def from_tensor(t) -> NpuMemref:
    """Descriptor of a torch tensor: the storage pointer, its offset and strides."""
    code = _codes().get(t.dtype)
    if code is None:
        raise TypeError(f"unsupported tensor dtype {t.dtype}")
    if t.dim() > 4:
        raise ValueError("npu_memref holds at most rank 4")
    m = NpuMemref()
    base = t.untyped_storage().data_ptr()
    m.allocated = base
    m.aligned = base
    m.offset = t.storage_offset()
    for i, (s, st) in enumerate(zip(t.shape, t.stride())):
        m.sizes[i] = s
        m.strides[i] = st
    m.rank = t.dim()
    m.dtype = code
    return m


def absent() -> NpuMemref:
    """An optional operand that is not present (null data pointer)."""
    m = NpuMemref()
    m.rank = 1
    return m


def ref(m: NpuMemref):
    return C.byref(m)
