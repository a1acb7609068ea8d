"""Mirror of Inferno.jl's ``GGUF`` module (src/GGUF.jl) on the library's
native reader (inferno.jl_amd/csrc/gguf.hip).

``read_gguf(path)`` parses the header and tensor infos of a memory-mapped
GGUF file (src/GGUF.jl:119-165); ``get_tensor_raw_bytes(file, name)`` returns
a tensor's bytes (src/GGUF.jl:186-205, sized by the tensor's block type: the
reference returns 4 bytes per element for every type); ``upload(file, name)``
puts a Q4_K / Q5_K / Q6_K / Q8_0 tensor into the device weight registry, as
the keep-quantized load of src/LoaderCPU.jl:125-163 keeps it quantized, and
returns the registry handle.  Missing tensors raise like the reference's
``error("Tensor not found: $name")``.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import check, lib


@dataclass
class TensorInfo:
    name: str
    dimensions: tuple        # ne0 first, as in the file
    type: int                # GGML type id (src/GGUF.jl:25-60)
    offset: int              # relative to the data section
    nbytes: int              # 0 when the type's block size is unknown


@dataclass
class GGUFFile:
    handle: int
    version: int
    alignment: int
    data_offset: int
    tensors: dict = field(default_factory=dict)

    def close(self) -> None:
        if self.handle:
            check(lib().ihip_gguf_close(self.handle))
            self.handle = 0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def read_gguf(path) -> GGUFFile:
    h = C.c_uint64(0)
    check(lib().ihip_gguf_open(str(path).encode(), C.byref(h)))
    ver, al, off, n = C.c_uint32(0), C.c_uint64(0), C.c_uint64(0), C.c_int64(0)
    check(lib().ihip_gguf_info(h, C.byref(ver), C.byref(al), C.byref(off), C.byref(n)))
    f = GGUFFile(h.value, ver.value, al.value, off.value)
    name = C.create_string_buffer(1 << 16)
    t, nd, o, nb = C.c_int(0), C.c_int(0), C.c_uint64(0), C.c_uint64(0)
    dims = (C.c_int64 * 4)()
    for i in range(n.value):
        check(lib().ihip_gguf_tensor_info(h, i, name, len(name), C.byref(t), C.byref(nd), dims,
                                          C.byref(o), C.byref(nb)))
        nm = name.value.decode()
        f.tensors[nm] = TensorInfo(nm, tuple(dims[d] for d in range(nd.value)), t.value, o.value,
                                   nb.value)
    return f


def get_tensor_raw_bytes(file: GGUFFile, name: str) -> np.ndarray:
    info = file.tensors.get(name)
    if info is None:
        raise _lib.IHIPArgumentError(_lib.IHIP_ERR_INVALID, f"Tensor not found: {name}")
    out = np.empty(info.nbytes, np.uint8)
    check(lib().ihip_gguf_tensor_bytes(file.handle, name.encode(), out.ctypes.data, out.size))
    return out


def upload(file: GGUFFile, name: str) -> int:
    """Registry handle of the device copy (release with ihip_weight_release)."""
    h = C.c_uint64(0)
    check(lib().ihip_gguf_upload(file.handle, name.encode(), C.byref(h)))
    return h.value


def upload_group(file: GGUFFile, names) -> int:
    """Registry handle of the named tensors (one type, one ne0) uploaded back
    to back as one weight of their summed rows: one GEMV over it computes
    every member's outputs (ihip_gguf_upload_group)."""
    arr = (C.c_char_p * len(names))(*[n.encode() for n in names])
    h = C.c_uint64(0)
    check(lib().ihip_gguf_upload_group(file.handle, arr, len(names), C.byref(h)))
    return h.value


def device_ptr(handle: int) -> int:
    p = C.c_void_p(0)
    check(lib().ihip_weight_device_ptr(handle, C.byref(p)))
    return p.value
