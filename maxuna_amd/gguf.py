"""Quantised weight containers in raw GGUF layout, resident in HBM.

`ExpertStack` mirrors the reference's `ExpertStack` (src/gguf.rs:247-276): the
stacked `[n_expert, n_out, k]` expert tensor kept in its quantised GGUF block
layout, whose device buffer the kernels index by expert id.  `base_off` is the
byte offset of the first block inside the buffer (gguf.rs:264-270).  A shared
expert / plain linear is an ExpertStack with n_expert == 1 (the reference's
`QLinear`, gguf.rs:207-242).
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum

import torch

import ctypes as C

from ._lib import ExpertStackC, GgufTensorC


class GgmlDType(IntEnum):
    """GGML type ids (the subset this path has kernels for)."""

    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14

    @property
    def block_size(self) -> int:
        return 32 if self is GgmlDType.Q8_0 else 256

    @property
    def type_size(self) -> int:
        return {GgmlDType.Q8_0: 34, GgmlDType.Q4_K: 144, GgmlDType.Q5_K: 176, GgmlDType.Q6_K: 210}[self]


def row_bytes(dtype: GgmlDType, k: int) -> int:
    if k % dtype.block_size:
        raise ValueError(f"k ({k}) is not a multiple of {dtype.name} block size {dtype.block_size}")
    return k // dtype.block_size * dtype.type_size


@dataclass
class ExpertStack:
    """Raw GGUF blocks of `[n_expert, n_out, k]` in a device uint8 buffer."""

    buffer: torch.Tensor  # uint8, on the GPU
    dtype: GgmlDType
    n_expert: int
    n_out: int
    k: int
    base_off: int = 0

    @property
    def row_bytes(self) -> int:
        return row_bytes(self.dtype, self.k)

    @property
    def expert_bytes(self) -> int:
        return self.n_out * self.row_bytes

    @property
    def nbytes(self) -> int:
        return self.n_expert * self.expert_bytes

    def to_c(self) -> ExpertStackC:
        return ExpertStackC(self.buffer.data_ptr(), self.base_off, int(self.dtype), 0,
                            self.n_expert, self.n_out, self.k)

    @staticmethod
    def empty(dtype: GgmlDType, n_expert: int, n_out: int, k: int, device="cuda") -> "ExpertStack":
        nbytes = n_expert * n_out * row_bytes(dtype, k)
        return ExpertStack(torch.empty(nbytes, dtype=torch.uint8, device=device), dtype, n_expert,
                           n_out, k)

    def expert_view(self, e: int) -> torch.Tensor:
        """The raw bytes of expert e (a view)."""
        o = self.base_off + e * self.expert_bytes
        return self.buffer[o:o + self.expert_bytes]


def null_stack() -> ExpertStackC:
    return ExpertStackC(None, 0, 0, 0, 0, 0, 0)


# ---- GGUF files ---------------------------------------------------------------------
# value types of the GGUF metadata (public GGUF layout)
GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL = range(8)
GGUF_STRING, GGUF_ARRAY, GGUF_U64, GGUF_I64, GGUF_F64 = 8, 9, 10, 11, 12
GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30


@dataclass
class GgufTensor:
    """One entry of a GGUF tensor table.  `shape` is in the candle/PyTorch order
    (outermost first), i.e. reversed ggml `ne`: an expert stack is
    (n_expert, n_out, k)."""

    name: str
    ggml_type: int
    shape: tuple
    offset: int  # absolute file offset
    nbytes: int
    _c: object = None


class GgufFile:
    """A GGUF v2/v3 file opened by the native reader (mx_gguf_*).  Mirrors what
    the reference host reads through candle's gguf_file::Content
    (src/gguf.rs:554-687, config.rs:115-130)."""

    def __init__(self, path):
        from ._lib import check, lib
        self.path = str(path)
        self._h = C.c_void_p()
        check(lib().mx_gguf_open(self.path.encode(), C.byref(self._h)))
        n = lib().mx_gguf_tensor_count(self._h)
        self.tensors: dict[str, GgufTensor] = {}
        for i in range(n):
            t = GgufTensorC()
            check(lib().mx_gguf_tensor_at(self._h, i, C.byref(t)))
            shape = tuple(int(t.ne[d]) for d in range(t.n_dims))[::-1]
            name = t.name.decode()
            self.tensors[name] = GgufTensor(name, t.ggml_type, shape, int(t.offset), int(t.nbytes), t)

    def close(self):
        if self._h:
            from ._lib import lib
            lib().mx_gguf_close(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def version(self) -> int:
        from ._lib import lib
        return int(lib().mx_gguf_version(self._h))

    @property
    def alignment(self) -> int:
        from ._lib import lib
        return int(lib().mx_gguf_alignment(self._h))

    def has(self, key: str) -> bool:
        from ._lib import lib
        return lib().mx_gguf_kv_type(self._h, key.encode()) >= 0

    def get_int(self, key: str, default=None):
        from ._lib import check, lib
        if default is not None and not self.has(key):
            return default
        v = C.c_int64()
        check(lib().mx_gguf_get_int(self._h, key.encode(), C.byref(v)))
        return int(v.value)

    def get_float(self, key: str, default=None):
        from ._lib import check, lib
        if default is not None and not self.has(key):
            return default
        v = C.c_double()
        check(lib().mx_gguf_get_float(self._h, key.encode(), C.byref(v)))
        return float(v.value)

    def get_bool(self, key: str, default=None):
        return bool(self.get_int(key, None if default is None else int(default)))

    def get_str(self, key: str, default=None):
        from ._lib import check, lib
        if default is not None and not self.has(key):
            return default
        v = C.c_char_p()
        check(lib().mx_gguf_get_string(self._h, key.encode(), C.byref(v)))
        return v.value.decode()

    def array_info(self, key: str):
        """(element type, count) of an array-valued key."""
        from ._lib import check, lib
        et, cnt = C.c_int32(), C.c_uint64()
        check(lib().mx_gguf_get_array(self._h, key.encode(), C.byref(et), C.byref(cnt)))
        return int(et.value), int(cnt.value)

    def tensor(self, name: str) -> GgufTensor:
        t = self.tensors.get(name)
        if t is None:
            from ._lib import MaxunaError
            raise MaxunaError(13, f"tensor {name} not found")
        return t

    def read_host(self, name: str):
        """The raw bytes of a tensor as a numpy uint8 array."""
        import numpy as np
        from ._lib import check, lib
        t = self.tensor(name)
        buf = np.empty(t.nbytes, dtype=np.uint8)
        check(lib().mx_gguf_read_host(self._h, C.byref(t._c), buf.ctypes.data, buf.nbytes))
        return buf

    def read_device(self, name: str, device="cuda", align: int = 256) -> torch.Tensor:
        """The raw bytes of a tensor uploaded into a fresh device buffer (pinned,
        double-buffered file read + DMA, mx_gguf_read)."""
        from ._lib import check, lib
        from .ops import _stream
        t = self.tensor(name)
        buf = torch.empty(max(t.nbytes, 1), dtype=torch.uint8, device=device)
        if buf.data_ptr() % align:
            raise RuntimeError("device allocation is not aligned")
        check(lib().mx_gguf_read(self._h, C.byref(t._c), buf.data_ptr(), buf.numel(), _stream()))
        return buf

    def dense_f32(self, name: str, device="cuda") -> torch.Tensor:
        """A small dense tensor as f32 on the device (F32 / F16 / BF16), shaped as
        stored; the reference's `dense_f32` (gguf.rs)."""
        import numpy as np
        t = self.tensor(name)
        raw = self.read_host(name)
        if t.ggml_type == GGML_F32:
            arr = raw.view(np.float32)
        elif t.ggml_type == GGML_F16:
            arr = raw.view(np.float16).astype(np.float32)
        elif t.ggml_type == GGML_BF16:
            arr = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        else:
            from ._lib import MaxunaError
            raise MaxunaError(3, f"{name}: ggml type {t.ggml_type} is not a dense float type")
        return torch.from_numpy(arr.reshape(t.shape).copy()).to(device)

    def expert_stack(self, name: str, device="cuda") -> ExpertStack:
        """A rank-3 [n_expert, n_out, k] (or rank-2 [n_out, k] -> n_expert 1)
        quantised tensor in HBM (gguf.rs:554-658)."""
        from ._lib import MaxunaError
        t = self.tensor(name)
        try:
            dt = GgmlDType(t.ggml_type)
        except ValueError:
            raise MaxunaError(3, f"{name}: no expert kernels for ggml type {t.ggml_type}") from None
        if len(t.shape) == 3:
            n_expert, n_out, k = t.shape
        elif len(t.shape) == 2:
            n_expert, (n_out, k) = 1, t.shape
        else:
            raise MaxunaError(2, f"{name} is not a rank-3 expert stack: {list(t.shape)}")
        return ExpertStack(self.read_device(name, device), dt, n_expert, n_out, k)


def _gguf_value(kind: int, v) -> bytes:
    import struct
    fmt = {GGUF_U8: "<B", GGUF_I8: "<b", GGUF_U16: "<H", GGUF_I16: "<h", GGUF_U32: "<I", GGUF_I32: "<i",
           GGUF_F32: "<f", GGUF_BOOL: "<?", GGUF_U64: "<Q", GGUF_I64: "<q", GGUF_F64: "<d"}
    if kind == GGUF_STRING:
        b = v.encode()
        return struct.pack("<Q", len(b)) + b
    if kind == GGUF_ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_gguf_value(et, x) for x in items)
    return struct.pack(fmt[kind], v)


def write_gguf(path, metadata: dict, tensors: list, version: int = 3, alignment: int = 32) -> None:
    """Writes a GGUF file (public layout).  metadata: {key: (gguf value type,
    value)} (arrays: (GGUF_ARRAY, (element type, [values]))); tensors: a list of
    (name, ggml_type, shape in candle order (outermost first), raw bytes)."""
    import struct
    meta = dict(metadata)
    if alignment != 32:
        meta["general.alignment"] = (GGUF_U32, alignment)
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, (kind, v) in meta.items():
        kb = key.encode()
        head += struct.pack("<Q", len(kb)) + kb + struct.pack("<I", kind) + _gguf_value(kind, v)
    offsets, off = [], 0
    for _, _, _, raw in tensors:
        offsets.append(off)
        off = (off + len(raw) + alignment - 1) // alignment * alignment
    for (name, gt, shape, _), o in zip(tensors, offsets):
        nb = name.encode()
        ne = list(shape)[::-1]
        head += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(ne))
        head += b"".join(struct.pack("<Q", d) for d in ne) + struct.pack("<IQ", gt, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (_, _, _, raw), o in zip(tensors, offsets):
            data = bytes(raw)
            f.write(data)
            f.write(b"\0" * ((-len(data)) % alignment))
