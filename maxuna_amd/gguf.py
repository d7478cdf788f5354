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

from ._lib import ExpertStackC


class GgmlDType(IntEnum):
    """GGML type ids (the subset this path has kernels for)."""

    Q8_0 = 8
    Q4_K = 12
    Q6_K = 14

    @property
    def block_size(self) -> int:
        return 32 if self is GgmlDType.Q8_0 else 256

    @property
    def type_size(self) -> int:
        return {GgmlDType.Q8_0: 34, GgmlDType.Q4_K: 144, GgmlDType.Q6_K: 210}[self]


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
