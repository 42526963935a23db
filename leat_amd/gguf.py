"""GGUF files (leat/gguf.py:64-140): the metadata, the tensor index, and the tensors' data copied
to the GPU in one transfer as QTensors that view it, blocks exactly as stored.

Layout (ggml's docs/gguf.md, versions 2 and 3, little-endian): "GGUF", u32 version, u64 tensor
count, u64 metadata count; metadata entries (string key, u32 value type, value); tensor infos
(string name, u32 dimension count, u64 dimensions innermost first, u32 ggml type, u64 offset
into the data section); the data section at the next multiple of general.alignment (32 by
default). Strings are a u64 length and UTF-8 bytes; arrays a u32 element type, a u64 count and
the elements.
"""

from __future__ import annotations

import math
import mmap
import struct
from collections.abc import Iterable
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np
import torch

from leat_amd.quant import BLOCK, NATIVE, GGMLType, QTensor

# metadata value types: struct formats of the scalars; 8 a string, 9 an array
SCALAR_FORMATS = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
STRING, ARRAY = 8, 9
DEFAULT_ALIGNMENT = 32


@dataclass(frozen=True)
class TensorInfo:
    """A tensor of the index: its row-major shape (GGUF lists dimensions innermost first), and
    where its bytes lie in the file."""

    name: str
    type: GGMLType
    shape: tuple[int, ...]
    offset: int  # absolute byte offset in the file
    nbytes: int


class _Cursor:
    # reads little-endian values from a buffer, front to back
    def __init__(self, buf: memoryview):
        self.buf, self.at = buf, 0

    def take(self, fmt: str) -> Any:
        (value,) = struct.unpack_from("<" + fmt, self.buf, self.at)
        self.at += struct.calcsize("<" + fmt)
        return value

    def text(self) -> str:
        n = self.take("Q")
        raw = self.buf[self.at : self.at + n]
        if len(raw) != n:
            raise ValueError("GGUF: a string runs past the end of the file")
        self.at += n
        # bytes that are not UTF-8 on their own (a token's piece of a character) are replaced
        return str(raw, "utf-8", errors="replace")

    def value(self, kind: int) -> Any:
        if kind == STRING:
            return self.text()
        if kind == ARRAY:
            element, count = self.take("I"), self.take("Q")
            if element in SCALAR_FORMATS:
                fmt = f"<{count}{SCALAR_FORMATS[element]}"
                values = list(struct.unpack_from(fmt, self.buf, self.at))
                self.at += struct.calcsize(fmt)
                return values
            return [self.value(element) for _ in range(count)]
        if kind not in SCALAR_FORMATS:
            raise ValueError(f"GGUF: unknown metadata value type {kind}")
        return self.take(SCALAR_FORMATS[kind])


def parse(buf: memoryview) -> tuple[dict[str, Any], dict[str, TensorInfo]]:
    """The metadata and tensor index of a GGUF file's bytes."""
    if bytes(buf[:4]) != b"GGUF":
        raise ValueError("not a GGUF file")
    cur = _Cursor(buf)
    cur.at = 4
    version = cur.take("I")
    if version not in (2, 3):
        raise ValueError(f"unsupported GGUF version {version}")
    n_tensors, n_meta = cur.take("Q"), cur.take("Q")
    metadata = {}
    for _ in range(n_meta):
        key = cur.text()
        metadata[key] = cur.value(cur.take("I"))
    entries = []
    for _ in range(n_tensors):
        name = cur.text()
        dims = [cur.take("Q") for _ in range(cur.take("I"))]
        entries.append((name, dims, cur.take("I"), cur.take("Q")))
    alignment = metadata.get("general.alignment", DEFAULT_ALIGNMENT)
    if alignment <= 0 or alignment & (alignment - 1):
        raise ValueError(f"GGUF: alignment {alignment} is not a power of 2")
    data_start = -(-cur.at // alignment) * alignment
    tensors = {}
    for name, dims, type_id, offset in entries:
        try:
            ggml_type = GGMLType(type_id)
        except ValueError:
            raise ValueError(f"GGUF: tensor {name!r} has unknown ggml type {type_id}") from None
        elements, size = BLOCK[ggml_type]
        if dims and dims[0] % elements:  # blocks run along a row
            raise ValueError(f"GGUF: tensor {name!r} has rows of {dims[0]}, not whole blocks of {elements}")
        nbytes = math.prod(dims) // elements * size
        tensors[name] = TensorInfo(name, ggml_type, tuple(reversed(dims)), data_start + offset, nbytes)
    return metadata, tensors


@dataclass(frozen=True)
class GGUF:
    """An opened GGUF file: its metadata and tensor index; `load` copies tensor data to the GPU."""

    path: Path
    metadata: dict[str, Any]
    tensors: dict[str, TensorInfo]

    @staticmethod
    def open(path: str | Path) -> GGUF:
        path = Path(path)
        with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            with memoryview(mm) as buf:
                metadata, tensors = parse(buf)
            size = len(mm)
        for t in tensors.values():
            if t.offset + t.nbytes > size:
                raise ValueError(f"{path}: truncated: tensor {t.name!r} ends past the end of the file")
        return GGUF(path, metadata, tensors)

    def load(self, device="cuda", names: Iterable[str] | None = None) -> dict[str, QTensor]:
        """The named tensors (all by default) as QTensors on `device`: the file span holding them
        is copied in one transfer, and each tensor views its bytes there (block types as
        (blocks, bytes) uint8, F32/F16/BF16 as their values)."""
        infos = list(self.tensors.values()) if names is None else [self.tensors[n] for n in names]
        if not infos:
            return {}
        start = min(t.offset for t in infos)
        end = max(t.offset + t.nbytes for t in infos)
        span = np.memmap(self.path, dtype=np.uint8, mode="r", offset=start, shape=(end - start,))
        if torch.device(device).type == "cuda":  # through a pinned staging buffer: one DMA transfer
            staging = torch.empty(end - start, dtype=torch.uint8, pin_memory=True)
            np.copyto(staging.numpy(), span)
            data = staging.to(device, non_blocking=True)
        else:
            data = torch.from_numpy(np.array(span))
        out = {}
        for t in infos:
            raw = data[t.offset - start : t.offset - start + t.nbytes]
            if t.type in NATIVE:
                out[t.name] = QTensor(raw.view(NATIVE[t.type]), t.type, t.shape)
            else:
                out[t.name] = QTensor(raw.view(-1, BLOCK[t.type][1]), t.type, t.shape)
        if data.is_cuda:
            torch.cuda.current_stream(data.device).synchronize()
        return out
