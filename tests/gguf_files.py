"""Writes GGUF files for the tests, byte by byte from the format's layout (ggml's docs/gguf.md):
the reader (leat_amd/gguf.py) is checked against files whose every byte the test places."""

import struct

import numpy as np

STRING, ARRAY = 8, 9
# metadata value types of Python values: u32 for ints, f32 for floats
_KINDS = {bool: (7, "?"), int: (4, "I"), float: (6, "f")}


def _text(s: str) -> bytes:
    raw = s.encode()
    return struct.pack("<Q", len(raw)) + raw


def _value(v) -> tuple[int, bytes]:
    if isinstance(v, str):
        return STRING, _text(v)
    if isinstance(v, list):
        kind, _ = _value(v[0])
        body = b"".join(_value(x)[1] for x in v)
        return ARRAY, struct.pack("<IQ", kind, len(v)) + body
    kind, fmt = _KINDS[type(v)]
    return kind, struct.pack("<" + fmt, v)


def gguf_bytes(metadata: dict, tensors: list[tuple[str, int, tuple[int, ...], bytes]], alignment: int = 32,
               version: int = 3) -> bytes:  # fmt: skip
    """A GGUF file: metadata {key: value}; tensors (name, ggml type, row-major shape, data bytes),
    each placed at the next multiple of `alignment` of the data section."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, v in metadata.items():
        kind, body = _value(v)
        head += _text(key) + struct.pack("<I", kind) + body
    offset, blobs = 0, []
    for name, ggml_type, shape, data in tensors:
        offset = -(-offset // alignment) * alignment
        dims = tuple(reversed(shape))
        head += _text(name) + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
        head += struct.pack("<IQ", ggml_type, offset)
        blobs.append((offset, data))
        offset += len(data)
    start = -(-len(head) // alignment) * alignment
    body = bytearray(offset)
    for at, data in blobs:
        body[at : at + len(data)] = data
    return head + bytes(start - len(head)) + bytes(body)


def f32_bytes(values) -> bytes:
    return np.asarray(values, np.float32).tobytes()
