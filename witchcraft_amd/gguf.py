"""Minimal GGUF v3 writer/reader for the encoder's tensors (F32, F16, Q4_K).

The container the reference loads with candle's `VarBuilder::from_gguf_buffer`
(src/quantized_t5.rs:740-743) and writes with `gguf_file::write` and no metadata
(tools/quantize-tool/src/main.rs:33-35).  Dims are stored innermost first; tensor data
is aligned to 32 bytes (GGUF default `general.alignment`).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

GGML_F32 = 0
GGML_F16 = 1
GGML_Q4_K = 12
ALIGN = 32


@dataclass
class Tensor:
    name: str
    ggml_type: int
    shape: tuple  # outermost first, e.g. (N, K) for a weight W[N, K]
    data: bytes


def _nbytes(ggml_type: int, shape) -> int:
    ne = int(np.prod(shape))
    if ggml_type == GGML_F32:
        return ne * 4
    if ggml_type == GGML_F16:
        return ne * 2
    if ggml_type == GGML_Q4_K:
        return ne // 256 * 144
    raise ValueError(f"unsupported GGML type {ggml_type}")


def write_gguf(tensors: list[Tensor]) -> bytes:
    head = bytearray()
    head += b"GGUF" + struct.pack("<IQQ", 3, len(tensors), 0)
    offset = 0
    offsets = []
    for t in tensors:
        nb = _nbytes(t.ggml_type, t.shape)
        if len(t.data) != nb:
            raise ValueError(f"{t.name}: {len(t.data)} bytes, expected {nb}")
        name = t.name.encode()
        head += struct.pack("<Q", len(name)) + name
        head += struct.pack("<I", len(t.shape))
        for d in reversed(t.shape):
            head += struct.pack("<Q", d)
        head += struct.pack("<IQ", t.ggml_type, offset)
        offsets.append(offset)
        offset = (offset + nb + ALIGN - 1) // ALIGN * ALIGN
    data0 = (len(head) + ALIGN - 1) // ALIGN * ALIGN
    out = bytearray(data0 + offset)
    out[: len(head)] = head
    for t, off in zip(tensors, offsets):
        out[data0 + off: data0 + off + len(t.data)] = t.data
    return bytes(out)


def read_gguf(buf: bytes) -> dict[str, Tensor]:
    mv = memoryview(buf)
    if bytes(mv[:4]) != b"GGUF":
        raise ValueError("bad GGUF magic")
    version, nt, nkv = struct.unpack_from("<IQQ", mv, 4)
    pos = 24
    if nkv:
        raise ValueError("metadata key/values are not supported by this reader")
    infos = []
    for _ in range(nt):
        (ln,) = struct.unpack_from("<Q", mv, pos)
        pos += 8
        name = bytes(mv[pos: pos + ln]).decode()
        pos += ln
        (nd,) = struct.unpack_from("<I", mv, pos)
        pos += 4
        dims = struct.unpack_from(f"<{nd}Q", mv, pos)
        pos += 8 * nd
        ty, off = struct.unpack_from("<IQ", mv, pos)
        pos += 12
        infos.append((name, tuple(reversed(dims)), ty, off))
    data0 = (pos + ALIGN - 1) // ALIGN * ALIGN
    out = {}
    for name, shape, ty, off in infos:
        nb = _nbytes(ty, shape)
        out[name] = Tensor(name, ty, shape, bytes(mv[data0 + off: data0 + off + nb]))
    return out
