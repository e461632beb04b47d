"""Model fingerprint of a safetensors checkpoint — test infrastructure only (the checker).

Restates src/core/protocol/model_identity.cc:124-148 over the tensors in header order, as the
reference loader keeps them (loader/safetensors.cc:430-482: F32 and BF16 tensors only,
``__metadata__`` skipped, names cut to 127 bytes).  The byte hash is the published XXH64
(model_identity.cc:54-101 is XXH64), taken here from the independent ``xxhash`` package; only
the composition of the per-tensor values is restated.
"""

from __future__ import annotations

import json
import struct

import xxhash

_M = (1 << 64) - 1
P1 = 0x9E3779B185EBCA87
P2 = 0xC2B2AE3D27D4EB4F
P3 = 0x165667B19E3779F9
P4 = 0x85EBCA77C2B2AE63
P5 = 0x27D4EB2F165667C5


def _rotl(v: int, r: int) -> int:
    return ((v << r) | (v >> (64 - r))) & _M


def _round0(lane: int) -> int:
    return (_rotl((lane * P2) & _M, 31) * P1) & _M


def _combine(acc: int, value: int) -> int:
    # model_identity.cc:98-102
    return (_rotl(acc ^ _round0(value & _M), 27) * P1 + P4) & _M


def _avalanche(h: int) -> int:
    h ^= h >> 33
    h = (h * P2) & _M
    h ^= h >> 29
    h = (h * P3) & _M
    return h ^ (h >> 32)


def tensors_in_order(path: str):
    """(name, dtype_code, shape, raw bytes) of the F32/BF16 tensors in header order."""
    with open(path, "rb") as f:
        raw = f.read()
    (n,) = struct.unpack("<Q", raw[:8])
    header = json.loads(raw[8:8 + n])
    base = 8 + n
    out = []
    for name, entry in header.items():
        if name == "__metadata__" or entry["dtype"] not in ("F32", "BF16"):
            continue
        a, b = entry["data_offsets"]
        out.append((name, 1 if entry["dtype"] == "BF16" else 0, list(entry["shape"]),
                    raw[base + a:base + b]))
    return out


def fingerprint(path: str) -> str:
    tensors = tensors_in_order(path)
    first = _combine(0x243F6A8885A308D3, len(tensors))
    second = _combine(0x13198A2E03707344, len(tensors))
    for name, dtype, shape, data in tensors:
        name_hash = xxhash.xxh64_intdigest(name.encode()[:127], seed=P3)
        first = _combine(first, name_hash)
        second = _combine(second, _rotl(name_hash, 17))
        fmt = dtype | (len(shape) << 8)
        first = _combine(first, fmt)
        second = _combine(second, fmt ^ len(data))
        for s in shape:
            first = _combine(first, s)
            second = _combine(second, _rotl(s, 23))
        content = xxhash.xxh64_intdigest(data, seed=P5)
        first = _combine(first, content)
        second = _combine(second, _rotl(content, 31) ^ len(data))
    lo, hi = _avalanche(first), _avalanche(second)
    return (lo.to_bytes(8, "little") + hi.to_bytes(8, "little")).hex()
