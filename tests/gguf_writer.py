"""Minimal GGUF v3 writer for tests (the published layout: header, metadata,
tensor table, aligned data).  Test infrastructure only."""
import struct

import numpy as np

_TYPES = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7,
          "str": 8, "arr": 9, "u64": 10, "i64": 11, "f64": 12}
_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
        11: "<q", 12: "<d"}
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q8_0": 8, "BF16": 30}


def _str(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _val(vtype, v):
    t = _TYPES[vtype] if isinstance(vtype, str) else vtype
    if t == 8:
        return _str(v)
    if t == 9:
        etype, items = v
        et = _TYPES[etype]
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def write_gguf(path, kv, tensors, alignment=None, version=3, magic=b"GGUF"):
    """kv: list of (key, type name, value) -- arrays as ("arr", (elem type, items));
    tensors: list of (name, ggml type name, ne tuple (fastest first), bytes)."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kv) + (alignment is not None))
    meta = b""
    if alignment is not None:
        meta += _str("general.alignment") + struct.pack("<I", 4) + struct.pack("<I", alignment)
    for key, vtype, v in kv:
        meta += _str(key) + struct.pack("<I", _TYPES[vtype]) + _val(vtype, v)
    align = alignment or 32
    infos, data, off = b"", b"", 0
    for name, tname, ne, payload in tensors:
        infos += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        infos += struct.pack("<IQ", GGML[tname], off)
        data += payload
        off += len(payload)
        pad = (-off) % align
        data += b"\0" * pad
        off += pad
    body = head + meta + infos
    body += b"\0" * ((-len(body)) % align)
    with open(path, "wb") as f:
        f.write(body + data)


def f32_bytes(a):
    return np.ascontiguousarray(a, dtype="<f4").tobytes()


def f16_bytes(a):
    return np.ascontiguousarray(a, dtype="<f2").tobytes()


def bf16_bytes(a):
    """Round-to-nearest-even float32 -> bf16 bit patterns."""
    u = np.ascontiguousarray(a, dtype="<f4").view("<u4").astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype("<u2")
    return r.tobytes()
