"""GGUF reader for the sparse-conv weights of SAM 3D Objects checkpoints.

The reference loads its converted checkpoints through ggml's GGUF reader
(cpp_ggml/src/gguf_loader.cpp:66-120, ggml v0.21.0, not in the reference
tree).  This module reads the same files with numpy over a read-only memory
map (no copy until a tensor is used), following the published GGUF layout
(versions 2 and 3, little endian):

    magic "GGUF" | u32 version | u64 n_tensors | u64 n_kv
    n_kv x (string key, u32 type, value)
    n_tensors x (string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset)
    padding to general.alignment (default 32) | tensor data (offsets relative)

Strings are (u64 length, bytes).  ne[0] is the fastest-varying dimension,
so a tensor with ne = (a, b) is the row-major array [b, a].

`load_sparse_conv` attaches a conv tensor pair to a `SparseConv3d` in the
layouts the converter writes:
  "slat"  ne = (27*Cin, Cout): rows [Cout, 27*Cin]  (gguf_schema.py:330-338;
          SLAT flow blocks, `<block>.conv1.conv.weight`, slat_flow_graph.cpp:344)
  "mesh"  ne = (Cout*Cin, 27): rows [27, Cout*Cin]  (convert_sam3d_to_gguf.py:
          508-511; mesh decoder `<name>.out_layers.0.conv.weight`,
          mesh_decoder_graph.cpp:290-347)
  1x1x1   ne = (Cout*Cin, 1): the checkpoint buffer in saved order; the conv
          applies the spconv raw view W[co][ci] = buf[ci*Cout + co]
          (mesh_decoder_graph.cpp:349-384), as SparseConv3d(k=1) does for its
          own parameter.
F32 / F16 / BF16 tensors become the module's parameters; Q8_0 tensors
(34-byte blocks along ne[0]) are attached as blocks (`load_q8_0`), which the
bf16 path dequantises inside the GEMM.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass
from typing import Any, Dict, Optional

import numpy as np

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# metadata value types
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {
    _U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f",
    _BOOL: "<?", _U64: "<Q", _I64: "<q", _F64: "<d",
}

# ggml tensor types this reader exposes: type -> (name, block elements, block bytes)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_BF16 = 0, 1, 2, 8, 30
_TYPES = {
    GGML_F32: ("F32", 1, 4),
    GGML_F16: ("F16", 1, 2),
    GGML_Q4_0: ("Q4_0", 32, 18),
    GGML_Q8_0: ("Q8_0", 32, 34),
    GGML_BF16: ("BF16", 1, 2),
}


@dataclass(frozen=True)
class TensorInfo:
    name: str
    ne: tuple           # ggml dimensions, fastest first
    ggml_type: int
    offset: int         # absolute byte offset in the file
    nbytes: int

    @property
    def shape(self) -> tuple:
        """Row-major shape (slowest first)."""
        return tuple(reversed(self.ne))

    @property
    def type_name(self) -> str:
        return _TYPES[self.ggml_type][0] if self.ggml_type in _TYPES else f"type{self.ggml_type}"

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.ne:
            n *= d
        return n


class GGUFError(ValueError):
    pass


class GGUFReader:
    """Parses a GGUF file's metadata and tensor table; tensor data are numpy
    views of a read-only memory map."""

    def __init__(self, path: str):
        self.path = os.fspath(path)
        with open(self.path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            if size < 24:
                raise GGUFError(f"{self.path}: too small for a GGUF header")
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self._buf = memoryview(self._mm)
        self._pos = 0
        if bytes(self._buf[:4]) != GGUF_MAGIC:
            raise GGUFError(f"{self.path}: bad magic {bytes(self._buf[:4])!r}")
        self._pos = 4
        self.version = self._scalar(_U32)
        if self.version not in (2, 3):
            raise GGUFError(f"{self.path}: GGUF version {self.version} is not supported (2 or 3)")
        n_tensors = self._scalar(_U64)
        n_kv = self._scalar(_U64)
        self.kv: Dict[str, Any] = {}
        for _ in range(n_kv):
            key = self._string()
            vtype = self._scalar(_U32)
            self.kv[key] = self._value(vtype)
        infos = []
        for _ in range(n_tensors):
            name = self._string()
            n_dims = self._scalar(_U32)
            if n_dims > 4:
                raise GGUFError(f"{self.path}: tensor {name} has {n_dims} dimensions")
            ne = tuple(self._scalar(_U64) for _ in range(n_dims))
            gtype = self._scalar(_U32)
            off = self._scalar(_U64)
            infos.append((name, ne, gtype, off))
        align = int(self.kv.get("general.alignment", DEFAULT_ALIGNMENT))
        if align <= 0 or align & (align - 1):
            raise GGUFError(f"{self.path}: bad alignment {align}")
        self.alignment = align
        self.data_offset = (self._pos + align - 1) // align * align
        self.tensors: Dict[str, TensorInfo] = {}
        for name, ne, gtype, off in infos:
            if gtype in _TYPES:
                _, be, bb = _TYPES[gtype]
                n = 1
                for d in ne:
                    n *= d
                if ne and ne[0] % be:
                    raise GGUFError(f"{self.path}: tensor {name}: ne[0]={ne[0]} not a multiple of {be}")
                nbytes = n // be * bb
            else:
                nbytes = -1  # unknown type: listed, not readable
            start = self.data_offset + off
            if nbytes >= 0 and start + nbytes > size:
                raise GGUFError(f"{self.path}: tensor {name} runs past the end of the file")
            if name in self.tensors:
                raise GGUFError(f"{self.path}: duplicate tensor {name}")
            self.tensors[name] = TensorInfo(name, ne, gtype, start, nbytes)

    # ---- parsing helpers --------------------------------------------------
    def _take(self, n: int) -> memoryview:
        if self._pos + n > len(self._buf):
            raise GGUFError(f"{self.path}: truncated header")
        v = self._buf[self._pos:self._pos + n]
        self._pos += n
        return v

    def _scalar(self, vtype: int):
        fmt = _SCALAR[vtype]
        return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]

    def _string(self) -> str:
        n = self._scalar(_U64)
        return bytes(self._take(n)).decode("utf-8")

    def _value(self, vtype: int):
        if vtype in _SCALAR:
            return self._scalar(vtype)
        if vtype == _STR:
            return self._string()
        if vtype == _ARR:
            etype = self._scalar(_U32)
            n = self._scalar(_U64)
            return [self._value(etype) for _ in range(n)]
        raise GGUFError(f"{self.path}: unknown metadata type {vtype}")

    # ---- tensors ----------------------------------------------------------
    def __contains__(self, name: str) -> bool:
        return name in self.tensors

    def info(self, name: str) -> TensorInfo:
        try:
            return self.tensors[name]
        except KeyError:
            raise KeyError(f"{self.path}: no tensor {name!r}") from None

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes (uint8, a view of the mapping)."""
        t = self.info(name)
        if t.nbytes < 0:
            raise GGUFError(f"{self.path}: tensor {name} has unsupported type {t.ggml_type}")
        return np.frombuffer(self._mm, dtype=np.uint8, count=t.nbytes, offset=t.offset)

    def array(self, name: str) -> np.ndarray:
        """F32 / F16 tensors as float32 / float16 arrays in row-major shape,
        BF16 as uint16 bit patterns, block-quantized types as raw blocks
        [n_blocks, block_bytes] (uint8)."""
        t = self.info(name)
        raw = self.raw(name)
        if t.ggml_type == GGML_F32:
            return raw.view("<f4").reshape(t.shape)
        if t.ggml_type == GGML_F16:
            return raw.view("<f2").reshape(t.shape)
        if t.ggml_type == GGML_BF16:
            return raw.view("<u2").reshape(t.shape)
        _, be, bb = _TYPES[t.ggml_type]
        return raw.reshape(-1, bb)

    def close(self) -> None:
        """Releases the mapping; arrays still referring to it keep it alive
        until they are gone."""
        self._buf.release()
        try:
            self._mm.close()
        except BufferError:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _float_tensor(reader: GGUFReader, name: str):
    """F32 / F16 / BF16 tensor -> float32 torch tensor (CPU), flat."""
    import torch

    t = reader.info(name)
    a = reader.array(name)
    if t.ggml_type == GGML_BF16:
        return torch.from_numpy(a.astype(np.int32) << 16).view(torch.float32).reshape(-1).clone()
    if t.ggml_type in (GGML_F32, GGML_F16):
        return torch.from_numpy(np.array(a, dtype=np.float32)).reshape(-1)
    raise GGUFError(f"{reader.path}: tensor {name} is {t.type_name}, expected F32/F16/BF16")


def load_sparse_conv(module, reader: GGUFReader, name: str, layout: Optional[str] = None) -> None:
    """Loads `<name>.weight` (and `<name>.bias` when present) into a
    `SparseConv3d` / `SparseInverseConv3d`.  `layout` is "slat" (rows
    [Cout, taps*Cin]) or "mesh" (rows [taps, Cout*Cin]); None infers it from
    the tensor's shape (ne[1] == taps with taps > 1 means "mesh").  A 1x1x1
    conv's tensor is the checkpoint buffer in saved order either way."""
    import torch

    conv = module.conv
    cin, cout, taps = conv.in_channels, conv.out_channels, module._ntaps
    wname, bname = name + ".weight", name + ".bias"
    t = reader.info(wname)
    if t.n_elements != taps * cin * cout:
        raise GGUFError(f"{wname}: {t.n_elements} weights, the conv has {taps}x{cin}x{cout}")
    if layout is None:
        layout = "mesh" if taps > 1 and len(t.ne) == 2 and t.ne[1] == taps else "slat"
    if layout not in ("slat", "mesh"):
        raise ValueError("layout must be 'slat' or 'mesh'")
    expect = {"slat": (taps * cin, cout), "mesh": (cout * cin, taps)}[layout]
    if taps == 1:
        expect = (cout * cin, 1)
    if tuple(t.ne) != expect and not (taps == 1 and tuple(t.ne) in ((cin, cout), (cout * cin,))):
        raise GGUFError(f"{wname}: ggml ne {t.ne} does not match the {layout} layout {expect}")
    with torch.no_grad():
        if t.ggml_type == GGML_Q8_0:
            if taps == 1 and getattr(module, "_raw_view", False):
                # the raw-view transpose spans block boundaries: dequantise
                # once, as the reference does before its transpose
                blocks = torch.from_numpy(np.array(reader.raw(wname)))
                w = _dequant_q8_0_cpu(blocks)
                conv.weight.copy_(w.reshape(conv.weight.shape).to(conv.weight.dtype))
            else:
                module.load_q8_0(torch.from_numpy(np.array(reader.raw(wname))),
                                 layout="slat" if taps == 1 else layout)
        else:
            w = _float_tensor(reader, wname)
            if layout == "mesh" and taps > 1:
                # rows [taps, Cout, Cin] -> KRSC [Cout, taps, Cin]
                w = w.reshape(taps, cout, cin).permute(1, 0, 2)
            conv.weight.copy_(w.reshape(conv.weight.shape).to(conv.weight.dtype))
            module._q8 = None
        if bname in reader:
            b = _float_tensor(reader, bname)
            if b.numel() != cout:
                raise GGUFError(f"{bname}: {b.numel()} values, the conv has {cout} outputs")
            if conv.bias is None:
                raise GGUFError(f"{bname}: the conv was built without a bias")
            conv.bias.copy_(b.to(conv.bias.dtype))


def _dequant_q8_0_cpu(blocks):
    """f32(d) * q of ggml Q8_0 blocks (CPU, exact in F32)."""
    import torch

    b = blocks.reshape(-1, 34)
    d = b[:, :2].contiguous().view(torch.float16).float()
    q = b[:, 2:].contiguous().view(torch.int8).float()
    return (d * q).reshape(-1)
