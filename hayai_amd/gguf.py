"""GGUF model files on the host side of the FFN path.

`GgufCatalog` binds the library's catalog (hh_gguf_*, include/hayai_hip.h), which mirrors
the reference's GgufCatalog (crates/hayai-model/src/gguf_stream.rs:34-192) and
load_layer_pack_into (:451-638): open parses the header and tensor directory, `layer_pack`
gives the LayerPackLayout of a layer, `load_layer_pack` reads the layer's tensors into a
host buffer (a numpy array or a pinned streaming slot) in one batch of io_uring reads.

`write_gguf` writes GGUF v3 files (typed metadata, raw tensor payloads in any GGML type):
the counterpart of the reference's write_minimal_gguf (gguf.rs:683-735), extended to
quantized tensors so tests and benchmarks can build model files without a download.
"""
from __future__ import annotations

import ctypes as C
import os
import struct
from dataclasses import dataclass

import numpy as np

from . import _abi
from .engine import HipError, _check

GGUF_MAGIC = 0x46554747

# metadata value types (gguf.rs:633-676)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)

SLOTS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down", "attn_gate")


@dataclass
class TensorInfo:
    name: str
    dims: tuple
    type: int
    offset: int       # relative to the data section
    abs_offset: int   # in the file
    nbytes: int

    @property
    def ncols(self) -> int:
        return self.dims[0] if self.dims else 1

    @property
    def nrows(self) -> int:
        return self.dims[1] if len(self.dims) >= 2 else 1


@dataclass
class LayerPack:
    """LayerPackLayout (gguf_stream.rs:1416-1432) with each region's shape and type; slots
    in pack order (SLOTS)."""
    off: tuple
    len: tuple
    type: tuple
    cols: tuple
    rows: tuple
    total: int
    fused_gate_up: bool

    def region(self, slot: str) -> tuple[int, int]:
        i = SLOTS.index(slot)
        return self.off[i], self.len[i]

    @property
    def gate_off(self) -> int:
        return self.off[4]

    @property
    def up_off(self) -> int:
        return self.off[5]

    @property
    def down_off(self) -> int:
        return self.off[6]

    def ffn_layout(self):
        """The FFN part as the engine's LayerPackLayout (offsets inside this pack)."""
        from .engine import LayerPackLayout
        return LayerPackLayout(self.off[4], self.off[5], self.off[6], self.len[4], self.len[5], self.len[6],
                               self.total)


def _pack(lp: _abi.LayerPack) -> LayerPack:
    return LayerPack(tuple(lp.off), tuple(lp.len), tuple(lp.type), tuple(lp.cols), tuple(lp.rows), lp.total,
                     bool(lp.fused_gate_up))


def tensor_nbytes(ggml_type: int, dims) -> int:
    """tensor_nbytes (gguf.rs:240-284)."""
    lib = _abi.load()
    d = (C.c_uint64 * max(1, len(dims)))(*[int(v) for v in dims])
    out = C.c_uint64()
    _check(lib.hh_tensor_nbytes(ggml_type, d, len(dims), C.byref(out)))
    return out.value


class GgufCatalog:
    """An open GGUF file (header + tensor directory in memory, payloads read on demand)."""

    def __init__(self, path: str):
        self.lib = _abi.load()
        h = C.c_void_p()
        _check(self.lib.hh_gguf_open(os.fsencode(path), C.byref(h)))
        self.handle = h
        self.path = path
        info = _abi.GgufInfo()
        _check(self.lib.hh_gguf_header(self.handle, C.byref(info)))
        self.version = info.version
        self.io_uring = bool(info.io_uring)
        self.o_direct = bool(info.o_direct)
        self.alignment = info.alignment
        self.data_offset = info.data_offset
        self.header_bytes = info.header_bytes
        self.n_tensors = info.n_tensors
        self.n_metadata = info.n_metadata
        self.file_size = info.file_size

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.hh_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def _info(t: _abi.GgufTensor) -> TensorInfo:
        return TensorInfo(t.name.decode("utf-8", "replace"), tuple(t.dims[: t.n_dims]), t.type, t.offset,
                          t.abs_offset, t.nbytes)

    def tensors(self) -> list[TensorInfo]:
        out = []
        for i in range(self.n_tensors):
            t = _abi.GgufTensor()
            _check(self.lib.hh_gguf_tensor_at(self.handle, i, C.byref(t)))
            out.append(self._info(t))
        return out

    def tensor(self, name: str) -> TensorInfo:
        t = _abi.GgufTensor()
        _check(self.lib.hh_gguf_find(self.handle, name.encode(), C.byref(t)))
        return self._info(t)

    def _meta(self, fn, key, ctype):
        v = ctype()
        st = fn(self.handle, key.encode(), C.byref(v))
        if st == 8:  # HH_ERR_NOT_FOUND: absent or another type (the reference's None)
            return None
        _check(st)
        return v.value

    def meta_u32(self, key: str):
        return self._meta(self.lib.hh_gguf_meta_u32, key, C.c_uint32)

    def meta_u64(self, key: str):
        return self._meta(self.lib.hh_gguf_meta_u64, key, C.c_uint64)

    def meta_f32(self, key: str):
        return self._meta(self.lib.hh_gguf_meta_f32, key, C.c_float)

    def meta_str(self, key: str):
        p, n = C.c_char_p(), C.c_size_t()
        st = self.lib.hh_gguf_meta_str(self.handle, key.encode(), C.byref(p), C.byref(n))
        if st == 8:
            return None
        _check(st)
        return C.string_at(p, n.value).decode("utf-8", "replace")

    def layer_pack(self, layer: int) -> LayerPack:
        lp = _abi.LayerPack()
        _check(self.lib.hh_gguf_layer_pack(self.handle, layer, C.byref(lp)))
        return _pack(lp)

    def load_layer_pack(self, layer: int, dst: np.ndarray) -> LayerPack:
        """load_layer_pack_into: the layer's tensors into dst (a writable uint8 host array,
        e.g. a pinned slot's host_view()) at the returned layout's offsets."""
        if not (isinstance(dst, np.ndarray) and dst.flags.c_contiguous and dst.flags.writeable):
            raise HipError(2, "dst must be a writable contiguous numpy array")
        lp = _abi.LayerPack()
        _check(self.lib.hh_gguf_load_layer_pack(self.handle, layer, dst.ctypes.data_as(C.c_void_p), dst.nbytes,
                                                C.byref(lp)))
        return _pack(lp)

    def read_tensor(self, name: str, dst: np.ndarray | None = None) -> np.ndarray:
        """read_tensor_into: the tensor's bytes (into dst when given)."""
        if dst is None:
            dst = np.empty(self.tensor(name).nbytes, np.uint8)
        _check(self.lib.hh_gguf_read_tensor(self.handle, name.encode(), dst.ctypes.data_as(C.c_void_p), dst.nbytes))
        return dst


# ---------------------------------------------------------------------- writer -------

def _enc_string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}


def _enc_value(ty: int, v) -> bytes:
    if ty == STRING:
        return _enc_string(v)
    if ty == ARRAY:
        elem_ty, items = v
        return struct.pack("<IQ", elem_ty, len(items)) + b"".join(_enc_value(elem_ty, x) for x in items)
    return struct.pack(_SCALAR[ty], int(v) if ty != F32 and ty != F64 else float(v))


def _typed(v):
    if isinstance(v, tuple) and len(v) == 2 and isinstance(v[0], int) and not isinstance(v[0], bool):
        return v  # (type, value)
    if isinstance(v, bool):
        return BOOL, v
    if isinstance(v, int):
        return (U32, v) if 0 <= v < 2**32 else (I64 if v < 0 else U64, v)
    if isinstance(v, float):
        return F32, v
    if isinstance(v, str):
        return STRING, v
    raise TypeError(f"metadata value {v!r}: pass (type, value)")


def write_gguf(path: str, metadata, tensors, alignment: int = 32, version: int = 3) -> list[int]:
    """Write a GGUF file.  metadata: iterable of (key, value) where value is a str / int /
    float / bool or an explicit (type, value) pair (arrays: (ARRAY, (elem_type, items)));
    tensors: iterable of (name, dims, ggml_type, payload bytes), dims ne0 first.  Payloads
    are placed in order, each on an `alignment` boundary of the data section; a
    general.alignment key is written when alignment is not 32.  Returns the payloads'
    offsets within the data section."""
    meta = list(metadata)
    if alignment != 32 and not any(k == "general.alignment" for k, _ in meta):
        meta.append(("general.alignment", (U32, alignment)))
    tensors = [(n, d, t, p.tobytes() if isinstance(p, np.ndarray) else bytes(p)) for n, d, t, p in tensors]
    head = struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(meta))
    for k, v in meta:
        ty, val = _typed(v)
        head += _enc_string(k) + struct.pack("<I", ty) + _enc_value(ty, val)
    offsets, off = [], 0
    for _, _, _, payload in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += len(payload)
    for (name, dims, ty, _), o in zip(tensors, offsets):
        head += _enc_string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", int(d)) for d in dims)
        head += struct.pack("<IQ", ty, o)
    with open(path, "wb") as f:
        f.write(head)
        pos = len(head)
        pad = (-pos) % alignment
        f.write(b"\0" * pad)
        data_pos = 0
        for (_, _, _, payload), o in zip(tensors, offsets):
            f.write(b"\0" * (o - data_pos))
            f.write(payload)
            data_pos = o + len(payload)
    return offsets
