"""Host-side mirror of the reference's FFN device interface, over the C ABI.

Names and argument meaning follow the reference so parity tests read like its own tests:

* :class:`HipEngine` <- ``OpenClEngine`` (crates/hayai-opencl/src/context.rs:23-69) and its
  GEMV methods (compute.rs:39-461, async_gemv.rs:15-305);
* :class:`PendingGemv` <- ``PendingGemv`` (async_gemv.rs:15-57): ``wait()`` returns the
  outputs, dropping it waits;
* :class:`QuantMatrix` <- ``QuantMatrix`` (crates/hayai-model/src/quant.rs:31-54);
* :class:`LayerPackLayout` <- ``LayerPackLayout`` (crates/hayai-model/src/gguf_stream.rs:1416-1444).

Errors raise :class:`HipError` carrying the ABI status (``HH_ERR_INVALID`` for the
shape/size rejections of compute.rs:912-949, ``HH_ERR_KERNEL_MISSING`` for a GGML type with
no kernel -- never a CPU fallback, orchestrator.rs:403-409).
"""
from __future__ import annotations

import ctypes as C
import weakref
from dataclasses import dataclass

import numpy as np

from . import _abi

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS = 0, 1, 2, 8, 12, 14, 16, 18
ACT_SILU, ACT_GELU_TANH = 0, 1
BUF_DEVICE, BUF_PINNED_HOST = 0, 1
TYPE_NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k", IQ2_XXS: "iq2_xxs",
              IQ3_XXS: "iq3_xxs"}


class HipError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = status
        self.status_name = _abi.STATUS_NAMES.get(status, f"status {status}")
        super().__init__(f"{self.status_name}: {message}")


def _check(st: int) -> None:
    if st != _abi.HH_OK:
        lib = _abi.load()
        raise HipError(st, (lib.hh_last_error() or b"").decode(errors="replace"))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def row_bytes(ggml_type: int, n: int) -> int:
    out = C.c_size_t(0)
    _check(_abi.load().hh_row_bytes(ggml_type, n, C.byref(out)))
    return out.value


def validate_gemv_shape(ggml_type: int, m: int, n: int) -> None:
    _check(_abi.load().hh_validate_gemv_shape(ggml_type, m, n))


def validate_gemv_weights(ggml_type: int, m: int, n: int, weights_len: int) -> None:
    _check(_abi.load().hh_validate_gemv_weights(ggml_type, m, n, weights_len))


def device_count() -> int:
    n = C.c_int(0)
    _check(_abi.load().hh_device_count(C.byref(n)))
    return n.value


class DeviceBuffer:
    """A device (HBM) or pinned-host buffer owned by an engine."""

    def __init__(self, engine: "HipEngine", nbytes: int, kind: int = BUF_DEVICE):
        self.engine = engine
        self.nbytes = int(nbytes)
        self.kind = kind
        h = C.c_void_p()
        _check(engine.lib.hh_buf_alloc(engine.handle, self.nbytes, kind, C.byref(h)))
        self.handle = h
        engine._children.add(self)

    def write(self, data: np.ndarray, offset: int = 0) -> None:
        data = np.ascontiguousarray(data)
        _check(self.engine.lib.hh_buf_write(self.engine.handle, self.handle, offset, _ptr(data), data.nbytes))

    def read(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        _check(self.engine.lib.hh_buf_read(self.engine.handle, self.handle, offset, _ptr(out), out.nbytes))
        return out

    def fill(self, value: int, nbytes: int | None = None, offset: int = 0) -> None:
        n = self.nbytes - offset if nbytes is None else nbytes
        _check(self.engine.lib.hh_buf_fill(self.engine.handle, self.handle, offset, value, n))

    def copy_from(self, src: "DeviceBuffer", nbytes: int, dst_off: int = 0, src_off: int = 0) -> None:
        """Enqueue a buffer-to-buffer copy on the engine's compute stream."""
        _check(self.engine.lib.hh_buf_copy(self.engine.handle, self.handle, dst_off, src.handle, src_off, nbytes))

    def host_view(self) -> np.ndarray:
        """numpy view of a pinned buffer (HH_BUF_PINNED_HOST only)."""
        p = self.engine.lib.hh_buf_host_ptr(self.handle)
        if not p:
            raise HipError(2, "host_view on a device buffer")
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(self.nbytes,))

    def free(self) -> None:
        if self.handle:
            self.engine.lib.hh_buf_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class MirrorView:
    """Non-owning handle of a streamer's device mirror slot (usable wherever a
    DeviceBuffer is: ``handle`` and ``nbytes``); the streamer frees it."""

    def __init__(self, engine: "HipEngine", handle, nbytes: int):
        self.engine, self.handle, self.nbytes, self.kind = engine, handle, nbytes, BUF_DEVICE

    def read(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        _check(self.engine.lib.hh_buf_read(self.engine.handle, self.handle, offset, _ptr(out), out.nbytes))
        return out


class StreamingScratch:
    """Pinned-host ping-pong weight slots + device mirrors: StreamingScratch
    (crates/hayai-opencl/src/hetero_scratch.rs:48-71) on the pinned path."""

    def __init__(self, engine: "HipEngine", layer_bytes: int, k_chunk: int = 1, n_slots: int = 2):
        self.engine = engine
        self.layer_bytes = int(layer_bytes)
        self.block_k = max(1, int(k_chunk))
        self.n_slots = max(2, int(n_slots))
        h = C.c_void_p()
        _check(engine.lib.hh_streamer_create(engine.handle, self.layer_bytes, self.block_k, self.n_slots, C.byref(h)))
        self.handle = h
        engine._children.add(self)

    def slot_for(self, layer: int) -> int:
        out = C.c_size_t(0)
        _check(self.engine.lib.hh_streamer_slot_for(self.handle, layer, C.byref(out)))
        return out.value

    def weight_offset(self, layer: int, tensor_off: int) -> int:
        out = C.c_size_t(0)
        _check(self.engine.lib.hh_streamer_weight_offset(self.handle, layer, tensor_off, C.byref(out)))
        return out.value

    def host_slot(self, layer: int) -> np.ndarray:
        """prepare_host_write + host_slot: writable uint8 view of the layer's pinned region."""
        p = C.c_void_p()
        _check(self.engine.lib.hh_streamer_host_slot(self.handle, layer, C.byref(p)))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(self.layer_bytes,))

    def dma(self, layer: int, off: int = 0, length: int | None = None) -> None:
        """dma_ffn_keep_mapped: async copy of [off, off+length) of the layer into its mirror."""
        n = self.layer_bytes - off if length is None else length
        _check(self.engine.lib.hh_streamer_dma(self.handle, layer, off, n))

    def weight_bind(self, layer: int) -> tuple[MirrorView, int]:
        """(mirror slot, byte offset of the layer in it); compute waits for the slot's DMA."""
        b = C.c_void_p()
        off = C.c_size_t(0)
        _check(self.engine.lib.hh_streamer_bind(self.handle, layer, C.byref(b), C.byref(off)))
        return MirrorView(self.engine, b, self.block_k * self.layer_bytes), off.value

    def free(self) -> None:
        if self.handle:
            self.engine.lib.hh_streamer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PendingGemv:
    """In-flight GEMV; ``wait()`` returns y.  Dropping it waits first (async_gemv.rs:48-57)."""

    def __init__(self, engine: "HipEngine", handle, m: int):
        self.engine, self.handle, self.m = engine, handle, m
        engine._children.add(self)

    def wait(self) -> np.ndarray:
        y = np.empty(self.m, np.float32)
        _check(self.engine.lib.hh_pending_wait(self.handle, _ptr(y), self.m))
        self.close()
        return y

    def close(self) -> None:
        if self.handle:
            self.engine.lib.hh_pending_destroy(self.handle)
            self.handle = None

    free = close

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self, engine: "HipEngine"):
        self.engine = engine
        h = C.c_void_p()
        _check(engine.lib.hh_event_create(engine.handle, C.byref(h)))
        self.handle = h
        engine._children.add(self)

    def record(self) -> None:
        _check(self.engine.lib.hh_event_record(self.engine.handle, self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0)
        _check(self.engine.lib.hh_event_elapsed_ms(self.handle, end.handle, C.byref(ms)))
        return ms.value

    def free(self) -> None:
        if self.handle:
            self.engine.lib.hh_event_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Graph:
    """A captured sequence of enqueue-only calls (HipEngine.capture), replayed by launch()."""

    def __init__(self, engine: "HipEngine", handle: C.c_void_p):
        self.engine = engine
        self.handle = handle
        engine._children.add(self)

    def launch(self) -> None:
        _check(self.engine.lib.hh_graph_launch(self.handle))

    def free(self) -> None:
        if self.handle:
            self.engine.lib.hh_graph_destroy(self.handle)
            self.handle = None

    close = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class QuantMatrix:
    """Weight descriptor (quant.rs:31-54): y[nrows] = W . x[ncols] in GGML layout."""

    name: str
    ncols: int
    nrows: int
    ggml_type: int

    @property
    def row_bytes(self) -> int:
        return row_bytes(self.ggml_type, self.ncols)

    @property
    def nbytes(self) -> int:
        return self.nrows * self.row_bytes


@dataclass
class LayerPackLayout:
    """FFN byte offsets inside a contiguous layer pack (gguf_stream.rs:1416-1444)."""

    gate_off: int
    up_off: int
    down_off: int
    gate_len: int
    up_len: int
    down_len: int
    total: int

    @staticmethod
    def ffn_only(gate: QuantMatrix, up: QuantMatrix, down: QuantMatrix, align: int = 256) -> "LayerPackLayout":
        """Pack [gate, up, down] back to back (pack order, gguf_stream.rs:456-464), each
        region starting on an `align`-byte boundary."""
        def up_to(v):
            return (v + align - 1) // align * align
        g = 0
        u = up_to(g + gate.nbytes)
        d = up_to(u + up.nbytes)
        return LayerPackLayout(g, u, d, gate.nbytes, up.nbytes, down.nbytes, up_to(d + down.nbytes))

    def ffn_region(self, role: int) -> tuple[int, int]:
        r = role % 3
        return [(self.gate_off, self.gate_len), (self.up_off, self.up_len), (self.down_off, self.down_len)][r]


class HipEngine:
    """One MI355X device (OpenClEngine analogue)."""

    def __init__(self, device: int = 0):
        self.lib = _abi.load()
        # buffers, events and pending GEMVs of this engine; freed before the engine
        self._children = weakref.WeakSet()
        h = C.c_void_p()
        _check(self.lib.hh_engine_create(device, C.byref(h)))
        self.handle = h
        info = _abi.DeviceInfo()
        _check(self.lib.hh_engine_info(self.handle, C.byref(info)))
        self.device_info = info

    # ---------------------------------------------------------------- lifetime
    def close(self) -> None:
        if getattr(self, "handle", None):
            for child in list(self._children):
                child.free()
            self.lib.hh_engine_destroy(self.handle)
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

    @property
    def device_name(self) -> str:
        return self.device_info.name.decode()

    @property
    def arch(self) -> str:
        return self.device_info.arch.decode()

    @property
    def ffn_calls(self) -> int:
        return int(self.lib.hh_engine_ffn_calls(self.handle))

    def sync(self) -> None:
        _check(self.lib.hh_engine_sync(self.handle))

    # ---------------------------------------------------------------- buffers
    def alloc(self, nbytes: int, kind: int = BUF_DEVICE) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes, kind)

    def upload(self, data: np.ndarray) -> DeviceBuffer:
        data = np.ascontiguousarray(data)
        b = DeviceBuffer(self, data.nbytes)
        b.write(data)
        return b

    def event(self) -> Event:
        return Event(self)

    # ---------------------------------------------------------------- graphs
    def capture(self, fn) -> Graph:
        """Capture the enqueue-only calls fn() makes on this engine into a replayable graph
        (hh_graph_begin / hh_graph_end); the capture is closed even when fn raises."""
        _check(self.lib.hh_graph_begin(self.handle))
        try:
            fn()
        except BaseException:
            h = C.c_void_p()
            self.lib.hh_graph_end(self.handle, C.byref(h))
            if h:
                self.lib.hh_graph_destroy(h)
            raise
        h = C.c_void_p()
        _check(self.lib.hh_graph_end(self.handle, C.byref(h)))
        return Graph(self, h)

    # ---------------------------------------------------------------- GEMV (compute.rs)
    def ggml_gemv_dispatch(self, ggml_type: int, m: int, n: int, weights: np.ndarray, inp: np.ndarray) -> np.ndarray:
        """compute.rs:281-383: host weights uploaded per call."""
        w = np.ascontiguousarray(weights, dtype=np.uint8)
        x = np.ascontiguousarray(inp, dtype=np.float32)
        if x.size != n:
            raise HipError(2, f"input has {x.size} floats, expected n={n}")
        y = np.empty(m, np.float32)
        _check(self.lib.hh_gemv(self.handle, ggml_type, m, n, _ptr(w), w.nbytes, _ptr(x), _ptr(y)))
        return y

    def ggml_gemv_q4_0(self, m, n, weights, inp):
        return self.ggml_gemv_dispatch(Q4_0, m, n, weights, inp)

    def ggml_gemv_q4_k(self, m, n, weights, inp):
        return self.ggml_gemv_dispatch(Q4_K, m, n, weights, inp)

    def ggml_gemv_iq2_xxs(self, m, n, weights, inp):
        return self.ggml_gemv_dispatch(IQ2_XXS, m, n, weights, inp)

    def ggml_gemv_iq3_xxs(self, m, n, weights, inp):
        return self.ggml_gemv_dispatch(IQ3_XXS, m, n, weights, inp)

    def ggml_gemv_q8_0(self, m, n, weights, inp):
        return self.ggml_gemv_dispatch(Q8_0, m, n, weights, inp)

    def ggml_gemv_q6_k(self, m, n, weights, inp):
        return self.ggml_gemv_dispatch(Q6_K, m, n, weights, inp)

    def ggml_gemv_batched(self, ggml_type: int, m: int, n: int, weights: np.ndarray, inputs: np.ndarray,
                          batch: int) -> np.ndarray:
        """ggml_gemv_batched_q4_k (compute.rs:179-257), any type: inputs = batch*n floats,
        returns batch*m floats (token-major)."""
        w = np.ascontiguousarray(weights, dtype=np.uint8)
        x = np.ascontiguousarray(inputs, dtype=np.float32).reshape(-1)
        if x.size != batch * n:
            raise HipError(2, f"inputs have {x.size} floats, expected batch*n={batch * n}")
        y = np.empty(batch * m, np.float32)
        _check(self.lib.hh_gemv_batched(self.handle, ggml_type, m, n, _ptr(w), w.nbytes, _ptr(x), _ptr(y), batch))
        return y

    def ggml_gemv_batched_q4_k(self, m: int, n: int, weights: np.ndarray, inputs: np.ndarray, batch: int) -> np.ndarray:
        return self.ggml_gemv_batched(Q4_K, m, n, weights, inputs, batch)

    def gemv_batched_dev(self, ggml_type, m, n, w: DeviceBuffer, w_off, x: DeviceBuffer, x_off, batch,
                         y: DeviceBuffer, y_off) -> None:
        _check(self.lib.hh_gemv_batched_dev(self.handle, ggml_type, m, n, w.handle, w_off, x.handle, x_off, batch,
                                            y.handle, y_off))

    def ggml_gemv_dispatch_bound(self, ggml_type: int, m: int, n: int, weights: DeviceBuffer, weight_off: int,
                                 inp: np.ndarray) -> np.ndarray:
        """compute.rs:388-461: resident weights at a byte offset."""
        x = np.ascontiguousarray(inp, dtype=np.float32)
        if x.size != n:
            raise HipError(2, f"input has {x.size} floats, expected n={n}")
        y = np.empty(m, np.float32)
        _check(self.lib.hh_gemv_bound(self.handle, ggml_type, m, n, weights.handle, weight_off, _ptr(x), _ptr(y)))
        return y

    def ggml_gemv_async_from_device(self, ggml_type: int, m: int, n: int, weights: DeviceBuffer, weight_off: int,
                                    inp: np.ndarray) -> PendingGemv:
        """async_gemv.rs:103-121."""
        x = np.ascontiguousarray(inp, dtype=np.float32)
        if x.size != n:
            raise HipError(2, f"input has {x.size} floats, expected n={n}")
        h = C.c_void_p()
        _check(self.lib.hh_gemv_begin(self.handle, ggml_type, m, n, weights.handle, weight_off, _ptr(x), C.byref(h)))
        return PendingGemv(self, h, m)

    def gemv_dev(self, ggml_type, m, n, w: DeviceBuffer, w_off, x: DeviceBuffer, x_off, y: DeviceBuffer, y_off):
        _check(self.lib.hh_gemv_dev(self.handle, ggml_type, m, n, w.handle, w_off, x.handle, x_off, y.handle, y_off))

    def lut_matmul_q4(self, m: int, n: int, weights_q4: np.ndarray, lut, inp: np.ndarray) -> np.ndarray:
        """OpenClEngine::lut_matmul_q4 (compute.rs:45-128): Hayai's 4-bit LUT format, m rows of
        n/2 packed bytes indexing a 16-entry f32 LUT; host arrays, blocking."""
        w = np.ascontiguousarray(weights_q4, dtype=np.uint8)
        t = np.ascontiguousarray(lut, dtype=np.float32)
        x = np.ascontiguousarray(inp, dtype=np.float32)
        if t.size != 16:
            raise HipError(2, f"lut has {t.size} entries, expected 16")
        if x.size != n:
            raise HipError(2, f"input has {x.size} floats, expected n={n}")
        y = np.empty(m, np.float32)
        _check(self.lib.hh_lut_gemv(self.handle, m, n, _ptr(w), w.nbytes, _ptr(t), _ptr(x), _ptr(y)))
        return y

    def lut_gemv_dev(self, m, n, w: DeviceBuffer, w_off, lut: DeviceBuffer, lut_off, x: DeviceBuffer, x_off,
                     y: DeviceBuffer, y_off) -> None:
        _check(self.lib.hh_lut_gemv_dev(self.handle, m, n, w.handle, w_off, lut.handle, lut_off, x.handle, x_off,
                                        y.handle, y_off))

    def dequant_dev(self, ggml_type, w: DeviceBuffer, w_off, n, out: DeviceBuffer, out_off=0):
        _check(self.lib.hh_dequant_dev(self.handle, ggml_type, w.handle, w_off, n, out.handle, out_off))

    def dequant(self, ggml_type: int, data: np.ndarray, n: int) -> np.ndarray:
        """Dequantize host bytes through the device probe (bit-exact with hayai-model)."""
        w = self.upload(np.ascontiguousarray(data, dtype=np.uint8))
        out = self.alloc(max(4 * n, 4))
        self.dequant_dev(ggml_type, w, 0, n, out)
        return out.read(np.float32, n)

    # ---------------------------------------------------------------- FFN
    @staticmethod
    def ffn_desc(types, d_model, d_ff, layout: LayerPackLayout, act=ACT_SILU) -> _abi.FfnDesc:
        tg, tu, td = types
        return _abi.FfnDesc(tg, tu, td, act, d_model, d_ff, layout.gate_off, layout.up_off, layout.down_off)

    # ---------------------------------------------------------------- MoE
    @staticmethod
    def moe_desc(d_model: int, d_ff: int, n_experts: int, top_k: int, expert_stride: int, offs,
                 ggml_type: int = Q4_K, act: int = ACT_SILU, n_group: int = 0, topk_group: int = 0,
                 gating: int = 0, norm_topk_prob: bool = False,
                 routed_scaling_factor: float = 1.0, shared=None) -> _abi.MoeDesc:
        """MoeMeta (exec_plan.rs:244-271) + the resident expert layout (moe_infer.rs:330-339).
        shared: (shared_d_ff, (gate_off, up_off, down_off)) of the always-active shared expert
        (moe_infer.rs:456-493), offsets in the experts buffer; None: no shared expert."""
        g, u, dn = offs
        sd, (sg, su, sdn) = shared if shared is not None else (0, (0, 0, 0))
        return _abi.MoeDesc(ggml_type, act, d_model, d_ff, n_experts, top_k, expert_stride, g, u, dn, n_group,
                            topk_group, gating, int(norm_topk_prob), routed_scaling_factor, sd, sg, su, sdn)

    def route_experts(self, desc: _abi.MoeDesc, logits: np.ndarray, bias=None):
        """route_experts (moe_infer.rs:865-934) for logits of shape (T, n_experts): returns
        ids (T, top_k) int32 (-1 = empty slot) and weights (T, top_k) f32."""
        lg = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1, desc.n_experts)
        T = lg.shape[0]
        ids = np.empty((T, desc.top_k), np.int32)
        w = np.empty((T, desc.top_k), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        _check(self.lib.hh_route_experts(self.handle, C.byref(desc), _ptr(lg), None if b is None else _ptr(b), T,
                                         _ptr(ids), _ptr(w)))
        return ids, w

    def route_experts_dev(self, desc, logits: DeviceBuffer, logits_off, bias, bias_off, T, ids: DeviceBuffer,
                          ids_off, weights: DeviceBuffer, weights_off) -> None:
        _check(self.lib.hh_route_experts_dev(self.handle, C.byref(desc), logits.handle, logits_off,
                                             None if bias is None else bias.handle, bias_off, T, ids.handle, ids_off,
                                             weights.handle, weights_off))

    def moe_ffn_dev(self, desc, experts: DeviceBuffer, experts_off, x: DeviceBuffer, x_off, T, ids: DeviceBuffer,
                    ids_off, weights: DeviceBuffer, weights_off, y: DeviceBuffer, y_off) -> None:
        """The routed-expert FFN + combine (moe_infer.rs:342-455), enqueue only."""
        _check(self.lib.hh_moe_ffn_dev(self.handle, C.byref(desc), experts.handle, experts_off, x.handle, x_off, T,
                                       ids.handle, ids_off, weights.handle, weights_off, y.handle, y_off))

    def moe_dev(self, desc, experts: DeviceBuffer, experts_off, logits: DeviceBuffer, logits_off, bias, bias_off,
                x: DeviceBuffer, x_off, T, y: DeviceBuffer, y_off) -> None:
        _check(self.lib.hh_moe_dev(self.handle, C.byref(desc), experts.handle, experts_off, logits.handle, logits_off,
                                   None if bias is None else bias.handle, bias_off, x.handle, x_off, T, y.handle,
                                   y_off))

    def ffn(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, x: np.ndarray) -> np.ndarray:
        """ffn_begin_gate_up_scratch + ffn_finish_scratch (stream_infer.rs:3752-3864), one call."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.size != desc.d_model:
            raise HipError(2, f"x has {x.size} floats, expected d_model={desc.d_model}")
        y = np.empty(desc.d_model, np.float32)
        _check(self.lib.hh_ffn(self.handle, C.byref(desc), pack.handle, pack_off, _ptr(x), _ptr(y)))
        return y

    def ffn_batched(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, x: np.ndarray) -> np.ndarray:
        """The FFN op for a batch of tokens (rows of x), blocking; prefill_wave.rs:577-584."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != desc.d_model:
            raise HipError(2, f"x must be (batch, d_model={desc.d_model}), got {x.shape}")
        y = np.empty_like(x)
        _check(self.lib.hh_ffn_batched(self.handle, C.byref(desc), pack.handle, pack_off, _ptr(x), _ptr(y), x.shape[0]))
        return y

    def ffn_batched_dev(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, x: DeviceBuffer, x_off: int,
                        batch: int, y: DeviceBuffer, y_off: int) -> None:
        _check(self.lib.hh_ffn_batched_dev(self.handle, C.byref(desc), pack.handle, pack_off, x.handle, x_off, batch,
                                           y.handle, y_off))

    def ffn_dev(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, x: DeviceBuffer, x_off: int,
                y: DeviceBuffer, y_off: int) -> None:
        _check(self.lib.hh_ffn_dev(self.handle, C.byref(desc), pack.handle, pack_off, x.handle, x_off, y.handle,
                                   y_off))

    def ffn_block_begin_dev(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, norm: DeviceBuffer,
                            norm_off: int, eps: float, x: DeviceBuffer, x_off: int) -> None:
        """ffn_apply's first half (hybrid_infer.rs:895-918): rms_norm(x) then gate/up(+act)
        into the engine's FFN intermediate.  Enqueue only."""
        _check(self.lib.hh_ffn_block_begin_dev(self.handle, C.byref(desc), pack.handle, pack_off, norm.handle, norm_off,
                                               eps, x.handle, x_off))

    def ffn_block_finish_dev(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, res: DeviceBuffer,
                             res_off: int, y: DeviceBuffer, y_off: int) -> None:
        """ffn_apply's second half (:919-935): the down projection plus the residual, y = res +
        down (y may be res).  Enqueue only."""
        _check(self.lib.hh_ffn_block_finish_dev(self.handle, C.byref(desc), pack.handle, pack_off, res.handle, res_off,
                                                y.handle, y_off))

    def ffn_dev_noalloc(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, x: DeviceBuffer, x_off: int,
                        y: DeviceBuffer, y_off: int) -> None:
        """ffn_dev with its intermediate in the GPU's fixed scratch array (no allocation at
        call time; calls that overlap on one GPU race on that array).  Enqueue only."""
        _check(self.lib.hh_ffn_dev_noalloc(self.handle, C.byref(desc), pack.handle, pack_off, x.handle, x_off,
                                           y.handle, y_off))

    def ffn_block_dev(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, norm: DeviceBuffer,
                      norm_off: int, eps: float, x: DeviceBuffer, x_off: int, y: DeviceBuffer, y_off: int) -> None:
        """The FFN residual block (ffn_apply, hybrid_infer.rs:883-936): y = x + FFN(rms_norm(x,
        norm, eps)); y may be x.  Enqueue only."""
        _check(self.lib.hh_ffn_block_dev(self.handle, C.byref(desc), pack.handle, pack_off, norm.handle, norm_off,
                                         eps, x.handle, x_off, y.handle, y_off))

    def ffn_block_stack_dev(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, layer_stride: int,
                            n_layers: int, norm: DeviceBuffer, norm_off: int, norm_stride: int, eps: float,
                            x: DeviceBuffer, x_off: int, y: DeviceBuffer, y_off: int) -> None:
        """n_layers FFN residual blocks back to back (layer l's pack at pack_off + l * layer_stride,
        its norm at norm_off + 4 * l * norm_stride): y = x_L; y may be x.  Enqueue only."""
        _check(self.lib.hh_ffn_block_stack_dev(self.handle, C.byref(desc), pack.handle, pack_off, layer_stride,
                                               n_layers, norm.handle, norm_off, norm_stride, eps, x.handle, x_off,
                                               y.handle, y_off))

    def ffn_block(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, norm: np.ndarray, eps: float,
                  x: np.ndarray) -> np.ndarray:
        """ffn_apply on host activations: returns x + FFN(rms_norm(x, norm, eps)), blocking."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        norm = np.ascontiguousarray(norm, dtype=np.float32)
        if x.size != desc.d_model or norm.size != desc.d_model:
            raise HipError(2, f"x and norm must hold d_model={desc.d_model} floats")
        xb, nb = self.upload(x), self.upload(norm)
        try:
            self.ffn_block_dev(desc, pack, pack_off, nb, 0, eps, xb, 0, xb, 0)
            return xb.read(np.float32, desc.d_model)
        finally:
            xb.free()
            nb.free()

    def ffn_begin_dev(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, x: DeviceBuffer,
                      x_off: int) -> None:
        """ffn_begin_gate_up_scratch (stream_infer.rs:3752-3808): gate/up + activation into
        the engine's FFN intermediate, enqueue only."""
        _check(self.lib.hh_ffn_begin_dev(self.handle, C.byref(desc), pack.handle, pack_off, x.handle, x_off))

    def ffn_finish_dev(self, desc: _abi.FfnDesc, pack: DeviceBuffer, pack_off: int, y: DeviceBuffer,
                       y_off: int) -> None:
        """ffn_finish_scratch (stream_infer.rs:3809-3864): down projection of the pending
        intermediate, enqueue only."""
        _check(self.lib.hh_ffn_finish_dev(self.handle, C.byref(desc), pack.handle, pack_off, y.handle, y_off))

    def gateup_dev(self, types, d_ff: int, d_model: int, wg: DeviceBuffer, wg_off: int, wu: DeviceBuffer,
                   wu_off: int, x: DeviceBuffer, x_off: int, h: DeviceBuffer, h_off: int, act: int = ACT_SILU) -> None:
        """h = act(W_gate . x) * (W_up . x) (gate/up half of the FFN op), enqueue only."""
        tg, tu = types
        _check(self.lib.hh_gateup_dev(self.handle, tg, tu, d_ff, d_model, wg.handle, wg_off, wu.handle, wu_off,
                                      x.handle, x_off, h.handle, h_off, act))

    # ---------------------------------------------------------------- synthetic data
    def synth_weights_dev(self, ggml_type: int, dst: DeviceBuffer, off: int, n_blocks: int, seed: int,
                          lo: float, hi: float) -> None:
        _check(self.lib.hh_synth_weights_dev(self.handle, ggml_type, dst.handle, off, n_blocks, seed & ((1 << 64) - 1),
                                             lo, hi))
