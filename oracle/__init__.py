"""CPU oracle for the Hayai FFN GEMV hot path -- TEST INFRASTRUCTURE ONLY.

Thin numpy/ctypes wrapper over ``libhayai_oracle.so`` (built from ``hayai_oracle.c`` by
``oracle/Makefile``).  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package; the product (``hayai_amd``) never does.

Each function mirrors a reference function; the C source cites the file:line.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libhayai_oracle.so")

# GGML type ids (crates/hayai-model/src/gguf_types.rs:6-78)
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, IQ2_XXS, IQ3_XXS = 0, 1, 2, 8, 12, 14, 16, 18
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), IQ2_XXS: (256, 66),
         IQ3_XXS: (256, 98), F32: (1, 4), F16: (1, 2)}


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "libhayai_oracle.so"], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        P = C.c_void_p
        sz = C.c_size_t
        L.or_f16_to_f32.restype = C.c_float
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f16_to_f32_array.argtypes = [P, P, sz]
        L.or_f32_to_f16_ref.restype = C.c_uint16
        L.or_f32_to_f16_ref.argtypes = [C.c_float]
        L.or_row_bytes.argtypes = [C.c_int, sz, C.POINTER(sz)]
        L.or_validate_shape.argtypes = [C.c_int, sz, sz]
        L.or_validate_weights.argtypes = [C.c_int, sz, sz, sz]
        L.or_dequant.argtypes = [C.c_int, P, sz, sz, P]
        L.or_gemv.argtypes = [C.c_int, sz, sz, P, sz, P, P]
        L.or_gemv_f64.argtypes = [C.c_int, sz, sz, P, sz, P, P]
        L.or_gemv_batched.argtypes = [C.c_int, sz, sz, P, sz, sz, P, P]
        L.or_lut_matmul_q4.argtypes = [sz, sz, P, P, P, P]
        L.or_swiglu.argtypes = [P, P, P, sz]
        L.or_gelu_tanh.argtypes = [P, P, P, sz]
        L.or_ffn.argtypes = [C.c_int, C.c_int, C.c_int, sz, sz, P, sz, P, sz, P, sz, C.c_int, P, P, P]
        L.or_rms_norm.argtypes = [P, P, C.c_float, P, sz]
        L.or_ffn_block.argtypes = [C.c_int, C.c_int, C.c_int, sz, sz, P, sz, P, sz, P, sz, C.c_int, P, C.c_float,
                                   P, P]
        L.or_route_experts.argtypes = [P, C.c_int, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                       C.c_float, P, P]
        L.or_moe_token.argtypes = [C.c_int, sz, sz, P, sz, sz, sz, sz, C.c_int, P, P, P, P]
        L.or_moe_shared.argtypes = [C.c_int, sz, sz, P, P, P, P, P]
        L.or_quantize_q4_k.argtypes = [P, sz, P]
        L.or_quantize_act_q8.argtypes = [P, sz, P, P]
        L.or_ffn_q8.argtypes = [C.c_int, C.c_int, C.c_int, sz, sz, P, sz, P, sz, P, sz, C.c_int, P, P]
        L.or_get_scale_min_k4.argtypes = [C.c_int, P, P, P]
        L.or_iq2xxs_grid.argtypes = [P]
        L.or_iq3xxs_grid.argtypes = [P]
        L.or_ksigns.argtypes = [P]
        L.or_set_threads.argtypes = [C.c_int]
        L.or_set_mutation.argtypes = [C.c_int]
        L.or_max_threads.restype = C.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class OracleError(ValueError):
    pass


def _check(rc: int, what: str):
    if rc != 0:
        raise OracleError(f"{what}: invalid arguments (status {rc})")


def set_threads(n: int) -> None:
    lib().or_set_threads(int(n))


def set_mutation(m: int) -> None:
    """Plant a known mistake in the oracle (0 = none, 1 = FFN gate/up swapped, 2 = MoE expert
    id + 1); only the tests that show the oracle's pins catch such mistakes use this."""
    lib().or_set_mutation(int(m))


def max_threads() -> int:
    return int(lib().or_max_threads())


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def f32_to_f16_ref(v: float) -> int:
    return int(lib().or_f32_to_f16_ref(float(v)))


def row_bytes(t: int, n: int) -> int:
    out = C.c_size_t(0)
    _check(lib().or_row_bytes(t, n, C.byref(out)), "row_bytes")
    return out.value


def validate_shape(t: int, m: int, n: int) -> bool:
    return lib().or_validate_shape(t, m, n) == 0


def validate_weights(t: int, m: int, n: int, nbytes: int) -> bool:
    return lib().or_validate_weights(t, m, n, nbytes) == 0


def dequant(t: int, data: np.ndarray, n: int) -> np.ndarray:
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(n, np.float32)
    _check(lib().or_dequant(t, _p(data), data.size, n, _p(out)), "dequant")
    return out


def gemv(t: int, m: int, n: int, w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.size != n:
        raise OracleError("gemv: x has the wrong length")
    y = np.empty(m, np.float32)
    _check(lib().or_gemv(t, m, n, _p(w), w.size, _p(x), _p(y)), "gemv")
    return y


def gemv_f64(t: int, m: int, n: int, w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float64)
    y = np.empty(m, np.float64)
    _check(lib().or_gemv_f64(t, m, n, _p(w), w.size, _p(x), _p(y)), "gemv_f64")
    return y


def gemv_batched(t: int, m: int, n: int, w: np.ndarray, X: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, n)
    Y = np.empty((X.shape[0], m), np.float32)
    _check(lib().or_gemv_batched(t, m, n, _p(w), w.size, X.shape[0], _p(X), _p(Y)), "gemv_batched")
    return Y


def lut_matmul_q4(m: int, n: int, wq: np.ndarray, lut, x: np.ndarray) -> np.ndarray:
    wq = np.ascontiguousarray(wq, dtype=np.uint8)
    lut = np.ascontiguousarray(lut, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(m, np.float32)
    _check(lib().or_lut_matmul_q4(m, n, _p(wq), _p(lut), _p(x), _p(y)), "lut_matmul_q4")
    return y


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    h = np.empty_like(g)
    lib().or_swiglu(_p(g), _p(u), _p(h), g.size)
    return h


def gelu_tanh(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    h = np.empty_like(g)
    lib().or_gelu_tanh(_p(g), _p(u), _p(h), g.size)
    return h


def ffn(types, d_model: int, d_ff: int, wg, wu, wd, x, act: int = 0, return_h: bool = False):
    tg, tu, td = types
    wg, wu, wd = (np.ascontiguousarray(a, dtype=np.uint8) for a in (wg, wu, wd))
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(d_model, np.float32)
    h = np.empty(d_ff, np.float32)
    _check(lib().or_ffn(tg, tu, td, d_model, d_ff, _p(wg), wg.size, _p(wu), wu.size, _p(wd), wd.size,
                        act, _p(x), _p(y), _p(h)), "ffn")
    return (y, h) if return_h else y


def dequant_act_q8(x: np.ndarray) -> np.ndarray:
    """q * s of quantize_act_q8: the activation the batched int8 path computes with."""
    q, s = quantize_act_q8(x)
    return (q.astype(np.float32) * np.repeat(s, 32)).astype(np.float32)


def ffn_q8(types, d_model: int, d_ff: int, wg, wu, wd, x, act: int = 0) -> np.ndarray:
    """The batched int8 path's FFN: both GEMV inputs (x, and h before down) dequantized from
    their int8 per-32-block quantization."""
    tg, tu, td = types
    wg, wu, wd = (np.ascontiguousarray(a, dtype=np.uint8) for a in (wg, wu, wd))
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(d_model, np.float32)
    _check(lib().or_ffn_q8(tg, tu, td, d_model, d_ff, _p(wg), wg.size, _p(wu), wu.size, _p(wd), wd.size, act,
                           _p(x), _p(y)), "ffn_q8")
    return y


def rms_norm(x, w, eps: float) -> np.ndarray:
    """rms_norm (crates/hayai-cpu/src/attention.rs:142-147), out of place."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    if x.size != w.size:
        raise ValueError("x and w differ in length")
    y = np.empty_like(x)
    lib().or_rms_norm(_p(x), _p(w), eps, _p(y), x.size)
    return y


def ffn_block(types, d_model: int, d_ff: int, wg, wu, wd, norm, eps: float, x, act: int = 0) -> np.ndarray:
    """ffn_apply (crates/hayai-core/src/hybrid_infer.rs:883-936): x + FFN(rms_norm(x))."""
    tg, tu, td = types
    wg, wu, wd = (np.ascontiguousarray(a, dtype=np.uint8) for a in (wg, wu, wd))
    norm = np.ascontiguousarray(norm, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(d_model, np.float32)
    _check(lib().or_ffn_block(tg, tu, td, d_model, d_ff, _p(wg), wg.size, _p(wu), wu.size, _p(wd), wd.size, act,
                              _p(norm), eps, _p(x), _p(y)), "ffn_block")
    return y


def route_experts(scores, top_k: int, bias=None, n_group: int = 0, topk_group: int = 0, gating: int = 0,
                  norm_topk_prob: bool = False, routed_scaling_factor: float = 1.0):
    s = np.ascontiguousarray(scores, dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    ids = np.zeros(max(s.size, 1), np.int32)
    w = np.zeros(max(s.size, 1), np.float32)
    k = lib().or_route_experts(_p(s), s.size, None if b is None else _p(b), top_k, n_group, topk_group,
                               gating, int(norm_topk_prob), routed_scaling_factor, _p(ids), _p(w))
    return ids[:k].tolist(), w[:k]


def moe_token(t: int, d_model: int, d_ff: int, w, expert_stride: int, offs, ids, wts, x, acc=None, shared=None):
    """The routed experts of one token (moe_infer.rs:342-455) accumulated into acc, then the
    shared expert (:456-493) when shared = (shared_d_ff, wg, wu, wd) is given."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    wts = np.ascontiguousarray(wts, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    acc = np.zeros(d_model, np.float32) if acc is None else np.ascontiguousarray(acc, dtype=np.float32).copy()
    g_off, u_off, d_off = offs
    _check(lib().or_moe_token(t, d_model, d_ff, _p(w), expert_stride, g_off, u_off, d_off, ids.size,
                              _p(ids), _p(wts), _p(x), _p(acc)), "moe_token")
    if shared is not None:
        sdf, sg, su, sd = shared
        sg, su, sd = (np.ascontiguousarray(a, dtype=np.uint8) for a in (sg, su, sd))
        _check(lib().or_moe_shared(t, d_model, sdf, _p(sg), _p(su), _p(sd), _p(x), _p(acc)), "moe_shared")
    return acc


def quantize_q4_k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.size // 256 * 144, np.uint8)
    _check(lib().or_quantize_q4_k(_p(x), x.size, _p(out)), "quantize_q4_k")
    return out


def quantize_act_q8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(x.size, np.int8)
    s = np.zeros(x.size // 32, np.float32)
    _check(lib().or_quantize_act_q8(_p(x), x.size, _p(q), _p(s)), "quantize_act_q8")
    return q, s


def get_scale_min_k4(j: int, scales12) -> tuple[int, int]:
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    sc = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().or_get_scale_min_k4(j, _p(s), _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def iq2xxs_grid() -> np.ndarray:
    out = np.zeros(256, np.uint64)
    lib().or_iq2xxs_grid(_p(out))
    return out


def iq3xxs_grid() -> np.ndarray:
    out = np.zeros(256, np.uint32)
    lib().or_iq3xxs_grid(_p(out))
    return out


def ksigns() -> np.ndarray:
    out = np.zeros(128, np.uint8)
    lib().or_ksigns(_p(out))
    return out
