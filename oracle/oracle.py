"""ctypes bindings and numpy helpers around ``liboracle.so`` (fgqa_oracle.c).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

bf16 tensors are numpy ``uint16`` arrays holding bfloat16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# FGQA_ORACLE_LIB selects another build of the same oracle (the sanitizer
# build, `make -C oracle liboracle_san.so`); by default the optimised one.
_LIB_PATH = os.path.abspath(os.environ.get("FGQA_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so"))
_lib = None

_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-C", _HERE, "-B", "liboracle.so"], check=True,
                   stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.fgqa_oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.fgqa_oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.fgqa_oracle_bf16_to_f32.restype = ctypes.c_float
        L.fgqa_oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.fgqa_oracle_f32_to_bf16_array.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.fgqa_oracle_bf16_to_f32_array.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.fgqa_oracle_decode_bf16.restype = ctypes.c_int
        L.fgqa_oracle_decode_bf16.argtypes = [
            _u16p, _u16p, _u16p, ctypes.c_float, _u16p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.fgqa_oracle_prefill_bf16.restype = ctypes.c_int
        L.fgqa_oracle_prefill_bf16.argtypes = [
            _u16p, _u16p, _u16p, ctypes.c_float, _u16p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.fgqa_oracle_prefill_mla_bf16.restype = ctypes.c_int
        L.fgqa_oracle_prefill_mla_bf16.argtypes = [
            _u16p, _u16p, _u16p, ctypes.c_float, _u16p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.fgqa_oracle_sparse_prefill_bf16.restype = ctypes.c_int
        L.fgqa_oracle_sparse_prefill_bf16.argtypes = [
            _u16p, _u16p, _u16p, ctypes.c_float, _u16p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, _i32p, _i64p, ctypes.c_int,
            ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.fgqa_oracle_attention_f64.restype = ctypes.c_int
        L.fgqa_oracle_attention_f64.argtypes = [
            _u16p, _u16p, _u16p, ctypes.c_double, _f64p, _f64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.fgqa_oracle_prefill_backward_bf16.restype = ctypes.c_int
        L.fgqa_oracle_prefill_backward_bf16.argtypes = [
            _u16p, _u16p, _u16p, _u16p, _f32p, _u16p, ctypes.c_float, _f32p, _f32p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, _i64p, ctypes.c_int, _i32p, _i32p, ctypes.c_int]
        L.fgqa_oracle_prefill_swa_backward_bf16.restype = ctypes.c_int
        L.fgqa_oracle_prefill_swa_backward_bf16.argtypes = [
            _u16p, _u16p, _u16p, _u16p, _f32p, _u16p, ctypes.c_float, _f32p, _f32p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, _i64p, ctypes.c_int, _i32p, _i32p, ctypes.c_int]
        L.fgqa_oracle_attention_swa_backward_f64.restype = ctypes.c_int
        L.fgqa_oracle_attention_swa_backward_f64.argtypes = [
            _u16p, _u16p, _u16p, _u16p, _u16p, ctypes.c_double, _f64p, _f64p, _f64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, _i64p, ctypes.c_int, _f32p, ctypes.c_int]
        L.fgqa_oracle_attention_backward_f64.restype = ctypes.c_int
        L.fgqa_oracle_attention_backward_f64.argtypes = [
            _u16p, _u16p, _u16p, _u16p, _u16p, ctypes.c_double, _f64p, _f64p, _f64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, _i64p, ctypes.c_int, ctypes.c_int]
        L.fgqa_oracle_prefill_mla_backward_bf16.restype = ctypes.c_int
        L.fgqa_oracle_prefill_mla_backward_bf16.argtypes = [
            _u16p, _u16p, _u16p, _u16p, _f32p, _u16p, ctypes.c_float, _f32p, _f32p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, _i64p, ctypes.c_int, _i32p, _i32p, ctypes.c_int]
        L.fgqa_oracle_attention_mla_backward_f64.restype = ctypes.c_int
        L.fgqa_oracle_attention_mla_backward_f64.argtypes = [
            _u16p, _u16p, _u16p, _u16p, _u16p, ctypes.c_double, _f64p, _f64p, _f64p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, _i64p, ctypes.c_int, ctypes.c_int]
        L.fgqa_oracle_fp8e4m3_to_f32.restype = ctypes.c_float
        L.fgqa_oracle_fp8e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.fgqa_oracle_decode_paged.restype = ctypes.c_int
        L.fgqa_oracle_decode_paged.argtypes = [
            _u16p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, _i32p, ctypes.c_int64, ctypes.c_int,
            _i64p, _i64p, ctypes.c_float, ctypes.c_float, ctypes.c_float, _u16p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p, ctypes.c_int, ctypes.c_int]
        L.fgqa_oracle_prefill_swa_bf16.restype = ctypes.c_int
        L.fgqa_oracle_prefill_swa_bf16.argtypes = [
            _u16p, _u16p, _u16p, ctypes.c_float, _u16p, _f32p,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _i64p, _i64p, _i64p, _i64p, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int]
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None, ctype):
    if a is None:
        return ctypes.cast(None, ctypes.POINTER(ctype))
    return a.ctypes.data_as(ctypes.POINTER(ctype))


# ---------------------------------------------------------------- bf16 helpers
def f32_to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (numpy restatement of
    fgqa_oracle_f32_to_bf16; the two are checked against each other exhaustively)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(np.asarray(h, dtype=np.uint16))
    return (h.astype(np.uint32) << 16).view(np.float32)


def normal_bf16(seed: int, shape, sigma: float = 1.0, stream: int = 0) -> np.ndarray:
    """Seeded N(0, sigma^2) bf16 bits (numpy PCG64; `stream` separates Q/K/V)."""
    rng = np.random.default_rng([seed, stream])
    x = rng.standard_normal(size=shape, dtype=np.float32) * np.float32(sigma)
    return f32_to_bf16(x)


# ---------------------------------------------------------------- oracles
def decode(q, k, v, scale, seqlens=None, tile=128, nthreads=0, with_lse=True, p_bf16=True):
    """Decode oracle. q [B,Hq,D], k/v [B,S,Hkv,D] (uint16 bf16 bits).
    p_bf16=True rounds P to bf16 before P.V (the C++ reference); False keeps
    fp32 P (the torch tiled reference).
    Returns (o uint16 [B,Hq,D], lse float32 [B,Hq] or None)."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    B, Hq, D = q.shape
    _, S, Hkv, _ = k.shape
    o = np.empty((B, Hq, D), dtype=np.uint16)
    lse = np.empty((B, Hq), dtype=np.float32) if with_lse else None
    sl = None if seqlens is None else np.ascontiguousarray(seqlens, dtype=np.int32)
    rc = lib().fgqa_oracle_decode_bf16(
        _ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
        float(scale), _ptr(o, ctypes.c_uint16), _ptr(lse, ctypes.c_float),
        B, S, Hq, Hkv, D, _ptr(sl, ctypes.c_int32), int(tile), int(bool(p_bf16)), int(nthreads))
    if rc != 0:
        raise ValueError("fgqa_oracle_decode_bf16: invalid arguments")
    return o, lse


def _strides(a: np.ndarray, layout: str):
    """Element strides (b, s, h) of a 4-D array in `layout` ('bshd' or 'bhsd')."""
    st = [s // a.itemsize for s in a.strides]
    if layout == "bshd":
        return np.array([st[0], st[1], st[2]], dtype=np.int64)
    if layout == "bhsd":
        return np.array([st[0], st[2], st[1]], dtype=np.int64)
    raise ValueError(layout)


def _dims(a: np.ndarray, layout: str):
    B = a.shape[0]
    if layout == "bshd":
        return B, a.shape[1], a.shape[2], a.shape[3]
    return B, a.shape[2], a.shape[1], a.shape[3]


def prefill(q, k, v, scale, causal=True, layout="bshd", q_offset=0, nthreads=0):
    """Prefill oracle. layout 'bshd': q [B,Sq,Hq,D], k/v [B,Skv,Hkv,D];
    'bhsd': q [B,Hq,Sq,D], k/v [B,Hkv,Skv,D].  Returns (o in q's layout, lse [B,Hq,Sq])."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    B, Sq, Hq, D = _dims(q, layout)
    _, Skv, Hkv, _ = _dims(k, layout)
    o = np.empty_like(q)
    lse = np.empty((B, Hq, Sq), dtype=np.float32)
    qs, ks, vs, os_ = (_strides(x, layout) for x in (q, k, v, o))
    rc = lib().fgqa_oracle_prefill_bf16(
        _ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
        float(scale), _ptr(o, ctypes.c_uint16), _ptr(lse, ctypes.c_float),
        B, Sq, Skv, Hq, Hkv, D,
        _ptr(qs, ctypes.c_int64), _ptr(ks, ctypes.c_int64), _ptr(vs, ctypes.c_int64),
        _ptr(os_, ctypes.c_int64), int(bool(causal)), int(q_offset), int(nthreads))
    if rc != 0:
        raise ValueError("fgqa_oracle_prefill_bf16: invalid arguments")
    return o, lse


def prefill_mla(q, k, v, scale, causal=True, layout="bshd", q_offset=0, nthreads=0):
    """MLA prefill oracle: q/k rows of Dqk elements, v rows of Dv (may differ).
    layout 'bshd': q [B,Sq,Hq,Dqk], k [B,Skv,Hkv,Dqk], v [B,Skv,Hkv,Dv];
    'bhsd': heads before sequence.  Returns (o [.., Dv] in q's layout, lse [B,Hq,Sq])."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    B, Sq, Hq, Dqk = _dims(q, layout)
    _, Skv, Hkv, Dk = _dims(k, layout)
    Dv = v.shape[3]
    if Dk != Dqk:
        raise ValueError("prefill_mla: q and k head dims differ")
    o = np.empty(q.shape[:3] + (Dv,), dtype=np.uint16)
    lse = np.empty((B, Hq, Sq), dtype=np.float32)
    qs, ks, vs, os_ = (_strides(x, layout) for x in (q, k, v, o))
    rc = lib().fgqa_oracle_prefill_mla_bf16(
        _ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
        float(scale), _ptr(o, ctypes.c_uint16), _ptr(lse, ctypes.c_float),
        B, Sq, Skv, Hq, Hkv, Dqk, Dv,
        _ptr(qs, ctypes.c_int64), _ptr(ks, ctypes.c_int64), _ptr(vs, ctypes.c_int64),
        _ptr(os_, ctypes.c_int64), int(bool(causal)), int(q_offset), int(nthreads))
    if rc != 0:
        raise ValueError("fgqa_oracle_prefill_mla_bf16: invalid arguments")
    return o, lse


def sparse_prefill(q, k, v, idx, scale, causal=True, layout="bshd", q_offset=0, nthreads=0):
    """Sparse-index prefill oracle.  idx: int32 [B, Hkv, Sq, nsparse] (key index
    lists, -1 = empty slot).  Layouts of q/k/v as `prefill`.  Returns (o in q's
    layout, lse [B,Hq,Sq])."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    B, Sq, Hq, D = _dims(q, layout)
    _, Skv, Hkv, _ = _dims(k, layout)
    if idx.ndim != 4 or idx.shape[:3] != (B, Hkv, Sq):
        raise ValueError("sparse_prefill: idx must be [B, Hkv, Sq, nsparse]")
    o = np.empty_like(q)
    lse = np.empty((B, Hq, Sq), dtype=np.float32)
    qs, ks, vs, os_ = (_strides(x, layout) for x in (q, k, v, o))
    ist = np.array([idx.strides[0] // 4, idx.strides[1] // 4, idx.strides[2] // 4], dtype=np.int64)
    rc = lib().fgqa_oracle_sparse_prefill_bf16(
        _ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
        float(scale), _ptr(o, ctypes.c_uint16), _ptr(lse, ctypes.c_float),
        B, Sq, Skv, Hq, Hkv, D,
        _ptr(qs, ctypes.c_int64), _ptr(ks, ctypes.c_int64), _ptr(vs, ctypes.c_int64),
        _ptr(os_, ctypes.c_int64), _ptr(idx, ctypes.c_int32), _ptr(ist, ctypes.c_int64),
        idx.shape[3], int(bool(causal)), int(q_offset), int(nthreads))
    if rc != 0:
        raise ValueError("fgqa_oracle_sparse_prefill_bf16: invalid arguments")
    return o, lse


def attention_f64(q, k, v, scale, causal=False, causal_offset=0, seqlens=None,
                  layout="bshd", nthreads=0):
    """float64 softmax attention. Returns (o float64 [B,Sq,Hq,D], lse float64 [B,Hq,Sq])."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    B, Sq, Hq, D = _dims(q, layout)
    _, Skv, Hkv, _ = _dims(k, layout)
    o = np.empty((B, Sq, Hq, D), dtype=np.float64)
    lse = np.empty((B, Hq, Sq), dtype=np.float64)
    qs, ks, vs = (_strides(x, layout) for x in (q, k, v))
    sl = None if seqlens is None else np.ascontiguousarray(seqlens, dtype=np.int32)
    rc = lib().fgqa_oracle_attention_f64(
        _ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
        float(scale), _ptr(o, ctypes.c_double), _ptr(lse, ctypes.c_double),
        B, Sq, Skv, Hq, Hkv, D,
        _ptr(qs, ctypes.c_int64), _ptr(ks, ctypes.c_int64), _ptr(vs, ctypes.c_int64),
        _ptr(sl, ctypes.c_int32), int(bool(causal)), int(causal_offset), int(nthreads))
    if rc != 0:
        raise ValueError("fgqa_oracle_attention_f64: invalid arguments")
    return o, lse


def prefill_backward(q, k, v, o, lse, grad_o, scale, causal=True, layout="bshd",
                     rows=None, keys=None, want=("dq", "dk", "dv"), nthreads=0, window=0):
    """Backward oracle (restates src/python/Triton/flash_gqa_backward_kernel.py).
    q/o/grad_o and k/v in `layout`; lse float32 [B,Hq,Sq].  Returns the fp32
    accumulators (dq [B,Sq,Hq,D], dk, dv [B,Skv,Hkv,D], BSHD) -- round with
    f32_to_bf16 for the reference's bf16 outputs.  rows/keys = (first, end)
    limit which dq rows / dk,dv rows are computed (the others are NaN); an
    output not named in `want` is returned as None.  window > 0 (causal):
    the sliding-window backward (SWA/flash_swa_backward_kernel.py), with the
    forward's sink-adjusted lse.  v/o/grad_o rows narrower than q/k rows (MLA:
    192 and 128) give the MLA backward (flash_mla_backward_kernel.py); dv then
    has v's row length."""
    q, k, v, o, grad_o = (np.ascontiguousarray(x, dtype=np.uint16) for x in (q, k, v, o, grad_o))
    lse = np.ascontiguousarray(lse, dtype=np.float32)
    B, Sq, Hq, D = _dims(q, layout)
    _, Skv, Hkv, _ = _dims(k, layout)
    Dv = v.shape[-1]
    dq = np.full((B, Sq, Hq, D), np.nan, dtype=np.float32) if "dq" in want else None
    dk = np.full((B, Skv, Hkv, D), np.nan, dtype=np.float32) if "dk" in want else None
    dv = np.full((B, Skv, Hkv, Dv), np.nan, dtype=np.float32) if "dv" in want else None
    qs, ks, vs, os_, dos = (_strides(x, layout) for x in (q, k, v, o, grad_o))
    rr = None if rows is None else np.array(rows, dtype=np.int32)
    kk = None if keys is None else np.array(keys, dtype=np.int32)
    args = (_ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
            _ptr(o, ctypes.c_uint16), _ptr(lse, ctypes.c_float), _ptr(grad_o, ctypes.c_uint16),
            float(scale), _ptr(dq, ctypes.c_float), _ptr(dk, ctypes.c_float), _ptr(dv, ctypes.c_float),
            B, Sq, Skv, Hq, Hkv, D,
            _ptr(qs, ctypes.c_int64), _ptr(ks, ctypes.c_int64), _ptr(vs, ctypes.c_int64),
            _ptr(os_, ctypes.c_int64), _ptr(dos, ctypes.c_int64))
    tail = (_ptr(rr, ctypes.c_int32), _ptr(kk, ctypes.c_int32), int(nthreads))
    if Dv != D:
        if window > 0:
            raise ValueError("prefill_backward: the MLA backward has no window form")
        args = args[:16] + (Dv,) + args[16:]
        rc = lib().fgqa_oracle_prefill_mla_backward_bf16(*args, int(bool(causal)), *tail)
        if rc != 0:
            raise ValueError("fgqa_oracle_prefill_mla_backward_bf16: invalid arguments")
        return dq, dk, dv
    if window > 0:
        if not causal:
            raise ValueError("prefill_backward: a window needs causal=True")
        rc = lib().fgqa_oracle_prefill_swa_backward_bf16(*args, int(window), *tail)
    else:
        rc = lib().fgqa_oracle_prefill_backward_bf16(*args, int(bool(causal)), *tail)
    if rc != 0:
        raise ValueError("fgqa_oracle_prefill_backward_bf16: invalid arguments")
    return dq, dk, dv


def attention_backward_f64(q, k, v, grad_o, scale, causal=True, o=None, layout="bshd", nthreads=0,
                           window=0, sink=None):
    """Exact gradient of softmax attention in float64.  o=None: delta from P
    (the true gradient); o given (bf16 bits): delta = sum O*dO as the torch
    reference does.  window > 0 and/or sink (float32 [Hq]): causal
    sliding-window attention with the sink in the denominator.  v/grad_o rows
    narrower than q/k rows: the MLA gradient.  Returns (dq [B,Sq,Hq,D], dk
    [B,Skv,Hkv,D], dv [B,Skv,Hkv,Dv]) float64."""
    q, k, v, grad_o = (np.ascontiguousarray(x, dtype=np.uint16) for x in (q, k, v, grad_o))
    B, Sq, Hq, D = _dims(q, layout)
    _, Skv, Hkv, _ = _dims(k, layout)
    Dv = v.shape[-1]
    dq = np.empty((B, Sq, Hq, D), dtype=np.float64)
    dk = np.empty((B, Skv, Hkv, D), dtype=np.float64)
    dv = np.empty((B, Skv, Hkv, Dv), dtype=np.float64)
    qs, ks, vs, dos = (_strides(x, layout) for x in (q, k, v, grad_o))
    os_ = None
    if o is not None:
        o = np.ascontiguousarray(o, dtype=np.uint16)
        os_ = _strides(o, layout)
    args = (_ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
            _ptr(o, ctypes.c_uint16), _ptr(grad_o, ctypes.c_uint16), float(scale),
            _ptr(dq, ctypes.c_double), _ptr(dk, ctypes.c_double), _ptr(dv, ctypes.c_double),
            B, Sq, Skv, Hq, Hkv, D,
            _ptr(qs, ctypes.c_int64), _ptr(ks, ctypes.c_int64), _ptr(vs, ctypes.c_int64),
            _ptr(os_, ctypes.c_int64), _ptr(dos, ctypes.c_int64))
    if Dv != D:
        if window > 0 or sink is not None:
            raise ValueError("attention_backward_f64: the MLA gradient has no window / sink form")
        args = args[:15] + (Dv,) + args[15:]
        rc = lib().fgqa_oracle_attention_mla_backward_f64(*args, int(bool(causal)), int(nthreads))
        if rc != 0:
            raise ValueError("fgqa_oracle_attention_mla_backward_f64: invalid arguments")
        return dq, dk, dv
    if window > 0 or sink is not None:
        if not causal:
            raise ValueError("attention_backward_f64: a window or sink needs causal=True")
        w = int(window) if window > 0 else max(Sq, Skv) + 1
        sk = None if sink is None else np.ascontiguousarray(sink, dtype=np.float32)
        rc = lib().fgqa_oracle_attention_swa_backward_f64(*args, w, _ptr(sk, ctypes.c_float), int(nthreads))
    else:
        rc = lib().fgqa_oracle_attention_backward_f64(*args, int(bool(causal)), int(nthreads))
    if rc != 0:
        raise ValueError("fgqa_oracle_attention_backward_f64: invalid arguments")
    return dq, dk, dv


def fp8e4m3_to_f32(codes) -> np.ndarray:
    """uint8 OCP e4m3 codes -> float32 (via fgqa_oracle_fp8e4m3_to_f32)."""
    codes = np.asarray(codes, dtype=np.uint8)
    table = np.array([lib().fgqa_oracle_fp8e4m3_to_f32(c) for c in range(256)], dtype=np.float32)
    return table[codes]


def decode_paged(q, k_cache, v_cache, block_table, seqlens, scale, k_scale=1.0, v_scale=1.0,
                 tile=128, nthreads=0, with_lse=True):
    """Paged decode oracle.  q [B,Hq,D] uint16 bf16 bits; k/v caches
    [num_pages, page_size, Hkv, D] as uint16 (bf16) or uint8 (fp8 e4m3) arrays;
    block_table int32 [B, max_pages]; seqlens int32 [B].
    Returns (o uint16 [B,Hq,D], lse float32 [B,Hq] or None)."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    if k_cache.dtype != v_cache.dtype or k_cache.dtype not in (np.uint16, np.uint8):
        raise ValueError("k_cache / v_cache must both be uint16 (bf16) or uint8 (fp8)")
    kv_fp8 = int(k_cache.dtype == np.uint8)
    k_cache = np.ascontiguousarray(k_cache)
    v_cache = np.ascontiguousarray(v_cache)
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seqlens, dtype=np.int32)
    B, Hq, D = q.shape
    _, page_size, Hkv, _ = k_cache.shape
    ks = np.array([s // k_cache.itemsize for s in k_cache.strides[:3]], dtype=np.int64)
    vs = np.array([s // v_cache.itemsize for s in v_cache.strides[:3]], dtype=np.int64)
    o = np.empty((B, Hq, D), dtype=np.uint16)
    lse = np.empty((B, Hq), dtype=np.float32) if with_lse else None
    rc = lib().fgqa_oracle_decode_paged(
        _ptr(q, ctypes.c_uint16), k_cache.ctypes.data_as(ctypes.c_void_p), v_cache.ctypes.data_as(ctypes.c_void_p),
        kv_fp8, _ptr(bt, ctypes.c_int32), int(bt.shape[1]), int(page_size),
        _ptr(ks, ctypes.c_int64), _ptr(vs, ctypes.c_int64), float(scale), float(k_scale), float(v_scale),
        _ptr(o, ctypes.c_uint16), _ptr(lse, ctypes.c_float), B, Hq, Hkv, D, _ptr(sl, ctypes.c_int32),
        int(tile), int(nthreads))
    if rc != 0:
        raise ValueError("fgqa_oracle_decode_paged: invalid arguments")
    return o, lse


def prefill_swa(q, k, v, scale, window, sink=None, layout="bshd", q_offset=0, nthreads=0):
    """Sliding-window (+ sink) prefill oracle.  sink: float32 [Hq] or None.
    Returns (o in q's layout, lse [B,Hq,Sq])."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    B, Sq, Hq, D = _dims(q, layout)
    _, Skv, Hkv, _ = _dims(k, layout)
    o = np.empty_like(q)
    lse = np.empty((B, Hq, Sq), dtype=np.float32)
    sk = None if sink is None else np.ascontiguousarray(sink, dtype=np.float32)
    qs, ks, vs, os_ = (_strides(x, layout) for x in (q, k, v, o))
    rc = lib().fgqa_oracle_prefill_swa_bf16(
        _ptr(q, ctypes.c_uint16), _ptr(k, ctypes.c_uint16), _ptr(v, ctypes.c_uint16),
        float(scale), _ptr(o, ctypes.c_uint16), _ptr(lse, ctypes.c_float),
        B, Sq, Skv, Hq, Hkv, D,
        _ptr(qs, ctypes.c_int64), _ptr(ks, ctypes.c_int64), _ptr(vs, ctypes.c_int64),
        _ptr(os_, ctypes.c_int64), int(window), _ptr(sk, ctypes.c_float), int(q_offset), int(nthreads))
    if rc != 0:
        raise ValueError("fgqa_oracle_prefill_swa_bf16: invalid arguments")
    return o, lse
