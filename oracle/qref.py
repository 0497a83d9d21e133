"""ctypes binding of the CPU oracle (liboracle.so built from this folder).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP library and the
timed CPU baseline. Only tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg may import it; the product never does.

The C sources restate candle's CPU path as SwarmLLM vendors it
(vendor/candle/candle-core/src/quantized/{k_quants,avx,utils}.rs); see
qref.h for the map.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

Q4_0, Q8_0, Q4_K, Q6_K, Q8_K, IQ4_NL, MXFP4 = 2, 8, 12, 14, 15, 20, 39
BLOCK = {Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256, Q8_K: 256, IQ4_NL: 32, MXFP4: 32}
TYPE_SIZE = {Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q8_K: 292, IQ4_NL: 18, MXFP4: 17}
VEC_DOT = {Q4_0: Q8_0, Q8_0: Q8_0, Q4_K: Q8_K, Q6_K: Q8_K, IQ4_NL: Q8_0, MXFP4: Q8_0}


def build() -> str:
    """Compile liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.qref_f32_to_f16.argtypes, L.qref_f32_to_f16.restype = [ctypes.c_float], ctypes.c_uint16
        L.qref_f16_to_f32.argtypes, L.qref_f16_to_f32.restype = [ctypes.c_uint16], ctypes.c_float
        L.qref_from_float.argtypes, L.qref_from_float.restype = [I, P, P, I64], I
        L.qref_to_float.argtypes, L.qref_to_float.restype = [I, P, P, I64], I
        L.qref_vec_dot.argtypes, L.qref_vec_dot.restype = [I, I64, P, P], ctypes.c_float
        L.qref_vec_dot_unopt.argtypes, L.qref_vec_dot_unopt.restype = [I, I64, P, P], ctypes.c_float
        L.qref_vec_dot_rows.argtypes, L.qref_vec_dot_rows.restype = [I, I64, P, P, I, P, I], None
        L.qref_matmul.argtypes, L.qref_matmul.restype = [I, I64, I64, I64, P, P, P, I], I
        L.qref_matmul_prequantized.argtypes = [I, I64, I64, I64, P, P, P, I]
        L.qref_matmul_prequantized.restype = I
        L.qref_matmul_upstream.argtypes, L.qref_matmul_upstream.restype = [I, I64, I64, I64, P, P, P], I
        L.qref_quantize_rows.argtypes, L.qref_quantize_rows.restype = [I, I64, I64, P, P, I], I
        L.qref_wire_bytes.argtypes, L.qref_wire_bytes.restype = [I64], I64
        L.qref_wire_encode.argtypes, L.qref_wire_encode.restype = [P, I64, P], None
        L.qref_wire_decode.argtypes, L.qref_wire_decode.restype = [P, I64, I64, P], I
        for f in ("qref_silu_mul", "qref_swiglu_oai_mul", "qref_gelu_mul"):
            getattr(L, f).argtypes, getattr(L, f).restype = [P, P, P, I64], None
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def nbytes(qtype: int, n: int) -> int:
    return n // BLOCK[qtype] * TYPE_SIZE[qtype]


def from_float(qtype: int, x: np.ndarray) -> np.ndarray:
    """Blocks (as uint8 bytes) of ``x`` quantized as ``qtype``: the type's from_float."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(nbytes(qtype, x.size), dtype=np.uint8)
    if lib().qref_from_float(qtype, _p(x), _p(out), x.size) != 0:
        raise ValueError(f"from_float: type {qtype}, {x.size} values")
    return out


def to_float(qtype: int, blocks: np.ndarray, n: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    assert blocks.size >= nbytes(qtype, n)
    out = np.empty(n, dtype=np.float32)
    if lib().qref_to_float(qtype, _p(blocks), _p(out), n) != 0:
        raise ValueError(f"to_float: type {qtype}, {n} values")
    return out


def vec_dot(qtype: int, n: int, xs: np.ndarray, ys: np.ndarray) -> np.float32:
    return np.float32(lib().qref_vec_dot(qtype, n, _p(np.ascontiguousarray(xs)), _p(np.ascontiguousarray(ys))))


def vec_dot_unopt(qtype: int, n: int, xs: np.ndarray, ys: np.ndarray) -> np.float32:
    return np.float32(
        lib().qref_vec_dot_unopt(qtype, n, _p(np.ascontiguousarray(xs)), _p(np.ascontiguousarray(ys))))


def quantize_rows(qtype: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """The activation rows as the driver quantizes them (VecDotType blocks)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    vt = VEC_DOT[qtype]
    out = np.zeros(m * nbytes(vt, k), dtype=np.uint8)
    if lib().qref_quantize_rows(qtype, m, k, _p(x), _p(out), threads) != 0:
        raise ValueError("quantize_rows")
    return out


def matmul(qtype: int, x: np.ndarray, w: np.ndarray, n: int, threads: int = 0) -> np.ndarray:
    """k_quants::matmul: x [m, k] f32 against n weight rows of k values (bytes ``w``)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    w = np.ascontiguousarray(w, dtype=np.uint8)
    assert w.size >= n * nbytes(qtype, k)
    dst = np.empty((m, n), dtype=np.float32)
    if lib().qref_matmul(qtype, m, k, n, _p(x), _p(w), _p(dst), threads) != 0:
        raise ValueError("matmul")
    return dst


def matmul_prequantized(qtype: int, xq: np.ndarray, m: int, k: int, w: np.ndarray, n: int,
                        threads: int = 0) -> np.ndarray:
    dst = np.empty((m, n), dtype=np.float32)
    rc = lib().qref_matmul_prequantized(qtype, m, k, n, _p(np.ascontiguousarray(xq)),
                                        _p(np.ascontiguousarray(w)), _p(dst), threads)
    if rc != 0:
        raise ValueError("matmul_prequantized")
    return dst


def matmul_upstream(qtype: int, x: np.ndarray, w: np.ndarray, n: int) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    dst = np.empty((m, n), dtype=np.float32)
    if lib().qref_matmul_upstream(qtype, m, k, n, _p(x), _p(np.ascontiguousarray(w)), _p(dst)) != 0:
        raise ValueError("matmul_upstream")
    return dst


def f32_to_f16_bits(x: float) -> int:
    return int(lib().qref_f32_to_f16(float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().qref_f16_to_f32(int(h)))


def wire_bytes(n: int) -> int:
    """q8_0_byte_len_checked (src/inference/quant.rs:98-104): -1 on overflow."""
    return int(lib().qref_wire_bytes(n))


def wire_encode(x: np.ndarray) -> np.ndarray:
    """quantize_q8_0 (src/inference/quant.rs:24-60): the wire bytes of ``x``."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.zeros(max(wire_bytes(x.size), 0), dtype=np.uint8)
    if x.size:
        lib().qref_wire_encode(_p(x), x.size, _p(out))
    return out


def wire_decode(b: np.ndarray, n: int) -> np.ndarray:
    """dequantize_q8_0 (src/inference/quant.rs:65-92); ValueError on a length mismatch."""
    b = np.ascontiguousarray(b, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    if lib().qref_wire_decode(_p(b) if b.size else 0, b.size, n, _p(out) if n else 0) != 0:
        raise ValueError(f"wire_decode: {b.size} bytes for {n} values")
    return out


def glu(activation: str, gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """act(gate) * up in f32 as the reference's CPU path evaluates it
    (src/inference/fast_math.rs: silu_mul_into :48-60, swiglu_oai_mul_into
    :84-104, gelu_mul_into :62-76), elementwise over arrays of one shape."""
    fn = {"silu": "qref_silu_mul", "swiglu_oai": "qref_swiglu_oai_mul", "gelu": "qref_gelu_mul"}[activation]
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    if g.shape != u.shape:
        raise ValueError("glu: gate and up must have one shape")
    out = np.empty_like(g)
    if g.size:
        getattr(lib(), fn)(_p(g), _p(u), _p(out), g.size)
    return out


def round_f16(x: np.ndarray) -> np.ndarray:
    """f32 values rounded to f16 (to nearest even, subnormals kept), back in
    f32: T(v) with T = half in the reference's tensor-core MoE kernel
    (moe_wmma_gguf.cu:60-165) and its caller's to_dtype(F16)."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """f32 values rounded to bf16 (to nearest even on the f32 bits), back in
    f32: T(v) with T = nv_bfloat16 in the same kernel. NaN stays NaN."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    b = a.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = a[nan]
    return out


def moe_prefill(qtype: int, stack: np.ndarray, num_experts: int, n: int, k: int, x: np.ndarray, bf16: bool,
                sorted_ids: np.ndarray, expert_ids: np.ndarray, topk_w, topk: int, size_m: int = -1) -> np.ndarray:
    """moe_gemm_gguf_prefill (candle-kernels/src/moe/moe_wmma_gguf.cu:191-371):
    entry i (pair p = sorted_ids[i], expert e = expert_ids[i], both in range)
    gives row p = scale_p * sum_j T(x[in_p][j]) T(w_e[.][j]) with T the
    rounding to f16 (bf16 when `bf16`) of the input value and of the weight's
    to_float value (:60-165, dequantize_block_warp), scale_p = topk_w[p] or 1
    (:356-367), in_p = p with topk_w else p // topk (:267). Summed here in
    f64 (the kernel's f32 tensor-core sum differs from it by rounding only).
    Rows no entry writes are NaN. size_m: the routing's entry count (pairs
    at or past it are out of range); -1 for len(sorted_ids), less to check a
    sample of a routing's entries."""
    rnd = round_bf16 if bf16 else round_f16
    size_m = len(sorted_ids) if size_m < 0 else size_m
    per = nbytes(qtype, n * k)
    out = np.full((size_m, n), np.nan, dtype=np.float32)
    wcache = {}
    for i in range(len(sorted_ids)):
        p, e = int(sorted_ids[i]), int(expert_ids[i])
        if not (0 <= p < size_m and 0 <= e < num_experts):
            continue
        if e not in wcache:
            w = to_float(qtype, stack[e * per:(e + 1) * per], n * k).reshape(n, k)
            wcache[e] = rnd(w).astype(np.float64)
        row = p if topk_w is not None else p // topk
        xr = rnd(np.asarray(x[row], dtype=np.float32)).astype(np.float64)
        with np.errstate(invalid="ignore"):  # 0 * inf weights give NaN, as in the kernel
            y = wcache[e] @ xr
        scale = np.float64(np.float32(topk_w[p])) if topk_w is not None else 1.0
        out[p] = (y * scale).astype(np.float32)
    return out
