"""CPU emulation (numpy) of the approximate weight operands of three kernels,
to pin their parity margins on weights of any scale pattern:

  - the single-pass Q4_K GEMM (swarmllm_amd/csrc/gemm_q4k_sp.hip): the weight
    enters the int8 matrix cores as w8 = floor((sc (q - 8) + 2) / 4), and
    per super-block
        out += 4 d dy sum_i w8_i y_i
             + sum_j f16(dy S_j 2^-8) f16((8 d sc_j - dmin m_j) 2^8)
    (S_j the activation codes' sum over sub-block j, the f16 products exact
    in f32 and summed in f32);
  - the single-pass Q6_K GEMM (same file): w8 = floor((m_j (q - 32) + 128) /
    256) with m_j = floor((127 sc_j + 8) / 16), and per super-block
        out += T f16(dy / 2) f16(d 4096 / 127 * 128) / 64,  T = sum_i w8_i y_i;
  - the few-row Q6_K kernel's single-product form (gemm_q6k_skinny.hip, from
    k = 2048): the same w8, out += f32(f32(d 4096 / 127) dy) T in f32.

Here dy already carries the GEMMs' per-row power-of-two factor (exact) and is
the Q8_K scale of the activation (BlockQ8K::from_float, the oracle's
quantize_rows); y its int8 codes. The block layouts are parsed here from the
GGUF bytes (BlockQ4K / BlockQ6K, vendor/candle/candle-core/src/quantized/
k_quants.rs:2031-2111, 2598-2727), independently of the oracle, and
mode="exact" replaces each rounded operand by the exact one so a test can
check the parsing against the oracle's own product.

TEST INFRASTRUCTURE: only tests import this.
"""
from __future__ import annotations

import numpy as np


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def q8k_fields(xq: np.ndarray, m: int, k: int):
    """BlockQ8K rows (292 bytes: f32 d, 256 int8 codes, 16 int16 sums) ->
    dy (m, nsb) f32, y (m, nsb, 256) int64."""
    nsb = k // 256
    b = xq.reshape(m, nsb, 292)
    dy = b[:, :, 0:4].copy().view("<f4").reshape(m, nsb)
    y = b[:, :, 4:260].view(np.int8).astype(np.int64)
    return dy, y


def q4k_fields(wq: np.ndarray, n: int, k: int):
    """BlockQ4K rows -> d, dmin (n, nsb) f32; sc, mn (n, nsb, 8) int64 (the
    six-bit scales and mins of get_scale_min_k4); q (n, nsb, 256) int64
    codes in element order (64-value chunk c: low nibbles of qs[32c..32c+32]
    for its first 32 values, sub-block 2c; high nibbles for the next 32,
    sub-block 2c + 1)."""
    nsb = k // 256
    b = wq.reshape(n, nsb, 144)
    d = b[:, :, 0:2].copy().view("<f2").astype(np.float32).reshape(n, nsb)
    dmin = b[:, :, 2:4].copy().view("<f2").astype(np.float32).reshape(n, nsb)
    s = b[:, :, 4:16].astype(np.int64)
    sc = np.empty((n, nsb, 8), np.int64)
    mn = np.empty((n, nsb, 8), np.int64)
    for j in range(8):
        if j < 4:
            sc[:, :, j] = s[:, :, j] & 63
            mn[:, :, j] = s[:, :, j + 4] & 63
        else:
            sc[:, :, j] = (s[:, :, j + 4] & 0xF) | ((s[:, :, j - 4] >> 6) << 4)
            mn[:, :, j] = (s[:, :, j + 4] >> 4) | ((s[:, :, j] >> 6) << 4)
    qs = b[:, :, 16:144].astype(np.int64).reshape(n, nsb, 4, 32)
    q = np.concatenate([qs & 0xF, qs >> 4], axis=3).reshape(n, nsb, 256)
    return d, dmin, sc, mn, q


def q6k_fields(wq: np.ndarray, n: int, k: int):
    """BlockQ6K rows -> d (n, nsb) f32; sc (n, nsb, 16) int64 (int8 scale of
    each 16-value group); q (n, nsb, 256) int64 unsigned six-bit codes in
    element order (BlockQ6K::to_float's layout)."""
    nsb = k // 256
    b = wq.reshape(n, nsb, 210)
    ql = b[:, :, 0:128].astype(np.int64)
    qh = b[:, :, 128:192].astype(np.int64)
    sc = b[:, :, 192:208].view(np.int8).astype(np.int64)
    d = b[:, :, 208:210].copy().view("<f2").astype(np.float32).reshape(n, nsb)
    q = np.empty((n, nsb, 256), np.int64)
    for h in range(2):
        L0 = ql[:, :, 64 * h:64 * h + 32]
        L1 = ql[:, :, 64 * h + 32:64 * h + 64]
        H = qh[:, :, 32 * h:32 * h + 32]
        base = 128 * h
        q[:, :, base:base + 32] = (L0 & 0xF) | ((H & 3) << 4)
        q[:, :, base + 32:base + 64] = (L1 & 0xF) | (((H >> 2) & 3) << 4)
        q[:, :, base + 64:base + 96] = (L0 >> 4) | (((H >> 4) & 3) << 4)
        q[:, :, base + 96:base + 128] = (L1 >> 4) | (((H >> 6) & 3) << 4)
    return d, sc, q


def _blocksum(a_sb: np.ndarray, b_sb: np.ndarray) -> np.ndarray:
    """sum_i a[m, s, i] b[n, s, i] -> (m, n, nsb), exact for integer inputs."""
    m, nsb, _ = a_sb.shape
    n = b_sb.shape[0]
    out = np.empty((m, n, nsb), np.float64)
    for s in range(nsb):
        out[:, :, s] = a_sb[:, s, :].astype(np.float64) @ b_sb[:, s, :].astype(np.float64).T
    return out


def q4k_single_pass(wq: np.ndarray, n: int, k: int, xq: np.ndarray, m: int, mode: str = "kernel") -> np.ndarray:
    """The single-pass Q4_K GEMM's output (m, n) f64. mode="exact": the
    weight operand sc (q - 8) exact and the min term in f64 (the reference's
    integer sums, scaled in f64)."""
    d, dmin, sc, mn, q = q4k_fields(wq, n, k)
    dy, y = q8k_fields(xq, m, k)
    nsb = k // 256
    scv = np.repeat(sc, 32, axis=2)  # (n, nsb, 256) the scale of each element's sub-block
    v = scv * (q - 8)
    w8 = v if mode == "exact" else np.floor_divide(v + 2, 4)
    T = _blocksum(y, w8)  # (m, n, nsb)
    S = y.reshape(m, nsb, 8, 32).sum(axis=3)  # (m, nsb, 8)
    d64 = d.astype(np.float64)[None, :, :]
    dy64 = dy.astype(np.float64)[:, None, :]
    main = (1.0 if mode == "exact" else 4.0) * d64 * dy64 * T
    if mode == "exact":
        coef = 8.0 * d.astype(np.float64)[:, :, None] * sc - dmin.astype(np.float64)[:, :, None] * mn  # (n, nsb, 8)
        mint = np.einsum("msj,nsj->mns", dy.astype(np.float64)[:, :, None] * S, coef)
        return (main + mint).sum(axis=2)
    # the f16 operands of the per-super-block product (row factor omitted:
    # a power of two, exact unless the f16 values leave the normal range)
    a = _f16(dy[:, :, None] * S.astype(np.float32) * np.float32(1.0 / 256))  # (m, nsb, 8)
    with np.errstate(over="ignore"):
        bq = _f16((np.float32(8.0) * d[:, :, None] * sc.astype(np.float32) - dmin[:, :, None] * mn.astype(np.float32))
                  * np.float32(256.0))
    mint = np.einsum("msj,nsj->mns", a.astype(np.float64), bq.astype(np.float64))
    return (main + mint).sum(axis=2)


def q6k_w8(sc: np.ndarray, q: np.ndarray) -> np.ndarray:
    """w8 = floor((m_j (q - 32) + 128) / 256), m_j = floor((127 sc_j + 8) / 16)."""
    mj = np.floor_divide(127 * sc + 8, 16)
    return np.floor_divide(np.repeat(mj, 16, axis=2) * (q - 32) + 128, 256)


def q6k_single_product(wq: np.ndarray, n: int, k: int, xq: np.ndarray, m: int, form: str) -> np.ndarray:
    """Output (m, n) f64 of a Q6_K product: form "gemm" (the single-pass
    GEMM, its scales in f16), "few_rows" (the few-row kernel's single-product
    form, scales in f32) or "exact" (sc (q - 32) exact, scaled in f64)."""
    d, sc, q = q6k_fields(wq, n, k)
    dy, y = q8k_fields(xq, m, k)
    if form == "exact":
        T = _blocksum(y, np.repeat(sc, 16, axis=2) * (q - 32))
        return (d.astype(np.float64)[None] * dy.astype(np.float64)[:, None, :] * T).sum(axis=2)
    T = _blocksum(y, q6k_w8(sc, q))
    eff = np.float32(4096.0 / 127.0)
    if form == "gemm":
        s = (_f16(dy * np.float32(0.5)).astype(np.float64)[:, None, :] *
             _f16(d * eff * np.float32(128.0)).astype(np.float64)[None] / 64.0)
    elif form == "few_rows":
        s = (d * eff)[None].astype(np.float32) * dy[:, None, :].astype(np.float32)
        s = s.astype(np.float64)
    else:
        raise ValueError(form)
    return (s * T).sum(axis=2)


def skewed_weights(rng: np.random.Generator, n: int, k: int, unit: int, factor: float, std: float = 0.02):
    """N(0, std) weights with one `unit`-value sub-block (32: a Q4_K
    sub-block; 16: a Q6_K group) per 256-value super-block scaled by
    `factor`: sub-block (3 s) mod (256 / unit) of super-block s, the same in
    every row. Returns (w, big) with big the (k,) mask of the scaled values."""
    w = (rng.standard_normal((n, k)) * std).astype(np.float32)
    per = 256 // unit
    big = np.zeros(k, bool)
    for s in range(k // 256):
        j = (3 * s) % per
        big[256 * s + unit * j:256 * s + unit * (j + 1)] = True
    w[:, big] *= np.float32(factor)
    return w, big


def concentrated_activations(rng: np.random.Generator, m: int, k: int, big: np.ndarray, unit: int) -> np.ndarray:
    """Activations that avoid the scaled sub-blocks (x0.01 there) and put x20
    on one small sub-block of each super-block: the weights' small scales
    carry the product."""
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, big] *= np.float32(0.01)
    per = 256 // unit
    for s in range(k // 256):
        j = (3 * s + 1) % per
        x[:, 256 * s + unit * j:256 * s + unit * (j + 1)] *= np.float32(20.0)
    return x


def outlier_activations(rng: np.random.Generator, m: int, k: int) -> np.ndarray:
    """BASELINE C3's activations: N(0, 1) with 1% of the channels x20."""
    x = rng.standard_normal((m, k)).astype(np.float32)
    ch = rng.permutation(k)[: max(1, k // 100)]
    x[:, ch] *= np.float32(20.0)
    return x
