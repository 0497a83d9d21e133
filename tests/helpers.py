"""Shared helpers of the parity tests."""
from __future__ import annotations

import numpy as np

from oracle import qref

# GGUF ids, product <-> oracle
TYPES = {"Q8_0": 8, "Q4_K": 12, "Q6_K": 14, "IQ4_NL": 20, "MXFP4": 39}

# Tolerances of the path: max |y_gpu - y_cpu| /
# (||w_j|| * ||x_r||), w_j the CPU-dequantized weight row, x_r the f32 row.
TOL_MATVEC = 1e-3
TOL_GEMM = 2e-3


def normalised_error(y_gpu: np.ndarray, y_cpu: np.ndarray, w_deq: np.ndarray, x: np.ndarray) -> float:
    norm = np.linalg.norm(w_deq.astype(np.float64), axis=1)[None, :] * np.linalg.norm(x.astype(np.float64), axis=1)[:, None]
    norm = np.where(norm == 0, 1.0, norm)
    return float(np.max(np.abs(y_gpu.astype(np.float64) - y_cpu.astype(np.float64)) / norm))


def weights(rng: np.random.Generator, n: int, k: int, std: float = 0.02) -> np.ndarray:
    return (rng.standard_normal((n, k)) * std).astype(np.float32)


def special_rows(k: int) -> np.ndarray:
    """Rows that exercise the quantizers' edge cases: zeros, a constant, one
    outlier, ties in |x| of both signs, tiny (subnormal-scale) values,
    all-positive and all-negative runs, values near powers of two."""
    rows = []
    rows.append(np.zeros(k, np.float32))
    rows.append(np.full(k, 0.37, np.float32))
    r = np.full(k, 0.01, np.float32); r[k // 3] = 5.0; rows.append(r)
    r = np.linspace(-1, 1, k, dtype=np.float32); r[5] = 2.0; r[6] = -2.0; rows.append(r)
    r = np.linspace(-1, 1, k, dtype=np.float32); r[9] = -3.0; r[200 % k] = 3.0; rows.append(r)
    rows.append((np.arange(k, dtype=np.float32) % 7 - 3) * np.float32(1e-39))
    rows.append(np.abs(np.sin(np.arange(k, dtype=np.float32))) + np.float32(0.5))
    rows.append(-np.abs(np.cos(np.arange(k, dtype=np.float32))) - np.float32(0.25))
    p = np.float32(2.0) ** np.arange(-6, 6, dtype=np.float32)
    r = np.resize(np.concatenate([p, np.nextafter(p, np.float32(0)), np.nextafter(p, np.float32(10))]), k)
    rows.append(r.astype(np.float32))
    return np.stack(rows).astype(np.float32)


def oracle_matmul(qtype: int, x: np.ndarray, wq: np.ndarray, n: int) -> np.ndarray:
    return qref.matmul(qtype, x, wq, n)
