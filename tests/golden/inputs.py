"""Input generators of the reference's own tests, restated in numpy.

Each function cites the reference test it follows (paths relative to the
reference checkout). They produce the inputs the known-answer values in
reference_kats.json were computed on.
"""
from __future__ import annotations

import numpy as np

M32 = 0xFFFFFFFF
M64 = 0xFFFFFFFFFFFFFFFF


class XorShift:
    """xorshift32: src/inference/mod.rs:1400-1410 (and :1643-1657)."""

    def __init__(self, seed: int):
        self.s = seed & M32

    def next(self) -> int:
        s = self.s
        s ^= (s << 13) & M32
        s ^= s >> 17
        s ^= (s << 5) & M32
        self.s = s
        return s

    def q8(self) -> int:
        """A Q8 byte within +-127 (src/inference/mod.rs:1653-1656)."""
        return ((self.next() % 255) - 127) & 0xFF


def fnv1a(data: bytes) -> int:
    h = 0xCBF29CE484222325
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & M64
    return h


def f32(v) -> np.float32:
    return np.float32(v)


def mxfp4_inputs():
    """src/inference/mod.rs:1439-1464: 9 MXFP4 blocks, 9 Q8_0 blocks, 192 values."""
    r = XorShift(0x12345678)
    x = bytearray()
    for b in range(9):
        e = 0 if b == 0 else (1 if b == 1 else 110 + r.next() % 30)
        x.append(e)
        x.extend((r.next() & 0xFF) for _ in range(16))
    y = bytearray()
    for _ in range(9):
        y.extend(int(0x2000 + r.next() % 0x2000).to_bytes(2, "little"))
        y.extend((r.next() & 0xFF) for _ in range(32))
    src = [f32(f32((r.next() % 20001) - 10000) / f32(997.0)) for _ in range(128)]
    src += [f32(0.0)] * 32
    src += [f32(f32((r.next() % 2001) - 1000) / f32(65536.0)) for _ in range(32)]
    return (np.frombuffer(bytes(x), np.uint8).copy(), np.frombuffer(bytes(y), np.uint8).copy(),
            np.array(src, dtype=np.float32))


def _to_quantize(r: XorShift, n: int) -> np.ndarray:
    """src/inference/mod.rs:1693-1704."""
    q = n // 4
    src = [f32(f32((r.next() % 20001) - 10000) / f32(997.0)) for _ in range(q)]
    src += [f32(0.0)] * q
    src += [f32(f32((r.next() % 2001) - 1000) / f32(65536.0)) for _ in range(q)]
    src += [f32(f32((r.next() % 2001) - 1000) / f32(500.0)) for _ in range(n - 3 * q)]
    out = np.array(src, dtype=np.float32)
    out[3 * q + 5] = 37.5
    return out


def iq4_inputs():
    """src/inference/mod.rs:1706-1764: IQ4_NL blocks, Q8_0 blocks, and the
    256 values IQ4_NL's quantizer is checked on. The IQ4_XS / Q8_K draws in
    between are made (and dropped) so the stream stays aligned."""
    r = XorShift(0x12345678)
    nl = bytearray()
    for b in range(9):
        d = 0x2000 + r.next() % 0x2000
        if b == 2:
            d |= 0x8000
        nl.extend(int(d).to_bytes(2, "little"))
        nl.extend((r.next() & 0xFF) for _ in range(16))
    q8 = bytearray()
    for _ in range(9):
        q8.extend(int(0x2000 + r.next() % 0x2000).to_bytes(2, "little"))
        q8.extend(r.q8() for _ in range(32))
    for _ in range(3):  # IQ4_XS super-blocks
        r.next()
        r.next()
        for _ in range(4 + 128):
            r.next()
    for _ in range(3):  # Q8_K blocks
        r.next()
        for _ in range(256):
            r.q8()
    nl_src = _to_quantize(r, 8 * 32)
    return (np.frombuffer(bytes(nl), np.uint8).copy(), np.frombuffer(bytes(q8), np.uint8).copy(), nl_src)


def lcg_noise(seed: int):
    """The LCG of src/inference/mod.rs:1297-1303 / :1353-1359:
    ((seed >> 33) as f32 / 2^31 - 0.5) * 2."""
    state = [seed & M64]

    def draw(n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        s = state[0]
        for i in range(n):
            s = (s * 6364136223846793005 + 1442695040888963407) & M64
            out[i] = (np.float32(s >> 33) / np.float32(2147483648.0) - np.float32(0.5)) * np.float32(2.0)
        state[0] = s
        return out

    return draw


def get_test_vector2(bound: float, size: int) -> np.ndarray:
    """get_test_vector2: tests/quantized_tests.rs:395-407."""
    v = np.arange(size, dtype=np.float32)
    half = np.float32(size / 2)
    return ((v - half) * np.float32(bound) / half).astype(np.float32)


def ggml_like_vector(offset: float, size: int = 32 * 128) -> np.ndarray:
    """create_ggml_like_vector: tests/quantized_tests.rs:430-434."""
    i = np.arange(size, dtype=np.float32) + np.float32(offset)
    return (np.float32(0.1) + np.float32(2.0) * np.cos(i).astype(np.float32)).astype(np.float32)


# ---- rand 0.9 StdRng (ChaCha12) for tests/quantized_tests.rs:1127-1148 -------
def _rotl(v, c):
    return ((v << c) | (v >> (32 - c))) & M32


def _chacha_block(key_words, counter, rounds=12):
    c = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574]
    st = c + list(key_words) + [counter & M32, (counter >> 32) & M32, 0, 0]
    x = list(st)

    def qr(a, b, cc, d):
        x[a] = (x[a] + x[b]) & M32; x[d] = _rotl(x[d] ^ x[a], 16)
        x[cc] = (x[cc] + x[d]) & M32; x[b] = _rotl(x[b] ^ x[cc], 12)
        x[a] = (x[a] + x[b]) & M32; x[d] = _rotl(x[d] ^ x[a], 8)
        x[cc] = (x[cc] + x[d]) & M32; x[b] = _rotl(x[b] ^ x[cc], 7)

    for _ in range(rounds // 2):
        qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15)
        qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14)
    return [(x[i] + st[i]) & M32 for i in range(16)]


class StdRng:
    """rand 0.9 `StdRng::seed_from_u64` (rand_core's PCG32 seed expansion into
    a ChaCha12 key, counter 0, stream 0) and `random::<f32>()`
    ((next_u32 >> 8) * 2^-24). A restatement: pinned by the f32 matmul KAT
    [1.262, 1.513, -0.208, 1.702] the reference asserts on these draws."""

    def __init__(self, seed: int):
        state = seed & M64
        key = []
        for _ in range(8):
            state = (state * 6364136223846793005 + 11634580027462260723) & M64
            xorshifted = (((state >> 18) ^ state) >> 27) & M32
            rot = state >> 59
            key.append(((xorshifted >> rot) | (xorshifted << ((32 - rot) & 31))) & M32)
        self.key = key
        self.counter = 0
        self.buf = []

    def next_u32(self) -> int:
        if not self.buf:
            self.buf = _chacha_block(self.key, self.counter)
            self.counter += 1
        return self.buf.pop(0)

    def random_f32(self, n: int) -> np.ndarray:
        return np.array([np.float32(self.next_u32() >> 8) * np.float32(2.0 ** -24) for _ in range(n)],
                        dtype=np.float32)


def random_tensors(m: int, k: int, n: int, seed: int = 314159265358979):
    """get_random_tensors: lhs [m, k], rhs [n, k], each rng.random::<f32>() - 0.5."""
    rng = StdRng(seed)
    lhs = (rng.random_f32(m * k) - np.float32(0.5)).astype(np.float32).reshape(m, k)
    rhs = (rng.random_f32(n * k) - np.float32(0.5)).astype(np.float32).reshape(n, k)
    return lhs, rhs


def rust_round(x):
    """f32::round: half away from zero."""
    x = np.asarray(x, dtype=np.float64)
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def round3(values):
    """round_vector: tests/quantized_tests.rs:410-415."""
    return [float(rust_round(np.float32(1000.0) * np.float32(v)) / 1000.0) for v in values]
