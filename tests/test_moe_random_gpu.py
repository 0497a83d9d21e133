"""Grouped expert products (qmm_moe_forward) at seeded random shapes and
routings: the type, the experts E, the weight rows n, the row length k, the
tokens and top-k, per-token or per-pair inputs with routing weights, drawn
from a fixed seed, so the grouped kernels' lines are crossed (MXFP4 rows of
up to 128 blocks: the matrix-core form; rows of fewer than 64 blocks, 64-126
blocks of an even count: the packed form, odd counts, past 4096 values: the
per-row form; the K-quants' run kernels).
Each entry is checked against the oracle's product of its pair (1e-3
normalised, the decode bound) and against qmm_forward of its pair bit for
bit (the reference's matmul_many equals per-job forward,
quantized/mod.rs:743-745)."""
import numpy as np
import pytest

from test_moe_gpu import (MOE_TYPES, check_against_forward, check_against_oracle, expert_stack, routing, t32)
from swarmllm_amd import moe_forward

pytestmark = pytest.mark.gpu

N_CASES = 32


def draw_cases():
    rng = np.random.default_rng(31337)
    names = list(MOE_TYPES)
    cases = []
    while len(cases) < N_CASES:
        name = names[int(rng.integers(len(names)))]
        if MOE_TYPES[name] in (12, 14):
            k = 256 * int(rng.integers(1, 33))  # to 8192
        else:
            k = 32 * int(rng.integers(1, 161))  # to 5120
        E = int(rng.integers(1, 17))
        n = int(rng.integers(1, 700))
        tokens = int(rng.integers(1, 9))
        topk = int(rng.integers(1, min(E, 4) + 1))
        if E * n * k > 40_000_000:
            continue
        weighted = bool(rng.integers(2))
        cases.append((name, E, n, k, tokens, topk, weighted, int(rng.integers(1 << 30))))
    return cases


CASES = draw_cases()


@pytest.mark.parametrize("name,E,n,k,tokens,topk,weighted,seed", CASES,
                         ids=[f"{c[0]}-E{c[1]}-n{c[2]}-k{c[3]}-t{c[4]}x{c[5]}{'-w' if c[6] else ''}" for c in CASES])
def test_moe_random_shape(name, E, n, k, tokens, topk, weighted, seed):
    qtype = MOE_TYPES[name]
    sorted_ids, expert_ids, topk_w = routing(tokens, E, topk, seed)
    stack = expert_stack(qtype, E, n, k, seed & 0xFFFF)
    rows = tokens * topk if weighted else tokens
    x = np.random.default_rng(seed).standard_normal((rows, k)).astype(np.float32)
    xs = t32(x)
    tw = topk_w if weighted else None
    out = moe_forward(xs, stack, t32(sorted_ids), t32(expert_ids), t32(topk_w) if weighted else None, topk)
    out = out.cpu().numpy()
    check_against_oracle(qtype, stack, x, out, sorted_ids, expert_ids, tw, topk)
    check_against_forward(stack, xs, out, sorted_ids, expert_ids, tw, topk)
