"""The CPU oracle of the prompt grouped product (qref.moe_prefill, the
reference's moe_gemm_gguf_prefill) pinned without a GPU: its roundings
against independent implementations (the oracle's C restatement of the
reference's f32 -> f16 conversion, torch's bf16 conversion), and the product
itself on inputs whose result is known exactly (one-hot input rows pick a
weight column; routing order and per-pair scales)."""
import numpy as np
import pytest
import torch

from oracle import qref

SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 65519.99, 1e-8, 5.96e-8, 2.98e-8, 6.1e-5, -6.1e-5,
                    1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 3.0e38, -3.4e38,
                    np.inf, -np.inf], dtype=np.float32)


def test_round_f16_is_the_references_conversion():
    rng = np.random.default_rng(7)
    x = np.concatenate([SPECIAL, rng.standard_normal(20000).astype(np.float32) * np.float32(100),
                        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-5)])
    got = qref.round_f16(x).astype(np.float16).view(np.uint16)
    want = np.array([qref.f32_to_f16_bits(v) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_round_bf16_is_torchs_conversion():
    rng = np.random.default_rng(8)
    x = np.concatenate([SPECIAL, rng.standard_normal(50000).astype(np.float32) * np.float32(10),
                        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-38)])
    got = qref.round_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7
    assert qref.round_bf16(np.float32([1.0 + 2.0 ** -8]))[0] == 1.0
    assert qref.round_bf16(np.float32([1.0 + 3 * 2.0 ** -8]))[0] == 1.0 + 2.0 ** -6
    assert np.isnan(qref.round_bf16(np.float32([np.nan]))[0])


def _stack(qtype, e, n, k, seed):
    rng = np.random.default_rng(seed)
    return np.concatenate([qref.from_float(qtype, (rng.standard_normal(n * k) * 0.02).astype(np.float32))
                           for _ in range(e)])


@pytest.mark.parametrize("qtype", [qref.Q8_0, qref.Q4_K, qref.Q6_K, qref.IQ4_NL, qref.MXFP4])
@pytest.mark.parametrize("bf16", [False, True])
def test_one_hot_rows_pick_rounded_weight_columns(qtype, bf16):
    e, n, k, topk, tokens = 3, 8, 256, 2, 4
    stack = _stack(qtype, e, n, k, 11 + qtype)
    sorted_ids = np.array([1, 6, 0, 3, 4, 2, 5, 7], np.int32)
    expert_ids = np.array([0, 0, 1, 1, 1, 2, 2, 2], np.int32)
    cols = [5, 130, 77, 255]  # token t's input row is e_{cols[t]}
    x = np.zeros((tokens, k), np.float32)
    for t, c in enumerate(cols):
        x[t, c] = 1.0
    out = qref.moe_prefill(qtype, stack, e, n, k, x, bf16, sorted_ids, expert_ids, None, topk)
    rnd = qref.round_bf16 if bf16 else qref.round_f16
    per = qref.nbytes(qtype, n * k)
    for p, ex in zip(sorted_ids, expert_ids):
        w = qref.to_float(qtype, stack[ex * per:(ex + 1) * per], n * k).reshape(n, k)
        assert np.array_equal(out[p], rnd(w[:, cols[p // topk]]) + 0.0), f"pair {p}"


def test_scales_inputs_and_order():
    qtype, e, n, k, topk = qref.Q4_K, 4, 16, 512, 2
    stack = _stack(qtype, e, n, k, 3)
    rng = np.random.default_rng(5)
    size_m = 12
    pairs = sorted((int(rng.integers(e)), p) for p in range(size_m))
    expert_ids = np.array([a for a, _ in pairs], np.int32)
    sorted_ids = np.array([b for _, b in pairs], np.int32)
    x = rng.standard_normal((size_m, k)).astype(np.float32)
    tw = rng.random(size_m).astype(np.float32)
    out = qref.moe_prefill(qtype, stack, e, n, k, x, False, sorted_ids, expert_ids, tw, topk)
    # per-pair inputs and scales: row p is pair p's own input times its weight
    per = qref.nbytes(qtype, n * k)
    p, ex = int(sorted_ids[3]), int(expert_ids[3])
    w = qref.round_f16(qref.to_float(qtype, stack[ex * per:(ex + 1) * per], n * k).reshape(n, k))
    want = (w.astype(np.float64) @ qref.round_f16(x[p]).astype(np.float64)) * np.float64(tw[p])
    assert np.allclose(out[p], want, rtol=1e-6, atol=1e-7)
    # entries in any order, and out-of-range entries writing nothing
    perm = rng.permutation(size_m)
    assert np.array_equal(out, qref.moe_prefill(qtype, stack, e, n, k, x, False, sorted_ids[perm],
                                                 expert_ids[perm], tw, topk))
    bad_e = expert_ids.copy()
    bad_e[0] = e
    got = qref.moe_prefill(qtype, stack, e, n, k, x, False, sorted_ids, bad_e, tw, topk)
    assert np.isnan(got[sorted_ids[0]]).all() and np.array_equal(np.delete(got, sorted_ids[0], 0),
                                                                  np.delete(out, sorted_ids[0], 0))
