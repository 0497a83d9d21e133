"""The C-ABI library without a GPU: it loads, exports every symbol
include/qmm.h declares, and its host-only entry points (sizes, layouts,
argument checks, the plan step of qmm_forward) answer as documented."""
import ctypes
import os
import re

import pytest

from swarmllm_amd import _lib
from swarmllm_amd._lib import lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "qmm.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qmm_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 15
    L = lib()
    for name in names:
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_type_registry():
    L = lib()
    assert [L.qmm_block_size(t) for t in (8, 12, 14, 20, 39)] == [32, 256, 256, 32, 32]
    assert L.qmm_block_size(2) == 0
    # GgmlDType::type_size x elements / block_size (quantized/mod.rs:421-461)
    assert L.qmm_type_bytes(12, 14336 * 4096) == 33_030_144
    assert L.qmm_type_bytes(14, 4096 * 14336) == 48_168_960
    assert L.qmm_type_bytes(8, 4096 * 4096) == 17_825_792
    assert L.qmm_type_bytes(39, 5760 * 2880) == 8_812_800
    assert L.qmm_type_bytes(20, 4096 * 4096) == 9_437_184
    assert L.qmm_type_bytes(12, 100) == 0


def test_activation_layouts():
    L = lib()
    assert L.qmm_act_layout(12, 1) == _lib.ACT_Q8K
    assert L.qmm_act_layout(14, 8) == _lib.ACT_Q8K
    for t in (8, 20, 39):
        assert L.qmm_act_layout(t, 1) == _lib.ACT_Q8_0
    assert L.qmm_act_layout(3, 1) == -1
    assert L.qmm_act_bytes(_lib.ACT_Q8K, 4096, 1) >= 4096 + 16 * 4 + 256 * 2
    assert L.qmm_act_bytes(_lib.ACT_Q8K, 100, 1) == 0
    co, so, uo = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    assert L.qmm_act_planes(_lib.ACT_Q8_0, 2880, 8, ctypes.byref(co), ctypes.byref(so), ctypes.byref(uo)) == 0
    assert co.value == 0 and so.value >= 8 * 2880 and uo.value >= so.value + 8 * 90 * 4
    assert so.value % 16 == 0 and uo.value % 16 == 0


def test_forward_plans_without_a_device_and_rejects_bad_shapes():
    L = lib()
    need = ctypes.c_size_t(0)
    # plan only (launch = 0): no device touched
    st = L.qmm_forward(12, None, None, 4096, None, 14336, None, 0, ctypes.byref(need), 4096, 14336, 1, 0, 0)
    assert st == _lib.QMM_OK and need.value == L.qmm_act_bytes(_lib.ACT_Q8K, 4096, 1)
    # k not a multiple of the block, unknown type, no need pointer, bad ldd / stride
    assert L.qmm_forward(12, None, None, 100, None, 8, None, 0, ctypes.byref(need), 100, 8, 1, 0, 0) == _lib.QMM_UNSUPPORTED
    assert L.qmm_forward(3, None, None, 256, None, 8, None, 0, ctypes.byref(need), 256, 8, 1, 0, 0) == _lib.QMM_UNSUPPORTED
    assert L.qmm_forward(12, None, None, 256, None, 8, None, 0, None, 256, 8, 1, 0, 0) == _lib.QMM_UNSUPPORTED
    assert L.qmm_forward(12, None, None, 256, None, 4, None, 0, ctypes.byref(need), 256, 8, 1, 0, 0) == _lib.QMM_UNSUPPORTED
    assert L.qmm_forward(12, None, None, 128, None, 8, None, 0, ctypes.byref(need), 256, 8, 1, 0, 0) == _lib.QMM_UNSUPPORTED
    # no activation rows, no weight rows (the host API returns an empty output before calling)
    assert L.qmm_forward(12, None, None, 256, None, 8, None, 0, ctypes.byref(need), 256, 8, 0, 0, 0) == _lib.QMM_UNSUPPORTED
    assert L.qmm_forward(12, None, None, 256, None, 8, None, 0, ctypes.byref(need), 256, 0, 1, 0, 0) == _lib.QMM_UNSUPPORTED
    # a launch with too small a workspace is refused before anything is enqueued
    assert L.qmm_forward(12, None, None, 256, None, 8, None, 0, ctypes.byref(need), 256, 8, 1, 1, 0) == \
        _lib.QMM_WORKSPACE_TOO_SMALL
    assert L.qmm_matvec(12, None, None, None, 8, 256, 8, L.qmm_matvec_max_rows() + 1, 0) == _lib.QMM_UNSUPPORTED


def test_moe_plans_without_a_device_and_rejects_bad_routing_shapes():
    L = lib()
    need = ctypes.c_size_t(0)
    # C4 gate_up plan: 8 tokens x top-4, per-token inputs; no device touched
    st = L.qmm_moe_forward(39, None, 32, None, 2880, None, None, None, 4, None, 5760, None, 0, ctypes.byref(need),
                           2880, 5760, 32, 0, 0)
    act = (L.qmm_act_bytes(_lib.ACT_Q8_0, 2880, 8) + 255) // 256 * 256
    assert st == _lib.QMM_OK and need.value == act + 4 * (1 + 3 * 32)
    # per-pair inputs (routing weights given) quantize one row per entry
    fake_w = ctypes.c_void_p(16)
    st = L.qmm_moe_forward(39, None, 32, None, 2880, None, None, fake_w, 4, None, 2880, None, 0, ctypes.byref(need),
                           2880, 2880, 32, 0, 0)
    assert st == _lib.QMM_OK and need.value == (L.qmm_act_bytes(_lib.ACT_Q8_0, 2880, 32) + 255) // 256 * 256 + 4 * 97
    # Q4_K / Q6_K experts quantize the activation per 256 values (Q8_K planes)
    for t in (12, 14):
        st = L.qmm_moe_forward(t, None, 128, None, 2048, None, None, None, 8, None, 768, None, 0,
                               ctypes.byref(need), 2048, 768, 32, 0, 0)
        assert st == _lib.QMM_OK
        assert need.value == (L.qmm_act_bytes(_lib.ACT_Q8K, 2048, 4) + 255) // 256 * 256 + 4 * 97
    # size_m not a multiple of topk without weights, K-quant rows past 16384
    # values, no experts
    assert L.qmm_moe_forward(39, None, 32, None, 2880, None, None, None, 4, None, 5760, None, 0, ctypes.byref(need),
                             2880, 5760, 30, 0, 0) == _lib.QMM_UNSUPPORTED
    assert L.qmm_moe_forward(12, None, 32, None, 16640, None, None, None, 4, None, 64, None, 0, ctypes.byref(need),
                             16640, 64, 32, 0, 0) == _lib.QMM_UNSUPPORTED
    assert L.qmm_moe_forward(39, None, 0, None, 2880, None, None, None, 4, None, 64, None, 0, ctypes.byref(need),
                             2880, 64, 32, 0, 0) == _lib.QMM_UNSUPPORTED


def test_fault_injection_is_host_side_and_one_shot():
    L = lib()
    need = ctypes.c_size_t(0)
    L.qmm_fail_next_launch()
    # the plan step is not a launch: the flag survives it
    assert L.qmm_forward(12, None, None, 256, None, 8, None, 0, ctypes.byref(need), 256, 8, 1, 0, 0) == _lib.QMM_OK
    assert L.qmm_forward(12, None, None, 256, None, 8, None, 0, ctypes.byref(need), 256, 8, 1, 1, 0) == _lib.QMM_NO_ROOM
    # once only: the next launch goes on to its own checks
    assert L.qmm_forward(12, None, None, 256, None, 8, None, 0, ctypes.byref(need), 256, 8, 1, 1, 0) == \
        _lib.QMM_WORKSPACE_TOO_SMALL


def test_available_is_false_without_a_gfx950():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is present")
    assert lib().qmm_available() == 0


def test_mmq_lines_default_and_force_dmmv_flag():
    """The few-rows line as the reference draws it (K-quants from 4 rows,
    2 MiB; the 32-value formats keep the decode kernels to 8 rows), no row
    cap, captured products allowed; set_force_dmmv is a process flag."""
    L = lib()
    rows, nbytes = ctypes.c_int64(0), ctypes.c_int64(0)
    for t, fewest in ((12, 4), (14, 4), (8, 9), (20, 9), (39, 9)):
        assert L.qmm_mmq_few_rows_line(t, ctypes.byref(rows), ctypes.byref(nbytes)) == _lib.QMM_OK
        assert (rows.value, nbytes.value) == (fewest, 2 << 20)
    assert L.qmm_mmq_few_rows_line(3, ctypes.byref(rows), ctypes.byref(nbytes)) == _lib.QMM_UNSUPPORTED
    assert L.qmm_mmq_max_rows() == 2**63 - 1 and L.qmm_mmq_captured() == 1
    assert L.qmm_force_dmmv() == 0
    L.qmm_set_force_dmmv(1)
    assert L.qmm_force_dmmv() == 1
    L.qmm_set_force_dmmv(0)
    assert L.qmm_force_dmmv() == 0


def _knobs_in_child(env: dict) -> list:
    """The lines a fresh process reads with `env` added (the environment is read once)."""
    import json
    import os
    import subprocess
    import sys
    code = ("import ctypes, json; from swarmllm_amd._lib import lib; L = lib(); r, b = ctypes.c_int64(), "
            "ctypes.c_int64(); out = []\n"
            "for t in (12, 8):\n"
            "    L.qmm_mmq_few_rows_line(t, ctypes.byref(r), ctypes.byref(b)); out.append([r.value, b.value])\n"
            "out.append([L.qmm_mmq_max_rows(), L.qmm_mmq_captured()]); print(json.dumps(out))")
    full = dict(os.environ)
    for k in list(full):
        if k.startswith("SWARMLLM_QMATMUL_MMQ"):
            del full[k]
    full.update(env)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, "-c", code], env=full, cwd=root, capture_output=True, text=True,
                         timeout=120, check=True)
    return json.loads(res.stdout.strip().splitlines()[-1])


def test_mmq_switches_read_from_the_environment():
    assert _knobs_in_child({}) == [[4, 2 << 20], [9, 2 << 20], [2**63 - 1, 1]]
    got = _knobs_in_child({"SWARMLLM_QMATMUL_MMQ_MIN_ROWS": "3", "SWARMLLM_QMATMUL_MMQ_FEW_ROWS_BYTES": "0",
                           "SWARMLLM_QMATMUL_MMQ_MAX_ROWS": "100", "SWARMLLM_QMATMUL_MMQ_CAPTURED": "off"})
    assert got == [[3, 0], [3, 0], [100, 0]]
    # off in any of its spellings; counts that do not parse leave the default
    for off in ("dp4a", "0", "off", "false"):
        assert _knobs_in_child({"SWARMLLM_QMATMUL_MMQ": off})[2] == [0, 1]
    got = _knobs_in_child({"SWARMLLM_QMATMUL_MMQ": "on", "SWARMLLM_QMATMUL_MMQ_MIN_ROWS": "-1",
                           "SWARMLLM_QMATMUL_MMQ_FEW_ROWS_BYTES": "2 MiB", "SWARMLLM_QMATMUL_MMQ_MAX_ROWS": "x",
                           "SWARMLLM_QMATMUL_MMQ_CAPTURED": "1"})
    assert got == [[4, 2 << 20], [9, 2 << 20], [2**63 - 1, 1]]
