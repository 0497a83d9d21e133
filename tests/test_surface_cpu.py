"""Host-side parts of the device arm's surface without a GPU: the row size
of a gathered table, the accumulate_in_f32 and prepare entries' answers for
a type not covered, and the reference's switches this build accepts without
effect (CANDLE_DEQUANTIZE_ALL[_F16], SWARMLLM_QMATMUL_CUBLAS*)."""
import ctypes

import pytest

from swarmllm_amd import qtensor
from swarmllm_amd._lib import QMM_OK, QMM_UNSUPPORTED, lib


def test_gather_row_bytes():
    L = lib()
    rb = ctypes.c_size_t(0)
    for t, hidden, want in ((12, 4096, 16 * 144), (14, 512, 2 * 210), (8, 2880, 90 * 34), (39, 96, 3 * 17),
                            (20, 32, 18), (0, 7, 28), (1, 5, 10), (30, 3, 6)):
        assert L.qmm_gather_row_bytes(t, hidden, ctypes.byref(rb)) == QMM_OK
        assert rb.value == want, (t, hidden)
    for t, hidden in ((12, 200), (8, 33), (3, 256), (12, 0)):
        assert L.qmm_gather_row_bytes(t, hidden, ctypes.byref(rb)) == QMM_UNSUPPORTED


def test_accumulate_in_f32_and_prepare_answer_for_the_types():
    L = lib()
    for t in (8, 12, 14, 20, 39):
        assert L.qmm_accumulate_in_f32(t) == QMM_OK
    for t in (0, 2, 13, 100):
        assert L.qmm_accumulate_in_f32(t) == QMM_UNSUPPORTED
        assert L.qmm_prepare(t) == QMM_UNSUPPORTED


@pytest.mark.parametrize("name,value,on", [("CANDLE_DEQUANTIZE_ALL", "1", True), ("CANDLE_DEQUANTIZE_ALL", "0", False),
                                           ("CANDLE_DEQUANTIZE_ALL_F16", "", False),
                                           ("CANDLE_DEQUANTIZE_ALL_F16", "yes", True),
                                           ("SWARMLLM_QMATMUL_CUBLAS", "0", True),
                                           ("SWARMLLM_QMATMUL_CUBLAS_MIN_ROWS", "128", True),
                                           ("SWARMLLM_QMATMUL_CUBLAS_ACC", "32", True)])
def test_inactive_knobs_are_accepted_and_reported(monkeypatch, name, value, on):
    for k in qtensor.INACTIVE_KNOBS:
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv(name, value)
    assert qtensor.inactive_knobs_set() == ([name] if on else [])
    monkeypatch.setattr(qtensor, "_KNOBS_REPORTED", False)
    if on:
        with pytest.warns(RuntimeWarning, match=name):
            qtensor._report_inactive_knobs()
    else:
        qtensor._report_inactive_knobs()
    # reported once a process
    qtensor._report_inactive_knobs()
