"""Host-side mirror of candle's quantized tensor API on the MI355X library.

Names, argument meaning and error behaviour follow
vendor/candle/candle-core/src/quantized/mod.rs (GgmlDType :294-461,
QTensor :76-1129, QMatMul :1131-1273, matmul_many :746-780): a QTensor
holds GGUF blocks of an [n, k] weight in device memory; QMatMul.forward(x)
returns x · Wᵀ with x [..., k] f32 contiguous and the result [..., n].

Device memory and streams come from torch (plumbing only); every product,
quantization and dequantization runs in libqmm's HIP kernels through the C
ABI of include/qmm.h.
"""
from __future__ import annotations

import ctypes
import enum
import os
import warnings
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import X_BF16, X_F16, X_F32, check, lib


class GgmlDType(enum.IntEnum):
    """GGUF type ids (mod.rs:319-371): the five formats the products take, and
    F32 / F16 / BF16, which a GGUF file holds beside them (norms, biases) and
    a QTensor stores but no product reads."""

    F32 = 0
    F16 = 1
    Q8_0 = 8
    Q4K = 12
    Q6K = 14
    Iq4Nl = 20
    BF16 = 30
    Mxfp4 = 39

    def block_size(self) -> int:
        return {0: 1, 1: 1, 30: 1, 8: 32, 20: 32, 39: 32, 12: 256, 14: 256}[int(self)]

    def type_size(self) -> int:
        return {0: 4, 1: 2, 30: 2, 8: 34, 12: 144, 14: 210, 20: 18, 39: 17}[int(self)]

    def is_quantized(self) -> bool:
        return int(self) not in (0, 1, 30)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def fill_normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0, device="cuda") -> torch.Tensor:
    """n f32 values from N(mean, std), reproducible from seed (on the device)."""
    out = torch.empty(n, dtype=torch.float32, device=device)
    check("qmm_fill_normal", lib().qmm_fill_normal(_ptr(out), n, seed, mean, std, _stream()))
    return out


class QTensor:
    """GGUF blocks of a weight on the device (mod.rs:76): [n, k] for a
    product, [E, n, k] for a stack of expert weights (one n x k matrix per
    expert, back to back, as stack_some / load_quantized_entries build them,
    mod.rs:989-1025)."""

    def __init__(self, data: torch.Tensor, shape: Sequence[int], dtype: GgmlDType):
        """The blocks of `shape` in `data` (uint8, on the device): exactly their
        bytes, or a storage that holds padding past them (QTensor.alloc)."""
        dtype = GgmlDType(dtype)
        shape = tuple(int(d) for d in shape)
        if len(shape) < 1:
            raise ValueError(f"QTensor: shape {shape} has no dims")
        k = shape[-1]
        qk = dtype.block_size()
        if k % qk:
            raise ValueError(f"quantized tensor must have their last dim divisible by block size {shape} {qk}")
        nel = 1
        for d in shape:
            nel *= d
        want = nel // qk * dtype.type_size()
        if data.dtype != torch.uint8 or data.numel() < want or not data.is_cuda:
            raise ValueError(f"QTensor: {data.numel()} device bytes for {shape} {dtype.name} (want {want})")
        self.storage_ = data.contiguous()
        self.data_ = self.storage_[:want]
        self.shape = shape
        self.dtype = dtype

    @staticmethod
    def alloc(shape: Sequence[int], dtype: GgmlDType, device="cuda") -> "QTensor":
        """Zeroed blocks of `shape` in a device buffer padded by 512 values'
        worth of blocks past them, as the reference pads every device weight
        (MATRIX_ROW_PADDING, quantized/cuda.rs:43, 1846-1870)."""
        dtype = GgmlDType(dtype)
        nel = 1
        for d in shape:
            nel *= int(d)
        padded = lib().qmm_padded_bytes(int(dtype), nel)
        if padded == 0 and nel:
            raise ValueError(f"QTensor.alloc: {list(shape)} is not a whole number of {dtype.name} blocks")
        return QTensor(torch.zeros(max(padded, 1), dtype=torch.uint8, device=device), shape, dtype)

    def padded_bytes(self) -> int:
        """Bytes of the device storage, padding included."""
        return self.storage_.numel()

    def elem_count(self) -> int:
        nel = 1
        for d in self.shape:
            nel *= d
        return nel

    @staticmethod
    def from_data(raw: bytes, shape: Sequence[int], dtype: GgmlDType, device="cuda") -> "QTensor":
        """Blocks from the bytes a GGUF holds them as (QStorage::from_data,
        mod.rs:119-163), in a padded device buffer (cuda::load_quantized)."""
        q = QTensor.alloc(shape, dtype, device)
        if len(raw) != q.data_.numel():
            raise ValueError(f"from_data: {len(raw)} bytes for {list(shape)} {GgmlDType(dtype).name}")
        if len(raw):
            q.data_.copy_(torch.frombuffer(bytearray(raw), dtype=torch.uint8))
        return q

    @staticmethod
    def stack_some(slots: int, parts: Sequence[tuple], device="cuda") -> "QTensor":
        """A [slots, rows, cols] stack holding each (slot, QTensor) part at its
        slot, the other slots zero (QTensor::stack_some / cuda::
        load_quantized_entries, mod.rs:989-1025, cuda.rs:2101-2127): every
        part of one type and 2-D shape; the stack padded as a device weight."""
        if not parts:
            raise ValueError("stack_some: no parts")
        first = parts[0][1]
        if len(first.shape) != 2:
            raise ValueError(f"stack_some: parts must be 2-D, got {first.shape}")
        rows, cols = first.shape
        out = QTensor.alloc((slots, rows, cols), first.dtype, device)
        eb = first.data_.numel()
        for slot, t in parts:
            if t.dtype != first.dtype or t.shape != first.shape:
                raise ValueError(f"stack_some: part {slot} is {t.dtype.name} {t.shape}, not {first.dtype.name} "
                                 f"{first.shape}")
            if not 0 <= slot < slots:
                raise ValueError(f"stack_some: slot {slot} of {slots}")
            out.data_[slot * eb:(slot + 1) * eb].copy_(t.data_)
        return out

    @staticmethod
    def quantize(w: torch.Tensor, dtype: GgmlDType) -> "QTensor":
        """QTensor::quantize (mod.rs:850-880), on the device, bit-exact to from_float."""
        dtype = GgmlDType(dtype)
        if w.dim() != 2:
            raise ValueError("quantize: a 2-D weight [n, k]")
        n, k = w.shape
        if k % dtype.block_size():
            raise ValueError(f"quantize: last dim {k} not divisible by block size {dtype.block_size()}")
        if not dtype.is_quantized():
            raise ValueError(f"quantize: {dtype.name} is not a block format")
        w = w.to(device="cuda", dtype=torch.float32).contiguous()
        nel = n * k
        q = QTensor.alloc((n, k), dtype, w.device)
        sb = lib().qmm_quantize_scratch_bytes(int(dtype), nel)
        scratch = torch.empty(max(sb, 1), dtype=torch.uint8, device=w.device)
        check("qmm_quantize_weights",
              lib().qmm_quantize_weights(int(dtype), _ptr(w), _ptr(q.data_), nel, _ptr(scratch), sb, _stream()))
        return q

    @staticmethod
    def quantize_onto(src: torch.Tensor, dtype: GgmlDType, device="cuda") -> "QTensor":
        """QTensor::quantize_onto (mod.rs:907-932): `src` on the CPU, quantized
        into a QTensor on `device` (any shape whose last dim is a whole number
        of blocks), bit-exact to from_float; the quantization runs on the device."""
        dtype = GgmlDType(dtype)
        if src.device.type != "cpu":
            raise ValueError(f"`quantize_onto` expects a `src` to be on the cpu, got {src.device}.")
        shape = tuple(src.shape)
        qk = dtype.block_size()
        if not shape or shape[-1] % qk:
            raise ValueError(f"quantized tensor must have their last dim divisible by block size {shape} {qk}")
        if not dtype.is_quantized():
            raise ValueError(f"quantize_onto: {dtype.name} is not a block format")
        flat = src.to(torch.float32).contiguous().reshape(-1).to(device)
        nel = flat.numel()
        if nel % qk:
            raise ValueError(f"tensor size ({shape}) is not divisible by block size {qk}")
        q = QTensor.alloc(shape, dtype, device)
        if nel:
            sb = lib().qmm_quantize_scratch_bytes(int(dtype), nel)
            scratch = torch.empty(max(sb, 1), dtype=torch.uint8, device=flat.device)
            check("qmm_quantize_weights", lib().qmm_quantize_weights(int(dtype), _ptr(flat), _ptr(q.data_), nel,
                                                                     _ptr(scratch), sb, _stream()))
        return q

    def gather_rows(self, ids: torch.Tensor, check_ids: bool = True) -> "QTensor":
        """QTensor::gather_rows (mod.rs:1039-1091): the rows `ids` (u32, on
        the table's device) of a [vocab, hidden] table, as a QTensor
        [len(ids), hidden] holding the same blocks (qmm_gather_rows). Rows must
        be a whole number of blocks. An id past the vocabulary raises
        ValueError, as the reference's host path does; that check reads a
        device counter back (a synchronization), and check_ids=False skips it
        (such a row then holds zeros, as does a row of id 0xFFFFFFFF)."""
        if len(self.shape) != 2:
            raise ValueError("gather_rows expects a 2-D [vocab, hidden] tensor")
        vocab, hidden = self.shape
        block = self.dtype.block_size()
        if hidden % block:
            raise ValueError(f"gather_rows: hidden {hidden} is not a whole number of {block}-element blocks")
        if ids.dtype != torch.uint32:
            raise ValueError(f"gather_rows: ids must be u32, got {ids.dtype}")
        if ids.device != self.data_.device:
            raise ValueError("gather_rows: ids must be on the same device")
        flat = ids.contiguous().reshape(-1)
        n_ids = flat.numel()
        L = lib()
        rb = ctypes.c_size_t(0)
        check("qmm_gather_row_bytes", L.qmm_gather_row_bytes(int(self.dtype), hidden, ctypes.byref(rb)))
        out = QTensor.alloc((n_ids, hidden), self.dtype, self.data_.device)
        if n_ids == 0:
            return out
        bad = torch.zeros(1, dtype=torch.int32, device=self.data_.device) if check_ids else None
        check("qmm_gather_rows", L.qmm_gather_rows(int(self.dtype), _ptr(self.data_), self.data_.numel(), vocab, hidden,
                                                   _ptr(flat), n_ids, _ptr(out.data_), out.data_.numel(),
                                                   _ptr(bad) if bad is not None else None, _stream()))
        if bad is not None and int(bad.item()):
            host = flat.cpu().to(torch.int64)
            first = int(host[(host >= vocab) & (host != 0xFFFFFFFF)][0])
            raise ValueError(f"gather_rows: id {first} out of range for vocabulary {vocab}")
        return out

    def device_ptr(self) -> int:
        """The device address of the blocks (QTensor::device_ptr, mod.rs:1120-1127)."""
        return self.data_.data_ptr()

    def indexed_moe_forward(self, x: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
        """QTensor::indexed_moe_forward (mod.rs:1093-1118, the card's
        cuda.rs:1236-1376) in its layout: weights [E, n, k], x [batch, topk or
        1, k] f32, ids [batch, topk] (u32, or int32 / int64 below 2^31)
        naming each token's experts; returns [batch, topk, n] with
        out[b, j] = x[b, j or 0] . W[ids[b, j]]. Served by qmm_moe_forward:
        entry i = b * topk + j pairs slot i with expert ids[b, j] (entries
        sorted by expert on the device, any order giving the same result);
        per-slot inputs (x's middle dim topk) take scale 1 per slot, which
        makes the routing read one input row per slot; a shared input (middle
        dim 1) reads row b for every slot of token b. An expert id out of
        range leaves its row zero, as the reference's zeroed output does."""
        if len(self.shape) != 3:
            raise ValueError(f"indexed_moe_forward: weights [E, n, k], not {self.shape}")
        e, n, k = self.shape
        if ids.dim() != 2:
            raise ValueError(f"indexed_moe_forward: ids [batch, topk], not {tuple(ids.shape)}")
        batch, topk = ids.shape
        if x.dim() != 3 or x.shape[0] != batch or x.shape[1] not in (1, topk) or x.shape[2] != k:
            raise ValueError(f"indexed_moe_forward: x [batch={batch}, {topk} or 1, {k}], not {tuple(x.shape)}")
        if x.dtype != torch.float32:
            raise ValueError("Expected f32")
        out = torch.zeros((batch, topk, n), dtype=torch.float32, device=x.device)
        if batch * topk == 0:
            return out
        flat_ids = ids.reshape(-1)
        if flat_ids.dtype == torch.uint32:
            flat_ids = flat_ids.to(torch.int64)
        expert_ids, order = torch.sort(flat_ids.to(torch.int64), stable=True)
        expert_ids = expert_ids.clamp(-1, 2 ** 31 - 1).to(torch.int32).contiguous()
        sorted_ids = order.to(torch.int32).contiguous()
        per_slot = x.shape[1] == topk and topk > 1
        xs = x.contiguous().reshape(-1, k)
        tw = torch.ones(batch * topk, dtype=torch.float32, device=x.device) if per_slot else None
        L = lib()
        st = _stream()
        need = ctypes.c_size_t(0)
        args = (int(self.dtype), _ptr(self.data_), e, _ptr(xs), k, _ptr(sorted_ids), _ptr(expert_ids),
                _ptr(tw) if tw is not None else None, topk, _ptr(out), n)
        check("qmm_moe_forward", L.qmm_moe_forward(*args, None, 0, ctypes.byref(need), k, n, batch * topk, 0, st))
        buf = torch.empty(max(need.value, 256), dtype=torch.uint8, device=x.device)
        check("qmm_moe_forward", L.qmm_moe_forward(*args, _ptr(buf), buf.numel(), ctypes.byref(need), k, n,
                                                   batch * topk, 1, st))
        return out

    def dequantize(self) -> torch.Tensor:
        return self._dequant(False)

    def dequantize_f16(self) -> torch.Tensor:
        return self._dequant(True)

    def _dequant(self, f16: bool) -> torch.Tensor:
        if not self.dtype.is_quantized():
            # F32 / F16 / BF16 storage: the values themselves
            src = {0: torch.float32, 1: torch.float16, 30: torch.bfloat16}[int(self.dtype)]
            vals = self.data_.view(src).reshape(self.shape)
            return vals.to(torch.float16 if f16 else torch.float32)
        out = torch.empty(self.shape, dtype=torch.float16 if f16 else torch.float32, device=self.data_.device)
        check("qmm_dequantize", lib().qmm_dequantize(int(self.dtype), _ptr(self.data_), _ptr(out), int(f16),
                                                     self.elem_count(), _stream()))
        return out

    def data(self) -> bytes:
        """The GGUF bytes (QTensor::data)."""
        return self.data_.cpu().numpy().tobytes()

    def storage_size_in_bytes(self) -> int:
        return self.data_.numel()

    def __repr__(self) -> str:
        return f"QTensor[{list(self.shape)}; {self.dtype.name}]"


@dataclass
class Workspace:
    """The device buffers the products of one weight quantize their activation
    into: one buffer per (device, stream), kept and grown as needed. Products
    on one stream run in order, so they can share a buffer; products of the
    same weight on two streams may run at once and get a buffer each, and a
    buffer outgrown on a stream is released on that stream, after the work
    already queued there (the reference allocates its temporaries per call)."""

    def __init__(self) -> None:
        self._bufs = {}

    def get(self, nbytes: int, device) -> torch.Tensor:
        device = torch.device(device)
        stream = torch.cuda.current_stream(device)
        key = (device.index, stream.cuda_stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            with torch.cuda.stream(stream):
                buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


# The reference's switches for arms this build does not have, accepted and
# without effect here (reported once, when the first QMatMul is made):
#   CANDLE_DEQUANTIZE_ALL / CANDLE_DEQUANTIZE_ALL_F16 (mod.rs:1138-1180): the
#     weight dequantized to f32 / f16 at QMatMul::from_arc and multiplied as
#     a plain tensor; here every weight stays quantized;
#   SWARMLLM_QMATMUL_CUBLAS / _MIN_ROWS / _ACC (cuda.rs:285-324, 455-470): a
#     prompt's product dequantized to f16 for cuBLAS from 64 rows; here the
#     int8 matrix-core kernels serve every row count, summing in int32 / f32;
#   SWARMLLM_LOAD_PINNED / SWARMLLM_LOAD_READ act in the loader (qmm_gguf_load).
INACTIVE_KNOBS = ("CANDLE_DEQUANTIZE_ALL", "CANDLE_DEQUANTIZE_ALL_F16", "SWARMLLM_QMATMUL_CUBLAS",
                  "SWARMLLM_QMATMUL_CUBLAS_MIN_ROWS", "SWARMLLM_QMATMUL_CUBLAS_ACC")
_KNOBS_REPORTED = False


def inactive_knobs_set() -> List[str]:
    """Those of INACTIVE_KNOBS set in the environment (the reference reads
    CANDLE_DEQUANTIZE_ALL[_F16] as on when non-empty and not "0")."""
    out = []
    for name in INACTIVE_KNOBS:
        v = os.environ.get(name)
        if v is None:
            continue
        if name.startswith("CANDLE_") and (v == "" or v == "0"):
            continue
        out.append(name)
    return out


def _report_inactive_knobs() -> None:
    global _KNOBS_REPORTED
    if _KNOBS_REPORTED:
        return
    _KNOBS_REPORTED = True
    on = inactive_knobs_set()
    if on:
        warnings.warn(f"{', '.join(on)}: accepted with no effect; every product here runs on the quantized "
                      "weights' own kernels", RuntimeWarning, stacklevel=3)


class QMatMul:
    """QMatMul::QTensor (mod.rs:1131-1273, Module::forward :1360-1383)."""

    def __init__(self, qtensor: QTensor):
        _report_inactive_knobs()
        self.qtensor = qtensor
        self._ws = Workspace()

    @staticmethod
    def from_qtensor(qtensor: QTensor) -> "QMatMul":
        return QMatMul(qtensor)

    def accumulate_in_f32(self) -> bool:
        """QMatMul::accumulate_in_f32 (mod.rs:1181-1200): keep this weight's
        products in f32. Every product here sums in int32 / f32 already, so
        nothing changes (qmm_accumulate_in_f32); True, as the reference
        answers for a weight it holds alone."""
        if self.qtensor.dtype.is_quantized():
            check("qmm_accumulate_in_f32", lib().qmm_accumulate_in_f32(int(self.qtensor.dtype)))
        return True

    def indexed_moe_forward(self, x: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
        """QMatMul::indexed_moe_forward (mod.rs:1265-1272): QTensor.indexed_moe_forward."""
        return self.qtensor.indexed_moe_forward(x, ids)

    def forward(self, xs: torch.Tensor) -> torch.Tensor:
        """x [..., k] f32 -> [..., n]; the CustomOp1 shape rules of cpu_fwd (mod.rs:1280-1333)."""
        if len(self.qtensor.shape) != 2:
            raise ValueError(f"QMatMul::forward: a [n, k] weight, not {self.qtensor.shape}")
        n, k = self.qtensor.shape
        if xs.dim() < 1 or xs.shape[-1] != k:
            raise ValueError(f"input tensor {tuple(xs.shape)} incompatible with {self.qtensor.shape}")
        if xs.dtype != torch.float32:
            raise ValueError("Expected f32")
        if not xs.is_contiguous():
            raise ValueError(f"input tensor is not contiguous {tuple(xs.shape)}")
        rows = xs.numel() // k
        out = torch.empty((*xs.shape[:-1], n), dtype=torch.float32, device=xs.device)
        if rows == 0:
            return out
        need = ctypes.c_size_t(0)
        L = lib()
        t = int(self.qtensor.dtype)
        st = _stream()
        check("qmm_forward", L.qmm_forward(t, _ptr(self.qtensor.data_), _ptr(xs), k, _ptr(out), n, None, 0,
                                           ctypes.byref(need), k, n, rows, 0, st))
        ws = self._ws.get(need.value, xs.device)
        check("qmm_forward", L.qmm_forward(t, _ptr(self.qtensor.data_), _ptr(xs), k, _ptr(out), n, _ptr(ws),
                                           ws.numel(), ctypes.byref(need), k, n, rows, 1, st))
        return out

    __call__ = forward

    @staticmethod
    def forward_shared(xs: torch.Tensor, ws: Sequence["QMatMul"]) -> List[torch.Tensor]:
        """Several weights against ONE activation, quantized once for all of
        them (mod.rs:1221-1263): one qmm_forward_shared call per group of
        weights of the same type; a single weight is a plain forward."""
        if len(ws) <= 1:
            return [w.forward(xs) for w in ws]
        k = ws[0].qtensor.shape[1]
        if any(w.qtensor.shape[1] != k for w in ws):
            raise ValueError("forward_shared: every weight must have the activation's k")
        if xs.dim() < 1 or xs.shape[-1] != k:
            raise ValueError(f"input tensor {tuple(xs.shape)} incompatible with k={k}")
        if xs.dtype != torch.float32:
            raise ValueError("Expected f32")
        if not xs.is_contiguous():
            raise ValueError(f"input tensor is not contiguous {tuple(xs.shape)}")
        rows = xs.numel() // k
        outs = [torch.empty((*xs.shape[:-1], w.qtensor.shape[0]), dtype=torch.float32, device=xs.device)
                for w in ws]
        if rows == 0:
            return outs
        L = lib()
        st = _stream()
        by_type = {}
        for i, w in enumerate(ws):
            by_type.setdefault(int(w.qtensor.dtype), []).append(i)
        for t, idx in by_type.items():
            cnt = len(idx)
            wp = (ctypes.c_void_p * cnt)(*[ws[i].qtensor.data_.data_ptr() for i in idx])
            ns = (ctypes.c_int64 * cnt)(*[ws[i].qtensor.shape[0] for i in idx])
            dp = (ctypes.c_void_p * cnt)(*[outs[i].data_ptr() for i in idx])
            ld = (ctypes.c_int64 * cnt)(*[ws[i].qtensor.shape[0] for i in idx])
            need = ctypes.c_size_t(0)
            check("qmm_forward_shared", L.qmm_forward_shared(t, cnt, wp, ns, dp, ld, _ptr(xs), k, None, 0,
                                                             ctypes.byref(need), k, rows, 0, st))
            buf = ws[idx[0]]._ws.get(need.value, xs.device)
            check("qmm_forward_shared", L.qmm_forward_shared(t, cnt, wp, ns, dp, ld, _ptr(xs), k, _ptr(buf),
                                                             buf.numel(), ctypes.byref(need), k, rows, 1, st))
        return outs


#: the gated activations of an MLP (src/inference/layers/mod.rs:583-632)
ACTIVATIONS = {"silu": _lib.GLU_SILU, "swiglu_oai": _lib.GLU_SWIGLU_OAI, "gelu": _lib.GLU_GELU}


def forward_glu(xs: torch.Tensor, gate: "QMatMul", up: "QMatMul", activation: str = "silu") -> torch.Tensor:
    """act(xs · gateᵀ) * (xs · upᵀ): the gate and up products of an MLP sharing
    one quantized activation and the gated activation between them, written
    once (qmm_forward_glu: one launch for Q4_K at 1-2 rows; otherwise the
    shared products and the elementwise GLU). The reference's forward_block
    (src/inference/layers/mod.rs:583-632): forward_shared of ffn_up and
    ffn_gate, then silu_mul / swiglu_oai_mul / gelu(gate) * up."""
    if activation not in ACTIVATIONS:
        raise ValueError(f"activation must be one of {sorted(ACTIVATIONS)}")
    gq, uq = gate.qtensor, up.qtensor
    if gq.shape != uq.shape or gq.dtype != uq.dtype:
        raise ValueError("forward_glu: gate and up must have one shape and type")
    n, k = gq.shape
    if xs.dim() < 1 or xs.shape[-1] != k:
        raise ValueError(f"input tensor {tuple(xs.shape)} incompatible with k={k}")
    if xs.dtype != torch.float32:
        raise ValueError("Expected f32")
    if not xs.is_contiguous():
        raise ValueError(f"input tensor is not contiguous {tuple(xs.shape)}")
    rows = xs.numel() // k
    out = torch.empty((*xs.shape[:-1], n), dtype=torch.float32, device=xs.device)
    if rows == 0:
        return out
    L = lib()
    st = _stream()
    t, act = int(gq.dtype), ACTIVATIONS[activation]
    need = ctypes.c_size_t(0)
    check("qmm_forward_glu", L.qmm_forward_glu(t, act, None, None, None, k, None, n, None, 0, ctypes.byref(need), k, n,
                                               rows, 0, st))
    buf = gate._ws.get(need.value, xs.device)
    check("qmm_forward_glu", L.qmm_forward_glu(t, act, gq.data_.data_ptr(), uq.data_.data_ptr(), _ptr(xs), k,
                                               _ptr(out), n, _ptr(buf), buf.numel(), ctypes.byref(need), k, n, rows,
                                               1, st))
    return out


def glu(gate: torch.Tensor, up: torch.Tensor, activation: str = "silu") -> torch.Tensor:
    """act(gate) * up elementwise (qmm_glu): the reference's silu_mul /
    swiglu_oai_mul / gelu product (src/inference/fast_math.rs:48-130)."""
    if activation not in ACTIVATIONS:
        raise ValueError(f"activation must be one of {sorted(ACTIVATIONS)}")
    if gate.shape != up.shape or gate.dtype != torch.float32 or up.dtype != torch.float32:
        raise ValueError("glu: gate and up must be f32 tensors of one shape")
    if not (gate.is_contiguous() and up.is_contiguous()) or not (gate.is_cuda and up.is_cuda):
        raise ValueError("glu: contiguous GPU tensors")
    out = torch.empty_like(gate)
    n = gate.numel()
    if n:
        check("qmm_glu", lib().qmm_glu(ACTIVATIONS[activation], _ptr(gate), _ptr(up), _ptr(out), n, _stream()))
    return out


# Tokens up to which a card's grouped expert products run one row per pair
# (qmm_moe_forward); above it a prompt's run on the matrix cores
# (qmm_moe_forward_prefill): MOE_CARD_ONE_ROW_MAX_TOKENS and the caller's
# choice in MoeFfn::stacked_products (src/inference/layers/mod.rs:475, 2753).
MOE_CARD_ONE_ROW_MAX_TOKENS = 8

_X_DTYPES = {torch.float16: X_F16, torch.bfloat16: X_BF16, torch.float32: X_F32}


def moe_prompt_on_tensor_cores() -> bool:
    """prompt_on_tensor_cores (src/inference/layers/mod.rs:1232-1235): the
    prompt kernel unless SWARMLLM_MOE_CARD_PROMPT=rows, read once."""
    global _PROMPT_ON
    if _PROMPT_ON is None:
        _PROMPT_ON = os.environ.get("SWARMLLM_MOE_CARD_PROMPT") != "rows"
    return _PROMPT_ON


_PROMPT_ON: Optional[bool] = None


def moe_uses_prompt_kernel(tokens: int) -> bool:
    """The caller's choice of kernel for a chunk of `tokens` tokens
    (src/inference/layers/mod.rs:2753)."""
    return tokens > MOE_CARD_ONE_ROW_MAX_TOKENS and moe_prompt_on_tensor_cores()


def moe_forward(xs: torch.Tensor, experts: QTensor, sorted_ids: torch.Tensor, expert_ids: torch.Tensor,
                topk_weights: Optional[torch.Tensor], topk: int, prompt: bool = False,
                workspace: Optional[Workspace] = None) -> torch.Tensor:
    """The grouped expert products of moe_gemm_gguf / moe_gemm_gguf_prefill as
    layers::moe_card calls them (moe_card.rs:48-170; candle-kernels/src/moe/
    moe_gguf.cu:149-252, moe_wmma_gguf.cu:450-535): experts [E, n, k] in
    GGUF blocks; routing entry i pairs sorted_ids[i] (token * topk + k-th
    choice) with expert_ids[i]; xs holds one row per pair when topk_weights is
    given (each output row then scaled by its pair's weight), else one row per
    token. Returns [len(sorted_ids), n] f32, row p the product of pair p.
    prompt=False: one row per pair with the activation quantized
    (qmm_moe_forward; xs f32). prompt=True: the matrix-core product of the
    f16-rounded (bf16 for a bf16 xs) input and weights (qmm_moe_forward_prefill;
    xs f32, f16 or bf16)."""
    if len(experts.shape) != 3:
        raise ValueError(f"moe_forward: expert weights [E, n, k], not {experts.shape}")
    e, n, k = experts.shape
    ok_dtype = xs.dtype in _X_DTYPES if prompt else xs.dtype == torch.float32
    if not ok_dtype or xs.dim() != 2 or xs.shape[1] != k or not xs.is_contiguous():
        raise ValueError(f"moe_forward: input [rows, {k}] contiguous {'f32/f16/bf16' if prompt else 'f32'}, "
                         f"not {tuple(xs.shape)} {xs.dtype}")
    size_m = int(sorted_ids.numel())
    for name, t in (("sorted_ids", sorted_ids), ("expert_ids", expert_ids)):
        if t.dtype != torch.int32 or t.numel() != size_m or not t.is_contiguous():
            raise ValueError(f"moe_forward: {name} must be {size_m} contiguous int32")
    want_rows = size_m if topk_weights is not None else size_m // max(topk, 1)
    if xs.shape[0] != want_rows:
        raise ValueError(f"moe_forward: {xs.shape[0]} input rows, the routing reads {want_rows}")
    if topk_weights is not None and (topk_weights.dtype != torch.float32 or topk_weights.numel() != size_m):
        raise ValueError("moe_forward: topk_weights must be one f32 per routing entry")
    out = torch.empty((size_m, n), dtype=torch.float32, device=xs.device)
    if size_m == 0:
        return out
    L = lib()
    st = _stream()
    tw = _ptr(topk_weights) if topk_weights is not None else None
    need = ctypes.c_size_t(0)
    if prompt:
        fn, call = "qmm_moe_forward_prefill", L.qmm_moe_forward_prefill
        args = (int(experts.dtype), _ptr(experts.data_), e, _ptr(xs), _X_DTYPES[xs.dtype], k, _ptr(sorted_ids),
                _ptr(expert_ids), tw, topk, _ptr(out), n)
    else:
        fn, call = "qmm_moe_forward", L.qmm_moe_forward
        args = (int(experts.dtype), _ptr(experts.data_), e, _ptr(xs), k, _ptr(sorted_ids), _ptr(expert_ids), tw,
                topk, _ptr(out), n)
    check(fn, call(*args, None, 0, ctypes.byref(need), k, n, size_m, 0, st))
    buf = (workspace or Workspace()).get(need.value, xs.device)
    check(fn, call(*args, _ptr(buf), buf.numel(), ctypes.byref(need), k, n, size_m, 1, st))
    return out


def prepare(dtype: GgmlDType) -> None:
    """The set-up a first product of `dtype` would do, done now (before a
    graph capture): qmm_prepare (mmq_prepare_few_rows_once, cuda.rs:890-932)."""
    check("qmm_prepare", lib().qmm_prepare(int(GgmlDType(dtype))))


def prepared(dtype: GgmlDType) -> bool:
    return bool(lib().qmm_prepared(int(GgmlDType(dtype))))


def set_force_dmmv(flag: bool) -> None:
    """candle's quantized::cuda::set_force_dmmv (quantized/cuda.rs:29-33):
    while set, QMatMul.forward / forward_shared / forward_glu dequantize the
    weight against the f32 activation (no activation quantization)."""
    lib().qmm_set_force_dmmv(1 if flag else 0)


def mmq_few_rows_line(dtype: GgmlDType) -> Tuple[int, int]:
    """(fewest rows, least weight bytes) of a product of up to 8 rows that
    the matrix-core kernels take in this process, the environment read once
    (quantized/cuda.rs:850-872, mmq_few_rows_line)."""
    rows, nbytes = ctypes.c_int64(0), ctypes.c_int64(0)
    check("qmm_mmq_few_rows_line", lib().qmm_mmq_few_rows_line(int(dtype), ctypes.byref(rows), ctypes.byref(nbytes)))
    return rows.value, nbytes.value


def quantize_act(x: torch.Tensor, layout: int) -> torch.Tensor:
    """The activation rows quantized on the device (qmm_quantize_act); the raw buffer."""
    x = x.contiguous()
    k = x.shape[-1]
    rows = x.numel() // k
    L = lib()
    out = torch.zeros(L.qmm_act_bytes(layout, k, rows), dtype=torch.uint8, device=x.device)
    check("qmm_quantize_act", L.qmm_quantize_act(_ptr(x), _ptr(out), layout, k, rows, k, _stream()))
    return out


def act_planes(buf: torch.Tensor, layout: int, k: int, rows: int):
    """(codes int8 [rows, k], scales f32, sums) views of an activation buffer."""
    co, so, uo = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    check("qmm_act_planes", lib().qmm_act_planes(layout, k, rows, ctypes.byref(co), ctypes.byref(so), ctypes.byref(uo)))
    per_scale = 256 if layout == _lib.ACT_Q8K else 32
    codes = buf[co.value: co.value + rows * k].view(torch.int8).reshape(rows, k)
    scales = buf[so.value: so.value + rows * (k // per_scale) * 4].view(torch.float32).reshape(rows, -1)
    if layout == _lib.ACT_Q8K:
        sums = buf[uo.value: uo.value + rows * (k // 16) * 2].view(torch.int16).reshape(rows, -1)
    else:
        sums = buf[uo.value: uo.value + rows * (k // 32) * 4].view(torch.int32).reshape(rows, -1)
    return codes, scales, sums
