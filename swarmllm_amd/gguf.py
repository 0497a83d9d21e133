"""GGUF files into device QTensors, with the names of candle's gguf_file
module (vendor/candle/candle-core/src/quantized/gguf_file.rs): Content.read
parses a file (Content::read, :415-487) in libqmm's C++ reader, and
Content.tensor loads one tensor into a padded device buffer (Content::tensor
:489-500 -> ggml_file::qtensor_read -> cuda::load_quantized_read), read
through the library's pinned staging buffers (qmm_gguf_load).

The loader variants of quantized/cuda.rs:1966-2127 sit beside it:
Content.tensor_entries (chosen experts of a stack, straight from the file),
load_quantized_entries and load_quantized_beside (from host bytes),
pinned_load_chunks and with_pinned_load_staging."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, Callable, Dict, Optional, Sequence, Tuple, TypeVar

import torch

from ._lib import QMM_OK, QmmError, check, lib
from .qtensor import GgmlDType, QTensor, _stream

DEFAULT_ALIGNMENT = 32

# GGUF value type ids (gguf_file.rs:329-346)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_UNSIGNED = {U8: 0xFF, U16: 0xFFFF, U32: 0xFFFFFFFF, U64: 0xFFFFFFFFFFFFFFFF}


@dataclass
class TensorInfo:
    """A tensor's entry in the file (gguf_file.rs:55-60): ggml type id, shape
    (outermost first), offset from the tensor data, byte size (0 when the
    element count is not a whole number of blocks)."""

    ggml_dtype: int
    shape: Tuple[int, ...]
    offset: int
    nbytes: int
    index: int


class Content:
    """A parsed GGUF file: version, metadata, tensor infos, the tensor data's
    offset and the alignment it was rounded to."""

    def __init__(self, handle: int, path: str):
        self._h = ctypes.c_void_p(handle)
        self.path = path
        L = lib()
        self.version = L.qmm_gguf_version(self._h)
        self.alignment = int(L.qmm_gguf_alignment(self._h))
        self.tensor_data_offset = int(L.qmm_gguf_data_offset(self._h))
        self.metadata: Dict[str, Any] = {}
        for i in range(L.qmm_gguf_kv_count(self._h)):
            self.metadata[L.qmm_gguf_kv_key(self._h, i).decode("utf-8", errors="replace")] = self._value(i)
        self.tensor_infos: Dict[str, TensorInfo] = {}
        for i in range(L.qmm_gguf_tensor_count(self._h)):
            t, nd = ctypes.c_int(0), ctypes.c_int(0)
            dims = (ctypes.c_int64 * 4)()
            off, nb = ctypes.c_uint64(0), ctypes.c_uint64(0)
            check("qmm_gguf_tensor_info", L.qmm_gguf_tensor_info(self._h, i, ctypes.byref(t), ctypes.byref(nd), dims,
                                                                 ctypes.byref(off), ctypes.byref(nb)))
            name = L.qmm_gguf_tensor_name(self._h, i).decode("utf-8", errors="replace")
            self.tensor_infos[name] = TensorInfo(t.value, tuple(dims[d] for d in range(nd.value)), off.value, nb.value,
                                                 i)

    def _value(self, i: int):
        L = lib()
        et, n = ctypes.c_int(0), ctypes.c_int64(0)
        vt = L.qmm_gguf_kv_type(self._h, i, ctypes.byref(et), ctypes.byref(n))
        if vt == ARRAY:
            if et.value == ARRAY:
                return None  # arrays of arrays are parsed but not read element by element
            return [self._elem(i, j, et.value) for j in range(n.value)]
        return self._elem(i, 0, vt)

    def _elem(self, i: int, j: int, vt: int):
        iv, fv, sv = ctypes.c_int64(0), ctypes.c_double(0.0), ctypes.c_char_p()
        check("qmm_gguf_kv_get", lib().qmm_gguf_kv_get(self._h, i, j, ctypes.byref(iv), ctypes.byref(fv),
                                                        ctypes.byref(sv)))
        if vt == STRING:
            return (sv.value or b"").decode("utf-8", errors="replace")
        if vt in (F32, F64):
            return fv.value
        if vt == BOOL:
            return bool(iv.value)
        if vt in _UNSIGNED:
            return iv.value & _UNSIGNED[vt]
        return iv.value

    @staticmethod
    def read(path: str) -> "Content":
        """Content::read of the file at `path`; ValueError when it is not a
        GGUF file the reader takes (bad magic or version, an unknown value or
        ggml type, a truncated header)."""
        h = ctypes.c_void_p()
        st = lib().qmm_gguf_open(path.encode(), ctypes.byref(h))
        if st != QMM_OK or not h.value:
            raise ValueError(f"{path}: not a GGUF file libqmm reads")
        return Content(h.value, path)

    def tensor(self, name: str, device="cuda") -> QTensor:
        """Content::tensor: the named tensor in a padded device buffer."""
        info = self.tensor_infos.get(name)
        if info is None:
            raise ValueError(f"cannot find tensor info for {name}")
        try:
            dtype = GgmlDType(info.ggml_dtype)
        except ValueError:
            raise ValueError(f"{name}: ggml type {info.ggml_dtype} is not one a QTensor holds") from None
        if info.nbytes == 0 and any(info.shape):
            raise ValueError(f"{name}: {list(info.shape)} is not a whole number of {dtype.name} blocks")
        q = QTensor.alloc(info.shape, dtype, device)
        st = lib().qmm_gguf_load(self._h, info.index, q.storage_.data_ptr(), q.storage_.numel(), _stream())
        if st != QMM_OK:
            raise QmmError("qmm_gguf_load", st)
        return q

    def tensor_entries(self, name: str, slots: Sequence[int], device="cuda") -> QTensor:
        """The named [entries, ...] stack (one weight per entry, e.g. a layer's
        experts) in a padded device buffer holding only the entries `slots`,
        read from the file; every other entry stays zero and must never be
        read (qmm_gguf_load_entries; the file-side form of
        load_quantized_entries, cuda.rs:2101-2127)."""
        info = self.tensor_infos.get(name)
        if info is None:
            raise ValueError(f"cannot find tensor info for {name}")
        dtype = GgmlDType(info.ggml_dtype)
        if len(info.shape) < 2:
            raise ValueError(f"{name}: {list(info.shape)} is not a stack of entries")
        entries = info.shape[0]
        for s in slots:
            if not 0 <= int(s) < entries:
                raise ValueError(f"tensor_entries: slot {s} of {entries}")
        q = QTensor.alloc(info.shape, dtype, device)
        arr = (ctypes.c_int64 * max(len(slots), 1))(*[int(s) for s in slots])
        st = lib().qmm_gguf_load_entries(self._h, info.index, len(slots), arr, q.storage_.data_ptr(),
                                         q.storage_.numel(), _stream())
        if st != QMM_OK:
            raise QmmError("qmm_gguf_load_entries", st)
        return q

    def close(self) -> None:
        if self._h is not None and self._h.value:
            lib().qmm_gguf_close(self._h)
        self._h = None

    def __enter__(self) -> "Content":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pinned_load_chunks() -> int:
    """Chunks this process has copied to the device through the pinned
    staging pair (pinned_load_chunks, cuda.rs:1966-1972)."""
    return int(lib().qmm_pinned_load_chunks())


T = TypeVar("T")


def with_pinned_load_staging(load: Callable[[], T]) -> T:
    """with_pinned_load_staging (cuda.rs:1974-1996): run `load` with loads
    copied through two page-locked chunks. The library keeps its pinned pair
    for the process (SWARMLLM_LOAD_PINNED=0 switches it off), so every load
    is already inside such a scope; this runs `load` and returns its result."""
    return load()


def load_quantized_entries(dtype: GgmlDType, entries: int, entry_shape: Sequence[int],
                           parts: Sequence[Tuple[int, bytes]], device="cuda") -> QTensor:
    """load_quantized_entries (cuda.rs:2101-2127): a [entries, *entry_shape]
    stack holding the host bytes of each (slot, bytes) part at its slot,
    every other slot zero; each part exactly one entry's bytes."""
    dtype = GgmlDType(dtype)
    shape = (int(entries), *[int(d) for d in entry_shape])
    nel = 1
    for d in entry_shape:
        nel *= int(d)
    if nel % dtype.block_size():
        raise ValueError(f"load_quantized_entries: {list(entry_shape)} is not a whole number of {dtype.name} blocks")
    entry_bytes = nel // dtype.block_size() * dtype.type_size()
    for slot, raw in parts:
        if not 0 <= int(slot) < entries or len(raw) != entry_bytes:
            raise ValueError(f"load_quantized_entries: slot {slot} of {entries} with {len(raw)} bytes, "
                             f"expected {entry_bytes}")
    q = QTensor.alloc(shape, dtype, device)
    bufs = [ctypes.create_string_buffer(bytes(raw), len(raw)) if len(raw) else None for _, raw in parts]
    n = max(len(parts), 1)
    slots = (ctypes.c_int64 * n)(*[int(s) for s, _ in parts])
    ptrs = (ctypes.c_void_p * n)(*[ctypes.cast(b, ctypes.c_void_p).value if b is not None else None for b in bufs])
    st = lib().qmm_load_entries(int(dtype), int(entries), entry_bytes, len(parts), slots, ptrs, q.storage_.data_ptr(),
                                q.storage_.numel(), _stream())
    if st != QMM_OK:
        raise QmmError("qmm_load_entries", st)
    return q


def load_quantized_beside(data: bytes, shape: Sequence[int], dtype: GgmlDType,
                          copy_stream: Optional[torch.cuda.Stream] = None, device="cuda") -> QTensor:
    """load_quantized_beside (cuda.rs:2082-2099): a weight's GGUF bytes into
    a padded device buffer, copied on `copy_stream` (a side stream by
    default) beside the work of the current stream, which waits for it."""
    dtype = GgmlDType(dtype)
    q = QTensor.alloc(shape, dtype, device)
    if len(data) != q.data_.numel():
        raise ValueError(f"load_quantized_beside: {len(data)} bytes for {list(shape)} {dtype.name}")
    side = copy_stream if copy_stream is not None else torch.cuda.Stream(device=q.data_.device)
    # the buffer's zero-fill, on the current stream, lands before the side copy
    side.wait_stream(torch.cuda.current_stream(q.data_.device))
    buf = ctypes.create_string_buffer(bytes(data), max(len(data), 1))
    st = lib().qmm_load_beside(int(dtype), ctypes.cast(buf, ctypes.c_void_p).value, len(data), q.storage_.data_ptr(),
                               q.storage_.numel(), side.cuda_stream, _stream())
    if st != QMM_OK:
        raise QmmError("qmm_load_beside", st)
    return q
