"""GGUF files into device QTensors, with the names of candle's gguf_file
module (vendor/candle/candle-core/src/quantized/gguf_file.rs): Content.read
parses a file (Content::read, :415-487) in libqmm's C++ reader, and
Content.tensor loads one tensor into a padded device buffer (Content::tensor
:489-500 -> ggml_file::qtensor_read -> cuda::load_quantized_read), read
through the library's pinned staging buffers (qmm_gguf_load)."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, Dict, Tuple

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
