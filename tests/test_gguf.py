"""The GGUF reader (libqmm's C++ restatement of candle's gguf_file::
Content::read, gguf_file.rs:415-487) on the committed tiny files
(tests/golden/make_tiny_gguf.py) and on malformed variants of them. No GPU:
parsing is host code."""
import struct

import pytest

from golden import make_tiny_gguf as tiny
from swarmllm_amd._lib import lib
from swarmllm_amd.gguf import Content

GOLDEN = tiny.HERE


def test_committed_files_are_the_scripts_output():
    for name, (data, *_rest) in tiny.files().items():
        with open(f"{GOLDEN}/{name}", "rb") as f:
            assert f.read() == data, name


def expected_metadata(items):
    out = {}
    for key, vt, v, *et in items:
        if vt == tiny.STRING:
            v = v.rstrip("\x00")  # the reader drops trailing NULs (gguf_file.rs:120-135)
        if vt == tiny.ARRAY and et and et[0] == tiny.ARRAY:
            v = None  # arrays of arrays are parsed, not read element by element
        out[key] = v
    return out


@pytest.mark.parametrize("name", ["tiny_v3.gguf", "tiny_v1.gguf"])
def test_header_metadata_and_tensor_infos(name):
    data, infos, data_offset, meta, tensors = tiny.files()[name]
    c = Content.read(f"{GOLDEN}/{name}")
    assert c.version == (3 if "v3" in name else 1)
    assert c.alignment == (64 if "v3" in name else 32)
    assert c.tensor_data_offset == data_offset
    assert c.metadata == expected_metadata(meta)
    assert list(c.metadata) == [m[0] for m in meta]  # file order
    assert list(c.tensor_infos) == [t[0] for t in tensors]
    for (tname, t, shape), (off, b) in zip(tensors, infos):
        info = c.tensor_infos[tname]
        assert (info.ggml_dtype, info.shape, info.offset, info.nbytes) == (t, shape, off, len(b))


def write(tmp_path, data, name="f.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def small(metadata=None, tensors=None, version=3, alignment=32):
    return tiny.build(version, metadata if metadata is not None else [("a", tiny.U32, 1)],
                      tensors if tensors is not None else tiny.TENSORS_V1, alignment)[0]


def test_alignment_rules(tmp_path):
    # U8 / U16 / non-negative I32 alignments are used; a negative one, a
    # non-integer one or none falls back to 32 (gguf_file.rs:471-480)
    for vt, v, want in ((tiny.U8, 16, 16), (tiny.U16, 128, 128), (tiny.I32, 256, 256), (tiny.I32, -5, 32),
                        (tiny.F32, 64.0, 32), (tiny.STRING, "64", 32)):
        data = small([("general.alignment", vt, v)], alignment=want)
        c = Content.read(write(tmp_path, data))
        assert c.alignment == want
        assert c.tensor_data_offset % want == 0
        head_end = len(data) - sum(len(b) + (-len(b)) % want for _, b in tiny.build(
            3, [("general.alignment", vt, v)], tiny.TENSORS_V1, want)[1])
        assert c.tensor_data_offset == head_end


def test_either_magic_byte_order(tmp_path):
    data = bytearray(small())
    data[0:4] = struct.pack("<I", 0x47475546)
    assert Content.read(write(tmp_path, bytes(data))).version == 3


@pytest.mark.parametrize("case", ["magic", "version0", "version4", "truncated", "value_type", "ggml_type", "bool",
                                  "zero_alignment", "empty"])
def test_malformed_files_are_rejected(tmp_path, case):
    data = bytearray(small([("k", tiny.BOOL, True)]))
    if case == "magic":
        data[0:4] = b"GGML"
    elif case == "version0":
        data[4:8] = struct.pack("<I", 0)
    elif case == "version4":
        data[4:8] = struct.pack("<I", 4)
    elif case == "truncated":
        data = data[:40]
    elif case == "value_type":
        # the key "k" (u64 length 1, 1 byte) follows the 24-byte preamble; its type is next
        data[24 + 8 + 1:24 + 8 + 5] = struct.pack("<I", 13)
    elif case == "ggml_type":
        data = bytearray(small(tensors=[("x", 12, (1, 256))]))
        i = data.index(b"x") + 1 + 4 + 16  # name, n_dims, two u64 dims
        data[i:i + 4] = struct.pack("<I", 5)  # no ggml type has id 5
    elif case == "bool":
        data[24 + 8 + 1 + 4] = 2
    elif case == "zero_alignment":
        data = bytearray(small([("general.alignment", tiny.U32, 0)]))
    elif case == "empty":
        data = b""
    with pytest.raises(ValueError):
        Content.read(write(tmp_path, bytes(data)))


def test_repeated_keys_and_names_keep_the_last():
    data, _, _ = tiny.build(3, [("k", tiny.U32, 1), ("k", tiny.U32, 2)],
                            [("t", 8, (1, 32)), ("t", 8, (2, 32))], 32)
    import tempfile
    with tempfile.NamedTemporaryFile(suffix=".gguf") as f:
        f.write(data)
        f.flush()
        c = Content.read(f.name)
        assert c.metadata == {"k": 2}
        assert c.tensor_infos["t"].shape == (2, 32) and len(c.tensor_infos) == 1


def test_padded_bytes():
    L = lib()
    for t, bs, ts in ((12, 256, 144), (14, 256, 210), (8, 32, 34), (20, 32, 18), (39, 32, 17), (0, 1, 4), (1, 1, 2)):
        assert L.qmm_padded_bytes(t, 4 * bs) == 4 * ts + 512 // bs * ts
    assert L.qmm_padded_bytes(12, 100) == 0 and L.qmm_padded_bytes(5, 64) == 0


def test_sizes_past_int64_are_refused(tmp_path):
    """A tensor whose byte count passes INT64_MAX reads as 0 bytes (refused by
    the loader), and qmm_padded_bytes answers 0 for such a count."""
    L = lib()
    assert L.qmm_padded_bytes(0, 2 ** 62) == 0
    assert L.qmm_padded_bytes(0, 2 ** 60) == 2 ** 62 + 512 * 4
    assert L.qmm_padded_bytes(15, 2 ** 62) == 2 ** 54 * 292 + 2 * 292
    # F32 [2^22, 2^40]: 2^62 values, 2^64 bytes
    pre = struct.pack("<II", 0x46554747, 3) + struct.pack("<QQ", 1, 0)
    pre += tiny._str("huge", 3) + struct.pack("<I", 2) + struct.pack("<QQ", 2 ** 40, 2 ** 22) + struct.pack("<IQ", 0, 0)
    c = Content.read(write(tmp_path, pre))
    assert c.tensor_infos["huge"].nbytes == 0
    with pytest.raises(ValueError):
        c.tensor("huge")
