"""The GGUF v3 reader (rvm_gguf_open and friends in librvmoe.so) on the CPU, against the reference
parser's own test cases (runtime/tests/synthetic.rs:104-193): the same valid image with the same
views, every truncation refused, and each header, metadata and descriptor violation refused with
the reference's message. No kernel is launched.
"""
import struct

import numpy as np
import pytest

from gguf_builder import Builder, valid
from rosevine_amd import gguf


def err(b: Builder) -> str:
    with pytest.raises(gguf.GgufError) as e:
        gguf.Gguf(b.build())
    return str(e.value)


def test_valid_file_parses_with_exact_views(rvlib):
    data = valid().build()
    g = gguf.Gguf(data)
    assert g.info()["n_tensors"] == 2 and g.info()["version"] == 3
    ta, sa, oa, va = g.tensor("a")
    assert (ta, va.size) == (gguf.F32, 32)
    tb, sb, ob, vb = g.tensor("b")
    assert (tb, vb.size, sb) == (gguf.Q4_0, 36, [32, 2])
    assert ob == g.info()["data_offset"] + 32
    assert bytes(vb) == data[ob:ob + 36]
    assert g.meta_str("general.architecture") == "test"
    with pytest.raises(gguf.GgufError, match="missing tensor"):
        g.tensor("c")


def test_every_truncation_is_rejected(rvlib):
    data = valid().build()
    for n in range(len(data)):
        with pytest.raises(gguf.GgufError):
            gguf.Gguf(data[:n])


def test_header_violations(rvlib):
    bad = bytearray(valid().build())
    bad[0] = ord("X")
    with pytest.raises(gguf.GgufError, match="^bad magic$"):
        gguf.Gguf(bytes(bad))
    v2 = valid()
    v2.version = 2
    assert err(v2) == "expected GGUF version 3"
    assert err(Builder().data(0)) == "descriptor count limit exceeded"
    many = bytearray(valid().build())
    many[16:24] = struct.pack("<Q", 1 << 40)
    with pytest.raises(gguf.GgufError, match="descriptor count limit exceeded"):
        gguf.Gguf(bytes(many))


def test_metadata_violations(rvlib):
    assert err(valid().kv_str("general.architecture", "x")) == "duplicate metadata key"
    assert err(valid().kv_str("", "x")) == "empty metadata key"
    for align in [0, 3, 48, 1 << 21]:
        b = valid()
        b.kv[1] = ("general.alignment", struct.pack("<II", 4, align))
        assert err(b) == "invalid alignment", align
    assert err(valid().raw_kv("k", struct.pack("<I", 7) + bytes([2]))) == "invalid bool"
    assert err(valid().raw_kv("k", struct.pack("<IIQ", 9, 9, 1))) == "unsupported array element type"
    assert err(valid().raw_kv("k", struct.pack("<IIQ", 9, 4, 1 << 40))) == "array length limit exceeded"
    assert err(valid().raw_kv("k", struct.pack("<IIQ", 9, 8, 4_000_000))) == "truncated header"
    assert err(valid().raw_kv("k", struct.pack("<IQ", 8, 1 << 40))) == "string length limit exceeded"
    assert err(valid().raw_kv("k", struct.pack("<IQ", 8, 1) + bytes([0xFF]))) == "string is not UTF-8"
    assert err(valid().raw_kv("k", struct.pack("<I", 13))) == "unsupported metadata type"
    # arrays of numbers and strings, and multi-byte UTF-8, are accepted
    ok = valid().raw_kv("n", struct.pack("<IIQ", 9, 5, 3) + struct.pack("<3i", 1, -2, 3))
    ok = ok.raw_kv("s", struct.pack("<IIQ", 9, 8, 2) + struct.pack("<Q", 3) + "▁a".encode()[:3]
                   + struct.pack("<Q", 1) + b"b")
    assert gguf.Gguf(ok.build()).info()["n_tensors"] == 2


def test_tensor_descriptor_violations(rvlib):
    def base():
        return Builder().data(4096)

    assert err(base().tensor("x", [8], 0, 0).tensor("x", [8], 0, 32)) == "empty or duplicate tensor name"
    assert err(base().tensor("", [8], 0, 0)) == "empty or duplicate tensor name"
    assert err(base().tensor("x", [], 0, 0)) == "invalid tensor rank"
    assert err(base().tensor("x", [1, 1, 1, 1, 1], 0, 0)) == "invalid tensor rank"
    assert err(base().tensor("x", [8, 0], 0, 0)) == "invalid tensor shape"
    assert err(base().tensor("x", [33], 2, 0)) == "invalid tensor shape"
    assert err(base().tensor("x", [8], 1, 0)) == "unsupported tensor type"
    assert err(base().tensor("x", [8], 0, 16)) == "misaligned tensor offset"
    assert err(base().tensor("x", [1 << 40, 1 << 40], 0, 0)) == "tensor element count overflow"
    assert err(base().tensor("x", [16], 0, 0).tensor("y", [8], 0, 32)) == "overlapping or out-of-file tensor range"
    assert err(base().tensor("x", [2048], 0, 0)) == "overlapping or out-of-file tensor range"
    assert err(base().tensor("x", [8], 0, (1 << 64) - 32)) == "tensor range overflow"


def test_mapped_file(rvlib, tmp_path):
    data = valid().build()
    p = tmp_path / "m.gguf"
    p.write_bytes(data)
    g = gguf.Gguf(str(p))
    _, _, off, view = g.tensor("b")
    assert bytes(view) == data[off:off + 36]
    del view
    g.close()
    (tmp_path / "empty").write_bytes(b"")
    with pytest.raises(gguf.GgufError, match="empty file"):
        gguf.Gguf(str(tmp_path / "empty"))
    with pytest.raises(gguf.GgufError, match="not a regular file"):
        gguf.Gguf(str(tmp_path))
