"""The GGUF reader (tlh_gguf_*) against ggml's own (vendor/ggml/src/gguf.cpp,
compiled in oracle/_ref): files written by ggml's writer and by ours give the
same version, alignment, data offset, tensor names / types / shapes / offsets /
sizes and key-value pairs (types and values) through both readers, and both
refuse the same malformed files. A llama-architecture file round-trips its
config and weights (tensorlisp_amd.gguf.write_llama / decoder_config)."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from refs import decoder_tiny_config, decoder_weights, ref
from tensorlisp_amd import gguf
from tensorlisp_amd import native as N

needs_ref = pytest.mark.skipif(ref() is None, reason="oracle/_ref (compiled reference) not built here")


def ours(path):
    g = gguf.GgufFile(path)
    d = dict(version=g.version, alignment=g.alignment, data_offset=g.data_offset,
             tensors=[(t["name"], t["type"], t["ne"], t["offset"], t["bytes"]) for t in g.tensors], kv=g.kv)
    g.close()
    return d


def same(a, b):
    assert a["version"] == b["version"] and a["alignment"] == b["alignment"]
    assert a["data_offset"] == b["data_offset"]
    assert a["tensors"] == b["tensors"]
    assert list(a["kv"]) == list(b["kv"])
    for k in a["kv"]:
        (ta, va), (tb, vb) = a["kv"][k], b["kv"][k]
        assert ta == tb, k
        if isinstance(va, np.ndarray):
            np.testing.assert_array_equal(va, vb)
        else:
            assert va == vb, (k, va, vb)


@needs_ref
def test_reader_matches_ggml_on_files_ggml_writes(tmp_path):
    """Every scalar type, strings, numeric and string arrays, tensors of seven
    types and one to four dimensions. (ggml's writer places tensors at its
    context's alignment, 32, even when general.alignment says otherwise, and its
    reader then refuses the file: files with other alignments come from ours.)"""
    p = tmp_path / "sample.gguf"
    ref().gguf_write_sample(p, 0)
    want = ref().gguf_describe(p)
    assert want is not None and want["alignment"] == 32 and len(want["tensors"]) == 7
    same(ours(p), want)


@needs_ref
@pytest.mark.parametrize("alignment", [32, 128, 8])
def test_reader_matches_ggml_on_files_we_write(tmp_path, alignment):
    c = decoder_tiny_config()
    p = tmp_path / "tiny.gguf"
    gguf.write_llama(p, c, decoder_weights(c), alignment)
    same(ours(p), ref().gguf_describe(p))


def _header(version=3, n_tensors=0, n_kv=0):
    return b"GGUF" + struct.pack("<IqQ", version, n_tensors, n_kv)


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _tensor(name, ne, ty, off):
    return _s(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}q", *ne) + struct.pack("<iQ", ty, off)


MALFORMED = {
    "bad magic": b"GGUG" + struct.pack("<IqQ", 3, 0, 0),
    "version 1": _header(1),
    "version 4": _header(4),
    "other byte order": b"GGUF" + struct.pack(">I", 3) + struct.pack("<qQ", 0, 0),
    "truncated": _header(3, 0, 1) + _s("k"),
    "alignment not a power of 2": _header(3, 0, 1) + _s("general.alignment") + struct.pack("<iI", 4, 48),
    "alignment of the wrong type": _header(3, 0, 1) + _s("general.alignment") + struct.pack("<ii", 5, 64),
    "duplicate tensor": _header(3, 2, 0) + _tensor("a", [4], 0, 0) + _tensor("a", [4], 0, 32) + bytes(96),
    "offsets not consecutive": _header(3, 2, 0) + _tensor("a", [4], 0, 0) + _tensor("b", [4], 0, 64) + bytes(160),
    "row not whole blocks": _header(3, 1, 0) + _tensor("a", [16], 2, 0) + bytes(64),
    "five dimensions": _header(3, 1, 0) + _s("a") + struct.pack("<I", 5) + struct.pack("<5q", 1, 1, 1, 1, 1) +
    struct.pack("<iQ", 0, 0) + bytes(64),
    "data past the end": _header(3, 1, 0) + _tensor("a", [1024], 0, 0) + bytes(40),
    # element counts beyond an int64 (vendor/ggml/src/gguf.cpp:691-702), here in a middle tensor
    "element count overflows int64": _header(3, 3, 0) + _tensor("a", [8], 0, 0) +
    _tensor("b", [1 << 32, 1 << 31, 4], 0, 32) + _tensor("c", [8], 0, 64) + bytes(128),
}


@pytest.mark.parametrize("what", list(MALFORMED))
def test_malformed_files_are_refused(tmp_path, what):
    p = tmp_path / "bad.gguf"
    p.write_bytes(MALFORMED[what])
    with pytest.raises(N.TlhError, match="INVALID"):
        gguf.GgufFile(p)
    if ref() is not None and what != "data past the end":  # ggml checks data only when it loads it
        assert ref().gguf_describe(p) is None, what


def test_llama_file_round_trips_config_and_weights(tmp_path):
    c = decoder_tiny_config()
    w = decoder_weights(c)
    p = tmp_path / "tiny.gguf"
    gguf.write_llama(p, c, w)
    g = gguf.GgufFile(p)
    c2 = gguf.decoder_config(g, n_ctx=c.n_ctx)
    for f in ("n_embd", "n_head", "n_head_kv", "n_ff", "n_layer", "n_vocab", "n_ctx", "rope_base"):
        assert getattr(c2, f) == getattr(c, f), f
    assert np.float32(c2.eps) == np.float32(c.eps)
    assert [(n, t, ne) for n, t, ne in c2.weight_shapes()] == c.weight_shapes()
    for (name, _, _), a in zip(c.weight_shapes(), w):
        np.testing.assert_array_equal(g.read(gguf.gguf_name(name)).reshape(-1),
                                      np.ascontiguousarray(a).view(np.uint8).reshape(-1))
    g.close()


def test_unsized_type_is_unsupported(tmp_path):
    p = tmp_path / "iq.gguf"
    p.write_bytes(_header(3, 1, 0) + _tensor("a", [256], 16, 0) + bytes(512))  # 16 = iq2_xxs
    with pytest.raises(N.TlhError, match="UNSUPPORTED"):
        gguf.GgufFile(p)


def test_byte_count_that_would_wrap_is_refused(tmp_path):
    """2^62 f32 elements fit an int64 but their 2^64 bytes do not: the reader must not
    wrap the size (and with it every later offset and the layout's total)."""
    p = tmp_path / "wrap.gguf"
    p.write_bytes(_header(3, 2, 0) + _tensor("a", [1 << 31, 1 << 31], 0, 0) + _tensor("b", [8], 0, 0) + bytes(64))
    with pytest.raises(N.TlhError, match="INVALID"):
        gguf.GgufFile(p)
