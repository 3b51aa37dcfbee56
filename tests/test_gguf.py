"""The GGUF reader (csrc/gguf.cpp, include/spq4k_gguf.h) against the
reference's own reader and writer (vendor/ggml/src/gguf.cpp, compiled into
oracle/_ref): host only, no GPU.

1. Files written by the reference's writer (gguf_write_to_file): every
   metadata type, arrays of each (empty ones and string arrays included),
   tensors of many ggml types and 1 to 4 dimensions, several alignments,
   hundreds of tensors. The reader must report what gguf_init_from_file
   reports (version, alignment, data offset, every key/value, every tensor's
   name, type, shape, offset and size), and each tensor's bytes must be the
   bytes written.
2. Malformed files, made by a byte-level builder from a valid layout with one
   field changed: each must be rejected exactly when the reference rejects
   it. Two cases differ by design and are checked on their own: a
   general.alignment of the wrong type (the reference aborts the process;
   the reader returns -EINVAL) and tensor data past the end of the file (the
   reference's no_alloc reader reads no data and accepts it; the reader hands
   out pointers into the file and rejects it)."""
import os
import struct

import numpy as np
import pytest

from _gguf_ref import ARRAY, STRING, RefGguf

spq4k = pytest.importorskip("spq4k")

# (ggml type id, block values, block bytes) for the tensors written below
TYPES = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210),
         24: (1, 1), 26: (1, 4), 30: (1, 2), 39: (32, 17)}


@pytest.fixture(scope="module")
def rg(ref):
    return RefGguf(ref)


def _nbytes(t, ne):
    blk, size = TYPES[t]
    n = int(np.prod(ne))
    return n // blk * size


def _tensors(rng, spec):
    return [(name, t, ne, rng.integers(0, 256, _nbytes(t, ne), dtype=np.uint8)) for name, t, ne in spec]


def _kvs():
    kv = [("general.architecture", STRING, "llama"), ("test.u8", 0, 250), ("test.i8", 1, -7),
          ("test.u16", 2, 65000), ("test.i16", 3, -30000), ("test.u32", 4, 4000000000), ("test.i32", 5, -2000000000),
          ("test.f32", 6, 3.25), ("test.bool", 7, True), ("test.false", 7, False), ("test.u64", 10, 2 ** 63 + 5),
          ("test.i64", 11, -(2 ** 62)), ("test.f64", 12, -1.0e300), ("test.str.empty", STRING, ""),
          ("test.str.utf8", STRING, "grüße ☃")]
    for et in (0, 1, 2, 3, 4, 5, 6, 7, 10, 11, 12):
        items = [1, 0, 1] if et == 7 else list(range(-3 if et in (1, 3, 5, 11) else 0, 5))
        kv.append((f"test.arr.{et}", ARRAY, (et, items)))
    kv.append(("test.arr.empty", ARRAY, (4, [])))
    kv.append(("tokenizer.ggml.tokens", ARRAY, (STRING, ["<s>", "", "été", "x" * 300])))
    return kv


def _ours(path):
    with spq4k.Gguf(str(path)) as g:
        return {"version": g.version, "alignment": g.alignment, "data_offset": g.data_offset, "kv": g.kv(),
                "tensors": g.tensors(), "bytes": [g.tensor_bytes(i).copy() for i in range(len(g.tensors()))]}


def _same(ours, refv):
    assert ours["version"] == refv["version"]
    assert ours["alignment"] == refv["alignment"]
    assert ours["data_offset"] == refv["data_offset"]
    assert len(ours["kv"]) == len(refv["kv"])
    for (k, t, at, v), (rk, rt, rat, rv) in zip(ours["kv"], refv["kv"]):
        assert (k, t) == (rk, rt), (k, t, rk, rt)
        if t == ARRAY:
            assert at == rat, k
        if isinstance(rv, list):
            assert v == rv, k
        else:
            assert v.dtype == rv.dtype and v.tobytes() == rv.tobytes(), k
    assert len(ours["tensors"]) == len(refv["tensors"])
    for (name, t, ne, nd, off, nb), (rn, rt, rne, roff, rnb) in zip(ours["tensors"], refv["tensors"]):
        assert (name, t, ne, off, nb) == (rn, rt, rne, roff, rnb), (name, rn)
        last = max([j + 1 for j in range(4) if ne[j] != 1] + [1])
        assert nd == last                      # ggml_n_dims


def test_reference_written_file(rg, tmp_path):
    """gguf_write_to_file output (default alignment: the writer pads tensor
    offsets to 32 whatever general.alignment says, gguf.cpp:1244-1245)."""
    rng = np.random.default_rng(1)
    spec = [("token_embd.weight", 12, (512, 7)), ("blk.0.attn_norm.weight", 0, (33,)),
            ("blk.0.attn_q.weight", 12, (256, 9)), ("blk.0.attn_v.weight", 14, (768, 5)),
            ("blk.0.ffn_down.weight", 13, (512, 3)), ("blk.0.ffn_gate_exps.weight", 8, (96, 4, 6)),
            ("blk.1.scale", 1, (3, 1, 1, 5)), ("blk.1.q4_0", 2, (64, 3, 2, 2)), ("blk.1.ids", 26, (11,)),
            ("blk.1.i8", 24, (17, 3)), ("blk.1.bf16", 30, (7, 1, 1, 1)), ("blk.1.mxfp4", 39, (64, 2)),
            ("output.weight", 14, (256, 3))]
    tensors = _tensors(rng, spec)
    path = tmp_path / "m.gguf"
    assert rg.write(path, tensors, _kvs())
    refv = rg.read(path)
    assert refv is not None
    ours = _ours(path)
    _same(ours, refv)
    for (name, t, ne, data), got in zip(tensors, ours["bytes"]):
        np.testing.assert_array_equal(got, data, err_msg=name)


def test_many_tensors(rg, tmp_path):
    rng = np.random.default_rng(7)
    spec = [(f"blk.{i // 7}.t{i % 7}.weight", [0, 8, 12, 14][i % 4], ((i % 5 + 1) * 256, i % 3 + 1))
            for i in range(700)]
    tensors = _tensors(rng, spec)
    path = tmp_path / "many.gguf"
    assert rg.write(path, tensors)
    ours = _ours(path)
    _same(ours, rg.read(path))
    for (_, _, _, data), got in zip(tensors, ours["bytes"]):
        np.testing.assert_array_equal(got, data)
    with spq4k.Gguf(str(path)) as g:
        assert g.find_tensor("blk.50.t0.weight") == 350
        assert g.find_tensor("nope") == -1


# ---- malformed files ---------------------------------------------------------------------------
def _gstr(s):
    b = s if isinstance(s, bytes) else s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _gstr(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<iQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack("<" + {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q",
                              12: "d"}[t], v)


def _build(kvs, tensors, version=3, magic=b"GGUF", n_tensors=None, n_kv=None, alignment=32, data=None,
           raw_kv=None):
    """A GGUF byte image: kvs [(key, type, value)], tensors [(name, n_dims,
    ne list, type, offset)] (offset None = the running padded offset),
    data bytes after the aligned header (None = zeros of the right size)."""
    out = bytearray(magic) + struct.pack("<Iqq", version, len(tensors) if n_tensors is None else n_tensors,
                                         len(kvs) if n_kv is None else n_kv)
    for key, t, v in kvs:
        out += _gstr(key) + struct.pack("<i", t) + _value(t, v)
    if raw_kv:
        out += raw_kv
    size = 0
    for name, nd, ne, t, off in tensors:
        out += _gstr(name) + struct.pack("<I", nd) + b"".join(struct.pack("<q", x) for x in ne[:nd])
        out += struct.pack("<iQ", t, size if off is None else off)
        full = list(ne) + [1] * (4 - len(ne))
        blk, bs = TYPES.get(t, (1, 1))
        nb = int(np.prod(full)) // blk * bs if all(x >= 0 for x in full) else 0
        size += (nb + alignment - 1) // alignment * alignment
    out += b"\0" * ((-len(out)) % alignment)
    out += bytes(size) if data is None else data
    return bytes(out)


GOOD_T = [("a", 2, [256, 2], 12, None), ("b", 1, [64], 0, None)]
GOOD_KV = [("general.name", STRING, "x"), ("n", 4, 7)]


def _cases():
    c = {
        "valid": _build(GOOD_KV, GOOD_T),
        "valid_v2": _build(GOOD_KV, GOOD_T, version=2),
        "no_tensors": _build(GOOD_KV, []),
        "zero_row": _build(GOOD_KV, [("z", 2, [0, 3], 0, None)]),
        "bad_magic": _build(GOOD_KV, GOOD_T, magic=b"GGUG"),
        "version_0": _build(GOOD_KV, GOOD_T, version=0),
        "version_1": _build(GOOD_KV, GOOD_T, version=1),
        "version_4": _build(GOOD_KV, GOOD_T, version=4),
        "byte_swapped": _build(GOOD_KV, GOOD_T, version=0x03000000),
        "neg_tensors": _build(GOOD_KV, GOOD_T, n_tensors=-1),
        "neg_kv": _build(GOOD_KV, GOOD_T, n_kv=-2),
        "too_many_kv": _build(GOOD_KV, GOOD_T, n_kv=3),
        "dup_key": _build(GOOD_KV + [("n", 4, 8)], GOOD_T),
        "bad_kv_type": _build(GOOD_KV, GOOD_T, n_kv=3, raw_kv=_gstr("bad") + struct.pack("<i", 13) + b"\0" * 8),
        "nested_array": _build(GOOD_KV, GOOD_T, n_kv=3,
                               raw_kv=_gstr("nest") + struct.pack("<iiQ", ARRAY, ARRAY, 0)),
        "huge_string": _build(GOOD_KV, GOOD_T, n_kv=3,
                              raw_kv=_gstr("s") + struct.pack("<iQ", STRING, 1 << 40)),
        "array_past_end": _build(GOOD_KV, GOOD_T, n_kv=3,
                                 raw_kv=_gstr("arr") + struct.pack("<iiQ", ARRAY, 4, 1 << 28)),
        "dup_tensor": _build(GOOD_KV, GOOD_T + [("a", 1, [32], 0, None)]),
        "five_dims": _build(GOOD_KV, [("t", 5, [1, 1, 1, 1, 1], 0, None)]),
        "neg_dim": _build(GOOD_KV, [("t", 2, [32, -1], 0, None)]),
        "type_4": _build(GOOD_KV, [("t", 1, [32], 4, None)]),
        "type_31": _build(GOOD_KV, [("t", 1, [32], 31, None)]),
        "type_42": _build(GOOD_KV, [("t", 1, [32], 42, None)]),
        "type_neg": _build(GOOD_KV, [("t", 1, [32], -1, None)]),
        "ragged_row": _build(GOOD_KV, [("t", 2, [100, 2], 12, None)]),
        "bad_offset": _build(GOOD_KV, [("a", 2, [256, 2], 12, None), ("b", 1, [64], 0, 64)]),
        "name_64": _build(GOOD_KV, [("n" * 64, 1, [32], 0, None)]),
        "name_63": _build(GOOD_KV, [("n" * 63, 1, [32], 0, None)]),
        "align_48": _build(GOOD_KV + [("general.alignment", 4, 48)], GOOD_T, alignment=48),
        "align_0": _build(GOOD_KV + [("general.alignment", 4, 0)], GOOD_T, alignment=32),
        "align_64": _build(GOOD_KV + [("general.alignment", 4, 64)], GOOD_T, alignment=64),
    }
    # cuts inside the header (the tensor infos end at byte 148, before the padding)
    v = c["valid"]
    for cut in (3, 10, 24, 40, 100, 140, 147):
        c[f"cut_{cut}"] = v[:cut]
    return c


CASES = _cases()


@pytest.mark.parametrize("name", sorted(CASES))
def test_malformed_like_reference(rg, tmp_path, name):
    path = tmp_path / f"{name}.gguf"
    path.write_bytes(CASES[name])
    refv = rg.read(path)
    try:
        ours = _ours(path)
    except spq4k.Spq4kError as e:
        assert e.rc == -22, e
        ours = None
    assert (ours is None) == (refv is None), (name, "ours accepts" if ours else "ours rejects",
                                             "reference accepts" if refv else "reference rejects")
    if ours is not None:
        _same(ours, refv)


@pytest.mark.parametrize("alignment", [1, 2, 64, 256, 4096])
def test_alignments(rg, tmp_path, alignment):
    """general.alignment other than 32: offsets padded to it (byte builder),
    read identically by both readers, tensor bytes where the offsets say."""
    rng = np.random.default_rng(alignment)
    tens = [("a", 2, [256, 3], 12, None), ("b", 1, [5], 0, None), ("c", 3, [64, 2, 3], 8, None),
            ("d", 2, [768, 1], 14, None)]
    sizes = [3 * 144, 20, 6 * 2 * 34, 3 * 210]
    data = bytearray()
    for nb in sizes:
        blob = rng.integers(0, 256, nb, dtype=np.uint8).tobytes()
        data += blob + b"\0" * ((-nb) % alignment)
    path = tmp_path / "al.gguf"
    path.write_bytes(_build(GOOD_KV + [("general.alignment", 4, alignment)], tens, alignment=alignment,
                            data=bytes(data)))
    ours = _ours(path)
    _same(ours, rg.read(path))
    assert ours["data_offset"] % alignment == 0
    off = 0
    for nb, got in zip(sizes, ours["bytes"]):
        assert got.tobytes() == bytes(data[off:off + nb])
        off += nb + (-nb) % alignment


def test_alignment_of_wrong_type_rejected(tmp_path):
    """general.alignment must be a u32: the reference aborts on another type
    (gguf_get_val_u32's type assertion), the reader returns -EINVAL."""
    for t, v in ((5, 32), (10, 32), (STRING, "32"), (ARRAY, (4, [32]))):
        path = tmp_path / f"align_{t}.gguf"
        path.write_bytes(_build(GOOD_KV + [("general.alignment", t, v)], GOOD_T))
        with pytest.raises(spq4k.Spq4kError) as e:
            spq4k.Gguf(str(path))
        assert e.value.rc == -22


def test_data_past_end_rejected(rg, tmp_path):
    """Tensor data cut short: the reference's no_alloc reader accepts the
    header (it reads no data); the reader rejects the file, since it hands
    out pointers into it."""
    v = CASES["valid"]
    for cut in (len(v) - 1, len(v) - 256):
        path = tmp_path / f"short_{cut}.gguf"
        path.write_bytes(v[:cut])
        assert rg.read(path) is not None
        with pytest.raises(spq4k.Spq4kError) as e:
            spq4k.Gguf(str(path))
        assert e.value.rc == -22
    # exactly the tensor bytes, without the last tensor's padding: accepted by both
    path = tmp_path / "unpadded.gguf"
    tens = [("b", 1, [64], 0, None), ("a", 2, [256, 2], 12, None)]
    path.write_bytes(_build(GOOD_KV, tens, data=bytes(256 + 288)))
    assert rg.read(path) is not None
    with spq4k.Gguf(str(path)) as g:
        assert [t[4:] for t in g.tensors()] == [(0, 256), (256, 288)]


def test_missing_file_and_errno():
    with pytest.raises(spq4k.Spq4kError) as e:
        spq4k.Gguf("/nonexistent/model.gguf")
    assert e.value.rc == -2
