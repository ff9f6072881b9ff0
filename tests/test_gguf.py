"""The GGUF reader (include/hq_gguf.h) on the CPU: tensor tables and data views of files written by
tests/golden/gguf_writer.py, the same bytes as the reference's own reader finds (src/gguf.c, through
oracle/_ref/libref.so), the general.alignment rule, and refusal of malformed files."""
import os
import struct

import numpy as np
import pytest

import gguf_writer
import hq
import synth

pytestmark = []


def tensors():
    rng = synth.Rng(70)
    return [("blk.0.attn_q.weight", (512, 96), synth.Q8_0, synth.q8_0_blocks(rng, 96, 512)),
            ("blk.0.ffn_gate.weight", (1024, 40), synth.Q4_K, synth.q4_k_blocks(rng, 40, 1024)),
            ("blk.0.ffn_up.weight", (1024, 40), synth.Q6_K, synth.q6_k_blocks(rng, 40, 1024)),
            ("blk.0.attn_norm.weight", (512,), 0, np.arange(512, dtype=np.float32)),
            ("output.weight", (256, 3, 2), synth.Q8_0, synth.q8_0_blocks(rng, 6, 256))]


@pytest.mark.parametrize("alignment", [32, 64, 4096])
def test_tensor_table_and_views(tmp_path, alignment):
    path = tmp_path / "t.gguf"
    ts = tensors()
    gguf_writer.write(str(path), [("general.architecture", "str", "llama"), ("llama.block_count", "u32", 1)], ts,
                      alignment)
    g = hq.Gguf(path)
    info = g.tensors()
    assert [t["name"] for t in info] == [t[0] for t in ts]
    assert g.get_uint("llama.block_count") == 1
    raw = path.read_bytes()
    for t, (name, ne, gtype, data) in zip(info, ts):
        assert t["type"] == gtype and t["ne"][:len(ne)] == ne and t["n_dims"] == len(ne)
        assert t["offset"] % alignment == 0
        assert raw[t["offset"]:t["offset"] + data.nbytes] == np.ascontiguousarray(data).tobytes()
        if gtype:
            w = g.wmat(name, 0)
            assert (w.rows, w.cols, w.ggml_type) == (int(np.prod(ne[1:])), ne[0], gtype)
            assert np.array_equal(g.view_bytes(name), data.reshape(w.rows, -1))
    with pytest.raises(hq.HQError, match="ggml type 0"):
        g.wmat("blk.0.attn_norm.weight")
    with pytest.raises(hq.HQError, match="no tensor"):
        g.wmat("missing")
    g.close()


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref", "libref.so")),
                    reason="oracle/_ref/libref.so not built (needs /root/reference)")
def test_same_bytes_as_the_reference_reader(tmp_path, reference):
    path = tmp_path / "t.gguf"
    ts = tensors()
    gguf_writer.write(str(path), [("general.architecture", "str", "llama")], ts, 64)
    g = hq.Gguf(path)
    for name, ne, gtype, data in ts:
        if not gtype:
            continue
        rt, rne, rbytes = reference.gguf_tensor(path, name)
        w = g.wmat(name)
        assert rt == w.ggml_type and rne[0] == w.cols and int(np.prod(rne[1:])) == w.rows
        assert np.array_equal(g.view_bytes(name).ravel(), rbytes)
    g.close()


def _good_file(tmp_path):
    path = tmp_path / "good.gguf"
    gguf_writer.write(str(path), [("k", "u32", 7)], tensors()[:2])
    return path, bytearray(path.read_bytes())


def test_malformed_files_are_refused(tmp_path):
    path, raw = _good_file(tmp_path)
    cases = {
        "bad magic": b"GGUX" + bytes(raw[4:]),
        "version 1": bytes(raw[:4]) + struct.pack("<I", 1) + bytes(raw[8:]),
        "truncated header": bytes(raw[:40]),
        "huge tensor count": bytes(raw[:8]) + struct.pack("<Q", 1 << 40) + bytes(raw[16:]),
    }
    for what, data in cases.items():
        p = tmp_path / "bad.gguf"
        p.write_bytes(data)
        with pytest.raises(hq.HQError):
            hq.Gguf(p)
    # a non-power-of-two alignment
    p = tmp_path / "align.gguf"
    gguf_writer.write(str(p), [("general.alignment", "u32", 48)], tensors()[:1])
    with pytest.raises(hq.HQError, match="malformed"):
        hq.Gguf(p)
    # data cut short: the table parses, the view is refused
    p = tmp_path / "short.gguf"
    p.write_bytes(bytes(raw[:len(raw) - 100]))
    g = hq.Gguf(p)
    with pytest.raises(hq.HQError, match="outside the file"):
        g.wmat("blk.0.ffn_gate.weight")
    g.close()
    with pytest.raises(hq.HQError, match="cannot open"):
        hq.Gguf(tmp_path / "absent.gguf")


# ---- acceptance edge cases, written byte by byte: each file's expected verdict is stated here and,
# where oracle/_ref/libref.so is built, the reference's own reader (src/gguf.c:134-219) must agree.
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)


def _s(b):
    b = b if isinstance(b, bytes) else b.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, vtype, payload):
    return _s(key) + struct.pack("<I", vtype) + payload


def _arr(etype, n, body=b""):
    return struct.pack("<IQ", etype, n) + body


def _nested(depth, inner_type, inner_n, inner_body=b""):
    """An array value whose elements are arrays, `depth` levels of arrays in all, the innermost of
    `inner_n` elements of `inner_type`."""
    v = _arr(inner_type, inner_n, inner_body)
    for _ in range(depth - 1):
        v = _arr(ARR, 1, v)
    return v


def _tensor(name, ne, gtype=8, offset=0):
    return _s(name) + struct.pack("<I", len(ne)) + struct.pack("<%dQ" % len(ne), *ne) + struct.pack("<IQ", gtype, offset)


def _file(kvs, trs, version=3, n_kv=None, n_t=None, tail=b""):
    head = b"GGUF" + struct.pack("<IQQ", version, len(trs) if n_t is None else n_t, len(kvs) if n_kv is None else n_kv)
    return head + b"".join(kvs) + b"".join(trs) + tail


ACCEPTANCE = {
    # name: (file bytes, accepted)
    "plain": (_file([_kv("a", U32, struct.pack("<I", 1))], [_tensor("t", (32, 2))]), True),
    "every scalar type": (_file([_kv("k%d" % t, t, b"\1" * w) for t, w in
                                 [(U8, 1), (I8, 1), (U16, 2), (I16, 2), (U32, 4), (I32, 4), (F32, 4), (BOOL, 1),
                                  (U64, 8), (I64, 8), (F64, 8)]], []), True),
    "unknown value type": (_file([_kv("x", 13, b"\0" * 8)], []), False),
    "empty array of an unknown type": (_file([_kv("x", ARR, _arr(13, 0))], []), True),
    "array of an unknown type": (_file([_kv("x", ARR, _arr(13, 1, b"\0" * 8))], []), False),
    "array of strings": (_file([_kv("x", ARR, _arr(STR, 2, _s("ab") + _s("")))], []), True),
    "arrays nested 5 deep, scalars inside": (_file([_kv("x", ARR, _nested(5, U8, 3, b"abc"))], []), True),
    "arrays nested 5 deep, strings inside": (_file([_kv("x", ARR, _nested(5, STR, 1, _s("a")))], []), False),
    "arrays nested 5 deep, empty strings array": (_file([_kv("x", ARR, _nested(5, STR, 0))], []), True),
    "arrays nested 4 deep, strings inside": (_file([_kv("x", ARR, _nested(4, STR, 1, _s("a")))], []), True),
    "arrays nested 6 deep": (_file([_kv("x", ARR, _nested(6, U8, 1, b"a"))], []), False),
    "scalar array longer than the file": (_file([_kv("x", ARR, _arr(U32, 1 << 40))], []), False),
    "string longer than the file": (_file([_kv("x", STR, struct.pack("<Q", 1 << 50))], []), False),
    "key longer than the file": (_file([struct.pack("<Q", 1 << 50)], []), False),
    "truncated metadata": (_file([_kv("a", U32, b"\1\0")], []), False),
    "more metadata than written": (_file([_kv("a", U32, b"\1\0\0\0")], [], n_kv=2), False),
    "2^20 metadata entries promised": (_file([], [], n_kv=(1 << 20) + 1), False),
    "version 2": (_file([], [_tensor("t", (32,))], version=2), True),
    "version 4": (_file([], [], version=4), False),
    "name of 255 bytes": (_file([], [_tensor("n" * 255, (32,))]), True),
    "name of 256 bytes": (_file([], [_tensor("n" * 256, (32,))]), False),
    "0 dimensions": (_file([], [_tensor("t", ())]), True),
    "4 dimensions": (_file([], [_tensor("t", (32, 2, 2, 2))]), True),
    "5 dimensions": (_file([], [_tensor("t", (32, 1, 1, 1, 1))]), False),
    "zero extent": (_file([], [_tensor("t", (32, 0))]), False),
    "extent 2^32": (_file([], [_tensor("t", (32, 1 << 32))]), True),
    "extent 2^32 + 1": (_file([], [_tensor("t", (1, (1 << 32) + 1))]), False),
    "2^40 elements": (_file([], [_tensor("t", (1 << 20, 1 << 20))]), True),
    "2^40 + 2^20 elements": (_file([], [_tensor("t", (1 << 20, (1 << 20) + 1))]), False),
    "truncated tensor record": (_file([], [_tensor("t", (32, 2))[:-3]]), False),
    "alignment 64": (_file([_kv("general.alignment", U32, struct.pack("<I", 64))], [_tensor("t", (32,))]), True),
    "alignment 48": (_file([_kv("general.alignment", U32, struct.pack("<I", 48))], []), False),
    "alignment 0": (_file([_kv("general.alignment", U32, struct.pack("<I", 0))], []), False),
    "alignment 0 as u64 (ignored)": (_file([_kv("general.alignment", U64, struct.pack("<Q", 0))], []), True),
    "alignment 48 then 64 (the last counts)": (_file([_kv("general.alignment", U32, struct.pack("<I", 48)),
                                                      _kv("general.alignment", U32, struct.pack("<I", 64))], []), True),
    "alignment 64 then 48 (the last counts)": (_file([_kv("general.alignment", U32, struct.pack("<I", 64)),
                                                      _kv("general.alignment", U32, struct.pack("<I", 48))], []), False),
}


@pytest.mark.parametrize("case", sorted(ACCEPTANCE))
def test_acceptance_matches_the_reference_reader(tmp_path, request, case):
    data, accepted = ACCEPTANCE[case]
    path = tmp_path / "case.gguf"
    # past the records: bytes never parsed as a valid record (none where the case is a cut-off file)
    path.write_bytes(data + (b"" if case.startswith("truncated") else b"\xff" * 64))
    if accepted:
        hq.Gguf(path).close()
    else:
        with pytest.raises(hq.HQError, match="malformed|implausible|version"):
            hq.Gguf(path)
    if os.path.exists(os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref", "libref.so")):
        assert request.getfixturevalue("reference").gguf_accepts(path) == accepted


def _located(path, name, rows=2, cols=32):
    g = hq.Gguf(path)
    try:
        w = g.wmat(name)
        assert (w.rows, w.cols) == (rows, cols)
        return g.view_bytes(name).ravel().copy()
    finally:
        g.close()


@pytest.mark.parametrize("order", ["first", "second"])
def test_alignment_and_duplicate_names_locate_the_same_bytes(tmp_path, request, order):
    """The last u32 general.alignment sets the data start; of two tensors with one name the first
    record counts; both readers find the same bytes."""
    al = [64, 256] if order == "first" else [256, 64]
    kvs = [_kv("general.alignment", U32, struct.pack("<I", a)) for a in al]
    trs = [_tensor("w", (32, 2), 8, 0), _tensor("w", (32, 2), 8, 128), _tensor("z", (32, 2), 8, 256)]
    head = _file(kvs, trs)
    start = -(-len(head) // al[-1]) * al[-1]
    body = bytes(range(256)) * 2
    raw = head + b"\0" * (start - len(head)) + body[:384] + b"\xee" * 4096
    path = tmp_path / "dup.gguf"
    path.write_bytes(raw)
    got = _located(path, "w")
    assert got.tobytes() == raw[start:start + 68]
    assert _located(path, "z").tobytes() == raw[start + 256:start + 324]
    if os.path.exists(os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref", "libref.so")):
        ref = request.getfixturevalue("reference")
        for name in ("w", "z"):
            assert np.array_equal(ref.gguf_tensor(path, name)[2], _located(path, name))


def test_many_tensors_are_found_by_name(tmp_path):
    """The name-sorted index: 300 tensors written in a shuffled name order are each found at their
    own data (and a missing name between two present ones is refused)."""
    rng = np.random.default_rng(5)
    names = ["blk.%d.%s" % (i // 3, ("q", "k", "v")[i % 3]) for i in range(300)]
    order = rng.permutation(300)
    data = [np.full(68, i % 251, np.uint8) for i in range(300)]
    ts = [(names[i], (32, 2), synth.Q8_0, data[i]) for i in order]
    path = tmp_path / "many.gguf"
    gguf_writer.write(str(path), [], ts)
    g = hq.Gguf(path)
    for i in range(300):
        assert np.array_equal(g.view_bytes(names[i]).ravel(), data[i])
    with pytest.raises(hq.HQError, match="no tensor"):
        g.wmat("blk.1.r")
    g.close()
