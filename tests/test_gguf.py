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
