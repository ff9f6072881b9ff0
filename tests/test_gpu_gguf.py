"""On-disk GGUF -> HBM (include/hq_gguf.h + hq_mat_upload): matrices uploaded straight from the file
mapping through the pinned staging path come back byte for byte (rows in Hugging Face order) and
decode bit-exactly; a matrix larger than one 32 MiB staging chunk crosses chunk boundaries; and the
config-1 model read from its GGUF file runs through hip_backend_create to the golden logits."""
import ctypes as C

import numpy as np
import pytest

import gguf_writer
import synth
from conftest import max_abs, same_bits_nan_aware

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gpu]", *a, flush=True)


def test_upload_from_gguf_mapping(hqlib, oracle, tmp_path):
    import oracle as o
    rng = synth.Rng(80)
    ts = [("q8", (2560, 16384), synth.Q8_0, synth.q8_0_blocks(rng, 16384, 2560), 8),   # 44.6 MB: two chunks
          ("q4", (2560, 9728), synth.Q4_K, synth.q4_k_blocks(rng, 9728, 2560), 0),
          ("q6", (1024, 640), synth.Q6_K, synth.q6_k_blocks(rng, 640, 1024), 4),
          ("q4p", (512, 512), synth.Q4_K, synth.q4_k_blocks(rng, 512, 512), 8)]
    path = tmp_path / "m.gguf"
    gguf_writer.write(str(path), [("general.architecture", "str", "llama")], [t[:4] for t in ts], 64)
    g = hqlib.Gguf(path)
    for name, ne, gtype, blocks, perm in ts:
        rows, cols = ne[1], ne[0]
        say(f"upload {name} type={gtype} {rows}x{cols} perm={perm}")
        W = g.upload(name, perm)
        wm = o.WMat(3, rows, cols, blocks.ctypes.data, gtype, perm)
        src = np.array([oracle.lib.or_src_row(C.byref(wm), r) for r in range(rows)])
        assert np.array_equal(W.download(), blocks[src])
        sel = np.unique(np.concatenate([np.arange(0, 8), np.arange(rows - 8, rows), [rows // 2]]))
        got = np.concatenate([hqlib.dequant(W, int(r), 1) for r in sel])
        want = oracle.dequantize(np.ascontiguousarray(blocks), gtype, rows, cols, perm)[sel]
        assert same_bits_nan_aware(got, want)
        W.free()
    g.close()


def test_backend_from_gguf_file(hqlib, tmp_path):
    from test_oracle import load_golden
    model = synth.tiny_llama(1)
    path = tmp_path / "tiny.gguf"
    gguf_writer.write_tiny_llama(str(path), model)
    g = hqlib.Gguf(path)
    view = hqlib.RefModelView(model)
    c = model["cfg"]
    # every matrix of the model_t mirror now points into the file mapping (q/k with perm_heads)
    names = {"q": ("attn_q", c["n_heads"]), "k": ("attn_k", c["n_kv_heads"]), "v": ("attn_v", 0),
             "o": ("attn_output", 0), "gate": ("ffn_gate", 0), "up": ("ffn_up", 0), "down": ("ffn_down", 0)}
    for li in range(c["n_layers"]):
        for key, (gn, perm) in names.items():
            setattr(view.layers[li], key, g.wmat(f"blk.{li}.{gn}.weight", perm))
    view.m.embed, view.m.lm_head = g.wmat("token_embd.weight"), g.wmat("output.weight")
    gd = load_golden("tiny_llama.npz")
    say("hip_backend_create from the GGUF mapping")
    be = hqlib.HipBackend(view, 256)
    got = be.forward(gd["tokens"], gd["ids"])
    be.destroy()
    g.close()
    say(f"logits {got} golden {gd['logits']}")
    assert max_abs(got, gd["logits"]) <= 1e-2 and np.argmax(got) == np.argmax(gd["logits"])
