"""ctypes wrapper of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Loads oracle/liboracle.so (this project's C restatement, hq_oracle.c) and, when it was built,
oracle/_ref/libref.so (the reference's own CPU sources). Only tests/, bench.py's cpu_baseline
leg and __graft_entry__.smoke() import this module, and only as the checker.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")


class WMat(C.Structure):
    """Layout of the reference wmat_t (cleanroom-transformer/src/transformer.h:293-300)."""
    _fields_ = [("dtype", C.c_int), ("rows", C.c_uint32), ("cols", C.c_uint32), ("data", C.c_void_p),
                ("ggml_type", C.c_int), ("perm_heads", C.c_uint32)]


class Layer(C.Structure):
    _fields_ = [(n, WMat) for n in ("q", "k", "v", "o", "gate", "up", "down")] + [
        ("in_norm", C.c_void_p), ("post_norm", C.c_void_p)]


class Llama(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden", "n_layers", "intermediate", "vocab", "n_heads", "n_kv_heads",
                                          "head_dim", "rot_dim")] + [
        ("eps", C.c_float), ("rope_theta", C.c_float), ("embed", WMat), ("lm_head", WMat),
        ("final_norm", C.c_void_p), ("layers", C.c_void_p), ("rope_inv_freq", C.c_void_p)]


DT_GGML = 3
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


def wmat(blocks, gtype, rows, cols, perm_heads=0):
    """WMat over a C-contiguous uint8 block array (the caller keeps `blocks` alive)."""
    assert blocks.flags["C_CONTIGUOUS"] and blocks.dtype == np.uint8
    return WMat(DT_GGML, rows, cols, blocks.ctypes.data, gtype, perm_heads)


class Oracle:
    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library {path} is not built (make -C oracle)")
        L = self.lib = C.CDLL(path)
        L.or_f16_to_f32.restype = C.c_float
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_scale_min_k4.argtypes = [C.c_int, _u8p, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        L.or_dequant_sub32.argtypes = [C.c_int, _u8p, C.c_int, _f32p]
        L.or_dequantize_row.argtypes = [C.c_int, C.c_void_p, _f32p, C.c_uint64]
        L.or_src_row.restype = C.c_uint32
        L.or_src_row.argtypes = [C.POINTER(WMat), C.c_uint32]
        L.or_wmat_row_f32.argtypes = [C.POINTER(WMat), C.c_uint32, _f32p]
        L.or_dot.restype = C.c_float
        L.or_dot.argtypes = [_f32p, _f32p, C.c_size_t]
        L.or_matmul.argtypes = [C.POINTER(WMat), _f32p, C.c_size_t, _f32p, C.c_int]
        L.or_matmul_rows.argtypes = [C.POINTER(WMat), _f32p, C.c_size_t, _f32p, C.c_int, C.c_uint32, C.c_uint32]
        L.or_gather_dot.argtypes = [C.POINTER(WMat), _f32p, _u32p, C.c_size_t, C.c_size_t, _f32p]
        L.or_f16_to_f32_array.argtypes = [_u16p, _f32p, C.c_size_t]
        L.or_llama_forward.restype = C.c_int
        L.or_llama_forward.argtypes = [C.POINTER(Llama), _u32p, C.c_size_t, _u32p, C.c_uint32, _f32p]
        L.or_llama_forward_h.restype = C.c_int
        L.or_llama_forward_h.argtypes = [C.POINTER(Llama), _u32p, C.c_size_t, _u32p, C.c_uint32, _f32p, _f32p]

    def f16_to_f32(self, bits):
        bits = np.ascontiguousarray(bits, dtype=np.uint16)
        out = np.empty(bits.shape, dtype=np.float32)
        self.lib.or_f16_to_f32_array(bits.ravel(), out.reshape(-1), bits.size)
        return out

    def dequantize(self, blocks, gtype, rows, cols, perm_heads=0):
        """All rows in Hugging Face order, float32 [rows, cols]."""
        w = wmat(blocks, gtype, rows, cols, perm_heads)
        out = np.empty((rows, cols), dtype=np.float32)
        for r in range(rows):
            self.lib.or_wmat_row_f32(C.byref(w), r, out[r])
        return out

    def matmul(self, blocks, gtype, rows, cols, x, y=None, accumulate=False, perm_heads=0, row_range=None):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        w = wmat(blocks, gtype, rows, cols, perm_heads)
        if y is None:
            y = np.zeros((T, rows), dtype=np.float32)
        if row_range is None:
            self.lib.or_matmul(C.byref(w), x.reshape(-1), T, y.reshape(-1), int(accumulate))
        else:
            self.lib.or_matmul_rows(C.byref(w), x.reshape(-1), T, y.reshape(-1), int(accumulate), *row_range)
        return y

    def gather_dot(self, blocks, gtype, rows, cols, h, ids):
        h = np.ascontiguousarray(h, dtype=np.float32)
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        B, k = ids.shape
        out = np.empty((B, k), dtype=np.float32)
        w = wmat(blocks, gtype, rows, cols)
        self.lib.or_gather_dot(C.byref(w), h.reshape(-1), ids.reshape(-1), B, k, out.reshape(-1))
        return out

    def llama_forward(self, model, tokens, ids, hidden=False):
        """model: synth.tiny_llama() dict (blocks in llama.cpp storage order). With hidden=True also
        returns the final-normalised last position (the CPU backend's last_hidden)."""
        st, keep = llama_struct(model)
        logits = np.empty(len(ids), dtype=np.float32)
        h = np.empty(model["cfg"]["hidden"], dtype=np.float32)
        rc = self.lib.or_llama_forward_h(C.byref(st), np.ascontiguousarray(tokens, np.uint32), len(tokens),
                                         np.ascontiguousarray(ids, np.uint32), len(ids), logits, h)
        del keep
        if rc:
            raise ValueError("or_llama_forward: bad tokens or ids")
        return (logits, h) if hidden else logits


def llama_struct(model):
    """Llama struct over a synth.tiny_llama() dict; returns (struct, objects to keep alive). Layer
    matrices are Q8_0 unless model["types"] names another ggml type for them (e.g. {"up": Q6_K})."""
    c = model["cfg"]
    H, I = c["hidden"], c["intermediate"]
    qw, kvw = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    keep = []
    layers = (Layer * c["n_layers"])()
    shapes = {"q": (qw, H, c["n_heads"]), "k": (kvw, H, c["n_kv_heads"]), "v": (kvw, H, 0), "o": (H, qw, 0),
              "gate": (I, H, 0), "up": (I, H, 0), "down": (H, I, 0)}
    for li, L in enumerate(model["layers"]):
        for name, (r, k, perm) in shapes.items():
            setattr(layers[li], name, wmat(L[name], model.get("types", {}).get(name, 8), r, k, perm))
        layers[li].in_norm = L["in_norm"].ctypes.data
        layers[li].post_norm = L["post_norm"].ctypes.data
    keep.append(layers)
    st = Llama(H, c["n_layers"], I, c["vocab"], c["n_heads"], c["n_kv_heads"], c["head_dim"], c["rot_dim"],
               c["eps"], c["rope_theta"], wmat(model["embed"], 8, c["vocab"], H), wmat(model["lm_head"], 8, c["vocab"], H),
               model["final_norm"].ctypes.data, C.cast(layers, C.c_void_p).value)
    if model.get("rope_inv_freq") is not None:
        inv = np.ascontiguousarray(model["rope_inv_freq"], np.float32)
        assert inv.shape == (c["rot_dim"] // 2,)
        keep.append(inv)
        st.rope_inv_freq = inv.ctypes.data
    return st, keep


class Reference:
    """The reference's own CPU code (oracle/_ref/libref.so), where it was built."""

    def __init__(self, path=REF_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"reference library {path} is not built (needs /root/reference; make -C oracle)")
        L = self.lib = C.CDLL(path)
        L.ref_f16_to_f32.restype = C.c_float
        L.ref_f16_to_f32.argtypes = [C.c_uint16]
        L.ref_scale_min_k4.argtypes = [C.c_int, _u8p, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8)]
        L.ref_dequant_sub32.argtypes = [C.c_int, _u8p, C.c_int, _f32p]
        L.ggml_dequantize_row.argtypes = [C.c_int, C.c_void_p, _f32p, C.c_uint64]
        L.wmat_row_f32.argtypes = [C.POINTER(WMat), C.c_uint32, _f32p]
        L.wmat_src_row.restype = C.c_uint32
        L.wmat_src_row.argtypes = [C.POINTER(WMat), C.c_uint32]
        L.ref_dot.restype = C.c_float
        L.ref_dot.argtypes = [_f32p, _f32p, C.c_size_t]
        L.ref_matmul.argtypes = [C.POINTER(WMat), _f32p, C.c_size_t, _f32p, C.c_int]
        L.ref_last_error.restype = C.c_char_p
        L.ref_gguf_tensor.restype = C.c_int
        L.ref_gguf_tensor.argtypes = [C.c_char_p, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_uint64), C.c_void_p,
                                      C.c_size_t, C.POINTER(C.c_size_t)]
        L.ref_gguf_open_ok.restype = C.c_int
        L.ref_gguf_open_ok.argtypes = [C.c_char_p]
        L.ref_logits.restype = C.c_int
        L.ref_logits.argtypes = [C.c_char_p, _u32p, C.c_size_t, _u32p, C.c_uint32, _f32p, C.c_void_p]

    def dequantize(self, blocks, gtype, rows, cols, perm_heads=0):
        w = wmat(blocks, gtype, rows, cols, perm_heads)
        out = np.empty((rows, cols), dtype=np.float32)
        for r in range(rows):
            self.lib.wmat_row_f32(C.byref(w), r, out[r])
        return out

    def matmul(self, blocks, gtype, rows, cols, x, y=None, accumulate=False, perm_heads=0):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        w = wmat(blocks, gtype, rows, cols, perm_heads)
        if y is None:
            y = np.zeros((T, rows), dtype=np.float32)
        self.lib.ref_matmul(C.byref(w), x.reshape(-1), T, y.reshape(-1), int(accumulate))
        return y

    def gguf_tensor(self, path, name, cap=1 << 26):
        """(type, ne, data bytes) of a tensor as the reference's GGUF reader finds it."""
        t, ne, n = C.c_int(), (C.c_uint64 * 4)(), C.c_size_t()
        buf = np.empty(cap, np.uint8)
        if self.lib.ref_gguf_tensor(str(path).encode(), name.encode(), C.byref(t), ne, buf.ctypes.data, cap, C.byref(n)):
            raise RuntimeError("reference: " + (self.lib.ref_last_error() or b"?").decode())
        return t.value, tuple(ne), buf[:n.value].copy()

    def gguf_accepts(self, path):
        """Whether the reference's GGUF reader opens the file (header, metadata, tensor table)."""
        return self.lib.ref_gguf_open_ok(str(path).encode()) == 0

    def logits(self, gguf_path, tokens, ids, hidden_size=0):
        """Option logits of the reference CPU backend; with hidden_size > 0 also its last_hidden."""
        out = np.empty(len(ids), dtype=np.float32)
        h = np.empty(max(hidden_size, 1), dtype=np.float32)
        rc = self.lib.ref_logits(gguf_path.encode(), np.ascontiguousarray(tokens, np.uint32), len(tokens),
                                 np.ascontiguousarray(ids, np.uint32), len(ids), out,
                                 h.ctypes.data if hidden_size else None)
        if rc:
            raise RuntimeError("reference: " + (self.lib.ref_last_error() or b"?").decode())
        return (out, h) if hidden_size else out
