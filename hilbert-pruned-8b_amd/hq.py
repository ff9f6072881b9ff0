"""ctypes binding of libhq.so, the gfx950 quantized matmul path (C ABI: include/hq.h, hq_llama.h).

Python is plumbing here: it moves numpy arrays in and out of device buffers and calls the C ABI.
There is no fallback: if libhq.so is not built, or a call fails, an exception is raised.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhq.so")

Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 8, 10, 11, 12, 13, 14
DT_GGML = 3
BLOCK_VALUES = {Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}

# Every function declared in include/hq.h and include/hq_llama.h.
EXPORTS = (
    "hq_last_error", "hq_device_init", "hq_device_count", "hq_device_name", "hq_mat_upload", "hq_mat_free",
    "hq_mat_shape", "hq_mat_device_bytes", "hq_mat_download", "hq_dequant_f32", "hq_gemm", "hq_gemv",
    "hq_gather_dot", "hq_gather_dot_dev", "hq_matmul_host", "hq_malloc", "hq_free", "hq_memcpy_h2d",
    "hq_memcpy_d2h", "hq_memcpy_d2d", "hq_memset", "hq_stream_create", "hq_stream_destroy", "hq_stream_synchronize",
    "hq_device_synchronize", "hq_time_gemm", "hq_time_gemm_kernel", "hq_time_gather", "hq_gemm_tiles", "hq_llama_forward",
    "hq_embed_f32", "hq_gemm_kernel", "hq_gemm_noalloc", "hq_gemm_workspace_bytes", "hq_gemv_swiglu",
    "hq_gguf_open", "hq_gguf_close", "hq_gguf_n_tensors", "hq_gguf_tensor_info", "hq_gguf_find", "hq_gguf_get_uint",
    "hq_gguf_wmat", "hq_mat_upload_pair", "hq_gemm_swiglu", "hq_time_gemm_swiglu", "hq_time_read",
)
# include/hq_backend.h (no hq_ prefix: the names of the reference entry points they replace)
BACKEND_EXPORTS = ("hip_backend_create", "hip_selftest")


class WMat(C.Structure):
    """hq_wmat_t: field for field the reference wmat_t (cleanroom-transformer/src/transformer.h:293-300)."""
    _fields_ = [("dtype", C.c_int), ("rows", C.c_uint32), ("cols", C.c_uint32), ("data", C.c_void_p),
                ("ggml_type", C.c_int), ("perm_heads", C.c_uint32)]


class LlamaLayer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("q", "k", "v", "o", "gate", "up", "down")] + [
        ("in_norm", C.c_void_p), ("post_norm", C.c_void_p)]


class Llama(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden", "n_layers", "intermediate", "vocab", "n_heads", "n_kv_heads",
                                          "head_dim", "rot_dim")] + [
        ("eps", C.c_float), ("rope_theta", C.c_float), ("embed", C.c_void_p), ("lm_head", C.c_void_p),
        ("final_norm", C.c_void_p), ("layers", C.c_void_p), ("rope_inv_freq", C.c_void_p)]


# Layout mirrors of the reference's config_t, layer_t, st_set_t, model_t and backend_t
# (cleanroom-transformer/src/transformer.h:229-235, :278-364), as include/hq_backend.h declares them.
class RefConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden", "n_layers", "intermediate", "vocab", "n_heads", "n_kv_heads",
                                          "head_dim", "rot_dim", "lin_k_heads", "lin_v_heads", "lin_k_dim",
                                          "lin_v_dim", "conv_k", "arch")] + [
        ("eps", C.c_float), ("rope_theta", C.c_float), ("norm_offset", C.c_float), ("attn_gate", C.c_bool),
        ("qk_norm", C.c_bool), ("tied", C.c_bool), ("rope_llama3", C.c_bool), ("rope_factor", C.c_float),
        ("rope_low_freq", C.c_float), ("rope_high_freq", C.c_float), ("rope_orig_ctx", C.c_float),
        ("layer_type", C.c_uint8 * 256), ("n_full", C.c_uint32), ("n_linear", C.c_uint32)]


class RefLayer(C.Structure):
    _fields_ = [("type", C.c_uint32), ("slot", C.c_uint32), ("in_norm", C.c_void_p), ("post_norm", C.c_void_p)] + \
        [(n, WMat) for n in ("gate", "up", "down", "q", "k", "v", "o")] + \
        [("q_norm", C.c_void_p), ("k_norm", C.c_void_p)] + [(n, WMat) for n in ("qkv", "z", "b", "a", "out")] + \
        [(n, C.c_void_p) for n in ("conv_w", "A_log", "dt_bias", "lin_norm")]


class RefStSet(C.Structure):
    _fields_ = [("files", C.c_void_p), ("n_files", C.c_size_t), ("tensors", C.c_void_p), ("n_tensors", C.c_size_t)]


class RefModel(C.Structure):
    _fields_ = [("cfg", RefConfig), ("st", RefStSet), ("embed", WMat), ("lm_head", WMat), ("final_norm", C.c_void_p),
                ("layers", C.c_void_p), ("rope_inv_freq", C.c_void_p), ("gguf", C.c_void_p), ("source", C.c_char * 512)]


class RefBackend(C.Structure):
    pass


_BP = C.POINTER(RefBackend)
RefBackend._fields_ = [
    ("name", C.c_char_p), ("reset", C.CFUNCTYPE(C.c_int, _BP)),
    ("forward", C.CFUNCTYPE(C.c_int, _BP, C.c_void_p, C.c_size_t, C.c_void_p, C.c_uint32, C.c_void_p)),
    ("snapshot", C.CFUNCTYPE(C.c_int, _BP)), ("restore", C.CFUNCTYPE(C.c_int, _BP)),
    ("destroy", C.CFUNCTYPE(None, _BP)), ("pos", C.c_size_t), ("max_seq", C.c_size_t),
    ("last_hidden", C.CFUNCTYPE(C.c_int, _BP, C.c_void_p))]


class HQError(RuntimeError):
    pass


_lib = None


def load(path=LIB_PATH):
    """Load libhq.so once; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise HQError(f"{path} is not built: run __graft_entry__.build() (make -C hilbert-pruned-8b_amd/csrc)")
    L = C.CDLL(path)
    vp, i, sz, u32 = C.c_void_p, C.c_int, C.c_size_t, C.c_uint32
    sig = {
        "hq_last_error": (C.c_char_p, []),
        "hq_device_init": (i, [i]),
        "hq_device_count": (i, [C.POINTER(i)]),
        "hq_device_name": (i, [i, C.c_char_p, sz, C.c_char_p, sz]),
        "hq_mat_upload": (i, [C.POINTER(WMat), i, C.POINTER(vp)]),
        "hq_mat_free": (None, [vp]),
        "hq_mat_shape": (i, [vp, C.POINTER(u32), C.POINTER(u32), C.POINTER(i)]),
        "hq_mat_device_bytes": (sz, [vp]),
        "hq_mat_download": (i, [vp, vp, sz]),
        "hq_dequant_f32": (i, [vp, u32, u32, vp, vp]),
        "hq_gemm": (i, [vp, vp, i, vp, i, i, vp]),
        "hq_gemv": (i, [vp, vp, vp, i, i, vp]),
        "hq_gather_dot": (i, [vp, vp, vp, i, i, vp, vp]),
        "hq_gather_dot_dev": (i, [vp, vp, vp, i, i, vp, vp]),
        "hq_matmul_host": (i, [vp, vp, sz, vp, C.c_bool]),
        "hq_malloc": (i, [C.POINTER(vp), sz]),
        "hq_free": (i, [vp]),
        "hq_memcpy_h2d": (i, [vp, vp, sz, vp]),
        "hq_memcpy_d2h": (i, [vp, vp, sz, vp]),
        "hq_memcpy_d2d": (i, [vp, vp, sz, vp]),
        "hq_memset": (i, [vp, i, sz, vp]),
        "hq_stream_create": (i, [C.POINTER(vp)]),
        "hq_stream_destroy": (i, [vp]),
        "hq_stream_synchronize": (i, [vp]),
        "hq_device_synchronize": (i, []),
        "hq_time_gemm": (i, [C.POINTER(vp), i, vp, i, vp, i, i, i, vp, C.POINTER(C.c_float)]),
        "hq_time_gemm_kernel": (i, [C.POINTER(vp), i, vp, i, vp, i, i, i, vp, C.POINTER(C.c_float)]),
        "hq_time_gather": (i, [C.POINTER(vp), i, vp, vp, i, i, i, vp, i, i, vp, C.POINTER(C.c_float)]),
        "hq_time_read": (i, [C.POINTER(vp), i, sz, i, i, i, vp, C.POINTER(C.c_float)]),
        "hq_gemm_tiles": (None, [i, i, i, C.POINTER(i), C.POINTER(i)]),
        "hq_gemm_kernel": (None, [i, i, i, i, C.c_char_p, i]),
        "hq_llama_forward": (i, [C.POINTER(Llama), vp, sz, vp, u32, vp]),
        "hq_embed_f32": (i, [vp, vp, i, vp, vp]),
        "hq_gemm_noalloc": (i, [vp, vp, i, vp, i, i, vp]),
        "hq_gemv_swiglu": (i, [vp, vp, vp, vp, vp]),
        "hq_mat_upload_pair": (i, [C.POINTER(WMat), C.POINTER(WMat), i, C.POINTER(vp)]),
        "hq_gemm_swiglu": (i, [vp, vp, i, vp, vp]),
        "hq_time_gemm_swiglu": (i, [C.POINTER(vp), i, vp, i, vp, i, i, vp, C.POINTER(C.c_float)]),
        "hq_gguf_open": (i, [C.c_char_p, C.POINTER(vp)]),
        "hq_gguf_close": (None, [vp]),
        "hq_gguf_n_tensors": (sz, [vp]),
        "hq_gguf_tensor_info": (i, [vp, sz, C.POINTER(C.c_char_p), C.POINTER(i), C.POINTER(u32),
                                    C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
        "hq_gguf_find": (i, [vp, C.c_char_p, C.POINTER(sz)]),
        "hq_gguf_get_uint": (i, [vp, C.c_char_p, C.POINTER(C.c_uint64)]),
        "hq_gguf_wmat": (i, [vp, C.c_char_p, u32, C.POINTER(WMat)]),
        "hip_backend_create": (C.POINTER(RefBackend), [C.POINTER(RefModel), sz, i, C.c_bool]),
        "hip_selftest": (i, [C.POINTER(RefModel), i, sz, i]),
        "hq_gemm_workspace_bytes": (i, [i, i, u32, u32, i, C.POINTER(sz), C.POINTER(sz), C.POINTER(sz),
                                        C.POINTER(i)]),
    }
    for name in EXPORTS + BACKEND_EXPORTS:
        fn = getattr(L, name)
        fn.restype, fn.argtypes = sig[name]
    _lib = L
    return L


def _check(rc):
    if rc != 0:
        raise HQError(load().hq_last_error().decode(errors="replace"))


def last_error():
    return load().hq_last_error().decode(errors="replace")


def row_bytes(gtype, cols):
    return cols // BLOCK_VALUES[gtype] * BLOCK_BYTES[gtype]


def _ptr(a):
    return C.c_void_p(a.ctypes.data)


class DevBuf:
    """A device allocation (hq_malloc) with numpy copy helpers."""

    def __init__(self, nbytes):
        load()
        p = C.c_void_p()
        _check(_lib.hq_malloc(C.byref(p), max(int(nbytes), 16)))
        self.ptr, self.nbytes = p.value, int(nbytes)

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a, stream=None, offset=0):
        """Copy array a into the buffer at byte `offset` (synchronous)."""
        a = np.ascontiguousarray(a)
        assert 0 <= offset and offset + a.nbytes <= self.nbytes
        _check(_lib.hq_memcpy_h2d(self.ptr + offset, _ptr(a), a.nbytes, stream))

    def download(self, shape, dtype, stream=None, offset=0):
        """A new array of `shape` from the buffer's bytes at `offset` (synchronous)."""
        out = np.empty(shape, dtype=dtype)
        assert 0 <= offset and offset + out.nbytes <= self.nbytes
        _check(_lib.hq_memcpy_d2h(_ptr(out), self.ptr + offset, out.nbytes, stream))
        return out

    def zero(self, stream=None):
        _check(_lib.hq_memset(self.ptr, 0, self.nbytes, stream))

    def free(self):
        if self.ptr:
            _check(_lib.hq_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Mat:
    """A weight matrix resident in HBM (hq_mat_upload)."""

    def __init__(self, blocks, gtype, rows, cols, perm_heads=0, device=0):
        load()
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        if blocks.nbytes != rows * row_bytes(gtype, cols):
            raise HQError(f"blocks hold {blocks.nbytes} bytes, expected {rows * row_bytes(gtype, cols)}")
        w = WMat(DT_GGML, rows, cols, blocks.ctypes.data, gtype, perm_heads)
        h = C.c_void_p()
        _check(_lib.hq_mat_upload(C.byref(w), device, C.byref(h)))
        self.h, self.gtype, self.rows, self.cols = h.value, gtype, rows, cols

    @property
    def device_bytes(self):
        return _lib.hq_mat_device_bytes(self.h)

    def download(self):
        out = np.empty((self.rows, row_bytes(self.gtype, self.cols)), dtype=np.uint8)
        _check(_lib.hq_mat_download(self.h, _ptr(out), out.nbytes))
        return out

    def free(self):
        if self.h:
            _lib.hq_mat_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def device_init(device=0):
    _check(load().hq_device_init(device))


def device_name(device=0):
    n, a = C.create_string_buffer(256), C.create_string_buffer(64)
    _check(load().hq_device_name(device, n, 256, a, 64))
    return n.value.decode(), a.value.decode()


def synchronize():
    _check(load().hq_device_synchronize())


def dequant(W, row0=0, nrows=None, stream=None):
    nrows = W.rows - row0 if nrows is None else nrows
    out = DevBuf(nrows * W.cols * 4)
    _check(_lib.hq_dequant_f32(W.h, row0, nrows, out.ptr, stream))
    return out.download((nrows, W.cols), np.float32)


def gemm(W, A, M, C_buf, c_f32=True, accumulate=False, stream=None):
    """Device-pointer GEMM: A, C_buf are DevBuf (or raw pointers)."""
    a = A.ptr if isinstance(A, DevBuf) else A
    c = C_buf.ptr if isinstance(C_buf, DevBuf) else C_buf
    _check(_lib.hq_gemm(W.h, a, M, c, int(c_f32), int(accumulate), stream))


def gemm_noalloc(W, A, M, C_buf, c_f32=True, accumulate=False, stream=None):
    """hq_gemm_noalloc: as gemm(), with the GEMM workspace in the library's preallocated scratch."""
    a = A.ptr if isinstance(A, DevBuf) else A
    c = C_buf.ptr if isinstance(C_buf, DevBuf) else C_buf
    _check(_lib.hq_gemm_noalloc(W.h, a, M, c, int(c_f32), int(accumulate), stream))


def gemm_workspace_bytes(gtype, M, N, K, n_cu=256):
    """(partial bytes, counter bytes, sum bytes, fits hq_gemm_noalloc's scratch) of one M-row launch."""
    pb, cb, sb, fits = C.c_size_t(), C.c_size_t(), C.c_size_t(), C.c_int()
    _check(load().hq_gemm_workspace_bytes(gtype, M, N, K, n_cu, C.byref(pb), C.byref(cb), C.byref(sb), C.byref(fits)))
    return pb.value, cb.value, sb.value, bool(fits.value)


class PairMat:
    """hq_mat_upload_pair: gate and up of one FFN as one interleaved resident matrix."""

    def __init__(self, gate_blocks, up_blocks, gtype, rows, cols, device=0):
        load()
        g = np.ascontiguousarray(gate_blocks, dtype=np.uint8)
        u = np.ascontiguousarray(up_blocks, dtype=np.uint8)
        wg = WMat(DT_GGML, rows, cols, g.ctypes.data, gtype, 0)
        wu = WMat(DT_GGML, rows, cols, u.ctypes.data, gtype, 0)
        h = C.c_void_p()
        _check(_lib.hq_mat_upload_pair(C.byref(wg), C.byref(wu), device, C.byref(h)))
        self.h, self.gtype, self.rows, self.cols = h.value, gtype, rows, cols

    def free(self):
        if self.h:
            _lib.hq_mat_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def gemm_swiglu_np(pair, a_f16_bits):
    """hq_gemm_swiglu on numpy fp16 bits [M, K]: fp16 bits [M, rows] of silu(A gate^T) * (A up^T)."""
    a = np.ascontiguousarray(a_f16_bits, dtype=np.uint16)
    M = a.shape[0]
    dA, dO = DevBuf.from_array(a), DevBuf(M * pair.rows * 2)
    _check(_lib.hq_gemm_swiglu(pair.h, dA.ptr, M, dO.ptr, None))
    synchronize()
    out = dO.download((M, pair.rows), np.uint16)
    dA.free(), dO.free()
    return out


def time_gemm_swiglu(pairs, A, M, out, iters, reps, stream):
    arr = (C.c_void_p * len(pairs))(*[m.h for m in pairs])
    ms = C.c_float()
    _check(_lib.hq_time_gemm_swiglu(arr, len(pairs), A.ptr, M, out.ptr, iters, reps, stream.ptr, C.byref(ms)))
    return ms.value


def gemv_swiglu_np(gate, up, a_f16_bits):
    """hq_gemv_swiglu on a numpy fp16 row [cols]: fp16 bits [rows] of silu(gate . a) * (up . a)."""
    dA = DevBuf.from_array(np.ascontiguousarray(a_f16_bits, dtype=np.uint16))
    dO = DevBuf(gate.rows * 2)
    _check(_lib.hq_gemv_swiglu(gate.h, up.h, dA.ptr, dO.ptr, None))
    synchronize()
    out = dO.download((gate.rows,), np.uint16)
    dA.free(), dO.free()
    return out


def gemm_np(W, a_f16_bits, c_f32=True, c_init=None):
    """Convenience: numpy fp16 bits [M, K] in, numpy fp32 / fp16-bits [M, N] out (accumulate into c_init)."""
    a = np.ascontiguousarray(a_f16_bits, dtype=np.uint16)
    M = a.shape[0]
    dA = DevBuf.from_array(a)
    esize = 4 if c_f32 else 2
    dC = DevBuf(M * W.rows * esize)
    if c_init is not None:
        dC.upload(np.ascontiguousarray(c_init))
    gemm(W, dA, M, dC, c_f32, c_init is not None)
    synchronize()
    out = dC.download((M, W.rows), np.float32 if c_f32 else np.uint16)
    dA.free(), dC.free()
    return out


def gather_dot_np(W, h_f16_bits, ids, device_ids=False):
    h = np.ascontiguousarray(h_f16_bits, dtype=np.uint16)
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    B, k = ids.shape
    dH = DevBuf.from_array(h)
    dO = DevBuf(B * k * 4)
    if device_ids:
        dI = DevBuf.from_array(ids)
        _check(_lib.hq_gather_dot_dev(W.h, dH.ptr, dI.ptr, B, k, dO.ptr, None))
    else:
        _check(_lib.hq_gather_dot(W.h, dH.ptr, _ptr(ids), B, k, dO.ptr, None))
    synchronize()
    return dO.download((B, k), np.float32)


def matmul_host(W, x, y=None, accumulate=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    if y is None:
        y = np.zeros((T, W.rows), dtype=np.float32)
    _check(_lib.hq_matmul_host(W.h, _ptr(x), T, _ptr(y), bool(accumulate)))
    return y


def embed(W, ids):
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    out = DevBuf(len(ids) * W.cols * 4)
    _check(_lib.hq_embed_f32(W.h, _ptr(ids), len(ids), out.ptr, None))
    synchronize()
    return out.download((len(ids), W.cols), np.float32)


def gemm_tiles(gtype, M, N):
    r, c = C.c_int(), C.c_int()
    load().hq_gemm_tiles(gtype, M, N, C.byref(r), C.byref(c))
    return r.value, c.value


def gemm_kernel(gtype, M, N, K):
    """Name of the kernel that does the work of an M x N x K hq_gemm (as rocprofv3 lists it)."""
    buf = C.create_string_buffer(64)
    load().hq_gemm_kernel(gtype, M, N, K, buf, 64)
    return buf.value.decode()


class Stream:
    def __init__(self):
        p = C.c_void_p()
        _check(load().hq_stream_create(C.byref(p)))
        self.ptr = p.value

    def sync(self):
        _check(_lib.hq_stream_synchronize(self.ptr))

    def destroy(self):
        if self.ptr:
            _check(_lib.hq_stream_destroy(self.ptr))
            self.ptr = None


def time_read(bufs, nbytes, grid, iters, reps, stream):
    """hq_time_read: ms per launch of a pure streaming read of nbytes from bufs[i % len(bufs)]."""
    arr = (C.c_void_p * len(bufs))(*[b.ptr for b in bufs])
    ms = C.c_float()
    _check(_lib.hq_time_read(arr, len(bufs), nbytes, grid, iters, reps, stream.ptr, C.byref(ms)))
    return ms.value


def time_gemm(mats, A, M, C_buf, c_f32, iters, reps, stream):
    arr = (C.c_void_p * len(mats))(*[m.h for m in mats])
    ms = C.c_float()
    _check(_lib.hq_time_gemm(arr, len(mats), A.ptr, M, C_buf.ptr, int(c_f32), iters, reps, stream.ptr, C.byref(ms)))
    return ms.value


def time_gemm_kernel(mats, A, M, C_buf, c_f32, iters, reps, stream):
    """Average duration (ms) of the GEMM's main kernel alone (see hq_time_gemm_kernel)."""
    arr = (C.c_void_p * len(mats))(*[m.h for m in mats])
    ms = C.c_float()
    _check(_lib.hq_time_gemm_kernel(arr, len(mats), A.ptr, M, C_buf.ptr, int(c_f32), iters, reps, stream.ptr,
                                    C.byref(ms)))
    return ms.value


def time_gather(mats, H, ids_dev, n_sets, B, k, out, iters, reps, stream):
    arr = (C.c_void_p * len(mats))(*[m.h for m in mats])
    ms = C.c_float()
    _check(_lib.hq_time_gather(arr, len(mats), H.ptr, ids_dev.ptr, n_sets, B, k, out.ptr, iters, reps, stream.ptr,
                               C.byref(ms)))
    return ms.value


class LlamaModel:
    """Config-1 model resident on the GPU, from a synth.tiny_llama()-style dict (llama.cpp storage
    order for q/k rows; perm_heads un-permutes them at upload, as the reference's model.c:382)."""

    def __init__(self, model, device=0):
        c = model["cfg"]
        self.cfg = c
        H, I, V = c["hidden"], c["intermediate"], c["vocab"]
        qw, kvw = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
        self.mats = []

        def up(blocks, rows, cols, perm=0):
            m = Mat(blocks, Q8_0, rows, cols, perm, device)
            self.mats.append(m)
            return m.h

        self.norms = [np.ascontiguousarray(model["final_norm"], np.float32)]
        self.layers = (LlamaLayer * c["n_layers"])()
        shapes = {"q": (qw, H, c["n_heads"]), "k": (kvw, H, c["n_kv_heads"]), "v": (kvw, H, 0), "o": (H, qw, 0),
                  "gate": (I, H, 0), "up": (I, H, 0), "down": (H, I, 0)}
        for li, L in enumerate(model["layers"]):
            for name, (r, k, perm) in shapes.items():
                setattr(self.layers[li], name, up(L[name], r, k, perm))
            n_in = np.ascontiguousarray(L["in_norm"], np.float32)
            n_post = np.ascontiguousarray(L["post_norm"], np.float32)
            self.norms += [n_in, n_post]
            self.layers[li].in_norm = n_in.ctypes.data
            self.layers[li].post_norm = n_post.ctypes.data
        self.st = Llama(H, c["n_layers"], I, V, c["n_heads"], c["n_kv_heads"], c["head_dim"], c["rot_dim"], c["eps"],
                        c["rope_theta"], up(model["embed"], V, H), up(model["lm_head"], V, H),
                        self.norms[0].ctypes.data, C.cast(self.layers, C.c_void_p).value)
        if model.get("rope_inv_freq") is not None:
            self.inv_freq = np.ascontiguousarray(model["rope_inv_freq"], np.float32)
            assert self.inv_freq.shape == (c["rot_dim"] // 2,)
            self.st.rope_inv_freq = self.inv_freq.ctypes.data

    def forward(self, tokens, ids):
        tokens = np.ascontiguousarray(tokens, np.uint32)
        ids = np.ascontiguousarray(ids, np.uint32)
        logits = np.empty(len(ids), np.float32)
        _check(_lib.hq_llama_forward(C.byref(self.st), _ptr(tokens), len(tokens), _ptr(ids), len(ids),
                                     _ptr(logits)))
        return logits

    def free(self):
        for m in self.mats:
            m.free()
        self.mats = []


def rope_inv_freq(theta, rot_dim):
    """The reference's RoPE table without Llama 3.1 scaling (src/model.c:453-454): float32
    1 / powf(theta, 2k / rot_dim), computed with the C library's powf."""
    libm = C.CDLL("libm.so.6")
    libm.powf.restype, libm.powf.argtypes = C.c_float, [C.c_float, C.c_float]
    out = np.empty(rot_dim // 2, np.float32)
    for k in range(rot_dim // 2):
        e = np.float32(np.float32(2 * k) / np.float32(rot_dim))
        out[k] = np.float32(1.0) / np.float32(libm.powf(np.float32(theta), e))
    return out


class RefModelView:
    """A reference model_t (layout mirror RefModel) over a synth.tiny_llama()-style dict of Q8_0 /
    Q4_K block arrays, as the reference's model_load would fill it for a GGUF Llama model: q/k in
    llama.cpp storage order with perm_heads, every layer LAYER_FULL, RMSNorm offset 0. Keeps the
    arrays alive while the view exists. model["types"] may give other ggml types for the layer
    matrices by name (e.g. {"gate": Q4_K, "up": Q6_K}, as Q4_K_M files mix them)."""

    def __init__(self, model, gtype=Q8_0):
        c = model["cfg"]
        self.keep = []
        H, I, V = c["hidden"], c["intermediate"], c["vocab"]
        qw, kvw = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]

        types = model.get("types", {})

        def wm(blocks, rows, cols, perm=0, name=None):
            blocks = np.ascontiguousarray(blocks, np.uint8)
            self.keep.append(blocks)
            return WMat(DT_GGML, rows, cols, blocks.ctypes.data, types.get(name, gtype), perm)

        def vec(v):
            v = np.ascontiguousarray(v, np.float32)
            self.keep.append(v)
            return v.ctypes.data

        cfg = RefConfig()
        for k in ("hidden", "n_layers", "intermediate", "vocab", "n_heads", "n_kv_heads", "head_dim", "rot_dim"):
            setattr(cfg, k, c[k])
        cfg.arch, cfg.eps, cfg.rope_theta, cfg.norm_offset = 1, c["eps"], c["rope_theta"], 0.0
        cfg.n_full, cfg.n_linear = c["n_layers"], 0
        for li in range(c["n_layers"]):
            cfg.layer_type[li] = 1
        self.layers = (RefLayer * c["n_layers"])()
        for li, L in enumerate(model["layers"]):
            d = self.layers[li]
            d.type, d.slot = 1, li
            d.in_norm, d.post_norm = vec(L["in_norm"]), vec(L["post_norm"])
            d.q = wm(L["q"], qw, H, c["n_heads"])
            d.k = wm(L["k"], kvw, H, c["n_kv_heads"])
            d.v, d.o = wm(L["v"], kvw, H), wm(L["o"], H, qw)
            d.gate, d.up = wm(L["gate"], I, H, name="gate"), wm(L["up"], I, H, name="up")
            d.down = wm(L["down"], H, I, name="down")
        self.m = RefModel()
        self.m.cfg = cfg
        self.m.embed, self.m.lm_head = wm(model["embed"], V, H), wm(model["lm_head"], V, H)
        self.m.final_norm = vec(model["final_norm"])
        self.m.layers = C.cast(self.layers, C.c_void_p).value
        self.m.rope_inv_freq = vec(rope_inv_freq(c["rope_theta"], c["rot_dim"]))


class HipBackend:
    """hip_backend_create's backend_t, driven through its vtable exactly as the reference engine does."""

    def __init__(self, view, max_seq, device=0, keep_quantized=True):
        self.view = view
        p = load().hip_backend_create(C.byref(view.m), max_seq, device, keep_quantized)
        if not p:
            raise HQError(last_error())
        self.p = p

    @property
    def pos(self):
        return self.p.contents.pos

    def _call(self, rc):
        if rc != 0:
            raise HQError(last_error())

    def reset(self):
        self._call(self.p.contents.reset(self.p))

    def forward(self, tokens, ids=None):
        tokens = np.ascontiguousarray(tokens, np.uint32)
        n_ids = 0 if ids is None else len(ids)
        ids = None if ids is None else np.ascontiguousarray(ids, np.uint32)
        out = np.empty(n_ids, np.float32)
        self._call(self.p.contents.forward(self.p, tokens.ctypes.data, len(tokens),
                                           ids.ctypes.data if n_ids else None, n_ids,
                                           out.ctypes.data if n_ids else None))
        return out

    def snapshot(self):
        self._call(self.p.contents.snapshot(self.p))

    def restore(self):
        self._call(self.p.contents.restore(self.p))

    def last_hidden(self):
        out = np.empty(self.view.m.cfg.hidden, np.float32)
        self._call(self.p.contents.last_hidden(self.p, out.ctypes.data))
        return out

    def destroy(self):
        if self.p:
            self.p.contents.destroy(self.p)
            self.p = None


def hip_selftest(view, device=0, n_tokens=64, verbose=1):
    return load().hip_selftest(C.byref(view.m), device, n_tokens, verbose)


class Gguf:
    """hq_gguf_open: a read-only mapping of a GGUF file and its tensor table (include/hq_gguf.h)."""

    def __init__(self, path):
        h = C.c_void_p()
        _check(load().hq_gguf_open(str(path).encode(), C.byref(h)))
        self.h = h.value

    def tensors(self):
        out = []
        for i in range(_lib.hq_gguf_n_tensors(self.h)):
            name, t, nd = C.c_char_p(), C.c_int(), C.c_uint32()
            ne, off = (C.c_uint64 * 4)(), C.c_uint64()
            _check(_lib.hq_gguf_tensor_info(self.h, i, C.byref(name), C.byref(t), C.byref(nd), ne, C.byref(off)))
            out.append(dict(name=name.value.decode(), type=t.value, n_dims=nd.value, ne=tuple(ne), offset=off.value))
        return out

    def get_uint(self, key):
        v = C.c_uint64()
        _check(_lib.hq_gguf_get_uint(self.h, key.encode(), C.byref(v)))
        return v.value

    def wmat(self, name, perm_heads=0):
        w = WMat()
        _check(_lib.hq_gguf_wmat(self.h, name.encode(), perm_heads, C.byref(w)))
        return w

    def view_bytes(self, name):
        """The bytes of a quantized matrix as the mapping holds them (a copy)."""
        w = self.wmat(name)
        n = w.rows * row_bytes(w.ggml_type, w.cols)
        return np.ctypeslib.as_array((C.c_uint8 * n).from_address(w.data)).reshape(w.rows, -1).copy()

    def upload(self, name, perm_heads=0, device=0):
        """hq_mat_upload of the named matrix straight from the mapping."""
        w = self.wmat(name, perm_heads)
        m = Mat.__new__(Mat)
        h = C.c_void_p()
        _check(_lib.hq_mat_upload(C.byref(w), device, C.byref(h)))
        m.h, m.gtype, m.rows, m.cols = h.value, w.ggml_type, w.rows, w.cols
        return m

    def close(self):
        if self.h:
            _lib.hq_gguf_close(self.h)
            self.h = None
