"""CPU checks of the C ABI: libhq.so is built, loads, and exports every function the headers
declare; host-side argument validation and tile selection work without a GPU."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import hq
import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", f) for f in sorted(os.listdir(os.path.join(ROOT, "include"))) if f.endswith(".h")]


def declared_functions():
    names = set()
    for path in HEADERS:
        text = open(path).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b((?:hq|hip)_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_built_and_exports_every_declared_function():
    assert os.path.exists(hq.LIB_PATH), "libhq.so not built: run __graft_entry__.build()"
    lib = C.CDLL(hq.LIB_PATH)
    declared = declared_functions()
    assert len(declared) >= 25
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing
    assert declared == set(hq.EXPORTS + hq.BACKEND_EXPORTS), declared ^ set(hq.EXPORTS + hq.BACKEND_EXPORTS)


def test_binding_signatures_load():
    lib = hq.load()
    for name in hq.EXPORTS:
        assert getattr(lib, name).argtypes is not None


def test_wmat_layout_matches_reference_struct():
    # reference wmat_t: {dtype_t dtype; uint32_t rows, cols; const void *data; int ggml_type; uint32_t perm_heads}
    assert C.sizeof(hq.WMat) == 32
    assert [hq.WMat.__dict__[f].offset for f in ("dtype", "rows", "cols", "data", "ggml_type", "perm_heads")] == \
        [0, 4, 8, 16, 24, 28]


@pytest.mark.parametrize("dtype,gtype,rows,cols,perm,msg", [
    (0, 8, 4, 64, 0, "not a GGUF block type"),
    (3, 2, 4, 64, 0, "not supported"),
    (3, 8, 4, 48, 0, "whole number"),
    (3, 12, 4, 512 + 32, 0, "whole number"),
    (3, 8, 0, 64, 0, "whole number"),
    (3, 8, 6, 64, 4, "heads of even size"),
])
def test_upload_rejects_bad_descriptors_before_touching_a_device(dtype, gtype, rows, cols, perm, msg):
    lib = hq.load()
    buf = np.zeros(1 << 16, np.uint8)
    w = hq.WMat(dtype, rows, cols, buf.ctypes.data, gtype, perm)
    h = C.c_void_p()
    assert lib.hq_mat_upload(C.byref(w), 0, C.byref(h)) == -1
    assert msg in hq.last_error()
    assert h.value is None


def test_upload_rejects_matrices_of_4gib_or_more():
    """The kernels address one matrix through 32-bit buffer ranges: 3,000,000 Q4_K rows of 2560
    values (4.32e9 bytes) are refused before any device is touched."""
    lib = hq.load()
    buf = np.zeros(16, np.uint8)
    w = hq.WMat(3, 3_000_000, 2560, buf.ctypes.data, synth.Q4_K, 0)
    h = C.c_void_p()
    assert lib.hq_mat_upload(C.byref(w), 0, C.byref(h)) == -1
    assert "limited to 4 GiB" in hq.last_error()
    assert h.value is None


def test_gemm_workspace_bytes():
    """Workspace of one GEMM launch (computed on the host, no device): the K-split tile kernel keeps
    one fp32 tile per (tile, part) plus a counter per tile; the Stream-K kernel two 128 x 256 fp32
    tiles per CU; the large-M tile kernel only the activation sub-block sums; hq_gemm_noalloc's
    96 MiB scratch holds the BASELINE shapes and refuses larger."""
    # (M = 512, N = 2560, K = 9728: the 128 x 160 register-decode kernel, 4 x 16 tiles with K split
    # over 4 workgroups, no sub-block sums)
    pb, cb, sb, fits = hq.gemm_workspace_bytes(synth.Q4_K, 512, 2560, 9728)
    assert (pb, cb, sb, fits) == (64 * 4 * 128 * 160 * 4, 64 * 4, 0, True)
    # (M = 4095, N = 32: the Stream-K kernel, 4096 / 128 x 1 tiles; M = 4096, N = 2560, K = 9728: the
    # register-decode kernel as launches of one round each, no workspace)
    pb, cb, sb, fits = hq.gemm_workspace_bytes(synth.Q4_K, 4095, 32, 2560)
    assert (pb, cb, fits) == (2 * 256 * 128 * 256 * 4, 32 * 4, True)
    assert hq.gemm_workspace_bytes(synth.Q4_K, 4096, 2560, 9728) == (0, 0, 0, True)
    assert hq.gemm_workspace_bytes(synth.Q4_K, 4096, 9728, 2560) == (0, 0, 4096 * 10 * 32, True)
    # the 128 x 192 loader-wave kernel (M = 512, N = 9728): one round of tiles; its loader waves form
    # the sub-block sums in LDS, so no workspace at all
    assert hq.gemm_workspace_bytes(synth.Q4_K, 512, 9728, 2560) == (0, 0, 0, True)
    assert hq.gemm_workspace_bytes(synth.Q8_0, 512, 9728, 2560) == (0, 0, 0, True)
    assert hq.gemm_workspace_bytes(synth.Q4_K, 16384, 2560, 9216)[3]
    assert not hq.gemm_workspace_bytes(synth.Q4_K, 131072, 256, 9216)[3]  # 151 MB of sub-block sums
    # the k-quant tile kernel (Q6_K, M = 512, N = 2560, K = 9728): 4 x 16 tiles of 128 x 160 with K
    # split over 4 workgroups; the Q5_K tile kernel (M = 512, N = 9728): sub-block sums only; the Q4_K
    # tile kernel at M = 128 (one row tile): 102 tiles of 128 x 96 with K split over 2 workgroups, no
    # sums (it forms them itself); the Q8_0 tile kernel at M = 96: the same split
    assert hq.gemm_workspace_bytes(synth.Q6_K, 512, 2560, 9728) == (64 * 4 * 128 * 160 * 4, 64 * 4, 0, True)
    assert hq.gemm_workspace_bytes(synth.Q5_K, 512, 9728, 2560) == (0, 0, 512 * 10 * 32, True)
    assert hq.gemm_workspace_bytes(synth.Q4_K, 128, 9728, 2560) == (102 * 2 * 128 * 96 * 4, 102 * 4, 0, True)
    assert hq.gemm_workspace_bytes(synth.Q8_0, 96, 9728, 2560) == (102 * 2 * 128 * 96 * 4, 102 * 4, 0, True)
    with pytest.raises(hq.HQError, match="type 9"):
        hq.gemm_workspace_bytes(9, 512, 256, 256)
    with pytest.raises(hq.HQError, match="M = 1"):
        hq.gemm_workspace_bytes(synth.Q4_K, 1, 256, 256)


def test_gemm_kernel_names():
    """hq_gemm_kernel names the kernel the launch plan picks (the names rocprofv3 lists)."""
    cases = {(synth.Q4_K, 512, 9728, 2560): "k_gemm_q4_k_wr160", (synth.Q4_K, 256, 9728, 2560): "k_gemm_q4_k_wr160",
             (synth.Q4_K, 384, 13000, 2560): "k_gemm_q4_k_wr<3>", (synth.Q8_0, 512, 9728, 2560): "k_gemm_q8_0_wr",
             (synth.Q8_0, 2048, 9728, 2560): "k_gemm_q8_0_wr", (synth.Q8_0, 128, 9728, 2560): "k_gemm_q8_0_ws<3>",
             (synth.Q8_0, 65, 9728, 2560): "k_gemm_q8_0_ws<3>", (synth.Q8_0, 128, 4096, 4096): "k_gemm_q8_0_ws<2>",
             (synth.Q6_K, 96, 9728, 2560): "k_gemm_kq_ws<14, 3>", (synth.Q4_K, 128, 9728, 2560): "k_gemm_q4_k_ws<3>",
             (synth.Q4_K, 200, 9728, 2560): "k_gemm_q4_k_wr_ks160", (synth.Q5_K, 96, 9728, 2560): "k_gemm_q5_k_ws<3>",
             (synth.Q4_K, 4096, 9728, 2560): "k_gemm_q4_k_bt", (synth.Q4_K, 16384, 2560, 9216): "k_gemm_q4_k_bt",
             (synth.Q4_K, 16384, 1024, 2560): "k_gemm_q4_k_bt", (synth.Q4_K, 2048, 9728, 2560): "k_gemm_q4_k_wr160",
             (synth.Q4_K, 64, 9728, 2560): "k_gemm_q4_k_rb<1, 4, 3, 2>",
             (synth.Q4_K, 64, 2560, 9728): "k_gemm_q4_k_rb<1, 4, 3, 2>", (synth.Q4_K, 64, 1024, 2560): "k_gemm_q4_k<4, 2>", (synth.Q4_K, 32, 9728, 2560): "k_gemm_q4_k<2, 2>",
             (synth.Q4_K, 64, 9728, 2304): "k_gemm_q4_k<4, 2>",
             (synth.Q4_K, 512, 2560, 9728): "k_gemm_q4_k_wr_ks160",
             (synth.Q4_K, 100, 10996, 5120): "k_gemm_q4_k_wr_ks<3>", (synth.Q4_K, 256, 2560, 9728): "k_gemm_q4_k_ws<3>",
             (synth.Q4_K, 512, 1024, 2560): "k_gemm_q4_k_w<8>", (synth.Q4_K, 4096, 2560, 9728): "k_gemm_q4_k_wr160",
             (synth.Q4_K, 512, 19456, 2560): "k_gemm_q4_k_wr160", (synth.Q4_K, 1536, 9728, 2560): "k_gemm_q4_k_bt",
             (synth.Q8_0, 512, 2560, 9728): "k_gemm_q8_0_ws<5>", (synth.Q8_0, 256, 2560, 9728): "k_gemm_q8_0_ws<3>",
             (synth.Q8_0, 16, 9728, 2560): "k_gemm_q8_0_rb<1, 3, 2>", (synth.Q8_0, 64, 9728, 2560): "k_gemm_q8_0_rb<4, 3, 2>",
             (synth.Q8_0, 16, 2560, 9728): "k_gemm_q8_0_rb<1, 3, 2>", (synth.Q8_0, 16, 1024, 1024): "k_gemm_q8_0<1, 2>", (synth.Q4_K, 1, 9728, 2560): "k_gemv_q4_k_r<4>",
             (synth.Q4_K, 1, 2560, 9728): "k_gemv_q4_k_s<4>", (synth.Q4_K, 1, 100, 512): "k_gemv_q4_k_s<1>",
             (synth.Q4_K, 1, 9728, 256): "k_gemv_q4_k_s<16>", (synth.Q8_0, 1, 9728, 2560): "k_gemv_q8_0<2>",
             (synth.Q8_0, 1, 100, 512): "k_gemv_q8_0<1>",
             # k-quant GEMVs: rows per wave, 2 at N >= 8192; the activation vector in LDS but for Q5_K
             (synth.Q6_K, 1, 9728, 2560): "k_gemv_sb<14, 2, false, true>", (synth.Q3_K, 1, 2560, 9728): "k_gemv_sb<11, 1, false, true>",
             (synth.Q5_K, 1, 100, 2048): "k_gemv_sb<13, 1, false, false>", (synth.Q2_K, 1, 100, 20480): "k_gemv_sb<10, 1, false, true>",
             (synth.Q2_K, 1, 100, 33024): "k_gemv_sb<10, 1, false, false>",
             # Q6_K / Q3_K / Q2_K above M = 64: the LDS-decode tile kernel (template: the ggml type, tile width / 32)
             (synth.Q6_K, 512, 9728, 2560): "k_gemm_kq_ws<14, 5>", (synth.Q3_K, 128, 9728, 2560): "k_gemm_kq_ws<11, 2>",
             (synth.Q2_K, 512, 9728, 2560): "k_gemm_kq_ws<10, 5>",
             (synth.Q6_K, 64, 9728, 2560): "k_gemm_q6_k<4, 2>", (synth.Q5_K, 64, 9728, 2560): "k_gemm_kq<13, 4, 2>",
             # Q5_K above M = 64: the Q4_K LDS-decode tile kernel's Q5_K instance
             (synth.Q5_K, 512, 9728, 2560): "k_gemm_q5_k_ws<5>", (synth.Q5_K, 300, 9728, 2560): "k_gemm_q5_k_ws<4>",
             # Q4_K with N <= 32 at M >= 4096: the skinny kernel (template: 16-column blocks)
             (synth.Q4_K, 16384, 32, 2560): "k_gemm_q4_k_nn<2>", (synth.Q4_K, 4096, 9, 256): "k_gemm_q4_k_nn<1>",
             (synth.Q4_K, 4095, 32, 2560): "k_gemm_q4_k_w<8>",
             # special-scale cases: the narrow kernel at M = 16, the mid-M kernel with a 6-way K split
             (synth.Q4_K, 16, 9728, 2560): "k_gemm_q4_k<2, 2>", (synth.Q4_K, 48, 9728, 2560): "k_gemm_q4_k_rb<1, 4, 3, 2>",
             (synth.Q4_K, 350, 9728, 512): "k_gemm_q4_k_wr160"}
    for (gtype, M, N, K), name in cases.items():
        assert hq.gemm_kernel(gtype, M, N, K) == name, (gtype, M, N, K)


def test_gemm_tile_selection():
    # every M from 1 to 4096 gets a tile; M = 1 is the GEMV
    for gtype in (synth.Q8_0, synth.Q4_K):
        assert hq.gemm_tiles(gtype, 1, 9728) == (1, 16)
        for M in (2, 16, 17, 33, 64, 65, 512, 4096):
            r, c = hq.gemm_tiles(gtype, M, 9728)
            assert r in (16, 32, 64, 128, 256)
            assert r >= min(M, 128)
            if gtype == synth.Q4_K and M > 64:
                # Q4_K above M = 64: full-K tiles of 128 x 32NB when they fill the CUs (128 x 192 or
                # 128 x 160 with loader waves when one round of them does, or launches of one round
                # each do), 256 x 256 full-K tiles at large M when their rounds fill the CUs, else the
                # 8-wave Stream-K kernel (128 x 256)
                assert (r, c) in ((128, 256), (256, 256), (128, 192)) or (r == 128 and c in (64, 96, 128, 160))
            elif gtype == synth.Q8_0 and M > 64:
                # Q8_0 above M = 64: full-K tiles of 128 x 32NB when they fill >= 50 % of the CU
                # time (any number of rounds; 128 x 192 with loader waves when one round of them fills
                # >= 70 % of the CUs), else the narrow Stream-K kernel
                assert c == 128 or (r == 128 and c in (64, 96, 128, 160, 192))
            elif gtype == synth.Q8_0:
                # Q8_0 up to M = 64 at N >= 8192: the mid-M kernel's full-K tiles of 16/32/64 x 64
                assert (r, c) == (16 if M <= 16 else 32 if M <= 32 else 64, 64)
            else:
                assert c == 128
    # Stream-K balances any tile count over the CUs (narrow Q8_0 / Q4_K, few Q4_K tiles)
    assert hq.gemm_tiles(synth.Q8_0, 65, 9728) == (128, 128)
    assert hq.gemm_tiles(synth.Q8_0, 128, 9728) == (128, 64)
    assert hq.gemm_tiles(synth.Q4_K, 2, 9728) == (32, 128)
    # Q8_0 full-K tiles of 128 x 192 (loader waves, register decode): 4 x 51 in one launch at M = 512,
    # 16 x 51 as four launches of at most one round at M = 2048; 128 x 96 at M = 256 (102 of the
    # larger tiles would fill only 40 % of the CUs)
    assert hq.gemm_tiles(synth.Q8_0, 512, 9728) == (128, 192)
    assert hq.gemm_tiles(synth.Q8_0, 2048, 9728) == (128, 192)
    assert hq.gemm_tiles(synth.Q8_0, 256, 9728) == (128, 96)
    assert hq.gemm_tiles(synth.Q4_K, 65, 9728) == (128, 256)
    # full-K tiles: 4 x 61 tiles of 128 x 160 on 256 CUs; more tiles than CUs: at large M the 256 x 256
    # tiles when their rounds fill >= 3/4 of the CU time (M = 4096: 608 tiles in 3 rounds), else the
    # 128 x 160 tiles as launches of one round each (M = 2048: 16 x 61 in 4 launches; the 256 x 256
    # tiles would make 304 tiles in 2 rounds, 59 %), Stream-K where those fill < 70 % of the CU time
    assert hq.gemm_tiles(synth.Q4_K, 512, 9728) == (128, 160)  # k_gemm_q4_k_wr160: 244 tiles in one round
    assert hq.gemm_tiles(synth.Q4_K, 2048, 9728) == (128, 160)
    assert hq.gemm_tiles(synth.Q4_K, 512, 1024) == (128, 256)
    assert hq.gemm_tiles(synth.Q4_K, 4096, 9728) == (256, 256)


def test_synth_is_deterministic():
    a = synth.q4_k_blocks(synth.Rng(9), 4, 512)
    b = synth.q4_k_blocks(synth.Rng(9), 4, 512)
    assert np.array_equal(a, b)
    x = synth.activations_f16(synth.Rng(3), 2, 64)
    assert x.dtype == np.uint16 and np.isfinite(x.view(np.float16)).all()
    # fp16 scales |N(0,1)| * 2e-4 are non-negative and finite
    q = synth.q8_0_blocks(synth.Rng(4), 8, 256)
    d = q.reshape(-1, 34)[:, :2].copy().view(np.float16)
    assert (d >= 0).all() and np.isfinite(d).all()


# ------------------------------------------------------------------ HIP backend (include/hq_backend.h)
REF_SRC = "/root/reference/cleanroom-transformer/src"
LAYOUT_FIELDS = {
    ("config_t", "hq_ref_config_t"): ["hidden", "n_layers", "intermediate", "vocab", "n_heads", "n_kv_heads",
                                       "head_dim", "rot_dim", "lin_k_heads", "lin_v_heads", "lin_k_dim", "lin_v_dim",
                                       "conv_k", "arch", "eps", "rope_theta", "norm_offset", "attn_gate", "qk_norm",
                                       "tied", "rope_llama3", "rope_factor", "rope_low_freq", "rope_high_freq",
                                       "rope_orig_ctx", "layer_type", "n_full", "n_linear"],
    ("layer_t", "hq_ref_layer_t"): ["type", "slot", "in_norm", "post_norm", "gate", "up", "down", "q", "k", "v", "o",
                                     "q_norm", "k_norm", "qkv", "z", "b", "a", "out", "conv_w", "A_log", "dt_bias",
                                     "lin_norm"],
    ("st_set_t", "hq_ref_st_set_t"): ["files", "n_files", "tensors", "n_tensors"],
    ("model_t", "hq_ref_model_t"): ["cfg", "st", "embed", "lm_head", "final_norm", "layers", "rope_inv_freq", "gguf",
                                     "source"],
    ("backend_t", "hq_ref_backend_t"): ["name", "reset", "forward", "snapshot", "restore", "destroy", "pos", "max_seq",
                                         "last_hidden"],
    ("wmat_t", "hq_wmat_t"): ["dtype", "rows", "cols", "data", "ggml_type", "perm_heads"],
}


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_SRC, "transformer.h")), reason="needs /root/reference")
def test_backend_structs_match_reference_header(tmp_path):
    """Every mirror struct of include/hq_backend.h has the size and field offsets of the reference's
    own declaration (compiled together, checked with _Static_assert)."""
    import shutil
    import subprocess
    if not shutil.which("gcc"):
        pytest.skip("gcc not found")
    lines = ['#include <stddef.h>', '#include "transformer.h"', '#include "hq_backend.h"']
    for (ref, mine), fields in LAYOUT_FIELDS.items():
        lines.append(f'_Static_assert(sizeof({ref}) == sizeof({mine}), "size {mine}");')
        for f in fields:
            lines.append(f'_Static_assert(offsetof({ref}, {f}) == offsetof({mine}, {f}), "{mine}.{f}");')
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    r = subprocess.run(["gcc", "-std=c11", "-fsyntax-only", f"-I{REF_SRC}", f"-I{os.path.join(ROOT, 'include')}",
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]


def test_backend_ctypes_mirrors_match_header(tmp_path):
    """hq.py's ctypes mirrors (used by the tests) have the header's offsets."""
    import shutil
    import subprocess
    if not shutil.which("gcc"):
        pytest.skip("gcc not found")
    py = {"hq_ref_config_t": hq.RefConfig, "hq_ref_layer_t": hq.RefLayer, "hq_ref_st_set_t": hq.RefStSet,
          "hq_ref_model_t": hq.RefModel, "hq_ref_backend_t": hq.RefBackend, "hq_wmat_t": hq.WMat}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "hq_backend.h"', 'int main(void) {']
    for (_, mine), fields in LAYOUT_FIELDS.items():
        lines.append(f'printf("{mine} sizeof %zu\\n", sizeof({mine}));')
        for f in fields:
            lines.append(f'printf("{mine} {f} %zu\\n", offsetof({mine}, {f}));')
    lines.append("return 0; }")
    src, exe = tmp_path / "probe.c", tmp_path / "probe"
    src.write_text("\n".join(lines) + "\n")
    subprocess.run(["gcc", "-std=c11", f"-I{os.path.join(ROOT, 'include')}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    for line in filter(None, out):
        name, field, val = line.split()
        cls = py[name]
        got = C.sizeof(cls) if field == "sizeof" else getattr(cls, field).offset
        assert got == int(val), line


def test_backend_create_refuses_before_touching_a_device():
    lib = hq.load()
    m = hq.RefModel()
    assert not lib.hip_backend_create(C.byref(m), 16, 0, False)
    assert "keep_quantized" in hq.last_error()
    m.cfg.hidden, m.cfg.n_layers, m.cfg.vocab, m.cfg.n_heads, m.cfg.n_kv_heads = 64, 1, 100, 1, 1
    m.cfg.head_dim, m.cfg.intermediate, m.cfg.rot_dim = 64, 128, 64
    layers = (hq.RefLayer * 1)()
    layers[0].type = 0  # LAYER_LINEAR
    m.layers = C.cast(layers, C.c_void_p).value
    assert not lib.hip_backend_create(C.byref(m), 16, 0, True)
    assert "Gated-DeltaNet" in hq.last_error()
