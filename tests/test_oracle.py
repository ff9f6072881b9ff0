"""Pins the CPU oracle (oracle/hq_oracle.c) before anything is checked against it.

Three kinds of check, chosen so that a dropped term, a wrong shift or index, or a swapped operand
fails at least one:
  * bit-exact agreement with the reference's own CPU code compiled from its sources
    (oracle/_ref/libref.so; skipped where /root/reference is absent, e.g. on the GPU box);
  * committed golden vectors produced by that build (tests/golden/, always run);
  * closed forms: all 65536 fp16 patterns against numpy, the inverse of the 6-bit scale/min
    packing over every code, integer-valued blocks, zero scales, double-precision products.
"""
import os

import numpy as np
import pytest

import synth
from conftest import rel_l2, same_bits_nan_aware

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------ fp16 -> fp32 (ops_common.h:32-53)
def test_f16_all_patterns_match_numpy(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    finite = ~np.isnan(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    # NaN: sign, all-ones exponent and the 10-bit payload shifted into the top of the mantissa
    nan_bits = bits[~finite].astype(np.uint32)
    expect = ((nan_bits & 0x8000) << 16) | 0x7F800000 | ((nan_bits & 0x3FF) << 13)
    assert np.array_equal(got[~finite].view(np.uint32), expect)


def test_f16_all_patterns_match_reference(oracle, reference):
    for h in list(range(0, 65536, 7)) + [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0x7C01, 0x7E00, 0xFC00, 0x8001]:
        a = np.float32(oracle.lib.or_f16_to_f32(h))
        b = np.float32(reference.lib.ref_f16_to_f32(h))
        assert a.view(np.uint32) == b.view(np.uint32), hex(h)


# ------------------------------------------------------------------ 6-bit scale/min unpack (ggml_quant.h:51-59)
def pack_scale_min(s, m):
    """Inverse of the unpack: eight 6-bit scales and mins -> 12 bytes (llama.cpp's Q4_K packing).
    Bytes 0-3: s0-3 in bits 0-5, top 2 bits of s4-7; bytes 4-7: m0-3, top 2 bits of m4-7;
    bytes 8-11: low nibble = low 4 bits of s4-7, high nibble = low 4 bits of m4-7."""
    q = np.zeros(12, dtype=np.uint8)
    for i in range(4):
        q[i] = s[i] | ((s[i + 4] >> 4) << 6)
        q[i + 4] = m[i] | ((m[i + 4] >> 4) << 6)
        q[i + 8] = (s[i + 4] & 0xF) | ((m[i + 4] & 0xF) << 4)
    return q


def test_scale_min_every_code_round_trips(oracle):
    import ctypes as C
    s_out, m_out = C.c_uint8(), C.c_uint8()
    for j in range(8):
        for code in range(64):
            # put code in slot j as scale and (63 - code) as min; other slots take other values
            s = [(code + 7 * i) % 64 if i != j else code for i in range(8)]
            m = [(63 - code + 11 * i) % 64 if i != j else 63 - code for i in range(8)]
            q = pack_scale_min(s, m)
            oracle.lib.or_scale_min_k4(j, q, C.byref(s_out), C.byref(m_out))
            assert (s_out.value, m_out.value) == (s[j], m[j]), (j, code)


def test_scale_min_matches_reference(oracle, reference):
    import ctypes as C
    rng = synth.Rng(11)
    b = rng.bytes(12 * 4000).reshape(4000, 12)
    a1, a2, b1, b2 = C.c_uint8(), C.c_uint8(), C.c_uint8(), C.c_uint8()
    for row in b:
        row = np.ascontiguousarray(row)
        for j in range(8):
            oracle.lib.or_scale_min_k4(j, row, C.byref(a1), C.byref(a2))
            reference.lib.ref_scale_min_k4(j, row, C.byref(b1), C.byref(b2))
            assert (a1.value, a2.value) == (b1.value, b2.value)


# ------------------------------------------------------------------ block decode
def special_q8_0_blocks():
    """Q8_0 blocks with every interesting scale: subnormals, zero, +-max, inf, NaN, and q = -128."""
    rng = synth.Rng(21)
    scales = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0xBC00, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0x7C01,
              0x1234, 0x0200, 0x2E66]
    blk = np.zeros((len(scales), 34), dtype=np.uint8)
    for i, d in enumerate(scales):
        blk[i, 0], blk[i, 1] = d & 0xFF, d >> 8
        blk[i, 2:] = rng.bytes(32)
        blk[i, 2] = 0x80  # q = -128
        blk[i, 3] = 0x7F  # q = 127
        blk[i, 4] = 0x00
    return blk.reshape(1, -1)  # one row of 16 blocks (512 values)


def special_q4_k_blocks():
    """Q4_K super-blocks: zero / subnormal / negative d and dmin, all-zero and all-15 quants."""
    rng = synth.Rng(22)
    cases = [(0x0000, 0x1400), (0x1400, 0x0000), (0x0001, 0x0001), (0x03FF, 0x8400), (0xBC00, 0x3C00),
             (0x7BFF, 0x7BFF), (0x2E66, 0x2A00), (0x7C00, 0x0000)]
    blk = rng.bytes(len(cases) * 144).reshape(len(cases), 144)
    for i, (d, dm) in enumerate(cases):
        blk[i, 0:2] = [d & 0xFF, d >> 8]
        blk[i, 2:4] = [dm & 0xFF, dm >> 8]
    blk[1, 16:] = 0
    blk[2, 16:] = 0xFF
    return blk.reshape(2, -1)  # two rows of four super-blocks (1024 values)


def special_q6_k_blocks():
    """Q6_K super-blocks with d = 0, +-1, the smallest subnormal, the largest finite value, inf
    and NaN; scales at -128, 127, 0 and 1; quants all 0 (q = -32) in one block and all 63 (q = 31)
    in another."""
    rng = synth.Rng(53)
    ds = [0x0000, 0x3C00, 0xBC00, 0x0001, 0x7BFF, 0x7C00, 0x7E00, 0x1400]
    blk = rng.bytes(len(ds) * 210).reshape(len(ds), 210)
    for i, d in enumerate(ds):
        blk[i, 208:210] = [d & 0xFF, d >> 8]
    blk[1, 192:208] = np.array([-128, 127, 0, 1] * 4, np.int8).view(np.uint8)
    blk[2, :192] = 0
    blk[3, :192] = 0xFF
    return blk.reshape(2, -1)


def special_kquant_blocks(gtype):
    """Q2_K / Q3_K / Q5_K super-blocks whose fp16 scales are 0, +-1, the smallest subnormal, the
    largest finite value, inf, NaN and a typical value; one block with every other byte 0 and one
    with every other byte 0xFF (all quants and scale codes at their extremes)."""
    fp16_at = {synth.Q2_K: (80, 82), synth.Q3_K: (108,), synth.Q5_K: (0, 2)}[gtype]
    nbytes = synth.BLOCK_BYTES[gtype]
    rng = synth.Rng(60 + gtype)
    ds = [0x0000, 0x3C00, 0xBC00, 0x0001, 0x7BFF, 0x7C00, 0x7E00, 0x1400]
    blk = rng.bytes(len(ds) * nbytes).reshape(len(ds), nbytes)
    keep = np.ones(nbytes, bool)
    for o in fp16_at:
        keep[o:o + 2] = False
    blk[1, keep] = 0
    blk[2, keep] = 0xFF
    for i, d in enumerate(ds):
        for j, o in enumerate(fp16_at):
            v = d if j == 0 else ds[(i + 3) % len(ds)]
            blk[i, o:o + 2] = [v & 0xFF, v >> 8]
    return blk.reshape(2, -1)


SPECIAL_BLOCKS = {synth.Q8_0: lambda: special_q8_0_blocks(), synth.Q4_K: lambda: special_q4_k_blocks(),
                  synth.Q6_K: lambda: special_q6_k_blocks(), synth.Q2_K: lambda: special_kquant_blocks(synth.Q2_K),
                  synth.Q3_K: lambda: special_kquant_blocks(synth.Q3_K),
                  synth.Q5_K: lambda: special_kquant_blocks(synth.Q5_K)}


@pytest.mark.parametrize("gtype", [synth.Q8_0, synth.Q2_K, synth.Q3_K, synth.Q4_K, synth.Q5_K, synth.Q6_K])
def test_dequant_matches_reference(oracle, reference, gtype):
    rng = synth.Rng(31)
    rows, cols = 24, 1024
    blocks = synth.random_blocks(gtype, rng, rows, cols)
    assert same_bits_nan_aware(oracle.dequantize(blocks, gtype, rows, cols),
                               reference.dequantize(blocks, gtype, rows, cols))
    sp = SPECIAL_BLOCKS[gtype]()
    r = sp.shape[0]
    c = sp.shape[1] // synth.BLOCK_BYTES[gtype] * synth.BLOCK_VALUES[gtype]
    assert same_bits_nan_aware(oracle.dequantize(sp, gtype, r, c), reference.dequantize(sp, gtype, r, c))


def test_dequant_q6_k_closed_form(oracle):
    """Every 6-bit code under every int8 scale: y is the exact product d * sc * (q - 32) (25
    significant bits at most, exact in float64) rounded once to float32."""
    rng = synth.Rng(59)
    n_blocks = 256
    blk = rng.bytes(n_blocks * 210).reshape(n_blocks, 210)
    blk[:, 192:208] = np.arange(n_blocks * 16, dtype=np.int64).reshape(n_blocks, 16).astype(np.uint8)  # all 256 scales
    d = synth.f16_bits(np.abs(rng.normal(n_blocks)) * 1e-2)
    blk[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    got = oracle.dequantize(blk.reshape(8, -1), synth.Q6_K, 8, 32 * 256).reshape(n_blocks, 256)
    dv = d.view(np.float16).astype(np.float64)
    sc = blk[:, 192:208].view(np.int8).astype(np.float64)
    ql, qh = blk[:, :128].astype(np.int64), blk[:, 128:192].astype(np.int64)
    codes = set()
    for v in range(256):
        h, r, l = v // 128, (v % 128) // 32, v % 32
        lo = ql[:, 64 * h + 32 * (r % 2) + l]
        lo = (lo >> 4) if r >= 2 else (lo & 0xF)
        q = (lo | (((qh[:, 32 * h + l] >> (2 * r)) & 3) << 4)) - 32
        codes.update(q.tolist())
        want = (dv * sc[:, 8 * h + 2 * r + l // 16] * q).astype(np.float32)
        assert np.array_equal(got[:, v], want), v
    assert codes == set(range(-32, 32))


def test_dequant_q8_0_closed_form(oracle):
    """d = 1.0 gives the int8 values themselves; d = 2^-24 (smallest subnormal) gives q * 2^-24."""
    q = np.arange(-128, 128, dtype=np.int16).astype(np.int8)
    blk = np.zeros((8, 34), dtype=np.uint8)
    for b in range(8):
        blk[b, 2:] = q[32 * b:32 * b + 32].view(np.uint8)
    blk[:4, 0:2] = [0x00, 0x3C]  # 1.0
    blk[4:, 0:2] = [0x01, 0x00]  # 2^-24
    got = oracle.dequantize(blk.reshape(1, -1), synth.Q8_0, 1, 256)[0]
    want = np.concatenate([q[:128].astype(np.float64), q[128:].astype(np.float64) * 2.0 ** -24])
    assert np.array_equal(got.astype(np.float64), want)


def test_dequant_q4_k_closed_form(oracle):
    """Every (scale, min) code pair and every nibble: y = d*s*q - dmin*m computed in float64 and
    rounded once to float32 (both products are exact in float32)."""
    rng = synth.Rng(41)
    n_blocks = 64 * 8  # 64 x 64 code pairs, 8 sub-blocks each
    blk = np.zeros((n_blocks, 144), dtype=np.uint8)
    codes_s = np.zeros((n_blocks, 8), np.int64)
    codes_m = np.zeros((n_blocks, 8), np.int64)
    for b in range(n_blocks):
        s = [(b * 8 + j) % 64 for j in range(8)]
        m = [((b * 8 + j) // 64) % 64 for j in range(8)]
        codes_s[b], codes_m[b] = s, m
        blk[b, 4:16] = pack_scale_min(s, m)
        blk[b, 16:] = rng.bytes(128)
    d = synth.f16_bits(np.abs(rng.normal(n_blocks)) * 1e-3)
    dm = synth.f16_bits(np.abs(rng.normal(n_blocks)) * 1e-3)
    blk[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    blk[:, 2:4] = dm.view(np.uint8).reshape(-1, 2)
    got = oracle.dequantize(blk.reshape(8, -1), synth.Q4_K, 8, 64 * 256).reshape(n_blocks, 256)
    dv = d.view(np.float16).astype(np.float64)
    dmv = dm.view(np.float16).astype(np.float64)
    qs = blk[:, 16:]
    for sub in range(8):
        byte = qs[:, 32 * (sub // 2):32 * (sub // 2) + 32].astype(np.int64)
        q = (byte >> 4) if sub % 2 else (byte & 0xF)
        want = (dv[:, None] * codes_s[:, sub:sub + 1]) * q - (dmv[:, None] * codes_m[:, sub:sub + 1])
        assert np.array_equal(got[:, 32 * sub:32 * sub + 32], want.astype(np.float32)), sub


def test_dequant_q5_k_closed_form(oracle):
    """Every (scale, min) code pair, every 5-bit code: y = d*s*(lo + 16 hb) - dmin*m in float64,
    rounded once to float32 (both products are exact in float32). lo is the nibble of qs[32 (j/2) +
    l] (j odd: high), hb bit j of qh[l]."""
    rng = synth.Rng(43)
    n_blocks = 64 * 8
    blk = rng.bytes(n_blocks * 176).reshape(n_blocks, 176)
    codes_s = np.zeros((n_blocks, 8), np.int64)
    codes_m = np.zeros((n_blocks, 8), np.int64)
    for b in range(n_blocks):
        codes_s[b] = [(b * 8 + j) % 64 for j in range(8)]
        codes_m[b] = [((b * 8 + j) // 64) % 64 for j in range(8)]
        blk[b, 4:16] = pack_scale_min(list(codes_s[b]), list(codes_m[b]))
    d = synth.f16_bits(np.abs(rng.normal(n_blocks)) * 1e-3)
    dm = synth.f16_bits(np.abs(rng.normal(n_blocks)) * 1e-3)
    blk[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    blk[:, 2:4] = dm.view(np.uint8).reshape(-1, 2)
    got = oracle.dequantize(blk.reshape(8, -1), synth.Q5_K, 8, 64 * 256).reshape(n_blocks, 256)
    dv, dmv = d.view(np.float16).astype(np.float64), dm.view(np.float16).astype(np.float64)
    qh, qs = blk[:, 16:48].astype(np.int64), blk[:, 48:].astype(np.int64)
    codes = set()
    for sub in range(8):
        byte = qs[:, 32 * (sub // 2):32 * (sub // 2) + 32]
        q = ((byte >> 4) if sub % 2 else (byte & 0xF)) + 16 * ((qh >> sub) & 1)
        codes.update(np.unique(q).tolist())
        want = (dv[:, None] * codes_s[:, sub:sub + 1]) * q - (dmv[:, None] * codes_m[:, sub:sub + 1])
        assert np.array_equal(got[:, 32 * sub:32 * sub + 32], want.astype(np.float32)), sub
    assert codes == set(range(32))


def test_dequant_q2_k_closed_form(oracle):
    """Every (scale, min) nibble pair in every scale slot, every 2-bit code: y = d*s*q - dmin*m in
    float64 rounded once to float32. Value 128 h + 32 j + l takes bits 2j of qs[32 h + l] and the
    scale byte 8 h + 2 j + l / 16."""
    rng = synth.Rng(47)
    n_blocks = 256
    blk = rng.bytes(n_blocks * 84).reshape(n_blocks, 84)
    blk[:, :16] = (np.arange(n_blocks * 16).reshape(n_blocks, 16) % 256).astype(np.uint8)  # every byte value
    d = synth.f16_bits(np.abs(rng.normal(n_blocks)) * 1e-2)
    dm = synth.f16_bits(np.abs(rng.normal(n_blocks)) * 1e-2)
    blk[:, 80:82] = d.view(np.uint8).reshape(-1, 2)
    blk[:, 82:84] = dm.view(np.uint8).reshape(-1, 2)
    got = oracle.dequantize(blk.reshape(8, -1), synth.Q2_K, 8, 32 * 256).reshape(n_blocks, 256)
    dv, dmv = d.view(np.float16).astype(np.float64), dm.view(np.float16).astype(np.float64)
    sc, qs = blk[:, :16].astype(np.int64), blk[:, 16:80].astype(np.int64)
    for v in range(256):
        h, j, l = v // 128, (v % 128) // 32, v % 32
        q = (qs[:, 32 * h + l] >> (2 * j)) & 3
        b = sc[:, 8 * h + 2 * j + l // 16]
        want = dv * (b & 15) * q - dmv * (b >> 4)
        assert np.array_equal(got[:, v], want.astype(np.float32)), v


def pack_q3_k_scales(s):
    """16 six-bit Q3_K scale codes -> the 12 packed bytes (the inverse of the unpacking the oracle
    restates, written from the layout: low nibbles of codes 0-7 in bytes 0-7, of codes 8-15 in the
    high nibbles of bytes 0-7, top two bits of code 4g + i in bits 2g of byte 8 + i)."""
    out = np.zeros(12, np.uint8)
    for e, c in enumerate(s):
        g, i = divmod(e, 4)
        out[4 * (g & 1) + i] |= (c & 15) << (4 * (g >> 1))
        out[8 + i] |= (c >> 4) << (2 * g)
    return out


def test_dequant_q3_k_closed_form(oracle):
    """Every 6-bit scale code in every slot, every 3-bit code: y = d*(sc - 32)*q exactly (at most
    20 significant bits), with q = (2-bit field) - 4 unless the hmask bit is set."""
    rng = synth.Rng(49)
    n_blocks = 64
    blk = rng.bytes(n_blocks * 110).reshape(n_blocks, 110)
    codes = (np.arange(n_blocks * 16).reshape(n_blocks, 16) + np.arange(n_blocks)[:, None] * 5) % 64
    for b in range(n_blocks):
        blk[b, 96:108] = pack_q3_k_scales(codes[b])
    d = synth.f16_bits(np.abs(rng.normal(n_blocks)) * 1e-3)
    blk[:, 108:110] = d.view(np.uint8).reshape(-1, 2)
    got = oracle.dequantize(blk.reshape(8, -1), synth.Q3_K, 8, 8 * 256).reshape(n_blocks, 256)
    dv = d.view(np.float16).astype(np.float64)
    hm, qs = blk[:, :32].astype(np.int64), blk[:, 32:96].astype(np.int64)
    seen = set()
    for v in range(256):
        h, j, l = v // 128, (v % 128) // 32, v % 32
        q = ((qs[:, 32 * h + l] >> (2 * j)) & 3) - 4 * (1 - ((hm[:, l] >> (4 * h + j)) & 1))
        seen.update(q.tolist())
        want = dv * (codes[:, 8 * h + 2 * j + l // 16] - 32) * q
        assert np.array_equal(got[:, v].astype(np.float64), want), v
    assert seen == set(range(-4, 4))
    assert set(codes.ravel().tolist()) == set(range(64))


def test_src_row_is_llama_cpp_interleave(oracle):
    """Storage row 2i+j of a head holds HF row j*(hd/2)+i: check the permutation inverts that."""
    import ctypes as C
    import oracle as o
    for rows, heads in [(512, 8), (64, 1), (96, 3)]:
        w = o.WMat(3, rows, 32, 0, 8, heads)
        src = np.array([oracle.lib.or_src_row(C.byref(w), r) for r in range(rows)])
        assert sorted(src) == list(range(rows))
        hd = rows // heads
        for r in range(rows):
            head, within = divmod(src[r], hd)
            i, j = divmod(within, 2)  # storage index 2i + j
            assert r == head * hd + j * (hd // 2) + i


def test_src_row_matches_reference(oracle, reference):
    import ctypes as C
    import oracle as o
    for rows, heads in [(512, 8), (4096, 32), (1024, 8)]:
        w = o.WMat(3, rows, 32, 0, 8, heads)
        for r in range(rows):
            assert oracle.lib.or_src_row(C.byref(w), r) == reference.lib.wmat_src_row(C.byref(w), r)


# ------------------------------------------------------------------ dot / matmul (cpu_backend.c:28-54)
# quantized shapes of the reference selftest (cuda_backend.cu:1110) plus Q8_0 rows that end mid
# 256-value chunk (K = 1408, the config-1 FFN width) and a perm_heads matrix
MATMUL_CASES = [(synth.Q8_0, 40, 512, 5), (synth.Q8_0, 40, 512, 40), (synth.Q4_K, 40, 512, 5),
                (synth.Q4_K, 40, 512, 40), (synth.Q8_0, 33, 1408, 7), (synth.Q4_K, 130, 2560, 3),
                (synth.Q6_K, 40, 512, 5), (synth.Q6_K, 130, 2560, 3), (synth.Q2_K, 40, 512, 5),
                (synth.Q3_K, 40, 512, 5), (synth.Q5_K, 40, 512, 5), (synth.Q5_K, 130, 2560, 3)]


@pytest.mark.parametrize("gtype,N,K,T", MATMUL_CASES)
def test_matmul_matches_reference(oracle, reference, gtype, N, K, T):
    rng = synth.Rng(1000 + N + K + T)
    blocks = synth.random_blocks(gtype, rng, N, K)
    x = oracle.f16_to_f32(synth.activations_f16(rng, T, K))
    y0 = rng.normal(T * N).astype(np.float32).reshape(T, N)
    for acc in (False, True):
        a = oracle.matmul(blocks, gtype, N, K, x, y0.copy(), acc)
        b = reference.matmul(blocks, gtype, N, K, x, y0.copy(), acc)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    perm = 8 if N % 16 == 0 else 0
    a = oracle.matmul(blocks, gtype, N, K, x, perm_heads=perm)
    b = reference.matmul(blocks, gtype, N, K, x, perm_heads=perm)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("gtype,N,K,T", MATMUL_CASES)
def test_matmul_close_to_double(oracle, gtype, N, K, T):
    rng = synth.Rng(2000 + N + K + T)
    blocks = synth.random_blocks(gtype, rng, N, K)
    x = oracle.f16_to_f32(synth.activations_f16(rng, T, K))
    y = oracle.matmul(blocks, gtype, N, K, x)
    w = oracle.dequantize(blocks, gtype, N, K).astype(np.float64)
    ref = x.astype(np.float64) @ w.T
    assert rel_l2(y, ref) < 2e-6
    scale = np.abs(x.astype(np.float64)) @ np.abs(w.T)
    assert np.all(np.abs(y - ref) <= 1e-5 * scale + 1e-30)


def test_matmul_rows_slice_equals_full(oracle):
    rng = synth.Rng(3)
    blocks = synth.random_blocks(synth.Q4_K, rng, 64, 512)
    x = oracle.f16_to_f32(synth.activations_f16(rng, 4, 512))
    full = oracle.matmul(blocks, synth.Q4_K, 64, 512, x)
    part = oracle.matmul(blocks, synth.Q4_K, 64, 512, x, row_range=(16, 48))
    assert np.array_equal(part[:, 16:48], full[:, 16:48])
    assert not part[:, :16].any() and not part[:, 48:].any()


def test_dot_partial_order(oracle, reference):
    """The 8-partial combining order changes float results: check against the reference on
    inputs built to cancel, and on random lengths with tails."""
    rng = synth.Rng(5)
    for n in [1, 7, 8, 9, 63, 64, 65, 2560]:
        a = (rng.normal(n) * 1e4).astype(np.float32)
        b = rng.normal(n).astype(np.float32)
        a[::3] *= -1e3
        x = np.float32(oracle.lib.or_dot(a, b, n))
        y = np.float32(reference.lib.ref_dot(a, b, n))
        assert x.view(np.uint32) == y.view(np.uint32), n


def test_gather_equals_matmul_columns(oracle):
    rng = synth.Rng(6)
    V, K, B, k = 300, 512, 9, 5
    blocks = synth.random_blocks(synth.Q8_0, rng, V, K)
    h = oracle.f16_to_f32(synth.activations_f16(rng, B, K))
    ids = np.stack([rng.choice_without_replacement(V, k) for _ in range(B)]).astype(np.uint32)
    got = oracle.gather_dot(blocks, synth.Q8_0, V, K, h, ids)
    full = oracle.matmul(blocks, synth.Q8_0, V, K, h)
    assert np.array_equal(got, np.take_along_axis(full, ids.astype(np.int64), axis=1))


# ------------------------------------------------------------------ config-1 forward (cpu_backend.c:218-263)
@pytest.fixture(scope="module")
def tiny_model():
    return synth.tiny_llama(1)


def test_llama_forward_matches_reference(oracle, reference, tiny_model, tmp_path):
    import gguf_writer
    path = str(tmp_path / "tiny.gguf")
    gguf_writer.write_tiny_llama(path, tiny_model)
    tokens, ids = synth.tiny_llama_prompt(2)
    a, ha = oracle.llama_forward(tiny_model, tokens, ids, hidden=True)
    b, hb = reference.logits(path, tokens, ids, hidden_size=tiny_model["cfg"]["hidden"])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(ha.view(np.uint32), hb.view(np.uint32))  # last_hidden, bit for bit
    # a second prompt: shorter, repeated ids
    t2 = tokens[:17]
    i2 = np.array([5, 5, 31999, 0], np.uint32)
    assert np.array_equal(oracle.llama_forward(tiny_model, t2, i2).view(np.uint32),
                          reference.logits(path, t2, i2).view(np.uint32))


def test_llama_forward_gqa_matches_reference(oracle, reference, tmp_path):
    """Grouped-query attention (8 query heads over 2 kv heads, src/cpu_backend.c:110) and a prompt of
    300 tokens: the oracle forward is bit-exact with the reference's model_load + cpu_forward."""
    import gguf_writer
    cfg = dict(synth.TINY_LLAMA, n_layers=2, n_kv_heads=2, vocab=4096)
    model = synth.tiny_llama(3, cfg)
    path = str(tmp_path / "gqa.gguf")
    gguf_writer.write_tiny_llama(path, model)
    tokens, ids = synth.tiny_llama_prompt(4, T=300, vocab=cfg["vocab"], n_ids=8)
    a = oracle.llama_forward(model, tokens, ids)
    b = reference.logits(path, tokens, ids)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_llama_forward_rope_table_matches_reference(oracle, reference, tiny_model, tmp_path):
    """A RoPE table: the GGUF carries per-frequency divisors (rope_freqs.weight: 1 for the short
    wavelengths, 8 for the long ones, a ramp between, as Llama 3.1 files do), which the reference's
    model_load divides its table by (src/model.c:470-476); the oracle forward given that table
    (theta powers / divisors in float32) is bit-exact with it, and differs from the unscaled one."""
    import gguf_writer
    import hq
    c = tiny_model["cfg"]
    half = c["rot_dim"] // 2
    div = np.ones(half, np.float32)
    div[half // 2:] = 8.0
    div[half // 2 - 4:half // 2] = np.float32([1.5, 2.5, 4.0, 6.0])
    model = dict(tiny_model, rope_freqs=div)
    path = str(tmp_path / "rope.gguf")
    gguf_writer.write_tiny_llama(path, model)
    tokens, ids = synth.tiny_llama_prompt(2, T=64)
    inv = (hq.rope_inv_freq(c["rope_theta"], c["rot_dim"]) / div).astype(np.float32)
    a = oracle.llama_forward(dict(tiny_model, rope_inv_freq=inv), tokens, ids)
    b = reference.logits(path, tokens, ids)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert not np.array_equal(a, oracle.llama_forward(tiny_model, tokens, ids))


def test_llama_forward_rejects_bad_ids(oracle, tiny_model):
    with pytest.raises(ValueError):
        oracle.llama_forward(tiny_model, np.array([32000], np.uint32), np.array([1], np.uint32))
    with pytest.raises(ValueError):
        oracle.llama_forward(tiny_model, np.array([1], np.uint32), np.array([40000], np.uint32))


# ------------------------------------------------------------------ committed golden vectors
def load_golden(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.fail(f"golden fixture {name} missing: run tests/golden/make_golden.py")
    return np.load(path, allow_pickle=False)


@pytest.mark.parametrize("name", ["dequant_q8_0.npz", "dequant_q4_k.npz", "dequant_q6_k.npz", "dequant_q2_k.npz",
                                  "dequant_q3_k.npz", "dequant_q5_k.npz"])
def test_golden_dequant(oracle, name):
    g = load_golden(name)
    got = oracle.dequantize(g["blocks"], int(g["gtype"]), int(g["rows"]), int(g["cols"]), int(g["perm_heads"]))
    assert same_bits_nan_aware(got, g["values"])


@pytest.mark.parametrize("name", ["matmul_q8_0.npz", "matmul_q4_k.npz", "matmul_q6_k.npz", "matmul_q2_k.npz",
                                  "matmul_q3_k.npz", "matmul_q5_k.npz"])
def test_golden_matmul(oracle, name):
    g = load_golden(name)
    got = oracle.matmul(g["blocks"], int(g["gtype"]), int(g["rows"]), int(g["cols"]), g["x"], g["y0"].copy(),
                        bool(g["accumulate"]))
    assert np.array_equal(got.view(np.uint32), g["y"].view(np.uint32))


def test_golden_tiny_llama(oracle, tiny_model):
    g = load_golden("tiny_llama.npz")
    assert synth_digest(tiny_model) == str(g["model_sha256"]), "synth.tiny_llama(1) changed"
    got = oracle.llama_forward(tiny_model, g["tokens"], g["ids"])
    assert np.array_equal(got.view(np.uint32), g["logits"].view(np.uint32))


def synth_digest(model):
    import hashlib
    h = hashlib.sha256()
    for key in ("embed", "lm_head", "final_norm"):
        h.update(np.ascontiguousarray(model[key]).tobytes())
    for L in model["layers"]:
        for key in sorted(L):
            h.update(np.ascontiguousarray(L[key]).tobytes())
    return h.hexdigest()
