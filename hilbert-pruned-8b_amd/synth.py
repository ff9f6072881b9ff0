"""Deterministic synthetic inputs for the quantized matmul path.

Every generator is seeded and platform-independent (splitmix64 + Box-Muller in numpy), so the
same bytes are produced here, on the GPU box, in tests and in bench.py.

Block layouts (GGUF, little-endian; reference cleanroom-transformer/src/ggml_quant.h):
  Q8_0  34 B / 32 values : fp16 d, int8 q[32]                          (ggml_quant.h:95-99)
  Q4_K 144 B / 256 values: fp16 d, fp16 dmin, u8 scales[12], u8 qs[128] (ggml_quant.h:135-150)
  Q6_K 210 B / 256 values: u8 ql[128], u8 qh[64], int8 scales[16], fp16 d (ggml_quant.h:151-169)
  Q2_K  84 B / 256 values: u8 scales[16], u8 qs[64], fp16 d, fp16 dmin  (ggml_quant.h:100-111)
  Q3_K 110 B / 256 values: u8 hmask[32], u8 qs[64], u8 scales[12], fp16 d (ggml_quant.h:112-134)
  Q5_K 176 B / 256 values: fp16 d, fp16 dmin, u8 scales[12], u8 qh[32], u8 qs[128] (:135-150)

Workloads:
  config 2  Q8_0 9728x2560, q uniform in [-127, 127], d = fp16(|N(0,1)| * 2e-4)
  config 3  Q4_K 9728x2560 and 2560x9728, every byte of scales/qs uniform, d and dmin =
            fp16(|N(0,1)| * 1e-3)
  config 1  tiny Llama, weights N(0, 0.02) quantised to Q8_0 by absmax/127
  config 5  Q8_0 lm_head 151936x2560 (as config 2), 256 fp16 states, k ids per state
Activations are fp16(N(0,1)), returned as uint16 bit patterns.
"""
import numpy as np

Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 8, 10, 11, 12, 13, 14
KQUANTS = (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K)
BLOCK_VALUES = {Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
TYPE_NAMES = {Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K"}

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def row_bytes(gtype, cols):
    return cols // BLOCK_VALUES[gtype] * BLOCK_BYTES[gtype]


class Rng:
    """splitmix64 stream. Vectorised: draw(n) returns the next n 64-bit outputs."""

    def __init__(self, seed):
        self.state = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)

    def draw(self, n):
        with np.errstate(over="ignore"):
            idx = np.arange(1, n + 1, dtype=np.uint64)
            z = self.state + idx * np.uint64(0x9E3779B97F4A7C15)
            self.state = z[-1] if n else self.state
            z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
            z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
            return z ^ (z >> np.uint64(31))

    def bytes(self, n):
        words = self.draw((n + 7) // 8)
        return words.view(np.uint8)[:n].copy()

    def uniform(self, n):
        """float64 in [0, 1) with 53 random bits."""
        return (self.draw(n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)

    def normal(self, n):
        m = (n + 1) // 2
        u1 = self.uniform(m)
        u2 = self.uniform(m)
        r = np.sqrt(-2.0 * np.log1p(-u1))  # 1-u1 in (0, 1]
        th = 2.0 * np.pi * u2
        return np.concatenate([r * np.cos(th), r * np.sin(th)])[:n]

    def integers(self, lo, hi, n):
        """uniform integers in [lo, hi] (inclusive), via 64-bit multiply-shift."""
        span = hi - lo + 1
        return lo + ((self.draw(n) >> np.uint64(32)).astype(np.uint64) * np.uint64(span) >> np.uint64(32)).astype(
            np.int64)

    def choice_without_replacement(self, n_pool, k):
        """k distinct values of range(n_pool) (partial Fisher-Yates on the first k slots)."""
        out = {}
        res = np.empty(k, dtype=np.int64)
        r = self.draw(k)
        for i in range(k):
            j = i + int(r[i] % np.uint64(n_pool - i))
            vi, vj = out.get(i, i), out.get(j, j)
            out[i], out[j] = vj, vi
            res[i] = vj
        return res


def f16_bits(x):
    return np.asarray(x, dtype=np.float64).astype(np.float16).view(np.uint16)


def activations_f16(rng, m, k):
    """fp16(N(0,1)) [m, k] as uint16 bit patterns."""
    return f16_bits(rng.normal(m * k)).reshape(m, k)


def q8_0_blocks(rng, rows, cols, scale=2e-4):
    """Config-2 style Q8_0 blocks [rows, row_bytes] (uint8): q uniform in [-127, 127] (16 random
    bits per value, multiply-shift), d = fp16(|N(0,1)| * scale). Generated in row chunks."""
    out = np.empty((rows, row_bytes(Q8_0, cols)), dtype=np.uint8)
    per = cols // 32
    step = max(1, (1 << 22) // cols)
    for r0 in range(0, rows, step):
        r1 = min(rows, r0 + step)
        nb = (r1 - r0) * per
        blk = out[r0:r1].reshape(nb, 34)
        blk[:, 0:2] = f16_bits(np.abs(rng.normal(nb)) * scale).view(np.uint8).reshape(nb, 2)
        u = rng.bytes(nb * 64).view(np.uint16).astype(np.uint32)
        blk[:, 2:] = ((u * 255 >> 16).astype(np.int32) - 127).astype(np.int8).view(np.uint8).reshape(nb, 32)
    return out


def q4_k_blocks(rng, rows, cols, scale=1e-3):
    """Config-3 style Q4_K super-blocks [rows, row_bytes] (uint8)."""
    nb = rows * (cols // 256)
    blk = rng.bytes(nb * 144).reshape(nb, 144)
    d = f16_bits(np.abs(rng.normal(nb)) * scale)
    dm = f16_bits(np.abs(rng.normal(nb)) * scale)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = dm.view(np.uint8).reshape(nb, 2)
    return blk.reshape(rows, row_bytes(Q4_K, cols))


def q6_k_blocks(rng, rows, cols, scale=2e-5):
    """Q6_K super-blocks [rows, row_bytes] (uint8): ql, qh uniform bytes, int8 scales uniform in
    [-128, 127], d = fp16(|N(0,1)| * scale) (weights of a few 1e-2, as in real models)."""
    nb = rows * (cols // 256)
    blk = rng.bytes(nb * 210).reshape(nb, 210)
    blk[:, 208:210] = f16_bits(np.abs(rng.normal(nb)) * scale).view(np.uint8).reshape(nb, 2)
    return blk.reshape(rows, row_bytes(Q6_K, cols))


def _kquant_blocks(gtype, rng, rows, cols, fp16_at, scale):
    """Super-blocks of `gtype` with every byte uniform except the fp16 scales at byte offsets
    `fp16_at`, which are fp16(|N(0,1)| * scale)."""
    nb = rows * (cols // 256)
    blk = rng.bytes(nb * BLOCK_BYTES[gtype]).reshape(nb, BLOCK_BYTES[gtype])
    for o in fp16_at:
        blk[:, o:o + 2] = f16_bits(np.abs(rng.normal(nb)) * scale).view(np.uint8).reshape(nb, 2)
    return blk.reshape(rows, row_bytes(gtype, cols))


def q2_k_blocks(rng, rows, cols, scale=4e-3):
    """Q2_K super-blocks: scales and qs uniform bytes, d and dmin = fp16(|N(0,1)| * scale). The
    default scale gives d of a few 1e-3, the size a 2-bit quantiser picks for weights of standard
    deviation ~0.03 (d ~ 0.1 x the weights' standard deviation: the largest 16-value group range / 3,
    spread over 15 scale codes); the committed golden fixtures were written with scale 1e-2."""
    return _kquant_blocks(Q2_K, rng, rows, cols, (80, 82), scale)


def q3_k_blocks(rng, rows, cols, scale=5e-4):
    """Q3_K super-blocks: hmask, qs and the packed scales uniform bytes, d = fp16(|N(0,1)| * scale)."""
    return _kquant_blocks(Q3_K, rng, rows, cols, (108,), scale)


def q5_k_blocks(rng, rows, cols, scale=5e-4):
    """Q5_K super-blocks: scales, qh and qs uniform bytes, d and dmin = fp16(|N(0,1)| * scale)."""
    return _kquant_blocks(Q5_K, rng, rows, cols, (0, 2), scale)


def random_blocks(gtype, rng, rows, cols):
    gen = {Q8_0: q8_0_blocks, Q2_K: q2_k_blocks, Q3_K: q3_k_blocks, Q4_K: q4_k_blocks, Q5_K: q5_k_blocks,
           Q6_K: q6_k_blocks}
    return gen[gtype](rng, rows, cols)


def quantize_q8_0(w):
    """float [rows, cols] -> Q8_0 blocks by absmax/127 (round half away from zero), as llama.cpp's
    reference quantiser. Only used to build config-1 weights; both sides read the same blocks."""
    w = np.asarray(w, dtype=np.float32)
    rows, cols = w.shape
    x = w.reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    v = x * inv[:, None]
    q = np.clip(np.sign(v) * np.floor(np.abs(v) + np.float32(0.5)), -127, 127).astype(np.int8)
    blk = np.empty((x.shape[0], 34), dtype=np.uint8)
    blk[:, 0:2] = f16_bits(d).view(np.uint8).reshape(-1, 2)
    blk[:, 2:] = q.view(np.uint8)
    return blk.reshape(rows, row_bytes(Q8_0, cols))


# ---------------------------------------------------------------- config 1: tiny Llama

TINY_LLAMA = dict(hidden=512, n_layers=4, intermediate=1408, vocab=32000, n_heads=8, n_kv_heads=8, head_dim=64,
                  rot_dim=64, eps=1e-5, rope_theta=10000.0)


def tiny_llama(seed=1, cfg=None):
    """Config-1 model: dict of Q8_0 block arrays (llama.cpp storage order: q/k rows interleaved
    per head, as GGUF files hold them) and float32 norm vectors."""
    c = dict(TINY_LLAMA if cfg is None else cfg)
    rng = Rng(seed)
    H, I, V = c["hidden"], c["intermediate"], c["vocab"]
    qw, kvw = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]

    def mat(rows, cols):
        return quantize_q8_0((rng.normal(rows * cols) * 0.02).astype(np.float32).reshape(rows, cols))

    def norm(n):
        return (1.0 + 0.1 * rng.normal(n)).astype(np.float32)

    m = {"cfg": c, "embed": mat(V, H), "lm_head": mat(V, H), "final_norm": norm(H), "layers": []}
    for _ in range(c["n_layers"]):
        m["layers"].append({
            "in_norm": norm(H), "post_norm": norm(H),
            "q": mat(qw, H), "k": mat(kvw, H), "v": mat(kvw, H), "o": mat(H, qw),
            "gate": mat(I, H), "up": mat(I, H), "down": mat(H, I),
        })
    return m


def tiny_llama_prompt(seed=2, T=128, vocab=32000, n_ids=4):
    rng = Rng(seed)
    tokens = rng.integers(0, vocab - 1, T).astype(np.uint32)
    ids = rng.choice_without_replacement(vocab, n_ids).astype(np.uint32)
    return tokens, ids


# ---------------------------------------------------------------- config 4: hybrid layer list

def hybrid_4b_projections(reading="baseline"):
    """(name, N=out rows, K=in cols) per projection of the 32-layer hybrid (3 Gated-DeltaNet : 1 full
    attention), in model order.
    reading="baseline": BASELINE.json config 4's literal widths (attention Q 4096 / KV 1024,
      DeltaNet in/out 4096, FFN 9216, d=2560).
    reading="layer_weights": the reference's own list (cleanroom-transformer/src/shapes.c:12-39)
      for its Qwen3.5-4B config (tests/configs/qwen3.5-4b/config.json: hidden 2560, 16 heads of 256
      with the output gate, 4 kv heads, DeltaNet 16 key heads x 128 and 32 value heads x 128, FFN
      9216): q_proj 8192 (q and gate), k/v 1024, o 2560 x 4096; in_proj_qkv 8192, z 4096, b and a 32,
      out_proj 2560 x 4096."""
    H, I = 2560, 9216
    if reading == "baseline":
        lin = [("linear.in_proj", 4096, H), ("linear.out_proj", H, 4096)]
        full = [("attn.q", 4096, H), ("attn.k", 1024, H), ("attn.v", 1024, H), ("attn.o", H, 4096)]
    elif reading == "layer_weights":
        hd, nh, nkv, Dk, Dv = 256, 16, 4, 16 * 128, 32 * 128
        full = [("self_attn.q_proj", nh * hd * 2, H), ("self_attn.k_proj", nkv * hd, H),
                ("self_attn.v_proj", nkv * hd, H), ("self_attn.o_proj", H, nh * hd)]
        lin = [("linear_attn.in_proj_qkv", 2 * Dk + Dv, H), ("linear_attn.in_proj_z", Dv, H),
               ("linear_attn.in_proj_b", 32, H), ("linear_attn.in_proj_a", 32, H),
               ("linear_attn.out_proj", H, Dv)]
    else:
        raise ValueError(reading)
    ffn = [("mlp.gate", I, H), ("mlp.up", I, H), ("mlp.down", H, I)]
    layers = []
    for li in range(32):
        mix = full if li % 4 == 3 else lin
        layers.append([(f"layers.{li}.{n}", r, k) for n, r, k in mix + ffn])
    return layers
