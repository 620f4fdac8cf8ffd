"""Seeded synthetic inputs in the shapes of Trit's benchmark workloads.

Every value is a counter-based hash: element i of a tensor with seed s is
splitmix64(s + i * 0x9E3779B97F4A7C15), so whole tensors are generated at
once with numpy and the same seed gives the same bytes on every machine.
The CPU oracle and the GPU library are fed identical inputs. Uniforms take
the top 24 bits; integers use a multiply-shift; normals are Box-Muller in
float64, rounded to float32.
"""

from __future__ import annotations

import numpy as np

BASE_SEED = 0x9E3779B97F4A7C15
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M64 = (1 << 64) - 1


_CHUNK = 1 << 18


def _hash_into(seed: int, out: np.ndarray, offset: int) -> None:
    n = out.size
    with np.errstate(over="ignore"):
        z = np.arange(offset + 1, offset + 1 + n, dtype=np.uint64)
        z *= _GOLDEN
        z += np.uint64(seed & _M64)
        z ^= z >> np.uint64(30)
        z *= np.uint64(0xBF58476D1CE4E5B9)
        z ^= z >> np.uint64(27)
        z *= np.uint64(0x94D049BB133111EB)
        z ^= z >> np.uint64(31)
    out[...] = z


def _hash(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint64)
    for a in range(0, count, _CHUNK):
        _hash_into(seed, out[a:a + _CHUNK], a)
    return out


def _unit(seed: int, count: int, offset: int) -> np.ndarray:
    h = np.empty(count, np.uint64)
    _hash_into(seed, h, offset)
    return (h >> np.uint64(40)).astype(np.float64) * (1.0 / (1 << 24))


def uniform(seed: int, shape) -> np.ndarray:
    """float64 in [0, 1) with 24-bit resolution."""
    n = int(np.prod(shape))
    out = np.empty(n, np.float64)
    for a in range(0, n, _CHUNK):
        out[a:a + _CHUNK] = _unit(seed, min(_CHUNK, n - a), a)
    return out.reshape(shape)


def ints(seed: int, shape, lo: int, hi: int) -> np.ndarray:
    """int64 uniform in [lo, hi]."""
    n = int(np.prod(shape))
    out = np.empty(n, np.int64)
    span = np.uint64(hi - lo + 1)
    h = np.empty(min(n, _CHUNK), np.uint64)
    for a in range(0, n, _CHUNK):
        c = min(_CHUNK, n - a)
        _hash_into(seed, h[:c], a)
        with np.errstate(over="ignore"):
            out[a:a + c] = (((h[:c] >> np.uint64(32)) * span) >> np.uint64(32)).astype(np.int64)
    out += lo
    return out.reshape(shape)


def normal(seed: int, shape, offset: int = 0) -> np.ndarray:
    """float64 standard normals (Box-Muller); element i is the tensor's
    element offset + i."""
    n = int(np.prod(shape))
    out = np.empty(n, np.float64)
    for a in range(0, n, _CHUNK):
        c = min(_CHUNK, n - a)
        u1 = np.maximum(_unit(seed, c, offset + a), 1.0 / (1 << 25))
        u2 = _unit(seed ^ 0x5851F42D4C957F2D, c, offset + a)
        out[a:a + c] = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return out.reshape(shape)


def seed_for(config: int, tensor: int) -> int:
    """Seed of tensor number `tensor` of workload `config`."""
    return (BASE_SEED + (config << 32) + (tensor << 48)) & _M64


def f16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> IEEE binary16 bits, round to nearest even."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).view(np.uint16)


def q8_0_blocks(codes: np.ndarray, scale_bits: np.ndarray) -> np.ndarray:
    """GGUF Q8_0 bytes: per block of 32 codes, the f16 scale (LE) then the codes.

    codes: int8 [n, k]; scale_bits: uint16 [n, k/32]. Returns uint8 [n*k/32*34].
    """
    n, k = codes.shape
    nb = k // 32
    out = np.empty((n, nb, 34), dtype=np.uint8)
    out[:, :, 0:2] = scale_bits.astype("<u2").reshape(n, nb, 1).view(np.uint8)
    out[:, :, 2:] = codes.reshape(n, nb, 32).view(np.uint8)
    return out.reshape(-1)


def q8_0_matrix(seed: int, n: int, k: int, scale: str = "uniform", lo: float = 0.002, hi: float = 0.02,
                sigma: float = 0.02):
    """Random Q8_0 weights: codes uniform in [-127, 127] and one f16 scale per block.

    scale "uniform": U[lo, hi]; "normal": N(0, sigma)/127 (sign kept).
    Returns (codes int8 [n,k], scale bits uint16 [n,k/32]).
    """
    codes = ints(seed, (n, k), -127, 127).astype(np.int8)
    if scale == "uniform":
        d = lo + (hi - lo) * uniform(seed ^ 0x5555, (n, k // 32))
    else:
        d = normal(seed ^ 0x5555, (n, k // 32)) * sigma / 127.0
    return codes, f16_bits(d.astype(np.float32))


def q4_k_blocks(seed: int, n: int, k: int) -> np.ndarray:
    """Random GGUF Q4_K super-blocks (144 bytes per 256 values): 4-bit codes
    uniform in 0..15, 6-bit scales and mins uniform (all 12 scale bytes
    random), f16 d and dmin uniform in [1e-3, 1e-2]. Returns uint8 bytes."""
    nb = n * k // 256
    out = np.zeros((nb, 144), np.uint8)
    dd = (1e-3 + 9e-3 * uniform(seed, (nb, 2))).astype(np.float32)
    out[:, 0:4] = f16_bits(dd).view(np.uint8).reshape(nb, 4)
    out[:, 4:16] = ints(seed ^ 0x1111, (nb, 12), 0, 255).astype(np.uint8)
    out[:, 16:] = ints(seed ^ 0x2222, (nb, 128), 0, 255).astype(np.uint8)
    return out.reshape(-1)


GGML_SCALE_FIELDS = {2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 12: (0, 2), 13: (0, 2), 14: (208,)}
GGML_BLOCK_BYTES = {2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 12: (256, 144), 13: (256, 176),
                    14: (256, 210)}


def ggml_blocks(seed: int, ggml_type: int, n: int, k: int) -> np.ndarray:
    """Random blocks of a ggml block type: random code bytes, and each f16
    scale field (d, and the min where the type has one) set to a finite
    value in +-[0.0005, 0.004] (a 32nd of that for the K types, whose
    6-bit sub-block scales multiply it)."""
    values, size = GGML_BLOCK_BYTES[ggml_type]
    nb = n * k // values
    b = ints(seed, (nb, size), 0, 255).astype(np.uint8)
    for i, at in enumerate(GGML_SCALE_FIELDS[ggml_type]):
        mag = (0.0005 + 0.0035 * uniform(seed ^ (0x77 + i), nb)) / (32.0 if values == 256 else 1.0)
        sign = np.where(ints(seed ^ (0x99 + i), nb, 0, 1) == 0, -1.0, 1.0) if i else 1.0
        b[:, at:at + 2] = f16_bits((mag * sign).astype(np.float32)).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def ternary_matrix(seed: int, n: int, k: int):
    """Ternary codes 0/1/2 (w = -1/0/1) with probabilities .25/.5/.25 and one
    f32 scale per row uniform in [0.01, 0.05], held per (row, 128-group)."""
    u = uniform(seed, (n, k))
    codes = np.where(u < 0.25, 0, np.where(u < 0.75, 1, 2)).astype(np.uint8)
    row_scale = (0.01 + 0.04 * uniform(seed ^ 0x3333, (n, 1))).astype(np.float32)
    return codes, np.repeat(row_scale, k // 128, axis=1)


def activations(seed: int, m: int, k: int) -> np.ndarray:
    """float32 [m, k] standard normals."""
    return normal(seed, (m, k)).astype(np.float32)


QWEN3_06B = dict(d=1024, ffn=3072, layers=28, heads=16, kv_heads=8, head_dim=128, vocab=151936, eps=1e-6,
                 rope_base=1e6, qk_norm=1)


class LayerWeights:
    """One decoder layer: GGUF Q8_0 bytes of the stacked products and f32 norms."""

    def __init__(self, qkv, o, gate_up, down, norm_attn, norm_mlp, q_norm, k_norm):
        self.qkv, self.o, self.gate_up, self.down = qkv, o, gate_up, down
        self.norm_attn, self.norm_mlp, self.q_norm, self.k_norm = norm_attn, norm_mlp, q_norm, k_norm


class LmWeights:
    def __init__(self, cfg, layers, embed, final_norm):
        self.cfg, self.layers, self.embed, self.final_norm = cfg, layers, embed, final_norm

    def norms_packed(self):
        """Per layer norm_attn, norm_mlp, q_norm, k_norm; then the final norm."""
        parts = []
        for L in self.layers:
            parts += [L.norm_attn, L.norm_mlp]
            if self.cfg.get("qk_norm", 1):
                parts += [L.q_norm, L.k_norm]
        parts.append(self.final_norm)
        return np.concatenate(parts).astype(np.float32)


def _layer(args):
    cfg, config, base, sigma, norm_jitter = args
    d, ffn, hd = cfg["d"], cfg["ffn"], cfg["head_dim"]
    qkv_rows = (cfg["heads"] + 2 * cfg["kv_heads"]) * hd
    t = base

    def mat(n, k):
        nonlocal t
        t += 1
        codes, sbits = q8_0_matrix(seed_for(config, t), n, k, scale="normal", sigma=sigma)
        return q8_0_blocks(codes, sbits)

    def norm(n):
        nonlocal t
        t += 1
        if norm_jitter == 0.0:
            return np.ones(n, np.float32)
        return (1.0 + norm_jitter * (2 * uniform(seed_for(config, t), n) - 1)).astype(np.float32)

    return LayerWeights(
        qkv=mat(qkv_rows, d), o=mat(d, cfg["heads"] * hd), gate_up=mat(2 * ffn, d), down=mat(d, ffn),
        norm_attn=norm(d), norm_mlp=norm(d), q_norm=norm(hd), k_norm=norm(hd))


def _embed_rows(args):
    seed, r0, r1, d, sigma = args
    return f16_bits((normal(seed, (r1 - r0, d), offset=r0 * d) * sigma).astype(np.float32))


def lm_weights(cfg: dict, config: int = 1, sigma: float = 0.02, norm_jitter: float = 0.0,
               workers: int = 0) -> LmWeights:
    """Random weights of a Qwen3-style decoder (the full-loop workload's recipe).

    Linears: Q8_0 codes uniform in [-127, 127], block scales N(0, sigma)/127.
    Embeddings (tied head): f16 N(0, sigma). Norm weights 1 (plus optional
    uniform jitter, so tests see non-unit norms). Layers are generated on
    `workers` threads (0: up to 8; numpy releases the GIL in its array
    operations); the bytes do not depend on it.
    """
    d = cfg["d"]
    jobs = [(cfg, config, 16 * (i + 1), sigma, norm_jitter) for i in range(cfg["layers"])]
    if workers == 0:
        import os
        workers = min(8, os.cpu_count() or 1) if cfg["layers"] * cfg["d"] >= 8192 else 1
    from concurrent.futures import ThreadPoolExecutor

    if workers > 1:
        with ThreadPoolExecutor(workers) as pool:
            layers = list(pool.map(_layer, jobs))
    else:
        layers = [_layer(j) for j in jobs]
    t = 16 * (cfg["layers"] + 1)
    vocab = cfg["vocab"]
    parts = [(seed_for(config, t), r0, min(vocab, r0 + 8192), d, sigma) for r0 in range(0, vocab, 8192)]
    if workers > 1:
        with ThreadPoolExecutor(workers) as pool:
            embed = np.concatenate(list(pool.map(_embed_rows, parts)))
    else:
        embed = np.concatenate([_embed_rows(p) for p in parts])
    if norm_jitter == 0.0:
        final = np.ones(d, np.float32)
    else:
        final = (1.0 + norm_jitter * (2 * uniform(seed_for(config, t + 1), d) - 1)).astype(np.float32)
    return LmWeights(cfg, layers, np.ascontiguousarray(embed.reshape(cfg["vocab"], d)), final)


def prompt(config: int, n: int, vocab: int) -> np.ndarray:
    """n token ids uniform in [0, vocab)."""
    return ints(seed_for(config, 0xFFFF), n, 0, vocab - 1).astype(np.int32)


class AutoWeights:
    """A decoder at Trit's Auto precision for safetensors (src/cpu/gemm.rs:
    565-617; S1-mini's load): every linear int8 with an f32 scale per row and
    128 inputs, and the token table (tied head) as int8 storage with an f32
    scale per 32 values (Q8, f32 math). Norms and config come from `base`."""

    def __init__(self, base: LmWeights, linears, table):
        self.cfg, self.base = base.cfg, base
        self.linears = linears  # per layer: [(codes n x k int8, scales n x k/128 f32)] * 4
        self.table = table      # (codes vocab x d int8, scales vocab x d/32 f32)

    def norms_packed(self):
        return self.base.norms_packed()


def _int8_of_blocks(blocks: np.ndarray, n: int, k: int):
    """Int8 weights from Q8_0 blocks: the same codes, and for each 128-group
    the magnitude of its first block's scale (a positive f32 scale)."""
    b = np.asarray(blocks, np.uint8).reshape(n, k // 32, 34)
    codes = np.ascontiguousarray(b[:, :, 2:]).view(np.int8).reshape(n, k)
    half = np.ascontiguousarray(b[:, ::4, :2]).view(np.float16).reshape(n, k // 128)
    scales = np.maximum(np.abs(half.astype(np.float32)), np.float32(1e-6)).astype(np.float32)
    return codes, scales


def q8_table(values: np.ndarray):
    """Int8 storage of f32 rows, 32 values a scale, by ggml's Q8_0 rule
    (d = max|v| / 127, codes round(v / d) half away from zero), the scale
    kept in f32."""
    v = np.asarray(values, np.float32)
    n, k = v.shape
    g = v.reshape(n, k // 32, 32)
    d = (np.max(np.abs(g), axis=2) / np.float32(127.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = g * inv[:, :, None]
    codes = (np.sign(q) * np.floor(np.abs(q) + np.float32(0.5))).astype(np.int8)
    return codes.reshape(n, k), d


def auto_weights(base: LmWeights) -> AutoWeights:
    """The Auto-precision form of `base` (same codes, 128-group scales; the
    f16 table requantized to int8 storage)."""
    cfg = base.cfg
    d, ffn, hd = cfg["d"], cfg["ffn"], cfg["head_dim"]
    shapes = [((cfg["heads"] + 2 * cfg["kv_heads"]) * hd, d), (d, cfg["heads"] * hd), (2 * ffn, d), (d, ffn)]
    linears = [[_int8_of_blocks(m, n, k) for m, (n, k) in zip((L.qkv, L.o, L.gate_up, L.down), shapes)]
               for L in base.layers]
    table = q8_table(base.embed.view(np.float16).astype(np.float32))
    return AutoWeights(base, linears, table)
