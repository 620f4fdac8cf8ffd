"""ctypes view of the oracle library (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker or the timed CPU baseline.
"""

from __future__ import annotations

import ctypes as C
import math
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libtrit_oracle.so")

SCALAR, AVX2, AVX512 = 0, 1, 2

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = _bind(C.CDLL(LIB_PATH))
    return _lib


class LmConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("d", "ffn", "layers", "heads", "kv_heads", "head_dim", "vocab")] + [
        ("eps", C.c_float), ("rope_base", C.c_float), ("qk_norm", C.c_int), ("kv_f16", C.c_int),
        ("embedding_multiplier", C.c_float), ("attention_multiplier", C.c_float),
        ("residual_multiplier", C.c_float), ("logits_scaling", C.c_float)]


TABLE_F16, TABLE_F32, TABLE_Q8 = 0, 1, 2


def _bind(L):
    p, i, f, i64 = C.c_void_p, C.c_int, C.c_float, C.c_int64
    sig = {
        "or_isa_best": (i, []),
        "or_team_start": (i, [i, i]),
        "or_team_size": (i, []),
        "or_vnni_peak": (C.c_double, [i64]),
        "or_f32_to_f16": (C.c_uint16, [f]),
        "or_f16_to_f32": (f, [C.c_uint16]),
        "or_exp": (f, [f]),
        "or_silu": (None, [p, i64]),
        "or_quantize": (None, [i, p, i, i, i, i, p, p, p]),
        "or_q8_0_quantize": (None, [p, i64, p, p]),
        "or_q8_0_parse": (None, [p, i64, p, p]),
        "or_q4_k_expand": (None, [p, i64, p]),
        "or_ggml_expand": (i, [i, p, i64, p]),
        "or_f32_to_f16_n": (None, [p, i64, p]),
        "or_gelu": (None, [p, i64]),
        "or_layer_norm": (None, [p, i, i, p, p, f, p]),
        "or_conv_columns": (None, [p, i, i, i, i, i, i, p]),
        "or_f16_to_f32_n": (None, [p, i64, p]),
        "or_int8_new": (p, [i, i, i, i, i, p, p]),
        "or_int8_forward": (None, [p, p, i, p]),
        "or_int8_free": (None, [p]),
        "or_ternary_new": (p, [i, i, i, p, p]),
        "or_ternary_forward": (None, [p, p, i, p]),
        "or_ternary_free": (None, [p]),
        "or_ternary_from_base3": (i, [p, i, i, p]),
        "or_matmul_f16": (None, [i, p, i, i, p, i, p]),
        "or_matmul_f32": (None, [i, p, i, i, p, i, p]),
        "or_rmsnorm": (None, [p, i, f, p, i]),
        "or_rope_table": (None, [i, f, i, p, p]),
        "or_rope": (None, [p, i, i, i, i, i, f]),
        "or_attention": (None, [p, i, p, p, i, i, i, i, i, i, i, p]),
        "or_argmax": (i, [p, i]),
        "or_lm_new": (p, [i, C.POINTER(LmConfig)]),
        "or_lm_set_layer": (i, [p, i, p, p, p, p, p, p, p, p]),
        "or_lm_set_embed": (i, [p, p, p]),
        "or_lm_set_linear_int8": (i, [p, i, i, p, p]),
        "or_lm_set_linear_float": (i, [p, i, i, i, p]),
        "or_lm_set_table": (i, [p, i, i, p, p]),
        "or_lm_set_ffn_scales": (i, [p, p]),
        "or_lm_forward_rows": (i, [p, p, i, p]),
        "or_lm_truncate": (i, [p, i]),
        "or_lm_position": (i, [p]),
        "or_lm_embed_row": (i, [p, i, p]),
        "or_lm_generate": (i, [p, p, i, i, p, i, p, p]),
        "or_lm_forward": (i, [p, p, i, p]),
        "or_lm_reset": (None, [p]),
        "or_lm_free": (None, [p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def ptr(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(C.c_void_p)


def isa_best() -> int:
    return lib().or_isa_best()


def team_start(spread: int = 0, threads: int = 0) -> int:
    return lib().or_team_start(spread, threads)


def vnni_peak(iters: int = 10_000_000) -> float:
    """int8 multiply-adds per second of the team on register-resident
    vpdpbusd chains, 24 a thread (0 without AVX-512 VNNI); the best of three
    runs."""
    return lib().or_vnni_peak(iters)


def quantize(x: np.ndarray, group: int, half_scales: bool, isa: int = SCALAR):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = x.shape
    codes = np.empty((m, k), np.int8)
    scales = np.empty((m, k // group), np.float32)
    sums = np.empty((m, k // group), np.int32)
    lib().or_quantize(isa, ptr(x), m, k, group, int(half_scales), ptr(codes), ptr(scales), ptr(sums))
    return codes, scales, sums


def q8_0_parse(blocks: np.ndarray, n: int, k: int):
    codes = np.empty((n, k), np.int8)
    scales = np.empty((n, k // 32), np.float32)
    lib().or_q8_0_parse(ptr(np.ascontiguousarray(blocks, np.uint8)), n * k // 32, ptr(codes), ptr(scales))
    return codes, scales


def q8_0_quantize(values: np.ndarray):
    v = np.ascontiguousarray(values, np.float32).reshape(-1)
    codes = np.empty(v.size, np.int8)
    scales = np.empty(v.size // 32, np.float32)
    lib().or_q8_0_quantize(ptr(v), v.size, ptr(codes), ptr(scales))
    return codes, scales


def gelu(x):
    """The exact GELU as every Trit path computes it (src/cpu/v2/activation.rs:33-39)."""
    x = np.array(x, np.float32, copy=True, order="C")
    lib().or_gelu(ptr(x), x.size)
    return x


def layer_norm(x, w, b, eps=1e-5):
    """Norm::apply (src/layers.rs:50-121): rows of len(w)."""
    w = np.ascontiguousarray(w, np.float32)
    d = w.size
    x = np.ascontiguousarray(x, np.float32).reshape(-1, d)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(x)
    lib().or_layer_norm(ptr(x), x.shape[0], d, ptr(w), ptr(b), eps, ptr(out))
    return out


def conv_columns(x, kernel, stride, pad, out_frames):
    """conv_columns (src/layers.rs:613-634) of x (frames x channels)."""
    x = np.ascontiguousarray(x, np.float32)
    frames, channels = x.shape
    out = np.empty((out_frames, channels * kernel), np.float32)
    lib().or_conv_columns(ptr(x), frames, channels, kernel, stride, pad, out_frames, ptr(out))
    return out


class Encoder:
    """Encoder::encode (src/models/parts/audio_encoder.rs:111-138), the
    Whisper encoder Voxtral and MOSS run, composed of the oracle's pieces:
    im2col (kernel 3, stride 1, pad 1) -> conv1 -> GELU -> im2col (stride 2)
    -> conv2 -> GELU -> + learned positions; per layer a pre-norm attention
    block (stacked q/k/v, every position sees every other) and a pre-norm
    GELU MLP, each added to the rows; then the final norm. `products` are
    callables x -> x W^T + bias (the layer's own kind and order): conv1,
    conv2, then qkv, out, fc1, fc2 of each layer; `norms` per layer
    (attn w, b, ffn w, b), then the final (w, b)."""

    def __init__(self, cfg, products, positions, norms):
        self.cfg, self.products, self.positions, self.norms = cfg, products, positions, norms

    def encode(self, mel):
        c = self.cfg
        d, P, heads = c["d"], c["positions"], c["heads"]
        frames = 2 * P
        mel = np.ascontiguousarray(mel, np.float32).reshape(frames, c["mels"])
        h = gelu(self.products[0](conv_columns(mel, 3, 1, 1, frames)))
        x = gelu(self.products[1](conv_columns(h, 3, 2, 1, P)))
        x = (x + np.asarray(self.positions, np.float32).reshape(P, d)).astype(np.float32)
        hd = d // heads
        for l in range(c["layers"]):
            qkv_p, out_p, fc1_p, fc2_p = self.products[2 + 4 * l:6 + 4 * l]
            aw, ab, fw, fb = self.norms[4 * l:4 * l + 4]
            qkv = qkv_p(layer_norm(x, aw, ab))
            att = attention(qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:], heads, heads, hd, causal=False)
            x = (x + out_p(att)).astype(np.float32)
            x = (x + fc2_p(gelu(fc1_p(layer_norm(x, fw, fb))))).astype(np.float32)
        return layer_norm(x, self.norms[-2], self.norms[-1])


def sinusoids(rows, d, first=0, ln_timescale=math.log(10000.0), scale=1.0) -> np.ndarray:
    """sinusoids (src/layers.rs:257-270): row p is [sin | cos] of
    (first + p) * exp(-i * ln_timescale / (d/2 - 1)) for i < d/2, times
    scale, in float64 (the C library's sin, cos and exp, as Rust's f64
    calls them), then rounded to f32."""
    half = d // 2
    inc = ln_timescale / (half - 1.0)
    steps = [math.exp(-inc * i) for i in range(half)]
    out = np.zeros((rows, d), np.float32)
    for p in range(rows):
        pos = float(first + p)
        out[p, :half] = [math.sin(pos * e) * scale for e in steps]
        out[p, half:] = [math.cos(pos * e) * scale for e in steps]
    return out


def half_len(n):
    """Length after one kernel-3, stride-2, padding-1 convolution
    (qwen3_asr.rs:120-123): n / 2 rounded up."""
    return (n + 1) // 2


def conv2d_columns(m, bins, times, channels) -> np.ndarray:
    """conv2d's im2col (src/models/families/qwen3_asr.rs:408-428): a 3x3,
    stride-2, padding-1 convolution over a [bin][time][channel] map. Row
    bin' * times' + time' holds map[2 bin' + dy - 1][2 time' + dx - 1][c]
    at column c * 9 + 3 dy + dx, zero outside the map."""
    ob, ot = half_len(bins), half_len(times)
    m = np.asarray(m, np.float32).reshape(bins, times, channels)
    pad = np.zeros((bins + 2, times + 2, channels), np.float32)
    pad[1:-1, 1:-1] = m
    cols = np.empty((ob, ot, channels, 9), np.float32)
    for dy in range(3):
        for dx in range(3):
            cols[:, :, :, 3 * dy + dx] = pad[dy:dy + 2 * ob:2, dx:dx + 2 * ot:2, :]
    return cols.reshape(ob * ot, channels * 9)


class AsrEncoder:
    """The Qwen3-ASR audio encoder (AudioEncoder::encode and ::chunk,
    src/models/families/qwen3_asr.rs:321-405) composed of the oracle's
    pieces. The frames are cut into chunks of cfg["chunk"] (the last one
    shorter) and every chunk is zero padded to the longest; per chunk the
    [bin][time] map goes through three 3x3 stride-2 convolutions, each
    followed by GELU, then per time step the channel-major columns
    (channel * bins + bin) through conv_out, plus the sinusoid positions of
    the chunk's time steps; the kept rows (half^3 of each chunk's real
    length) are laid end to end. Per layer a pre-norm attention block whose
    rows see only the rows of their window (half^3(longest) *
    window_chunks rows) and a pre-norm GELU MLP; then ln_post, proj1, GELU,
    proj2. `products` are callables x -> x W^T + bias: the three
    convolutions, conv_out, then qkv, out, fc1, fc2 of each layer, then
    proj1 and proj2; `norms` per layer (attn w, b, ffn w, b), then ln_post's
    (w, b)."""

    def __init__(self, cfg, products, norms, positions=None):
        self.cfg, self.products, self.norms = cfg, products, norms
        self.positions = (sinusoids(cfg["max_positions"], cfg["d"]) if positions is None
                          else np.asarray(positions, np.float32))

    def rows(self, frames):
        c = self.cfg["chunk"]
        return sum(half_len(half_len(half_len(min(c, frames - s)))) for s in range(0, frames, c))

    def chunk(self, mel, frames):
        c = self.cfg
        length = mel.shape[0]
        m = np.zeros((c["mels"], frames), np.float32)
        m[:, :length] = mel.T
        bins, times, channels = c["mels"], frames, 1
        for conv in self.products[:3]:
            m = gelu(conv(conv2d_columns(m, bins, times, channels)))
            bins, times, channels = half_len(bins), half_len(times), m.shape[1]
        cols = m.reshape(bins, times, channels).transpose(1, 2, 0).reshape(times, channels * bins)
        return (self.products[3](np.ascontiguousarray(cols)) + self.positions[:times]).astype(np.float32)

    def encode(self, mel, frames):
        c = self.cfg
        d, heads = c["d"], c["heads"]
        mel = np.ascontiguousarray(mel, np.float32).reshape(frames, c["mels"])
        spans = [(s, min(c["chunk"], frames - s)) for s in range(0, frames, c["chunk"])]
        longest = max(n for _, n in spans)
        x = np.concatenate([self.chunk(mel[s:s + n], longest)[:half_len(half_len(half_len(n)))]
                            for s, n in spans]).astype(np.float32)
        t = x.shape[0]
        window = half_len(half_len(half_len(longest))) * c["window_chunks"]
        hd = d // heads
        for l in range(c["layers"]):
            qkv_p, out_p, fc1_p, fc2_p = self.products[4 + 4 * l:8 + 4 * l]
            aw, ab, fw, fb = self.norms[4 * l:4 * l + 4]
            qkv = qkv_p(layer_norm(x, aw, ab))
            att = np.empty((t, d), np.float32)
            for s in range(0, t, window):
                r = qkv[s:s + min(window, t - s)]
                att[s:s + r.shape[0]] = attention(r[:, :d], r[:, d:2 * d], r[:, 2 * d:], heads, heads, hd,
                                                  causal=False)
            x = (x + out_p(att)).astype(np.float32)
            x = (x + fc2_p(gelu(fc1_p(layer_norm(x, fw, fb))))).astype(np.float32)
        h = gelu(self.products[-2](layer_norm(x, self.norms[-2], self.norms[-1])))
        return self.products[-1](h).astype(np.float32)


def f32_to_f16(values) -> np.ndarray:
    """f32_to_f16 (src/cpu/tensors.rs:542-573) of every value: f16 bits."""
    v = np.ascontiguousarray(values, np.float32).reshape(-1)
    out = np.empty(v.size, np.uint16)
    lib().or_f32_to_f16_n(ptr(v), v.size, ptr(out))
    return out


def f16_to_f32(bits) -> np.ndarray:
    """f16_to_f32 (src/cpu/tensors.rs:575-595) of every f16 bit pattern."""
    b = np.ascontiguousarray(bits, np.uint16).reshape(-1)
    out = np.empty(b.size, np.float32)
    lib().or_f16_to_f32_n(ptr(b), b.size, ptr(out))
    return out


def f16_boundaries() -> np.ndarray:
    """Every f32 value where f32 -> f16 rounding can turn: each finite f16
    value, and the midpoint to the next one in magnitude with its f32
    neighbours (ties to even, the subnormal steps, the overflow edge at
    65520); then +-0, +-inf and NaNs."""
    h = np.arange(0x7C00, dtype=np.uint32)  # non-negative finite f16 values
    lo = h.astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)  # 0x7C00 is +inf
    hi[-1] = 65520.0 * 2 - 65504.0  # the step above 65504 (its midpoint is 65520)
    mid = ((lo + hi) / 2).astype(np.float32)  # exact in f32
    mb = mid.view(np.uint32)
    vals = np.concatenate([lo.astype(np.float32).view(np.uint32), mb - 1, mb, mb + 1])
    vals = np.unique(vals)
    vals = np.concatenate([vals, vals | np.uint32(0x80000000)])
    special = np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F800001, 0x477FF000, 0x477FEFFF,
                        0x00000001, 0x80000001, 0x33000000, 0x33000001, 0x387FE000], np.uint32)
    return np.concatenate([vals, special]).view(np.float32)


GGML_BLOCKS = {2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def ggml_expand(ggml_type: int, blocks: np.ndarray) -> np.ndarray:
    """ggml's block types (Q4_0 2, Q4_1 3, Q5_0 6, Q5_1 7, Q4_K 12, Q5_K 13,
    Q6_K 14) as f32 (src/cpu/ggml_quants.rs:103-245)."""
    values, size = GGML_BLOCKS[ggml_type]
    b = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    nb = b.size // size
    out = np.empty(nb * values, np.float32)
    assert lib().or_ggml_expand(ggml_type, ptr(b), nb, ptr(out)) == 0
    return out


def q4_k_expand(blocks: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    nb = b.size // 144
    out = np.empty(nb * 256, np.float32)
    lib().or_q4_k_expand(ptr(b), nb, ptr(out))
    return out


class Int8:
    def __init__(self, codes, scales, group: int, half_scales: bool, isa: int = SCALAR):
        codes = np.ascontiguousarray(codes, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        self.n, self.k = codes.shape
        self.h = lib().or_int8_new(isa, self.n, self.k, group, int(half_scales), ptr(codes), ptr(scales))
        assert self.h

    def __call__(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.k)
        out = np.empty((x.shape[0], self.n), np.float32)
        lib().or_int8_forward(self.h, ptr(x), x.shape[0], ptr(out))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_int8_free(self.h)


class Ternary:
    def __init__(self, codes, scales, isa: int = SCALAR):
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        self.n, self.k = codes.shape
        self.h = lib().or_ternary_new(isa, self.n, self.k, ptr(codes), ptr(scales))
        assert self.h

    def __call__(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.k)
        out = np.empty((x.shape[0], self.n), np.float32)
        lib().or_ternary_forward(self.h, ptr(x), x.shape[0], ptr(out))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_ternary_free(self.h)


def matmul_f16(x, w_bits, isa: int = SCALAR):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w_bits, np.uint16)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    lib().or_matmul_f16(isa, ptr(x), m, k, ptr(w), n, ptr(out))
    return out


def matmul_f32(x, w, isa: int = SCALAR):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    lib().or_matmul_f32(isa, ptr(x), m, k, ptr(w), n, ptr(out))
    return out


def rmsnorm(x, weight, eps):
    x = np.array(x, np.float32, copy=True, order="C")
    w = np.ascontiguousarray(weight, np.float32)
    d = w.size
    lib().or_rmsnorm(ptr(w), d, eps, ptr(x), x.size // d)
    return x


def rope_table(dims, base, positions):
    s = np.empty((positions, dims // 2), np.float32)
    c = np.empty((positions, dims // 2), np.float32)
    lib().or_rope_table(dims, base, positions, ptr(s), ptr(c))
    return s, c


def attention(q, k, v, heads, kv_heads, hd, causal=True):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    tq, tk = q.shape[0], k.shape[0]
    out = np.empty((tq, heads * hd), np.float32)
    lib().or_attention(ptr(q), q.shape[1], ptr(k), ptr(v), k.shape[1], tq, tk, heads, kv_heads, hd, int(causal),
                       ptr(out))
    return out


def attention_steps(q, caches, heads, kv_heads):
    """layers::attention_steps (src/layers.rs:505-562). For sequence b it
    makes the calls attention_with (src/layers.rs:442-504) makes for one
    query row that sees every key: qh = q * (1/sqrt(hd)), matmul_nn_into for
    the scores, softmax_rows over all tk keys, matmul_nn_into for p.V. So
    each output row is the oracle's attention of that row alone over the
    sequence's keys (tq = 1; causal or not, the row sees all tk keys)."""
    q = np.ascontiguousarray(q, np.float32)
    kvs = np.asarray(caches[0][0]).shape[1]
    hd = kvs // kv_heads
    d = heads * hd
    out = np.empty((q.shape[0], d), np.float32)
    for b, (k, v) in enumerate(caches):
        out[b] = attention(q[b:b + 1, :d], k, v, heads, kv_heads, hd, causal=False)[0]
    return out


def exp(x: float) -> float:
    return lib().or_exp(x)


def silu(x):
    x = np.array(x, np.float32, copy=True, order="C")
    lib().or_silu(ptr(x), x.size)
    return x


def argmax(v) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return lib().or_argmax(ptr(v), v.size)


class Lm:
    """CausalLm (src/models/parts/causal_lm.rs:93-481) with Q8_0 linears and
    a tied f16 table; kv_f16 rounds each appended key and value through f16
    (the device's f16 caches). Granite's multipliers come from cfg
    (embedding_multiplier, attention_multiplier, residual_multiplier,
    logits_scaling); other linear and table kinds are set afterwards."""

    def __init__(self, cfg: dict, weights, isa: int = SCALAR, kv_f16: bool = False):
        c = LmConfig(cfg["d"], cfg["ffn"], cfg["layers"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                     cfg["vocab"], cfg["eps"], cfg["rope_base"], int(cfg.get("qk_norm", 1)), int(kv_f16),
                     cfg.get("embedding_multiplier", 1.0), cfg.get("attention_multiplier") or 0.0,
                     cfg.get("residual_multiplier", 1.0), cfg.get("logits_scaling", 1.0))
        self.cfg = cfg
        self.h = lib().or_lm_new(isa, C.byref(c))
        assert self.h
        for li, L in enumerate(weights.layers):
            rc = lib().or_lm_set_layer(self.h, li, ptr(L.qkv), ptr(L.o), ptr(L.gate_up), ptr(L.down),
                                       ptr(L.norm_attn), ptr(L.norm_mlp), ptr(L.q_norm), ptr(L.k_norm))
            assert rc == 0
        assert lib().or_lm_set_embed(self.h, ptr(weights.embed), ptr(weights.final_norm)) == 0

    def set_linear_int8(self, layer, which, codes, scales):
        """Linear `which` (0 qkv, 1 o, 2 gate_up, 3 down) as Trit's int8
        weights (one f32 scale per row and 128 inputs)."""
        codes = np.ascontiguousarray(codes, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        assert lib().or_lm_set_linear_int8(self.h, layer, which, ptr(codes), ptr(scales)) == 0

    def set_linear_float(self, layer, which, weights):
        """Linear `which` as f32 or f16-bits (uint16) weights, f32 math."""
        w = np.ascontiguousarray(weights)
        kind = TABLE_F16 if w.dtype == np.uint16 else TABLE_F32
        w = np.ascontiguousarray(w, np.uint16 if kind == TABLE_F16 else np.float32)
        assert lib().or_lm_set_linear_float(self.h, layer, which, kind, ptr(w)) == 0

    def set_table(self, which, kind, data, scales=None):
        """Table 0 (the embedding) or 1 (the untied head; None ties it)."""
        if data is None:
            assert lib().or_lm_set_table(self.h, which, kind, None, None) == 0
            return
        dt = {TABLE_F16: np.uint16, TABLE_F32: np.float32, TABLE_Q8: np.int8}[kind]
        data = np.ascontiguousarray(data, dt)
        sc = None if scales is None else np.ascontiguousarray(scales, np.float32)
        assert lib().or_lm_set_table(self.h, which, kind, ptr(data), ptr(sc) if sc is not None else None) == 0
        self._keep = getattr(self, "_keep", []) + [data]

    def set_ffn_scales(self, scales):
        if scales is None:
            assert lib().or_lm_set_ffn_scales(self.h, None) == 0
            return
        s = np.ascontiguousarray(scales, np.float32)
        assert lib().or_lm_set_ffn_scales(self.h, ptr(s)) == 0

    def generate(self, prompt, max_new, stop=()):
        prompt = np.ascontiguousarray(prompt, np.int32)
        stop = np.ascontiguousarray(np.array(stop, np.int32).reshape(-1))
        out = np.empty(max(max_new, 1), np.int32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        n = lib().or_lm_generate(self.h, ptr(prompt), prompt.size, max_new, ptr(stop) if stop.size else None,
                                 stop.size, ptr(out), ptr(logits))
        assert n >= 0
        return out[:n].copy(), logits

    def reset(self):
        lib().or_lm_reset(self.h)

    def truncate(self, position):
        assert lib().or_lm_truncate(self.h, position) == 0

    @property
    def position(self):
        return lib().or_lm_position(self.h)

    def forward(self, tokens):
        tokens = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.cfg["vocab"], np.float32)
        assert lib().or_lm_forward(self.h, ptr(tokens), tokens.size, ptr(logits)) == 0
        return logits

    def forward_rows(self, rows):
        rows = np.ascontiguousarray(rows, np.float32).reshape(-1, self.cfg["d"])
        logits = np.empty(self.cfg["vocab"], np.float32)
        assert lib().or_lm_forward_rows(self.h, ptr(rows), rows.shape[0], ptr(logits)) == 0
        return logits

    def embed_row(self, token):
        out = np.empty(self.cfg["d"], np.float32)
        assert lib().or_lm_embed_row(self.h, int(token), ptr(out)) == 0
        return out

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_lm_free(self.h)
