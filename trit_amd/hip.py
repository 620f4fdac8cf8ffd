"""ctypes driver of libtrit_hip.so, shaped like Trit's Rust interface.

`Dense` mirrors src/cpu/gemm.rs's Dense (constructors per weight kind,
`forward(x, rows)`, `row(index)`); `CausalLm` and `Session` mirror
src/models/parts/causal_lm.rs (`generate`, `forward`, `greedy`). Every call
goes through the C ABI; there is no CPU fallback: a missing library or a
failed call raises.
"""

from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# TRIT_HIP_LIBRARY names another build of the library (the measurement
# build with the step's phase stamps: lib/libtrit_hip_stamps.so).
LIB_PATH = os.environ.get("TRIT_HIP_LIBRARY") or os.path.join(HERE, "lib", "libtrit_hip.so")

Q8_0, INT8, TERNARY, Q4_K, F16, F32, Q8 = 1, 2, 3, 4, 5, 6, 7
EXACT, KV_F32, TREE_SUMS = 1, 2, 4

_lib = None


class TritError(RuntimeError):
    pass


class LmConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("d", "ffn", "layers", "heads", "kv_heads", "head_dim", "vocab")] + [
        ("eps", C.c_float), ("rope_base", C.c_float), ("qk_norm", C.c_int),
        ("embedding_multiplier", C.c_float), ("attention_multiplier", C.c_float),
        ("residual_multiplier", C.c_float), ("logits_scaling", C.c_float)]

    @classmethod
    def of(cls, cfg: dict) -> "LmConfig":
        """From a config dict; Granite's keys as in causal_lm.rs:58-61
        (missing: 1, and no attention multiplier)."""
        return cls(cfg["d"], cfg["ffn"], cfg["layers"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                   cfg["vocab"], cfg["eps"], cfg["rope_base"], int(cfg.get("qk_norm", 1)),
                   cfg.get("embedding_multiplier", 1.0), cfg.get("attention_multiplier") or 0.0,
                   cfg.get("residual_multiplier", 1.0), cfg.get("logits_scaling", 1.0))


class EncoderConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("d", "layers", "heads", "ffn", "mels", "positions")]


ASR_FIELDS = ("d", "layers", "heads", "ffn", "mels", "channels", "chunk", "window_chunks", "out", "max_positions")


class AsrEncoderConfig(C.Structure):
    _fields_ = [(n, C.c_int) for n in ASR_FIELDS]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise TritError(f"{LIB_PATH} is missing: build it with `python -m trit_amd.build`")
        L = C.CDLL(LIB_PATH)
        p, i, f = C.c_void_p, C.c_int, C.c_float
        pp = C.POINTER(C.c_void_p)
        sig = {
            "trit_hip_version": (C.c_char_p, []),
            "trit_hip_step_stamps": (i, [i, i]),
            "trit_hip_step_stamps_read": (i, [p, p, i]),
            "trit_hip_last_error": (C.c_char_p, []),
            "trit_hip_init": (i, [i]),
            "trit_hip_layer_q8_0": (i, [i, i, p, p, pp]),
            "trit_hip_layer_int8": (i, [i, i, p, p, p, pp]),
            "trit_hip_layer_ternary": (i, [i, i, p, p, pp]),
            "trit_hip_layer_ternary_base3": (i, [i, i, p, p, pp]),
            "trit_hip_layer_q4_k": (i, [i, i, p, pp]),
            "trit_hip_layer_f16": (i, [i, i, p, p, pp]),
            "trit_hip_layer_f32": (i, [i, i, p, p, pp]),
            "trit_hip_layer_q8": (i, [i, i, p, p, p, pp]),
            "trit_hip_layer_q8_0_f32": (i, [i, i, p, p, pp]),
            "trit_hip_layer_ggml": (i, [i, i, i, p, p, i, pp]),
            "trit_hip_layer_forward": (i, [p, p, i, i, p]),
            "trit_hip_layer_forward_device": (i, [p, p, i, i, p, p]),
            "trit_hip_layer_forward_device_noalloc": (i, [p, p, i, i, p, p]),
            "trit_hip_layer_forward_timed": (i, [p, p, i, i, p, p, p, p]),
            "trit_hip_layer_info": (i, [p, C.POINTER(i), C.POINTER(i), C.POINTER(i), C.POINTER(C.c_int64)]),
            "trit_hip_layer_row": (i, [p, i, p]),
            "trit_hip_layer_free": (None, [p]),
            "trit_hip_decoder_new": (i, [C.POINTER(LmConfig), p, p, p, p, pp]),
            "trit_hip_decoder_free": (None, [p]),
            "trit_hip_decoder_save": (i, [p, C.c_char_p]),
            "trit_hip_decoder_load": (i, [C.c_char_p, C.POINTER(LmConfig), pp]),
            "trit_hip_decoder_set_ffn_scales": (i, [p, p]),
            "trit_hip_session_generate_additive": (i, [p, p, i, p, i, p, i, p]),
            "trit_hip_prefix_new": (i, [p, p, i, i, pp]),
            "trit_hip_prefix_free": (None, [p]),
            "trit_hip_session_prefill_prefixed": (i, [p, p, p, i, p]),
            "trit_hip_session_new": (i, [p, i, i, pp]),
            "trit_hip_session_prefill": (i, [p, p, i, p]),
            "trit_hip_session_prefill_rows": (i, [p, p, i, p]),
            "trit_hip_session_generate": (i, [p, i, p, i, p]),
            "trit_hip_session_generate_timed": (i, [p, i, p, i, p, p, p, p]),
            "trit_hip_session_reset": (i, [p]),
            "trit_hip_session_position": (i, [p]),
            "trit_hip_session_free": (None, [p]),
            "trit_hip_gguf_open": (i, [C.c_char_p, pp]),
            "trit_hip_gguf_free": (None, [p]),
            "trit_hip_gguf_tensor_count": (i, [p]),
            "trit_hip_gguf_tensor": (i, [p, i, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p), C.POINTER(i),
                                         C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
            "trit_hip_gguf_meta_u64": (i, [p, C.c_char_p, C.POINTER(C.c_uint64)]),
            "trit_hip_gguf_meta_f64": (i, [p, C.c_char_p, C.POINTER(C.c_double)]),
            "trit_hip_gguf_meta_str": (i, [p, C.c_char_p, C.POINTER(C.c_char_p)]),
            "trit_hip_decoder_from_gguf": (i, [C.c_char_p, C.c_char_p, C.POINTER(LmConfig), pp]),
            "trit_hip_attention": (i, [p, i, p, p, i, i, i, i, i, i, i, i, p]),
            "trit_hip_f32_to_f16": (i, [p, C.c_int64, p]),
            "trit_hip_f16_to_f32": (i, [p, C.c_int64, p]),
            "trit_hip_encoder_new": (i, [C.POINTER(EncoderConfig), p, p, p, p, p, pp]),
            "trit_hip_asr_encoder_new": (i, [C.POINTER(AsrEncoderConfig), p, p, p, p, p, p, pp]),
            "trit_hip_asr_encoder_free": (None, [p]),
            "trit_hip_asr_encoder_rows": (i, [p, i]),
            "trit_hip_asr_encoder_positions": (i, [p, p]),
            "trit_hip_asr_encoder_encode": (i, [p, p, i, p]),
            "trit_hip_encoder_free": (None, [p]),
            "trit_hip_encoder_encode": (i, [p, p, p]),
            "trit_hip_bpe_open": (i, [C.c_char_p, pp]),
            "trit_hip_bpe_parse": (i, [C.c_char_p, C.c_size_t, pp]),
            "trit_hip_bpe_free": (None, [p]),
            "trit_hip_bpe_id": (i, [p, C.c_char_p]),
            "trit_hip_bpe_encode": (i, [p, C.c_char_p, C.c_size_t, i, p, i]),
            "trit_hip_bpe_decode": (C.c_int64, [p, p, i, p, C.c_size_t]),
            "trit_hip_cleanup_system": (i, [p, p, i]),
            "trit_hip_cleanup_prompt": (i, [p, C.c_char_p, C.c_size_t, i, i, i, p, i]),
            "trit_hip_cleanup_parts": (C.c_int64, [p, C.c_char_p, C.c_size_t, i, p, C.c_size_t]),
            "trit_hip_attention_steps": (i, [p, i, p, p, p, i, i, i, i, p]),
            "trit_hip_attention_steps_device": (i, [p, i, p, p, p, i, i, i, i, p, p]),
        }
        for name, (res, args) in sig.items():
            if not hasattr(L, name):
                continue
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc is None or (isinstance(rc, int) and rc < 0):
        raise TritError(lib().trit_hip_last_error().decode())
    return rc


def ptr(a):
    if a is None:
        return None
    assert a.flags.c_contiguous
    return a.ctypes.data_as(C.c_void_p)


def init(device: int = 0):
    check(lib().trit_hip_init(device))


def attention(q, k, v, heads, kv_heads, hd, causal=True, flags=0):
    """layers::attention (src/layers.rs:343-504) on the device: q tq x qs,
    k and v tk x kvs f32 rows; returns tq x (heads * hd)."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty((q.shape[0], heads * hd), np.float32)
    check(lib().trit_hip_attention(ptr(q), q.shape[1], ptr(k), ptr(v), k.shape[1], q.shape[0], k.shape[0], heads,
                                   kv_heads, hd, int(causal), flags, ptr(out)))
    return out


def f32_to_f16(values):
    """f32 -> f16 bits on the device (trit_hip_f32_to_f16)."""
    v = np.ascontiguousarray(values, np.float32).reshape(-1)
    out = np.empty(v.size, np.uint16)
    check(lib().trit_hip_f32_to_f16(ptr(v), v.size, ptr(out)))
    return out


def f16_to_f32(bits):
    """f16 bits -> f32 on the device (trit_hip_f16_to_f32)."""
    b = np.ascontiguousarray(bits, np.uint16).reshape(-1)
    out = np.empty(b.size, np.float32)
    check(lib().trit_hip_f16_to_f32(ptr(b), b.size, ptr(out)))
    return out


def attention_steps(q, caches, heads, kv_heads):
    """layers::attention_steps (src/layers.rs:505-562) on the device: row b
    of q (sequences x qs) asks sequence b's cache (keys, values), each
    tk_b x (kv_heads * hd) f32; returns sequences x d, d = heads * hd."""
    q = np.ascontiguousarray(q, np.float32)
    sequences = q.shape[0]
    assert len(caches) == sequences
    ks = [np.ascontiguousarray(k, np.float32) for k, _ in caches]
    vs = [np.ascontiguousarray(v, np.float32) for _, v in caches]
    kvs = ks[0].shape[1]
    d = kvs // kv_heads * heads
    keys = (C.c_void_p * sequences)(*[k.ctypes.data for k in ks])
    values = (C.c_void_p * sequences)(*[v.ctypes.data for v in vs])
    tk = (C.c_int * sequences)(*[k.shape[0] for k in ks])
    out = np.empty((sequences, d), np.float32)
    check(lib().trit_hip_attention_steps(ptr(q), q.shape[1], keys, values, tk, sequences, d, heads, kv_heads,
                                         ptr(out)))
    return out


class Dense:
    """A layer on the device (src/cpu/gemm.rs:15-35)."""

    def __init__(self, handle, n, k):
        self.h, self.n, self.k = handle, n, k

    @staticmethod
    def _make(fn, n, k, *args):
        out = C.c_void_p()
        check(fn(n, k, *args, C.byref(out)))
        return Dense(out, n, k)

    @classmethod
    def q8_0(cls, n, k, blocks, bias=None):
        blocks = np.ascontiguousarray(blocks, np.uint8)
        assert blocks.size == n * k // 32 * 34
        bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        return cls._make(lib().trit_hip_layer_q8_0, n, k, ptr(blocks), ptr(bias))

    @classmethod
    def int8(cls, codes, scales, bias=None):
        codes = np.ascontiguousarray(codes, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        n, k = codes.shape
        return cls._make(lib().trit_hip_layer_int8, n, k, ptr(codes), ptr(scales), ptr(bias))

    @classmethod
    def ternary(cls, codes, scales):
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        n, k = codes.shape
        return cls._make(lib().trit_hip_layer_ternary, n, k, ptr(codes), ptr(scales))

    @classmethod
    def ternary_base3(cls, n, k, packed, scales):
        packed = np.ascontiguousarray(packed, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        return cls._make(lib().trit_hip_layer_ternary_base3, n, k, ptr(packed), ptr(scales))

    @classmethod
    def q4_k(cls, n, k, blocks):
        blocks = np.ascontiguousarray(blocks, np.uint8)
        assert blocks.size == n * k // 256 * 144
        return cls._make(lib().trit_hip_layer_q4_k, n, k, ptr(blocks))

    @classmethod
    def f16(cls, weights_bits, bias=None):
        w = np.ascontiguousarray(weights_bits, np.uint16)
        bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        n, k = w.shape
        return cls._make(lib().trit_hip_layer_f16, n, k, ptr(w), ptr(bias))

    @classmethod
    def f32(cls, weights, bias=None):
        """Dense::new (f32 weights, f32 math)."""
        w = np.ascontiguousarray(weights, np.float32)
        bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        n, k = w.shape
        return cls._make(lib().trit_hip_layer_f32, n, k, ptr(w), ptr(bias))

    @classmethod
    def q8(cls, codes, scales, bias=None):
        """Weights::Q8: int8 storage, an f32 scale per 32 values, f32 math."""
        codes = np.ascontiguousarray(codes, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        n, k = codes.shape
        return cls._make(lib().trit_hip_layer_q8, n, k, ptr(codes), ptr(scales), ptr(bias))

    @classmethod
    def q8_0_f32(cls, n, k, blocks, bias=None):
        """Q8_0 blocks with f32 math (Dense::table under Q8_0)."""
        blocks = np.ascontiguousarray(blocks, np.uint8)
        assert blocks.size == n * k // 32 * 34
        bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        return cls._make(lib().trit_hip_layer_q8_0_f32, n, k, ptr(blocks), ptr(bias))

    @classmethod
    def ggml(cls, n, k, ggml_type, blocks, bias=None, f32_math=False):
        """A GGUF tensor of ggml type `ggml_type` as Trit loads it under Auto
        precision (trit_hip_layer_ggml)."""
        blocks = np.ascontiguousarray(blocks, np.uint8)
        bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
        return cls._make(lib().trit_hip_layer_ggml, n, k, ggml_type, ptr(blocks), ptr(bias), int(f32_math))

    def forward(self, x, rows=None, relu=False):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.k)
        m = x.shape[0] if rows is None else rows
        y = np.empty((m, self.n), np.float32)
        check(lib().trit_hip_layer_forward(self.h, ptr(x), m, int(relu), ptr(y)))
        return y

    def row(self, index):
        out = np.empty(self.k, np.float32)
        check(lib().trit_hip_layer_row(self.h, index, ptr(out)))
        return out

    def info(self):
        n, k, kind, b = C.c_int(), C.c_int(), C.c_int(), C.c_int64()
        check(lib().trit_hip_layer_info(self.h, C.byref(n), C.byref(k), C.byref(kind), C.byref(b)))
        return {"n": n.value, "k": k.value, "kind": kind.value, "bytes": b.value}

    def free(self):
        if self.h:
            lib().trit_hip_layer_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class CausalLm:
    """The decoder on the device (src/models/parts/causal_lm.rs:93-481)."""

    def __init__(self, cfg: dict, linears, norms, embed: Dense, head: Dense | None = None):
        c = LmConfig.of(cfg)
        self.cfg = cfg
        arr = (C.c_void_p * len(linears))(*[l.h for l in linears])
        norms = np.ascontiguousarray(norms, np.float32)
        out = C.c_void_p()
        check(lib().trit_hip_decoder_new(C.byref(c), arr, ptr(norms), embed.h, head.h if head else None,
                                         C.byref(out)))
        self.h = out

    @classmethod
    def from_gguf(cls, path, prefix=None):
        """The decoder of a GGUF file (trit_hip_decoder_from_gguf)."""
        self = cls.__new__(cls)
        c = LmConfig()
        out = C.c_void_p()
        check(lib().trit_hip_decoder_from_gguf(str(path).encode(), prefix.encode() if prefix else None,
                                               C.byref(c), C.byref(out)))
        self.h = out
        self.cfg = cls._cfg_of(c)
        return self

    def save(self, path):
        """The device layouts to a weight-cache file (trit_hip_decoder_save)."""
        check(lib().trit_hip_decoder_save(self.h, str(path).encode()))

    @classmethod
    def load(cls, path):
        """A decoder from a weight-cache file (trit_hip_decoder_load)."""
        self = cls.__new__(cls)
        c = LmConfig()
        out = C.c_void_p()
        check(lib().trit_hip_decoder_load(str(path).encode(), C.byref(c), C.byref(out)))
        self.h = out
        self.cfg = cls._cfg_of(c)
        return self

    @staticmethod
    def _cfg_of(c):
        return dict(d=c.d, ffn=c.ffn, layers=c.layers, heads=c.heads, kv_heads=c.kv_heads, head_dim=c.head_dim,
                    vocab=c.vocab, eps=c.eps, rope_base=c.rope_base, qk_norm=c.qk_norm,
                    embedding_multiplier=c.embedding_multiplier, attention_multiplier=c.attention_multiplier or None,
                    residual_multiplier=c.residual_multiplier, logits_scaling=c.logits_scaling)

    def session(self, max_positions, flags=0):
        return Session(self, max_positions, flags)

    def generate(self, prompt, max_new, stop=(), flags=0, prefix=None):
        """CausalLm::generate (causal_lm.rs:217-249); `prefix` a Prefix of
        this decoder made with the same flags, or None."""
        s = self.session(len(prompt) + max_new + 1, flags)
        try:
            if prefix is None:
                s.prefill(prompt, want_logits=False)
            else:
                s.prefill_prefixed(prefix, prompt, want_logits=False)
            return s.generate(max_new, stop)
        finally:
            s.free()

    def prefix(self, tokens, flags=0):
        """CausalLm::prefix (causal_lm.rs:200-215): the keys and values of a
        prompt start that many calls share."""
        return Prefix(self, tokens, flags)

    def set_ffn_scales(self, scales):
        """CausalLm::set_ffn_scales (causal_lm.rs:304-307): layers x d
        scales on each layer's normed MLP input, or None."""
        if scales is None:
            check(lib().trit_hip_decoder_set_ffn_scales(self.h, None))
            return
        s = np.ascontiguousarray(scales, np.float32)
        assert s.size == self.cfg["layers"] * self.cfg["d"]
        check(lib().trit_hip_decoder_set_ffn_scales(self.h, ptr(s)))

    def generate_additive(self, prompt, audio, stop=(), flags=0):
        """CausalLm::generate_additive (causal_lm.rs:313-345): greedy tokens
        with audio rows (rows x d) added to every input."""
        audio = np.ascontiguousarray(audio, np.float32).reshape(-1, self.cfg["d"])
        s = self.session(max(audio.shape[0], 1), flags)
        try:
            return s.generate_additive(prompt, audio, stop)
        finally:
            s.free()

    def free(self):
        if self.h:
            lib().trit_hip_decoder_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Encoder:
    """Whisper's audio encoder on the device (src/models/parts/audio_encoder.rs):
    conv1 (d x 3 mels), conv2 (d x 3 d), then qkv, out, fc1, fc2 of each
    layer, as Dense layers with their biases; positions (positions x d);
    norms per layer attn w, b, ffn w, b, then the final w, b."""

    def __init__(self, cfg: dict, conv1: Dense, conv2: Dense, positions, linears, norms):
        c = EncoderConfig(*(cfg[k] for k in ("d", "layers", "heads", "ffn", "mels", "positions")))
        self.cfg = cfg
        pos = np.ascontiguousarray(positions, np.float32)
        arr = (C.c_void_p * len(linears))(*[l.h for l in linears])
        nrm = np.ascontiguousarray(np.concatenate([np.asarray(v, np.float32).reshape(-1) for v in norms]))
        out = C.c_void_p()
        check(lib().trit_hip_encoder_new(C.byref(c), conv1.h, conv2.h, ptr(pos), arr, ptr(nrm), C.byref(out)))
        self.h = out

    def encode(self, mel):
        """Encoder::encode: positions x d of one 2 * positions x mels window."""
        c = self.cfg
        mel = np.ascontiguousarray(mel, np.float32).reshape(2 * c["positions"], c["mels"])
        out = np.empty((c["positions"], c["d"]), np.float32)
        check(lib().trit_hip_encoder_encode(self.h, ptr(mel), ptr(out)))
        return out

    def free(self):
        if self.h:
            lib().trit_hip_encoder_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class AsrEncoder:
    """The Qwen3-ASR audio encoder on the device (src/models/families/
    qwen3_asr.rs:284-405): convs (conv2d1, conv2d2, conv2d3), conv_out,
    then qkv, out, fc1, fc2 of each layer, then proj1 and proj2, as Dense
    layers with their biases; norms per layer attn w, b, ffn w, b, then
    ln_post's w, b. The sinusoid positions are made by the library."""

    def __init__(self, cfg: dict, convs, conv_out: Dense, linears, norms, proj1: Dense, proj2: Dense):
        c = AsrEncoderConfig(*(cfg[k] for k in ASR_FIELDS))
        self.cfg = cfg
        cv = (C.c_void_p * 3)(*[l.h for l in convs])
        arr = (C.c_void_p * len(linears))(*[l.h for l in linears])
        nrm = np.ascontiguousarray(np.concatenate([np.asarray(v, np.float32).reshape(-1) for v in norms]))
        out = C.c_void_p()
        check(lib().trit_hip_asr_encoder_new(C.byref(c), cv, conv_out.h, arr, ptr(nrm), proj1.h, proj2.h,
                                             C.byref(out)))
        self.h = out

    def rows(self, frames: int) -> int:
        return check(lib().trit_hip_asr_encoder_rows(self.h, frames))

    def positions(self):
        c = self.cfg
        out = np.empty((c["max_positions"], c["d"]), np.float32)
        check(lib().trit_hip_asr_encoder_positions(self.h, ptr(out)))
        return out

    def encode(self, mel, frames: int):
        """AudioEncoder::encode: rows x out from frames x mels features."""
        c = self.cfg
        mel = np.ascontiguousarray(mel, np.float32).reshape(frames, c["mels"])
        out = np.empty((self.rows(frames), c["out"]), np.float32)
        check(lib().trit_hip_asr_encoder_encode(self.h, ptr(mel), frames, ptr(out)))
        return out

    def free(self):
        if self.h:
            lib().trit_hip_asr_encoder_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Bpe:
    """Byte-level BPE from a tokenizer.json (src/text/bpe.rs): `encode`,
    `encode_plain`, `decode`, `id`, as Trit's Bpe."""

    def __init__(self, path=None, text=None):
        out = C.c_void_p()
        if text is not None:
            b = text.encode() if isinstance(text, str) else bytes(text)
            check(lib().trit_hip_bpe_parse(b, len(b), C.byref(out)))
        else:
            check(lib().trit_hip_bpe_open(str(path).encode(), C.byref(out)))
        self.h = out

    @staticmethod
    def _ids(call):
        n = check(call(None, 0))
        out = np.empty(max(n, 1), np.int32)
        check(call(ptr(out), n))
        return out[:n].tolist()

    def encode(self, text, plain=False):
        b = text.encode()
        return self._ids(lambda out, cap: lib().trit_hip_bpe_encode(self.h, b, len(b), int(plain), out, cap))

    def encode_plain(self, text):
        return self.encode(text, plain=True)

    def decode(self, ids):
        a = np.ascontiguousarray(ids, np.int32)
        n = check(lib().trit_hip_bpe_decode(self.h, ptr(a), a.size, None, 0))
        buf = C.create_string_buffer(n + 1)
        check(lib().trit_hip_bpe_decode(self.h, ptr(a), a.size, buf, n + 1))
        return buf.raw[:n].decode()

    def id(self, token):
        v = lib().trit_hip_bpe_id(self.h, token.encode())
        return None if v < 0 else v

    def cleanup_system(self):
        """The ids of the cleanup's shared system turn (src/cleanup.rs:156-158)."""
        return self._ids(lambda out, cap: lib().trit_hip_cleanup_system(self.h, out, cap))

    def cleanup_prompt(self, transcript, styling=2, structure=0, context=0):
        """The ids of one cleanup call (Cleaner::clean_part, src/cleanup.rs:280-301)."""
        b = transcript.encode()
        return self._ids(lambda out, cap: lib().trit_hip_cleanup_prompt(self.h, b, len(b), styling, structure,
                                                                        context, out, cap))

    def cleanup_parts(self, transcript, limit=800):
        """Cleaner::parts of the trimmed transcript (src/cleanup.rs:240-278)."""
        b = transcript.encode()
        n = check(lib().trit_hip_cleanup_parts(self.h, b, len(b), limit, None, 0))
        buf = C.create_string_buffer(max(n, 1))
        check(lib().trit_hip_cleanup_parts(self.h, b, len(b), limit, buf, n))
        return [p.decode() for p in buf.raw[:n].split(b"\0")[:-1]]

    def free(self):
        if self.h:
            lib().trit_hip_bpe_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Gguf:
    """A checked GGUF file (trit_hip_gguf_open; Gguf::open,
    src/models/gguf/mod.rs:155-226). Host only."""

    def __init__(self, path):
        out = C.c_void_p()
        check(lib().trit_hip_gguf_open(str(path).encode(), C.byref(out)))
        self.h = out

    def tensors(self):
        """[(name, ggml type name, dims (ne0 first), start, end)] in file order."""
        res = []
        for i in range(check(lib().trit_hip_gguf_tensor_count(self.h))):
            name, dtype, nd = C.c_char_p(), C.c_char_p(), C.c_int()
            dims = (C.c_int64 * 4)()
            start, end = C.c_int64(), C.c_int64()
            check(lib().trit_hip_gguf_tensor(self.h, i, C.byref(name), C.byref(dtype), C.byref(nd), dims,
                                             C.byref(start), C.byref(end)))
            res.append((name.value.decode(), dtype.value.decode(), list(dims[: min(nd.value, 4)]), start.value,
                        end.value))
        return res

    def u64(self, key):
        v = C.c_uint64()
        check(lib().trit_hip_gguf_meta_u64(self.h, key.encode(), C.byref(v)))
        return v.value

    def f64(self, key):
        v = C.c_double()
        check(lib().trit_hip_gguf_meta_f64(self.h, key.encode(), C.byref(v)))
        return v.value

    def str(self, key):
        v = C.c_char_p()
        check(lib().trit_hip_gguf_meta_str(self.h, key.encode(), C.byref(v)))
        return v.value.decode()

    def free(self):
        if self.h:
            lib().trit_hip_gguf_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Prefix:
    """Prefix (causal_lm.rs:118-122,200-215) on the device."""

    def __init__(self, lm: CausalLm, tokens, flags=0):
        self.lm = lm
        self.tokens = np.ascontiguousarray(tokens, np.int32)
        out = C.c_void_p()
        check(lib().trit_hip_prefix_new(lm.h, ptr(self.tokens), self.tokens.size, flags, C.byref(out)))
        self.h = out

    def free(self):
        if self.h:
            lib().trit_hip_prefix_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Session:
    def __init__(self, lm: CausalLm, max_positions, flags=0):
        self.lm = lm
        out = C.c_void_p()
        check(lib().trit_hip_session_new(lm.h, max_positions, flags, C.byref(out)))
        self.h = out

    def prefill(self, tokens, want_logits=True):
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.lm.cfg["vocab"], np.float32) if want_logits else None
        check(lib().trit_hip_session_prefill(self.h, ptr(t), t.size, ptr(logits)))
        return logits

    def prefill_rows(self, rows, want_logits=True):
        r = np.ascontiguousarray(rows, np.float32).reshape(-1, self.lm.cfg["d"])
        logits = np.empty(self.lm.cfg["vocab"], np.float32) if want_logits else None
        check(lib().trit_hip_session_prefill_rows(self.h, ptr(r), r.shape[0], ptr(logits)))
        return logits

    def prefill_prefixed(self, prefix: Prefix, tokens, want_logits=True):
        """The prompt of a fresh session from `prefix`'s caches when it
        starts with the prefix's tokens (trit_hip_session_prefill_prefixed)."""
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.lm.cfg["vocab"], np.float32) if want_logits else None
        check(lib().trit_hip_session_prefill_prefixed(self.h, prefix.h, ptr(t), t.size, ptr(logits)))
        return logits

    def generate_additive(self, prompt, audio, stop=()):
        """trit_hip_session_generate_additive on a fresh session."""
        t = np.ascontiguousarray(prompt, np.int32)
        audio = np.ascontiguousarray(audio, np.float32).reshape(-1, self.lm.cfg["d"])
        stop = np.ascontiguousarray(np.array(stop, np.int32).reshape(-1))
        rows = audio.shape[0]
        out = np.empty(max(rows - t.size + 1, 1), np.int32)
        n = check(lib().trit_hip_session_generate_additive(self.h, ptr(t), t.size, ptr(audio), rows,
                                                           ptr(stop) if stop.size else None, stop.size, ptr(out)))
        return out[:n].copy()

    def generate(self, max_new, stop=()):
        """Greedy tokens (trit_hip_session_generate); `self.persistent` then
        tells whether they ran on the persistent decode step."""
        stop = np.ascontiguousarray(np.array(stop, np.int32).reshape(-1))
        out = np.empty(max(max_new, 1), np.int32)
        persistent = C.c_int(0)
        n = check(lib().trit_hip_session_generate_timed(self.h, max_new, ptr(stop) if stop.size else None,
                                                        stop.size, ptr(out), None, None, C.byref(persistent)))
        self.persistent = bool(persistent.value & 1)
        # On the step: bit 1 when the attention runs on every block, each
        # key/value head's exchanges in one XCD's L2.
        self.step_layout = int(persistent.value)
        return out[:n].copy()

    def reset(self):
        check(lib().trit_hip_session_reset(self.h))

    @property
    def position(self):
        return check(lib().trit_hip_session_position(self.h))

    def free(self):
        if self.h:
            lib().trit_hip_session_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
