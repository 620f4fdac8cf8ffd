"""A float64 statement of the decoder architecture, written from the model
definition (Hugging Face Qwen3ForCausalLM / GraniteForCausalLM), not from
the oracle's C++: test infrastructure that pins the oracle's composition.

Per layer, for hidden states h (rows x d):
    x      = rmsnorm(h) * input_layernorm
    q,k,v  = x Wq^T, x Wk^T, x Wv^T              (heads, kv_heads, kv_heads)
    q,k    = per-head rmsnorm * q_norm / k_norm  (Qwen3 only)
    q,k    = rotary with rotate_half: pairs (i, i + hd/2),
             angle = position * theta^(-2i/hd)
    q      = q * attention scale (Granite's attention_multiplier, else
             1/sqrt(hd))
    scores = q k^T over the visible keys (causal), query head h reads key
             head h // (heads / kv_heads) (repeat_kv)
    h      = h + residual_multiplier * (softmax(scores) v) Wo^T
    x      = rmsnorm(h) * post_attention_layernorm (* ffn scale)
    h      = h + residual_multiplier * (silu(x Wgate^T) * (x Wup^T)) Wdown^T
logits = rmsnorm(h_last) * norm  Head^T / logits_scaling, with h starting
at embed[tokens] * embedding_multiplier.

`mistake` plants one plausible slip (to show that a check built on this
model fails for it): "swap_gate_up", "interleaved_rope", "mod_head_map",
"no_causal", "kv_f16_off".
"""

from __future__ import annotations

import numpy as np


def rmsnorm(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def silu(x):
    return x / (1.0 + np.exp(-x))


def rotary(x, positions, theta, mistake=None):
    """x: rows x heads x hd (float64)."""
    hd = x.shape[-1]
    half = hd // 2
    inv = theta ** (-np.arange(0, hd, 2, dtype=np.float64) / hd)
    ang = positions[:, None].astype(np.float64) * inv[None, :]
    cos, sin = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    if mistake == "interleaved_rope":
        a, b = x[..., 0::2], x[..., 1::2]
        out = np.empty_like(x)
        out[..., 0::2] = a * cos - b * sin
        out[..., 1::2] = b * cos + a * sin
        return out
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * cos - b * sin, b * cos + a * sin], axis=-1)


class Model:
    """Weights as float64 arrays; `layers` is a list of dicts with q, k, v, o,
    gate, up, down (row-major [out][in]), input_norm, post_norm, q_norm,
    k_norm; `embed` vocab x d; `head` (None: tied); `norm` d."""

    def __init__(self, cfg, layers, embed, norm, head=None, ffn_scales=None, kv_f16=False):
        self.cfg, self.layers, self.embed, self.norm = cfg, layers, embed, norm
        self.head = head
        self.ffn_scales = ffn_scales
        self.kv_f16 = kv_f16
        self.reset()

    def reset(self):
        self.keys = [[] for _ in self.layers]
        self.values = [[] for _ in self.layers]
        self.position = 0

    def forward_tokens(self, tokens, mistake=None):
        return self.forward_rows(self.embed[np.asarray(tokens)], mistake)

    def forward_rows(self, rows, mistake=None):
        c = self.cfg
        d, hd, H, KV = c["d"], c["head_dim"], c["heads"], c["kv_heads"]
        eps = c["eps"]
        h = np.array(rows, np.float64) * c.get("embedding_multiplier", 1.0)
        m = h.shape[0]
        pos = np.arange(self.position, self.position + m)
        att_mult = c.get("attention_multiplier")
        scale = att_mult if att_mult else 1.0 / np.sqrt(hd)
        res = c.get("residual_multiplier", 1.0)
        for li, L in enumerate(self.layers):
            x = rmsnorm(h, L["input_norm"], eps)
            q = (x @ L["q"].T).reshape(m, H, hd)
            k = (x @ L["k"].T).reshape(m, KV, hd)
            v = (x @ L["v"].T).reshape(m, KV, hd)
            if c.get("qk_norm", 1):
                q = rmsnorm(q, L["q_norm"], eps)
                k = rmsnorm(k, L["k_norm"], eps)
            q = rotary(q, pos, c["rope_base"], mistake) * scale
            k = rotary(k, pos, c["rope_base"], mistake)
            if self.kv_f16 and mistake != "kv_f16_off":
                k = k.astype(np.float16).astype(np.float64)
                v = v.astype(np.float16).astype(np.float64)
            self.keys[li].append(k)
            self.values[li].append(v)
            K = np.concatenate(self.keys[li])  # t x KV x hd
            V = np.concatenate(self.values[li])
            t = K.shape[0]
            group = H // KV
            out = np.empty((m, H, hd))
            for head in range(H):
                g = head % KV if mistake == "mod_head_map" else head // group
                s = q[:, head, :] @ K[:, g, :].T  # m x t
                if mistake != "no_causal":
                    visible = pos[:, None] >= np.arange(t)[None, :]
                    s = np.where(visible, s, -np.inf)
                s = s - s.max(axis=1, keepdims=True)
                p = np.exp(s)
                p = p / p.sum(axis=1, keepdims=True)
                out[:, head, :] = p @ V[:, g, :]
            h = h + res * (out.reshape(m, H * hd) @ L["o"].T)
            x = rmsnorm(h, L["post_norm"], eps)
            if self.ffn_scales is not None:
                x = x * self.ffn_scales[li]
            gate, up = x @ L["gate"].T, x @ L["up"].T
            if mistake == "swap_gate_up":
                gate, up = up, gate
            h = h + res * ((silu(gate) * up) @ L["down"].T)
        self.position += m
        last = rmsnorm(h[-1], self.norm, eps)
        head = self.embed if self.head is None else self.head
        return (head @ last) / c.get("logits_scaling", 1.0)
