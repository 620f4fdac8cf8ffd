"""A float64 statement of the Whisper audio encoder (the one Voxtral and
MOSS run), written from the model definition (Hugging Face
WhisperEncoder), not from the oracle's code: test infrastructure that pins
the oracle's composition.

    h = gelu(conv1d(mel, W1, b1, kernel 3, stride 1, padding 1))
    x = gelu(conv1d(h,   W2, b2, kernel 3, stride 2, padding 1)) + positions
    per layer:
        a = layernorm(x) ; q, k, v = a Wq^T + bq, a Wk^T, a Wv^T + bv
        x = x + (softmax(q k^T / sqrt(hd)) v) Wo^T + bo     (no mask)
        x = x + gelu(layernorm(x) W1^T + b1) W2^T + b2
    out = layernorm(x)

conv1d weights are [out][in][kernel]; gelu is the exact one (erf);
layernorm has eps 1e-5. `mistake` plants one plausible slip: "tanh_gelu",
"conv2_shift" (the stride-2 windows one frame late), "post_norm"
(norm after the residual add), "positions_before_gelu", "causal".
"""

from __future__ import annotations

import numpy as np
from scipy.special import erf


def gelu(x, mistake=None):
    if mistake == "tanh_gelu":
        return 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))
    return 0.5 * x * (1 + erf(x / np.sqrt(2)))


def layernorm(x, w, b, eps=1e-5):
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * w + b


def conv1d(x, w, b, stride):
    """x: frames x cin; w: cout x cin x 3; padding 1."""
    frames = x.shape[0]
    xp = np.concatenate([np.zeros((1, x.shape[1])), x, np.zeros((1, x.shape[1]))])
    out_frames = (frames + 2 - 3) // stride + 1
    out = np.empty((out_frames, w.shape[0]))
    for t in range(out_frames):
        window = xp[t * stride:t * stride + 3]  # 3 x cin
        out[t] = np.einsum("oik,ki->o", w, window) + b
    return out


def encode(cfg, p, mel, mistake=None):
    """p: float64 weights (conv1_w cout x mels x 3, conv1_b, conv2_w, conv2_b,
    positions, layers: list of dicts q, k, v, o, fc1, fc2 ([out][in]), bq,
    bv, bo, b1, b2, attn_w, attn_b, ffn_w, ffn_b), norm_w, norm_b."""
    d, heads = cfg["d"], cfg["heads"]
    hd = d // heads
    h = gelu(conv1d(mel, p["conv1_w"], p["conv1_b"], 1), mistake)
    if mistake == "positions_before_gelu":
        x = gelu(conv1d(h, p["conv2_w"], p["conv2_b"], 2) + p["positions"], mistake)
    elif mistake == "conv2_shift":
        # The stride-2 windows one frame late (padding at the wrong end).
        x = gelu(conv1d(h, p["conv2_w"], p["conv2_b"], 1), mistake)[1::2] + p["positions"]
    else:
        x = gelu(conv1d(h, p["conv2_w"], p["conv2_b"], 2), mistake) + p["positions"]
    P = x.shape[0]
    for L in p["layers"]:
        a = x if mistake == "post_norm" else layernorm(x, L["attn_w"], L["attn_b"])
        q = (a @ L["q"].T + L["bq"]).reshape(P, heads, hd)
        k = (a @ L["k"].T).reshape(P, heads, hd)
        v = (a @ L["v"].T + L["bv"]).reshape(P, heads, hd)
        s = np.einsum("qhe,khe->hqk", q, k) / np.sqrt(hd)
        if mistake == "causal":
            s = s + np.triu(np.full((P, P), -np.inf), 1)[None]
        s = np.exp(s - s.max(axis=-1, keepdims=True))
        s = s / s.sum(axis=-1, keepdims=True)
        att = np.einsum("hqk,khe->qhe", s, v).reshape(P, d)
        x = x + att @ L["o"].T + L["bo"]
        if mistake == "post_norm":
            x = layernorm(x, L["attn_w"], L["attn_b"])
        f = x if mistake == "post_norm" else layernorm(x, L["ffn_w"], L["ffn_b"])
        x = x + gelu(f @ L["fc1"].T + L["b1"], mistake) @ L["fc2"].T + L["b2"]
        if mistake == "post_norm":
            x = layernorm(x, L["ffn_w"], L["ffn_b"])
    return layernorm(x, p["norm_w"], p["norm_b"])
