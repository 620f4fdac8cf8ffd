"""A float64 statement of the Qwen3-ASR audio encoder, written from the
model definition (the Hugging Face Qwen3-ASR / Qwen3-Omni audio tower), not
from the oracle's code: test infrastructure that pins the oracle's
composition.

    the frames cut into chunks of `chunk`, each zero padded to the longest;
    per chunk, the (1, mels, frames) image through
        h = gelu(conv2d(h, W_i, b_i, 3x3, stride 2, padding 1))  i = 1, 2, 3
    (channels c, bins f, times t) -> permute to (t, c, f) -> rows of c * f
        x = rows W_out^T (+ b_out) + sinusoids[:t]
    the first ceil^3(real frames / 2) rows of each chunk, end to end;
    per layer:
        a = layernorm(x); q, k, v = a W_q^T + b_q, a W_k^T + b_k, a W_v^T + b_v
        x = x + attention(q, k, v, rows see only the rows of their window) W_o^T + b_o
        x = x + gelu(layernorm(x) W_1^T + b_1) W_2^T + b_2
    out = gelu(layernorm(x) P_1^T + p_1) P_2^T + p_2

conv2d weights are [out][in][bin tap][time tap]; windows hold
ceil^3(longest / 2) * window_chunks rows; sinusoids row p is
[sin | cos](p * 10000^(-i / (d/2 - 1))); gelu is the exact one (erf);
layernorm has eps 1e-5. `mistake` plants one plausible slip: "taps_transposed",
"bin_major" (features f * c + c), "global_attention", "positions_offset"
(rows 1.. of the table), "pad_own_length" (the short chunk padded to its
own length).
"""

from __future__ import annotations

import numpy as np
from scipy.special import erf


def gelu(x):
    return 0.5 * x * (1 + erf(x / np.sqrt(2)))


def layernorm(x, w, b, eps=1e-5):
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * w + b


def conv2d(img, w, b, transposed=False):
    """img: cin x F x T; w: cout x cin x 3 x 3; stride 2, padding 1."""
    cin, F, T = img.shape
    if transposed:
        w = w.transpose(0, 1, 3, 2)
    pad = np.zeros((cin, F + 2, T + 2))
    pad[:, 1:-1, 1:-1] = img
    fo, to = (F - 1) // 2 + 1, (T - 1) // 2 + 1
    out = np.empty((w.shape[0], fo, to))
    for y in range(fo):
        for x in range(to):
            out[:, y, x] = np.einsum("oikl,ikl->o", w, pad[:, 2 * y:2 * y + 3, 2 * x:2 * x + 3]) + b
    return out


def sinusoids(rows, d):
    half = d // 2
    inc = np.log(10000.0) / (half - 1)
    ang = np.arange(rows)[:, None] * np.exp(-inc * np.arange(half))[None, :]
    return np.concatenate([np.sin(ang), np.cos(ang)], axis=1)


def attention(q, k, v, heads):
    t, d = q.shape
    hd = d // heads
    out = np.empty((t, d))
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[:, sl] @ k[:, sl].T / np.sqrt(hd)
        s = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, sl] = (s / s.sum(axis=1, keepdims=True)) @ v[:, sl]
    return out


def encode(cfg, p, mel, frames, mistake=None):
    """p: float64 weights: convs (three (w, b)), conv_out (w, b), layers
    (dicts q, k, v, o, fc1, fc2 as [out][in]; bq, bk, bv, bo, b1, b2,
    attn_w, attn_b, ffn_w, ffn_b), post_w, post_b, proj1 (w, b), proj2
    (w, b). mel: frames x mels."""
    d, heads, C = cfg["d"], cfg["heads"], cfg["chunk"]
    half3 = lambda n: (((n + 1) // 2 + 1) // 2 + 1) // 2
    spans = [(s, min(C, frames - s)) for s in range(0, frames, C)]
    longest = max(n for _, n in spans)
    table = sinusoids(cfg["max_positions"] + 1, d)
    rows = []
    for s, n in spans:
        width = n if mistake == "pad_own_length" else longest
        img = np.zeros((1, cfg["mels"], width))
        img[0, :, :n] = mel[s:s + n].T
        for w, b in p["convs"]:
            img = gelu(conv2d(img, w, b, mistake == "taps_transposed"))
        c, f, t = img.shape
        feats = img.transpose(2, 1, 0) if mistake == "bin_major" else img.transpose(2, 0, 1)
        x = feats.reshape(t, c * f) @ p["conv_out"][0].T + p["conv_out"][1]
        x = x + table[1:t + 1] if mistake == "positions_offset" else x + table[:t]
        rows.append(x[:half3(n)])
    x = np.concatenate(rows)
    t = x.shape[0]
    window = t if mistake == "global_attention" else half3(longest) * cfg["window_chunks"]
    for L in p["layers"]:
        a = layernorm(x, L["attn_w"], L["attn_b"])
        q, k, v = a @ L["q"].T + L["bq"], a @ L["k"].T + L["bk"], a @ L["v"].T + L["bv"]
        att = np.concatenate([attention(q[s:s + window], k[s:s + window], v[s:s + window], heads)
                              for s in range(0, t, window)])
        x = x + att @ L["o"].T + L["bo"]
        x = x + gelu(layernorm(x, L["ffn_w"], L["ffn_b"]) @ L["fc1"].T + L["b1"]) @ L["fc2"].T + L["b2"]
    h = gelu(layernorm(x, p["post_w"], p["post_b"]) @ p["proj1"][0].T + p["proj1"][1])
    return h @ p["proj2"][0].T + p["proj2"][1]
