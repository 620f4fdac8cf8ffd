"""Builds a device decoder (CausalLm) from host weights through the C ABI."""

from __future__ import annotations

from . import hip


def build_decoder(w) -> hip.CausalLm:
    """Layers are created one at a time and released once the decoder holds them."""
    cfg = w.cfg
    d, ffn, hd = cfg["d"], cfg["ffn"], cfg["head_dim"]
    qkv_rows = (cfg["heads"] + 2 * cfg["kv_heads"]) * hd
    linears = []
    for L in w.layers:
        linears += [hip.Dense.q8_0(qkv_rows, d, L.qkv), hip.Dense.q8_0(d, cfg["heads"] * hd, L.o),
                    hip.Dense.q8_0(2 * ffn, d, L.gate_up), hip.Dense.q8_0(d, ffn, L.down)]
    embed = hip.Dense.f16(w.embed)
    lm = hip.CausalLm(cfg, linears, w.norms_packed(), embed)
    for layer in linears:
        layer.free()
    embed.free()
    return lm
