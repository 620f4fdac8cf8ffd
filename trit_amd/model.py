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


def build_decoder_auto(w) -> hip.CausalLm:
    """A device decoder at Trit's Auto precision (synth.AutoWeights): int8
    linears (Dense::int8) and a tied int8-storage table (Dense::q8)."""
    linears = [hip.Dense.int8(codes, scales) for layer in w.linears for codes, scales in layer]
    table = hip.Dense.q8(*w.table)
    lm = hip.CausalLm(w.cfg, linears, w.norms_packed(), table)
    for layer in linears:
        layer.free()
    table.free()
    return lm
