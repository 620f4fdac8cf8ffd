"""A decoder from a GGUF file (trit_hip_decoder_from_gguf) against the
decoder built from the same weights layer by layer: the same device layouts,
so exact-mode logits are bit-identical and the persistent step's tokens
equal; with Q4_K linears and with an untied head too."""

import numpy as np
import pytest

from tests import gguf_writer as G
from trit_amd import hip, model, synth

pytestmark = pytest.mark.gpu

QS = dict(d=1024, ffn=3072, layers=2, heads=16, kv_heads=8, head_dim=128, vocab=3000, eps=1e-6, rope_base=1e6,
          qk_norm=1)


@pytest.fixture(scope="module")
def weights(gpu):
    return synth.lm_weights(QS, config=93, sigma=0.1, norm_jitter=0.2)


def exact_logits(lm, p, steps=6):
    s = lm.session(64, hip.EXACT)
    logits = s.prefill(p)
    return logits, s.generate(steps)


def test_gguf_decoder_matches(weights, tmp_path):
    print("case gguf decoder (qwen3 shapes, tied head)", flush=True)
    path = tmp_path / "lm.gguf"
    G.write_decoder(path, weights)
    lm = hip.CausalLm.from_gguf(path)
    assert {k: lm.cfg[k] for k in QS if k not in ("eps", "rope_base")} == {k: QS[k] for k in QS
                                                                          if k not in ("eps", "rope_base")}
    ref = model.build_decoder(weights)
    p = synth.prompt(93, 30, QS["vocab"])
    a, ta = exact_logits(lm, p)
    b, tb = exact_logits(ref, p)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert ta.tolist() == tb.tolist()
    # The persistent step (fast mode) on both.
    s, r = lm.session(64, 0), ref.session(64, 0)
    s.prefill(p, want_logits=False)
    r.prefill(p, want_logits=False)
    gs, gr = s.generate(16), r.generate(16)
    assert s.persistent and r.persistent
    assert gs.tolist() == gr.tolist()


def test_gguf_decoder_q4_k_and_untied_head(weights, tmp_path):
    print("case gguf decoder (Q4_K gate and up, untied head)", flush=True)
    c = QS
    d, ffn = c["d"], c["ffn"]
    gate = synth.q4_k_blocks(synth.seed_for(93, 901), ffn, d)
    up = synth.q4_k_blocks(synth.seed_for(93, 902), ffn, d)
    head = synth.f16_bits((synth.normal(synth.seed_for(93, 903), (c["vocab"], d)) * 0.1).astype(np.float32))
    path = tmp_path / "lm_q4k.gguf"
    G.write_decoder(path, weights, untied_head=head,
                    replace={"dec.blocks.1.ffn.gate.weight": (G.GGML["Q4_K"], [d, ffn], gate.tobytes()),
                             "dec.blocks.1.ffn.up.weight": (G.GGML["Q4_K"], [d, ffn], up.tobytes())})
    lm = hip.CausalLm.from_gguf(path)
    hd, qkv_rows = c["head_dim"], (c["heads"] + 2 * c["kv_heads"]) * c["head_dim"]
    linears = []
    for i, L in enumerate(weights.layers):
        gu = hip.Dense.q4_k(2 * ffn, d, np.concatenate([gate, up])) if i == 1 else hip.Dense.q8_0(2 * ffn, d, L.gate_up)
        linears += [hip.Dense.q8_0(qkv_rows, d, L.qkv), hip.Dense.q8_0(d, c["heads"] * hd, L.o), gu,
                    hip.Dense.q8_0(d, ffn, L.down)]
    ref = hip.CausalLm(c, linears, weights.norms_packed(), hip.Dense.f16(weights.embed), hip.Dense.f16(head))
    p = synth.prompt(94, 30, c["vocab"])
    a, ta = exact_logits(lm, p)
    b, tb = exact_logits(ref, p)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert ta.tolist() == tb.tolist()


def test_gguf_decoder_errors(weights, tmp_path):
    path = tmp_path / "bad.gguf"
    G.write_decoder(path, weights, arch="whisper")
    with pytest.raises(hip.TritError, match="no language model block"):
        hip.CausalLm.from_gguf(path)
    lm = hip.CausalLm.from_gguf(path, prefix="stt.qwen3_asr.decoder")  # named explicitly
    lm.free()
    d = QS["d"]
    G.write_decoder(path, weights, replace={"dec.blocks.0.attn.o.weight": (G.GGML["Q6_K"], [QS["heads"] * 128, d],
                                                                           b"\0" * (d * QS["heads"] * 128 // 256 * 210))})
    with pytest.raises(hip.TritError, match="attn.o.weight is Q6_K; the device loader reads Q8_0 and Q4_K"):
        hip.CausalLm.from_gguf(path)
