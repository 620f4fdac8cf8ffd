"""A decoder from a GGUF file (trit_hip_decoder_from_gguf) against the
decoder built from the same weights layer by layer (the same device
layouts, so exact-mode logits are bit-identical and the persistent step's
tokens equal; with Q4_K linears and with an untied head too), and a file of
mixed ggml types against the oracle."""

import numpy as np
import pytest

from trit_amd import gguf_writer as G
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
    G.write_decoder(path, weights, replace={"dec.blocks.0.attn.o.weight": (G.GGML["BF16"], [QS["heads"] * 128, d],
                                                                           b"\0" * (d * QS["heads"] * 128 * 2))})
    with pytest.raises(hip.TritError, match="attn.o.weight is BF16; the device loader reads F32, F16, Q8_0"):
        hip.CausalLm.from_gguf(path)


def q8_0_bytes(codes, scales):
    """Q8_0 blocks (f16 d, then 32 codes) of codes n x k and f16-exact scales."""
    codes = np.asarray(codes, np.int8).reshape(-1, 32)
    d = np.asarray(scales, np.float32).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return np.concatenate([d, codes.view(np.uint8)], axis=1).reshape(-1)


def test_gguf_types_against_oracle(weights, tmp_path):
    """A GGUF file with the tensor types a llama.cpp quantization mixes --
    Q6_K, Q5_0 and Q4_K linears, F16 q/k/v, an F32 token table and a Q8_0
    untied head -- built on the device as Trit builds it under Auto:
    the block types requantized to Q8_0 codes, F16 linears and both tables
    with f32 math. Logits (EXACT, and the f16-cache default) and greedy
    tokens are the oracle's for the same rules, bit for bit."""
    print("case gguf decoder with mixed ggml types against the oracle", flush=True)
    from oracle import oracle as O

    c = QS
    d, ffn, hd, vocab = c["d"], c["ffn"], c["head_dim"], c["vocab"]
    qd, kd = c["heads"] * hd, c["kv_heads"] * hd
    seed = lambda i: synth.seed_for(95, 1000 + i)
    o0 = synth.ggml_blocks(seed(1), 14, d, qd)  # Q6_K attn.o of layer 0
    down1 = synth.ggml_blocks(seed(2), 6, d, ffn)  # Q5_0 ffn.down of layer 1
    gate1 = synth.ggml_blocks(seed(3), 12, ffn, d)  # Q4_K gate of layer 1
    up1 = synth.ggml_blocks(seed(4), 3, ffn, d)  # Q4_1 up of layer 1: stacked parts of two types are refused
    qkv1 = synth.f16_bits(synth.activations(seed(5), qd + 2 * kd, d) * np.float32(0.02))  # F16 q/k/v of layer 1
    embed = synth.activations(seed(6), vocab, d) * np.float32(0.1)  # F32 token table
    hcodes, hsb = synth.q8_0_matrix(seed(7), vocab, d)
    head_blocks = synth.q8_0_blocks(hcodes, hsb)  # Q8_0 untied head
    ggml = lambda t, n, k, b: (G.GGML[t], [k, n], b.tobytes())
    repl = {
        "dec.blocks.0.attn.o.weight": ggml("Q6_K", d, qd, o0),
        "dec.blocks.1.ffn.down.weight": ggml("Q5_0", d, ffn, down1),
        "dec.blocks.1.ffn.gate.weight": ggml("Q4_K", ffn, d, gate1),
        "dec.blocks.1.ffn.up.weight": ggml("Q4_K", ffn, d, synth.ggml_blocks(seed(4), 12, ffn, d)),
        "dec.blocks.1.attn.q.weight": ggml("F16", qd, d, qkv1[:qd]),
        "dec.blocks.1.attn.k.weight": ggml("F16", kd, d, qkv1[qd:qd + kd]),
        "dec.blocks.1.attn.v.weight": ggml("F16", kd, d, qkv1[qd + kd:]),
        "dec.token_embd.weight": ggml("F32", vocab, d, embed),
        "dec.output.weight": ggml("Q8_0", vocab, d, head_blocks),
    }
    path = tmp_path / "mixed.gguf"
    G.write_decoder(path, weights, untied_head=weights.embed, replace=repl)
    lm = hip.CausalLm.from_gguf(path)

    # The oracle under the same rules: block types become Q8_0 blocks of the
    # requantized expansion; F16 q/k/v f32 math; the tables f32 and Q8.
    def requant(t, n, k, b):
        codes, scales = O.q8_0_quantize(O.ggml_expand(t, b))
        return q8_0_bytes(codes, scales)

    layers = []
    for i, L in enumerate(weights.layers):
        o = requant(14, d, qd, o0) if i == 0 else L.o
        down = requant(6, d, ffn, down1) if i == 1 else L.down
        gu = (np.concatenate([requant(12, ffn, d, gate1),
                              requant(12, ffn, d, synth.ggml_blocks(seed(4), 12, ffn, d))]) if i == 1 else L.gate_up)
        layers.append(synth.LayerWeights(L.qkv, o, gu, down, L.norm_attn, L.norm_mlp, L.q_norm, L.k_norm))
    w2 = synth.LmWeights(c, layers, weights.embed, weights.final_norm)
    refs = [O.Lm(c, w2, O.isa_best()), O.Lm(c, w2, O.isa_best(), kv_f16=True)]
    for r in refs:
        r.set_linear_float(1, 0, qkv1)
        r.set_table(0, O.TABLE_F32, embed)
        r.set_table(1, O.TABLE_Q8, hcodes, hsb.view(np.float16).astype(np.float32))
    p = synth.prompt(95, 28, vocab)
    for flags, r in ((hip.EXACT, refs[0]), (0, refs[1])):
        r.reset()
        want_logits = r.forward(p)
        s = lm.session(64, flags)
        got_logits = s.prefill(p)
        assert np.array_equal(got_logits.view(np.uint32), want_logits.view(np.uint32)), flags
        got = s.generate(10)
        want = []
        logits = want_logits
        for _ in range(10):
            t = O.argmax(logits)
            want.append(t)
            logits = r.forward(np.array([t]))
        assert got.tolist() == want, flags
    # Stacked parts of two types are refused, as one layer takes one type.
    repl["dec.blocks.1.ffn.up.weight"] = ggml("Q4_1", ffn, d, up1)
    G.write_decoder(path, weights, untied_head=weights.embed, replace=repl)
    with pytest.raises(hip.TritError, match="stacked rows take one type"):
        hip.CausalLm.from_gguf(path)


def test_weight_cache(weights, tmp_path):
    """The device weight-cache file: a decoder saved and loaded again (Q8_0,
    Q4_K and float-math layers, an untied head) gives the same logits bit
    for bit and the same tokens; a file of another key, a damaged one and a
    cut one fail the load."""
    print("case weight cache file", flush=True)
    c = QS
    d, ffn = c["d"], c["ffn"]
    gate = synth.q4_k_blocks(synth.seed_for(93, 911), ffn, d)
    up = synth.q4_k_blocks(synth.seed_for(93, 912), ffn, d)
    head = synth.activations(synth.seed_for(93, 913), c["vocab"], d) * np.float32(0.1)
    path = tmp_path / "lm.gguf"
    G.write_decoder(path, weights, untied_head=weights.embed,
                    replace={"dec.blocks.1.ffn.gate.weight": (G.GGML["Q4_K"], [d, ffn], gate.tobytes()),
                             "dec.blocks.1.ffn.up.weight": (G.GGML["Q4_K"], [d, ffn], up.tobytes()),
                             "dec.output.weight": (G.GGML["F32"], [d, c["vocab"]], head.tobytes())})
    lm = hip.CausalLm.from_gguf(path)
    cache = tmp_path / "weights.bin"
    lm.save(cache)
    again = hip.CausalLm.load(cache)
    assert again.cfg["d"] == d and again.cfg["layers"] == c["layers"]
    p = synth.prompt(96, 30, c["vocab"])
    a, ta = exact_logits(lm, p)
    b, tb = exact_logits(again, p)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert ta.tolist() == tb.tolist()
    s1, s2 = lm.session(64, 0), again.session(64, 0)
    s1.prefill(p, want_logits=False)
    s2.prefill(p, want_logits=False)
    assert s1.generate(12).tolist() == s2.generate(12).tolist()
    raw = bytearray(cache.read_bytes())
    bad = tmp_path / "bad.bin"
    for what, data in (("damaged", raw[:len(raw) // 2] + bytes([raw[len(raw) // 2] ^ 1]) + raw[len(raw) // 2 + 1:]),
                       ("cut short", raw[:len(raw) - 100]),
                       ("made by", raw[:16] + b"X" + raw[17:])):
        bad.write_bytes(bytes(data))
        with pytest.raises(hip.TritError, match=what):
            hip.CausalLm.load(bad)
