"""The persistent decode step with the linear and table kinds Trit's callers
load: int8 linears (an f32 scale per row and 128 inputs; int8 activations in
128-groups) and int8-storage (Q8) tables with f32 math -- Trit's Auto
precision, S1-mini's load (src/cpu/gemm.rs:565-617, src/cleanup.rs:187-215)
-- and Q8_0 linears under a Q8 head. Each runs on the step
(Session.persistent) and gives the f16-cache oracle's prompt logits and
greedy tokens bit for bit; the same model in EXACT mode (the per-kernel
loop, f32 caches) gives the f32-cache oracle's."""

import numpy as np
import pytest

from oracle import oracle as O
from trit_amd import hip, model, synth

pytestmark = pytest.mark.gpu

# Qwen3-0.6B's layer shapes with two layers.
QS = dict(d=1024, ffn=3072, layers=2, heads=16, kv_heads=8, head_dim=128, vocab=3000, eps=1e-6, rope_base=1e6,
          qk_norm=1)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def rel(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def greedy(ref, logits, n):
    out = []
    while len(out) < n:
        t = O.argmax(logits)
        out.append(t)
        logits = ref.forward(np.array([t]))
    return out


def auto_oracle(w, kv_f16):
    """The oracle's CausalLm at Auto precision: int8 linears, a tied Q8 table."""
    ref = O.Lm(w.cfg, w.base, O.isa_best(), kv_f16=kv_f16)
    for li, layer in enumerate(w.linears):
        for which, (codes, scales) in enumerate(layer):
            ref.set_linear_int8(li, which, codes, scales)
    ref.set_table(0, O.TABLE_Q8, *w.table)
    return ref


def check(lm, ref, p, n, flags=0, max_pos=96):
    ref.reset()
    want_logits = ref.forward(p)
    s = lm.session(max_pos, flags)
    logits = s.prefill(p)
    got = s.generate(n)
    assert s.persistent == (flags == 0), "the persistent step should run exactly in the default mode"
    assert same_bits(logits, want_logits), rel(logits, want_logits)
    assert got.tolist() == greedy(ref, want_logits, n)
    s.free()
    return got


@pytest.fixture(scope="module")
def auto_qs(gpu):
    base = synth.lm_weights(QS, config=140, sigma=0.1, norm_jitter=0.2)
    w = synth.auto_weights(base)
    return w, model.build_decoder_auto(w)


def test_auto_precision_on_the_step(auto_qs):
    """Int8 linears and a tied Q8 table (S1-mini's Auto load) on the step."""
    print("case step: int8 linears, tied Q8 table", flush=True)
    w, lm = auto_qs
    got = check(lm, auto_oracle(w, True), synth.prompt(140, 40, QS["vocab"]), 24)
    print(f"tokens {got[:8].tolist()} ...", flush=True)
    assert len(set(got.tolist())) > 4  # a stream that moves


def test_auto_precision_exact(auto_qs):
    """The same model in EXACT mode (f32 caches, the per-kernel loop)."""
    print("case per-kernel loop: int8 linears, tied Q8 table, exact", flush=True)
    w, lm = auto_qs
    check(lm, auto_oracle(w, False), synth.prompt(141, 33, QS["vocab"]), 12, flags=hip.EXACT)


def test_auto_precision_continues(auto_qs):
    """Two generate calls on one session continue each other (the second
    starts from the first one's last choice: the step's second launch takes
    the candidates the first one left), a prompt longer than one key block,
    and a stop token."""
    print("case step: int8 linears, two calls and a stop token", flush=True)
    w, lm = auto_qs
    ref = auto_oracle(w, True)
    p = synth.prompt(142, 70, QS["vocab"])
    ref.reset()
    want = greedy(ref, ref.forward(p), 30)
    s = lm.session(128, 0)
    s.prefill(p)
    a = s.generate(12)
    b = s.generate(18)
    assert s.persistent
    assert a.tolist() == want[:12] and b.tolist() == want[11:29]
    s.reset()
    s.prefill(p)
    stop = want[9]
    c = s.generate(30, stop=[stop])
    assert c.tolist() == want[:want.index(stop)]


def test_q8_head_on_the_step(gpu):
    """Q8_0 linears, an f16 embedding and an untied Q8 head."""
    print("case step: Q8_0 linears, f16 table, Q8 head", flush=True)
    base = synth.lm_weights(QS, config=143, sigma=0.1, norm_jitter=0.2)
    codes, scales = synth.q8_table(synth.activations(synth.seed_for(143, 9001), QS["vocab"], QS["d"]) * 0.05)
    linears = []
    d, ffn, hd = QS["d"], QS["ffn"], QS["head_dim"]
    for L in base.layers:
        linears += [hip.Dense.q8_0((QS["heads"] + 2 * QS["kv_heads"]) * hd, d, L.qkv),
                    hip.Dense.q8_0(d, QS["heads"] * hd, L.o), hip.Dense.q8_0(2 * ffn, d, L.gate_up),
                    hip.Dense.q8_0(d, ffn, L.down)]
    lm = hip.CausalLm(QS, linears, base.norms_packed(), hip.Dense.f16(base.embed), hip.Dense.q8(codes, scales))
    ref = O.Lm(QS, base, O.isa_best(), kv_f16=True)
    ref.set_table(1, O.TABLE_Q8, codes, scales)
    check(lm, ref, synth.prompt(143, 37, QS["vocab"]), 20)


def test_int8_linears_f16_table(gpu):
    """Int8 linears under a tied f16 table."""
    print("case step: int8 linears, tied f16 table", flush=True)
    base = synth.lm_weights(QS, config=144, sigma=0.1, norm_jitter=0.2)
    w = synth.auto_weights(base)
    linears = [hip.Dense.int8(c, s) for layer in w.linears for c, s in layer]
    lm = hip.CausalLm(QS, linears, base.norms_packed(), hip.Dense.f16(base.embed))
    ref = O.Lm(QS, base, O.isa_best(), kv_f16=True)
    for li, layer in enumerate(w.linears):
        for which, (c, s) in enumerate(layer):
            ref.set_linear_int8(li, which, c, s)
    check(lm, ref, synth.prompt(144, 29, QS["vocab"]), 20)


def test_auto_precision_full_loop(gpu):
    """S1-mini's configuration: Qwen3-0.6B's shape (28 layers, vocab 151936)
    at Auto precision, a 256-token prompt and 128 greedy steps on the
    persistent step; prompt logits and every token bit for bit the
    f16-cache oracle's."""
    print("case step: s1-mini auto precision, 28 layers, 256 + 128", flush=True)
    cfg = dict(synth.QWEN3_06B)
    base = synth.lm_weights(cfg, config=12, sigma=0.1, norm_jitter=0.2)
    w = synth.auto_weights(base)
    lm = model.build_decoder_auto(w)
    p = synth.prompt(12, 256, cfg["vocab"])
    s = lm.session(256 + 128 + 1, 0)
    logits = s.prefill(p)
    got = s.generate(128)
    assert s.persistent and len(got) == 128
    ref = auto_oracle(w, True)
    ref.reset()
    want_logits = ref.forward(p)
    assert same_bits(logits, want_logits), rel(logits, want_logits)
    print(f"{len(set(got.tolist()))} distinct tokens", flush=True)
    assert got.tolist() == greedy(ref, want_logits, 128)


def test_auto_precision_long_session(auto_qs):
    """A cleanup-length session at Auto precision: a 900-token prompt and
    160 greedy steps (past 512 positions: the keys in rounds of 512)."""
    print("case step: int8 linears, tied Q8 table, 900 + 160", flush=True)
    w, lm = auto_qs
    got = check(lm, auto_oracle(w, True), synth.prompt(145, 900, QS["vocab"]), 160, max_pos=1100)
    assert len(set(got.tolist())) > 4
