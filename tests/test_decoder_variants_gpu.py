"""The decoder's other entry points against the oracle's CausalLm:
Granite's multipliers, per-layer MLP input scales (set_ffn_scales), added
input rows (generate_additive) and shared prompt starts (prefix).

Bars as for the plain token loop: EXACT (f32 caches) bit for bit the
oracle; the default (f16 caches) bit for bit the f16-cache oracle; greedy
tokens identical. TREE_SUMS is held to TREE_RTOL of the f16-cache oracle's
logits.
"""

import copy

import numpy as np
import pytest

from oracle import oracle as O
from trit_amd import hip, model, synth

pytestmark = pytest.mark.gpu

TREE_RTOL = 5e-2

SMALL = dict(d=256, ffn=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000, eps=1e-6, rope_base=1e6,
             qk_norm=1)
# Granite: no q/k norms, every multiplier away from 1.
GRANITE = dict(SMALL, qk_norm=0, embedding_multiplier=12.0, attention_multiplier=0.0078125 * 2,
               residual_multiplier=0.22, logits_scaling=8.0)
# Qwen3-0.6B's layer shapes with two layers: plain sessions run the persistent step.
QS = dict(d=1024, ffn=3072, layers=2, heads=16, kv_heads=8, head_dim=128, vocab=3000, eps=1e-6, rope_base=1e6,
          qk_norm=1)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def rel(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def oracles(cfg, w):
    """(f32-cache oracle, f16-cache oracle)."""
    return O.Lm(cfg, w, O.isa_best()), O.Lm(cfg, w, O.isa_best(), kv_f16=True)


def pick(flags, ref, ref16):
    return ref if flags & (hip.EXACT | hip.KV_F32) else ref16


def greedy(ref, logits, n, stop=()):
    """CausalLm::greedy (causal_lm.rs:284-302) on the oracle's caches."""
    out = []
    while len(out) < n:
        t = O.argmax(logits)
        if t in stop:
            break
        out.append(t)
        logits = ref.forward(np.array([t]))
    return out


def check_run(lm, ref, flags, p, n, max_pos=96):
    """Prefill logits and greedy tokens of a session against the oracle."""
    ref.reset()
    want_logits = ref.forward(p)
    s = lm.session(max_pos, flags)
    logits = s.prefill(p)
    got = s.generate(n)
    want = greedy(ref, want_logits, n)
    if flags & hip.TREE_SUMS:
        print(f"tree sums: prompt logits vs the oracle {rel(logits, want_logits):.3g}", flush=True)
        assert rel(logits, want_logits) < TREE_RTOL
    else:
        assert same_bits(logits, want_logits), rel(logits, want_logits)
        assert got.tolist() == want
    s.free()
    return got


@pytest.fixture(scope="module")
def granite(gpu):
    w = synth.lm_weights(GRANITE, config=110, sigma=0.2, norm_jitter=0.2)
    return w, model.build_decoder(w), *oracles(GRANITE, w)


@pytest.mark.parametrize("flags", [0, hip.EXACT, hip.KV_F32, hip.TREE_SUMS])
def test_granite_multipliers(granite, flags):
    """Embedding, attention and residual multipliers and the logits scaling
    (causal_lm.rs:387,420-424,438-442,456,474-478)."""
    print(f"case granite multipliers flags={flags}", flush=True)
    w, lm, ref, ref16 = granite
    p = synth.prompt(110, 33, GRANITE["vocab"])
    check_run(lm, pick(flags, ref, ref16), flags, p, 16)


def test_granite_matters(granite):
    """The multipliers change the logits (a Qwen-style run of the same
    weights differs), so the parity above is not vacuous."""
    print("case granite multipliers change the result", flush=True)
    w, lm, ref, ref16 = granite
    plain_w = copy.copy(w)
    plain_w.cfg = {k: v for k, v in GRANITE.items() if not k.endswith(("_multiplier", "_scaling"))}
    plain = model.build_decoder(plain_w)
    p = synth.prompt(110, 33, GRANITE["vocab"])
    a = lm.session(64, hip.EXACT).prefill(p)
    b = plain.session(64, hip.EXACT).prefill(p)
    assert rel(a, b) > 1e-2


@pytest.fixture(scope="module")
def scaled(gpu):
    w = synth.lm_weights(SMALL, config=111, sigma=0.2, norm_jitter=0.2)
    scales = (1.0 + 0.5 * synth.normal(111, (SMALL["layers"], SMALL["d"]))).astype(np.float32)
    return w, model.build_decoder(w), scales


@pytest.mark.parametrize("flags", [0, hip.EXACT, hip.TREE_SUMS])
def test_ffn_scales(scaled, flags):
    """set_ffn_scales (causal_lm.rs:304-307,458-464): the normed MLP input
    times each layer's scales; removing them restores the plain model, also
    in a session whose captured step was made with them."""
    print(f"case ffn scales flags={flags}", flush=True)
    w, lm, scales = scaled
    ref, ref16 = oracles(SMALL, w)
    r = pick(flags, ref, ref16)
    p = synth.prompt(111, 29, SMALL["vocab"])
    r.set_ffn_scales(scales)
    lm.set_ffn_scales(scales)
    try:
        with_scales = check_run(lm, r, flags, p, 14)
        s = lm.session(96, flags)
        s.prefill(p)
        a = s.generate(6)
        r.set_ffn_scales(None)
        lm.set_ffn_scales(None)
        check_run(lm, r, flags, p, 14)
        # The same session: its step is captured again without the scales.
        s.reset()
        s.prefill(p)
        b = s.generate(14)
        r.reset()
        want = greedy(r, r.forward(p), 14)
        if not flags & hip.TREE_SUMS:
            assert a.tolist() == with_scales.tolist()[:6]
            assert b.tolist() == want
    finally:
        lm.set_ffn_scales(None)


def oracle_additive(ref, prompt, audio, stop=()):
    """CausalLm::generate_additive (causal_lm.rs:313-345) on the oracle."""
    ref.reset()
    n, rows = len(prompt), audio.shape[0]
    if n == 0 or rows < n:
        return []
    x = np.stack([ref.embed_row(t) for t in prompt]) + audio[:n]
    token = O.argmax(ref.forward_rows(x))
    out = []
    for position in range(n, rows):
        if token in stop:
            return out
        out.append(token)
        x = ref.embed_row(token) + audio[position]
        token = O.argmax(ref.forward_rows(x[None]))
    if token not in stop:
        out.append(token)
    return out


@pytest.fixture(scope="module")
def qshape(gpu):
    w = synth.lm_weights(QS, config=112, sigma=0.1, norm_jitter=0.2)
    return w, model.build_decoder(w), *oracles(QS, w)


@pytest.mark.parametrize("flags", [0, hip.EXACT])
def test_generate_additive(qshape, flags):
    """Audio rows added to the prompt's embeddings and to each new token's:
    tokens identical to the oracle's; a stop token ends the call; the
    session decodes on the persistent step again afterwards."""
    print(f"case generate_additive flags={flags}", flush=True)
    w, lm, ref, ref16 = qshape
    r = pick(flags, ref, ref16)
    d = QS["d"]
    p = synth.prompt(112, 12, QS["vocab"])
    audio = (0.1 * synth.normal(113, (40, d))).astype(np.float32)
    want = oracle_additive(r, p.tolist(), audio)
    s = lm.session(48, flags)
    got = s.generate_additive(p, audio)
    print(f"additive tokens {len(got)}: {got[:8].tolist()} ...", flush=True)
    assert len(got) == 40 - 12 + 1 and got.tolist() == want
    # Without the audio the tokens differ (the rows are used).
    r.reset()
    plain = greedy(r, r.forward(p), len(want))
    assert plain != want
    # A stop token: the tokens before it.
    stop = [want[7]]
    s.reset()
    got2 = s.generate_additive(p, audio, stop=stop)
    assert got2.tolist() == oracle_additive(r, p.tolist(), audio, stop)
    assert got2.tolist() == want[: want.index(stop[0])]
    # Back to a plain generate on the same session.
    s.reset()
    s.prefill(p)
    g = s.generate(10)
    # Both modes decode on the step: 48 positions, within the f32-cache
    # instance's 512.
    assert s.persistent
    r.reset()
    assert g.tolist() == greedy(r, r.forward(p), 10)
    s.free()


# Granite's multipliers on Qwen3-0.6B's layer shapes: the persistent step
# takes them in the default (Trit-order) instance.
GRANITE_QS = dict(QS, qk_norm=0, embedding_multiplier=12.0, attention_multiplier=0.0078125 * 2,
                  residual_multiplier=0.22, logits_scaling=8.0)


def check_step(lm, ref16, p, n, max_pos=96):
    """The default mode on the persistent step: prompt logits and every
    greedy token bit for bit the f16-cache oracle's."""
    ref16.reset()
    want_logits = ref16.forward(p)
    s = lm.session(max_pos, 0)
    logits = s.prefill(p)
    got = s.generate(n)
    assert s.persistent, "the persistent step did not run"
    assert same_bits(logits, want_logits), rel(logits, want_logits)
    assert got.tolist() == greedy(ref16, want_logits, n)
    s.free()
    return got


def test_granite_on_the_step(gpu):
    """Embedding, attention and residual multipliers and the logits scaling
    inside the persistent step (causal_lm.rs:387,420-424,438-442,456)."""
    print("case granite multipliers on the persistent step", flush=True)
    w = synth.lm_weights(GRANITE_QS, config=114, sigma=0.1, norm_jitter=0.2)
    lm = model.build_decoder(w)
    ref16 = O.Lm(GRANITE_QS, w, O.isa_best(), kv_f16=True)
    got = check_step(lm, ref16, synth.prompt(114, 40, GRANITE_QS["vocab"]), 24)
    print(f"granite step tokens {got[:8].tolist()} ...", flush=True)


def test_ffn_scales_on_the_step(qshape):
    """set_ffn_scales inside the persistent step: the normed MLP input times
    each layer's scales; removing them gives the plain model again."""
    print("case ffn scales on the persistent step", flush=True)
    w, lm, ref, ref16 = qshape
    scales = (1.0 + 0.5 * synth.normal(115, (QS["layers"], QS["d"]))).astype(np.float32)
    p = synth.prompt(115, 30, QS["vocab"])
    ref16.set_ffn_scales(scales)
    lm.set_ffn_scales(scales)
    try:
        a = check_step(lm, ref16, p, 20)
    finally:
        ref16.set_ffn_scales(None)
        lm.set_ffn_scales(None)
    b = check_step(lm, ref16, p, 20)
    assert a.tolist() != b.tolist()  # the scales are used


def test_generate_additive_edges(qshape):
    """No tokens for an empty prompt or fewer rows than the prompt; one
    token when the rows end with the prompt; errors for a used session and
    for rows beyond the session's positions."""
    print("case generate_additive edge cases", flush=True)
    w, lm, ref, ref16 = qshape
    d = QS["d"]
    p = synth.prompt(114, 6, QS["vocab"])
    audio = (0.1 * synth.normal(115, (6, d))).astype(np.float32)
    s = lm.session(16, 0)
    assert s.generate_additive(p[:0], audio).tolist() == []
    assert s.generate_additive(p, audio[:5]).tolist() == []
    one = s.generate_additive(p, audio)
    assert one.tolist() == oracle_additive(ref16, p.tolist(), audio) and len(one) == 1
    with pytest.raises(hip.TritError, match="reset"):
        s.generate_additive(p, audio)
    s.reset()
    with pytest.raises(hip.TritError, match="exceed"):
        s.generate_additive(p, np.zeros((17, d), np.float32))
    s.free()


@pytest.mark.parametrize("flags", [0, hip.EXACT, hip.KV_F32])
def test_prefix(qshape, flags):
    """CausalLm::generate with a prefix (causal_lm.rs:200-249): the session
    takes the prefix's keys and values and runs the rest of the prompt; the
    logits and tokens are the oracle's for the whole prompt. A prompt that
    does not start with the prefix, or is no longer than it, runs whole."""
    print(f"case prefix flags={flags}", flush=True)
    w, lm, ref, ref16 = qshape
    r = pick(flags, ref, ref16)
    head = synth.prompt(116, 17, QS["vocab"])
    tail = synth.prompt(117, 11, QS["vocab"])
    p = np.concatenate([head, tail])
    pre = lm.prefix(head, flags)
    r.reset()
    r.forward(head)
    want_logits = r.forward(tail)
    want = greedy(r, want_logits, 12)
    s = lm.session(64, flags)
    logits = s.prefill_prefixed(pre, p)
    assert s.position == len(p)
    assert same_bits(logits, want_logits), rel(logits, want_logits)
    got = s.generate(12)
    assert got.tolist() == want
    assert lm.generate(p, 12, flags=flags, prefix=pre).tolist() == want
    # A prompt equal to the prefix, and one that differs in its first token.
    for q in (head, np.concatenate([[int(head[0]) ^ 1], head[1:], tail])):
        s.reset()
        r.reset()
        assert same_bits(s.prefill_prefixed(pre, q), r.forward(q))
    # An empty prefix is no prefix.
    empty = lm.prefix(np.zeros(0, np.int32), flags)
    s.reset()
    r.reset()
    assert same_bits(s.prefill_prefixed(empty, p), r.forward(p))
    s.free()
    pre.free()


def test_prefix_errors(qshape):
    print("case prefix errors", flush=True)
    w, lm, ref, ref16 = qshape
    head = synth.prompt(118, 9, QS["vocab"])
    p = np.concatenate([head, head[:3]])
    pre = lm.prefix(head, 0)
    s = lm.session(32, hip.EXACT)
    with pytest.raises(hip.TritError, match="flags"):
        s.prefill_prefixed(pre, p)
    s0 = lm.session(32, 0)
    s0.prefill(head[:2])
    with pytest.raises(hip.TritError, match="reset"):
        s0.prefill_prefixed(pre, p)
    other = model.build_decoder(w)
    s1 = other.session(32, 0)
    with pytest.raises(hip.TritError, match="another decoder"):
        s1.prefill_prefixed(pre, p)
    small = lm.session(10, 0)
    with pytest.raises(hip.TritError, match="exceed"):
        small.prefill_prefixed(pre, p)


def widened(L_blocks, n, k):
    """f32 values of Q8_0 blocks (codes times widened f16 scales)."""
    b = np.asarray(L_blocks, np.uint8).reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    codes = b[:, 2:].copy().view(np.int8).astype(np.float32)
    return (codes * d).reshape(n, k)


def build(w, kinds, embed=("f16",), head=None):
    """A device decoder with linears of `kinds` (per layer, per linear:
    "q8_0", "f16" or "f32") and the given tables; the matching oracle
    (f32 caches and f16 caches)."""
    cfg = w.cfg
    d, ffn, hd = cfg["d"], cfg["ffn"], cfg["head_dim"]
    qkv_rows = (cfg["heads"] + 2 * cfg["kv_heads"]) * hd
    shapes = [(qkv_rows, d), (d, cfg["heads"] * hd), (2 * ffn, d), (d, ffn)]
    refs = oracles(cfg, w)
    linears = []
    for li, L in enumerate(w.layers):
        for which, (blocks, (n, k)) in enumerate(zip((L.qkv, L.o, L.gate_up, L.down), shapes)):
            kind = kinds[li][which]
            if kind == "q8_0":
                linears.append(hip.Dense.q8_0(n, k, blocks))
                continue
            vals = widened(blocks, n, k)
            if kind == "f16":
                bits = synth.f16_bits(vals)
                linears.append(hip.Dense.f16(bits))
                for r in refs:
                    r.set_linear_float(li, which, bits)
            else:
                linears.append(hip.Dense.f32(vals))
                for r in refs:
                    r.set_linear_float(li, which, vals)

    def table(spec, which):
        kind = spec[0]
        if kind == "f16":
            data = w.embed if which == 0 else synth.f16_bits(synth.activations(900, cfg["vocab"], d) * 0.1)
            for r in refs:
                r.set_table(which, O.TABLE_F16, data)
            return hip.Dense.f16(data)
        if kind == "f32":
            data = synth.activations(901 + which, cfg["vocab"], d) * np.float32(0.1)
            for r in refs:
                r.set_table(which, O.TABLE_F32, data)
            return hip.Dense.f32(data)
        codes = synth.ints(902 + which, (cfg["vocab"], d), -127, 127).astype(np.int8)
        scales = (np.abs(synth.activations(903 + which, cfg["vocab"], d // 32)) * np.float32(0.002)).astype(np.float32)
        for r in refs:
            r.set_table(which, O.TABLE_Q8, codes, scales)
        return hip.Dense.q8(codes, scales)

    emb = table(embed, 0)
    hd_layer = table(head, 1) if head else None
    lm = hip.CausalLm(cfg, linears, w.norms_packed(), emb, hd_layer)
    return lm, refs


@pytest.fixture(scope="module")
def small_w(gpu):
    return synth.lm_weights(SMALL, config=120, sigma=0.2, norm_jitter=0.2)


@pytest.mark.parametrize("flags", [0, hip.EXACT, hip.TREE_SUMS])
def test_float_linears(small_w, flags):
    """f16 and f32 linears (Dense::half / Dense::new, f32 math in the 16-lane
    order) mixed with Q8_0 ones: the normed rows go to the product, and a
    float gate_up's SwiGLU runs after it."""
    print(f"case float linears flags={flags}", flush=True)
    kinds = [["f32", "q8_0", "f16", "q8_0"], ["q8_0", "f16", "f32", "f32"]]
    lm, (ref, ref16) = build(small_w, kinds)
    p = synth.prompt(120, 31, SMALL["vocab"])
    check_run(lm, pick(flags, ref, ref16), flags, p, 12)


@pytest.mark.parametrize("embed,head", [(("q8",), ("f32",)), (("f32",), None), (("q8",), None),
                                        (("f16",), ("q8",))])
@pytest.mark.parametrize("flags", [0, hip.EXACT])
def test_tables(small_w, embed, head, flags):
    """Token tables of f16, f32 and int8-storage (Q8) weights, tied or with
    an untied head (Dense::table, src/cpu/gemm.rs:376-409): rows widened for
    the embeddings (the chosen token's too), f32 math for the logits."""
    print(f"case tables embed={embed[0]} head={head[0] if head else 'tied'} flags={flags}", flush=True)
    kinds = [["q8_0"] * 4] * SMALL["layers"]
    lm, (ref, ref16) = build(small_w, kinds, embed, head)
    p = synth.prompt(121, 23, SMALL["vocab"])
    check_run(lm, pick(flags, ref, ref16), flags, p, 12)


def test_tables_refused(small_w, qshape):
    """A head of int8 activations is refused (a table never takes them); a
    Q8 head runs on the persistent step."""
    print("case table kinds refused / step fallback", flush=True)
    w = small_w
    cfg = w.cfg
    d, hd = cfg["d"], cfg["head_dim"]
    qkv_rows = (cfg["heads"] + 2 * cfg["kv_heads"]) * hd
    linears = []
    for L in w.layers:
        linears += [hip.Dense.q8_0(qkv_rows, d, L.qkv), hip.Dense.q8_0(d, cfg["heads"] * hd, L.o),
                    hip.Dense.q8_0(2 * cfg["ffn"], d, L.gate_up), hip.Dense.q8_0(d, cfg["ffn"], L.down)]
    int8_head = hip.Dense.int8(synth.ints(5, (cfg["vocab"], d), -127, 127).astype(np.int8),
                               np.full((cfg["vocab"], d // 128), 0.01, np.float32))
    with pytest.raises(hip.TritError, match="head must be a table"):
        hip.CausalLm(cfg, linears, w.norms_packed(), hip.Dense.f16(w.embed), int8_head)
    # The Qwen3-shaped model with a Q8 head: tokens as the oracle's, on the
    # persistent step.
    wq = qshape[0]
    lm, (ref, ref16) = build(wq, [["q8_0"] * 4] * QS["layers"], ("f16",), ("q8",))
    p = synth.prompt(122, 20, QS["vocab"])
    ref16.reset()
    want = greedy(ref16, ref16.forward(p), 10)
    s = lm.session(64, 0)
    s.prefill(p)
    got = s.generate(10)
    assert s.persistent
    assert got.tolist() == want
