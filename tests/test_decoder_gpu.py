"""The device token loop against the oracle's CausalLm.

Every session runs Trit's sum orders unless it asks for tree sums, so:
- EXACT (f32 keys and values): the oracle's logits and greedy tokens, bit
  for bit;
- the default (f16 keys and values): the logits and tokens of the oracle run
  with the same f16 caches (each appended key and value rounded through
  f16, the oracle's kv_f16), bit for bit -- prefill, the per-kernel loop and
  the persistent decode step alike;
- TREE_SUMS: norms and attention summed as parallel trees. Its int8
  activation codes differ from Trit's wherever a value lies within rounding
  of a code boundary, so it is held to TREE_RTOL of the f16-cache oracle,
  not to its bits.
"""

import numpy as np
import pytest

from oracle import oracle as O
from trit_amd import hip, model, synth

pytestmark = pytest.mark.gpu

TREE_RTOL = 5e-2


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


SMALL = dict(d=256, ffn=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000, eps=1e-6, rope_base=1e6,
             qk_norm=1)


@pytest.fixture(scope="module")
def small(gpu):
    w = synth.lm_weights(SMALL, config=90, sigma=0.2, norm_jitter=0.2)
    ref = O.Lm(SMALL, w)
    ref16 = O.Lm(SMALL, w, kv_f16=True)
    lm = model.build_decoder(w)
    return w, ref, lm, ref16


MID = dict(d=1024, ffn=2048, layers=2, heads=8, kv_heads=4, head_dim=128, vocab=2000, eps=1e-6, rope_base=1e6,
           qk_norm=1)


@pytest.fixture(scope="module")
def mid(gpu):
    """d 1024: the one-row decode products (k 1024 and 2048) run here."""
    w = synth.lm_weights(MID, config=96, sigma=0.1, norm_jitter=0.2)
    return w, O.Lm(MID, w, O.isa_best()), model.build_decoder(w), O.Lm(MID, w, O.isa_best(), kv_f16=True)


QS = dict(d=1024, ffn=3072, layers=2, heads=16, kv_heads=8, head_dim=128, vocab=3000, eps=1e-6, rope_base=1e6,
          qk_norm=1)


@pytest.fixture(scope="module")
def qshape(gpu):
    """Qwen3-0.6B's layer shapes with two layers: fits the persistent step."""
    w = synth.lm_weights(QS, config=95, sigma=0.1, norm_jitter=0.2)
    return w, O.Lm(QS, w, O.isa_best()), model.build_decoder(w), O.Lm(QS, w, O.isa_best(), kv_f16=True)


def test_mid_generate_exact(mid):
    print("case decoder mid exact", flush=True)
    w, ref, lm, _ = mid
    p = synth.prompt(96, 40, MID["vocab"])
    want, want_logits = ref.generate(p, 24)
    s = lm.session(80, hip.EXACT)
    logits = s.prefill(p)
    got = s.generate(24)
    assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
    assert got.tolist() == want.tolist()
    # The steps' logits: one more forward of the last token, both sides.
    ref.reset()
    ref.forward(np.concatenate([p, want[:-1]]))
    want_next = ref.forward(want[-1:])
    got_next = s.prefill(got[-1:])
    assert np.array_equal(got_next.view(np.uint32), want_next.view(np.uint32))


def test_mid_generate_kv_f32(mid):
    print("case decoder mid f32 caches", flush=True)
    w, ref, lm, _ = mid
    p = synth.prompt(97, 40, MID["vocab"])
    s = lm.session(80, hip.KV_F32)
    logits = s.prefill(p)
    got = s.generate(24)
    ref.reset()
    want_logits = ref.forward(p)
    assert same_bits(logits, want_logits), rel(logits, want_logits)
    check_tokens(got, ref, p, 24)


def rel(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def oracle_steps(ref, prompt, n):
    """The oracle's greedy tokens and, per step, the top-2 logit margin."""
    ref.reset()
    logits = ref.forward(prompt)
    tokens, margins = [], []
    for _ in range(n):
        top = np.sort(logits)[-2:]
        margins.append(float(top[1] - top[0]))
        t = int(np.argmax(logits))
        tokens.append(t)
        logits = ref.forward(np.array([t]))
    return tokens, margins


def check_tokens(got, ref, prompt, n):
    """Greedy tokens identical to the oracle's at every one of the n steps."""
    want, margins = oracle_steps(ref, prompt, n)
    same = sum(1 for g, w_ in zip(got.tolist(), want) if g == w_)
    print(f"tokens identical for {same} of {n} steps (least top-2 margin {min(margins):.4g})", flush=True)
    assert got.tolist() == want


def test_prefill_logits_exact(small):
    print("case decoder prefill exact", flush=True)
    w, ref, lm, _ = small
    p = synth.prompt(90, 37, SMALL["vocab"])
    ref.reset()
    want = ref.forward(p)
    s = lm.session(64, hip.EXACT)
    got = s.prefill(p)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rel(got, want)
    # Steps one token at a time continue the same caches.
    for t in [5, 999, 0]:
        want = ref.forward(np.array([t]))
        got = s.prefill(np.array([t]))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rel(got, want)
    s.free()


def test_prefill_in_parts_matches_one_forward(small):
    print("case decoder prefill parts", flush=True)
    w, ref, lm, _ = small
    p = synth.prompt(91, 20, SMALL["vocab"])
    s = lm.session(64, hip.EXACT)
    s.prefill(p[:7], want_logits=False)
    got = s.prefill(p[7:])
    ref.reset()
    ref.forward(p[:7])
    want = ref.forward(p[7:])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("flags", [hip.EXACT, 0, hip.KV_F32, hip.TREE_SUMS])
def test_generate(small, flags):
    print(f"case decoder generate flags={flags}", flush=True)
    w, ref32, lm, ref16 = small
    ref = ref32 if flags & (hip.EXACT | hip.KV_F32) else ref16
    p = synth.prompt(92, 25, SMALL["vocab"])
    want, want_logits = ref.generate(p, 30)
    s = lm.session(64, flags)
    logits = s.prefill(p)
    got = s.generate(30)
    print(f"rel {rel(logits, want_logits):.3g} tokens {got.tolist()[:10]} want {want.tolist()[:10]}", flush=True)
    if flags & hip.TREE_SUMS:
        assert rel(logits, want_logits) < TREE_RTOL
    else:
        assert same_bits(logits, want_logits), rel(logits, want_logits)
        assert got.tolist() == want.tolist()
    assert s.position == 25 + 29


def test_generate_stop(small):
    print("case decoder stop", flush=True)
    w, ref, lm, _ = small
    p = synth.prompt(93, 10, SMALL["vocab"])
    full, _ = ref.generate(p, 12)
    stop = [int(full[5])]
    want, _ = ref.generate(p, 12, stop=stop)
    s = lm.session(64, hip.EXACT)
    s.prefill(p)
    got = s.generate(12, stop=stop)
    assert got.tolist() == want.tolist()
    assert len(got) == list(full).index(stop[0])


def test_rows_prefill(small):
    """forward_rows / answer: embeddings given as rows."""
    print("case decoder rows", flush=True)
    w, ref, lm, _ = small
    p = synth.prompt(94, 9, SMALL["vocab"])
    rows = w.embed[p].view(np.float16).astype(np.float32)
    s = lm.session(32, hip.EXACT)
    got = s.prefill_rows(rows)
    ref.reset()
    want = ref.forward(p)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_errors(small):
    w, ref, lm, _ = small
    s = lm.session(8, 0)
    with pytest.raises(hip.TritError, match="exceed"):
        s.prefill(np.arange(9))
    with pytest.raises(hip.TritError, match="out of range"):
        s.prefill(np.array([SMALL["vocab"]]))
    with pytest.raises(hip.TritError, match="prefill a prompt first"):
        s.generate(3)


@pytest.mark.parametrize("flags", [0, hip.EXACT, hip.KV_F32, hip.TREE_SUMS])
def test_generate_long_prompt(small, flags):
    """Prompts over several 64-key attention splits."""
    print(f"case decoder long prompt flags={flags}", flush=True)
    w, ref32, lm, ref16 = small
    ref = ref32 if flags & (hip.EXACT | hip.KV_F32) else ref16
    p = synth.prompt(95, 150, SMALL["vocab"])
    want, want_logits = ref.generate(p, 20)
    s = lm.session(200, flags)
    logits = s.prefill(p)
    got = s.generate(20)
    print(f"rel {rel(logits, want_logits):.3g}", flush=True)
    if flags & hip.TREE_SUMS:
        assert rel(logits, want_logits) < TREE_RTOL
    else:
        assert same_bits(logits, want_logits), rel(logits, want_logits)
        assert got.tolist() == want.tolist()


def check_generate_default(w, ref16, lm, cfg, monkeypatch, layout=None):
    """Default-mode greedy tokens (Trit's sums, f16 caches) on the persistent
    step: logits and tokens bit for bit the f16-cache oracle's and the
    per-kernel loop's, positions, a stop token, a second generate call that
    continues the first, and the caches the steps wrote (one more token
    through the prompt path gives the oracle's logits bit for bit). layout:
    the step's layout flags the session must report (3: the attention on
    every block, each key/value head's exchanges in one XCD's L2)."""
    p = synth.prompt(98, 40, cfg["vocab"])
    s = lm.session(96, 0)
    logits = s.prefill(p)
    got = s.generate(24)
    assert s.persistent
    if layout is not None:
        assert s.step_layout == layout, s.step_layout
    assert len(got) == 24
    assert s.position == 40 + 23
    ref16.reset()
    want_logits = ref16.forward(p)
    assert same_bits(logits, want_logits), rel(logits, want_logits)
    check_tokens(got, ref16, p, 24)

    monkeypatch.setenv("TRIT_HIP_STEP", "0")
    k = lm.session(96, 0)
    k.prefill(p)
    kern = k.generate(24)
    assert not k.persistent
    monkeypatch.delenv("TRIT_HIP_STEP")
    assert got.tolist() == kern.tolist()

    nxt = np.array([int(got[-1])])
    after_step = s.prefill(nxt)
    after_kern = k.prefill(nxt)
    ref16.reset()
    ref16.forward(np.concatenate([p, got[:-1]]))
    want_after = ref16.forward(nxt)
    print(f"after the steps: vs the oracle {rel(after_step, want_after):.3g}", flush=True)
    assert same_bits(after_step, want_after)
    assert same_bits(after_kern, want_after)

    # A stop token ends the loop without being kept.
    s2 = lm.session(96, 0)
    s2.prefill(p)
    stop = [int(got[5])]
    cut = got.tolist().index(stop[0])
    got2 = s2.generate(24, stop=stop)
    assert got2.tolist() == got.tolist()[:cut]
    assert s2.position == 40 + cut

    # Two calls: the second starts from the first one's last choice.
    s3 = lm.session(96, 0)
    s3.prefill(p)
    a = s3.generate(10)
    b = s3.generate(10)
    assert a.tolist() == got.tolist()[:10]
    assert b.tolist() == got.tolist()[9:19]
    assert s3.position == 40 + 18


def check_generate_tree(w, ref16, lm, cfg, monkeypatch, persistent):
    """TREE_SUMS: the persistent step (tree sums) against the f16-cache
    oracle within TREE_RTOL, its stop and continuation behaviour, and the
    caches it wrote against the per-kernel tree loop's."""
    p = synth.prompt(98, 40, cfg["vocab"])
    s = lm.session(96, hip.TREE_SUMS)
    logits = s.prefill(p)
    got = s.generate(24)
    assert s.persistent == persistent
    assert len(got) == 24 and s.position == 40 + 23
    ref16.reset()
    want_logits = ref16.forward(p)
    print(f"tree sums: prompt logits vs the oracle {rel(logits, want_logits):.3g}", flush=True)
    assert rel(logits, want_logits) < TREE_RTOL
    nxt = np.array([int(got[-1])])
    after_step = s.prefill(nxt)
    ref16.reset()
    ref16.forward(np.concatenate([p, got[:-1]]))
    want_after = ref16.forward(nxt)
    print(f"tree sums: after the steps vs the oracle {rel(after_step, want_after):.3g}", flush=True)
    assert rel(after_step, want_after) < TREE_RTOL
    s2 = lm.session(96, hip.TREE_SUMS)
    s2.prefill(p)
    stop = [int(got[5])]
    got2 = s2.generate(24, stop=stop)
    assert got2.tolist() == got.tolist()[:got.tolist().index(stop[0])]
    s3 = lm.session(96, hip.TREE_SUMS)
    s3.prefill(p)
    a = s3.generate(10)
    b = s3.generate(10)
    assert a.tolist() == got.tolist()[:10] and b.tolist() == got.tolist()[9:19]


def test_step_default(qshape, monkeypatch):
    """The persistent decode step on Qwen3-0.6B's layer shapes in the
    default mode: Trit's sums, bit for bit, with the attention on every
    block (8 key/value heads: one an XCD)."""
    print("case decoder persistent step (qwen3 shapes, Trit's sums)", flush=True)
    w, ref, lm, ref16 = qshape
    check_generate_default(w, ref16, lm, QS, monkeypatch, layout=3)


def test_step_plain_launch(qshape, monkeypatch):
    """TRIT_HIP_STEP_LAUNCH=plain (the profiling option: the same step by an
    ordinary launch) gives the cooperative launch's tokens and the same
    logits after them."""
    print("case decoder persistent step (ordinary launch)", flush=True)
    w, ref, lm, ref16 = qshape
    p = synth.prompt(99, 33, QS["vocab"])
    out = []
    for plain in (False, True):
        if plain:
            monkeypatch.setenv("TRIT_HIP_STEP_LAUNCH", "plain")
        s = lm.session(96, 0)
        s.prefill(p)
        got = s.generate(20)
        assert s.persistent
        after = s.prefill(np.array([int(got[-1])]))
        out.append((got.tolist(), after))
        s.free()
    monkeypatch.delenv("TRIT_HIP_STEP_LAUNCH")
    assert out[0][0] == out[1][0]
    assert same_bits(out[0][1], out[1][1])


def test_step_default_two_blocks_a_head(qshape, monkeypatch):
    """The same with TRIT_HIP_STEP_LOCAL=0: the attention on two blocks a
    query head and every exchange at agent scope (the layout of models
    without one key/value head an XCD), bit for bit."""
    print("case decoder persistent step (qwen3 shapes, two blocks a head)", flush=True)
    w, ref, lm, ref16 = qshape
    monkeypatch.setenv("TRIT_HIP_STEP_LOCAL", "0")
    check_generate_default(w, ref16, lm, QS, monkeypatch, layout=1)


WIDE = dict(d=2048, ffn=6144, layers=2, heads=16, kv_heads=8, head_dim=128, vocab=3000, eps=1e-6, rope_base=1e6,
            qk_norm=1)


@pytest.fixture(scope="module")
def wide(gpu):
    """Qwen3-1.7B's layer shapes (d 2048, ffn 6144) with two layers: the
    step's wide-model layout (gate_up in the last waves, the down product in
    two rounds, the head's x from LDS)."""
    w = synth.lm_weights(WIDE, config=97, sigma=0.1, norm_jitter=0.2)
    return w, O.Lm(WIDE, w, O.isa_best()), model.build_decoder(w), O.Lm(WIDE, w, O.isa_best(), kv_f16=True)


def test_step_wide(wide, monkeypatch):
    """The persistent decode step on Qwen3-1.7B's layer shapes in the default
    mode: Trit's sums, bit for bit, on the step."""
    print("case decoder persistent step (qwen3 1.7b shapes, Trit's sums)", flush=True)
    w, ref, lm, ref16 = wide
    check_generate_default(w, ref16, lm, WIDE, monkeypatch, layout=3)


def test_step_wide_q4_k(wide, monkeypatch):
    """The same shapes with Q4_K linears on the step (the requantized codes)."""
    print("case decoder persistent step (qwen3 1.7b shapes, Q4_K linears)", flush=True)
    w = wide[0]
    ref, ref16, lm = q4_k_decoder(w, WIDE, 91)
    p = synth.prompt(91, 30, WIDE["vocab"])
    want, want_logits = ref16.generate(p, 16)
    s = lm.session(64, 0)
    logits = s.prefill(p)
    got = s.generate(16)
    assert s.persistent
    assert same_bits(logits, want_logits), rel(logits, want_logits)
    assert got.tolist() == want.tolist()


@pytest.mark.parametrize("flags,prompt,steps,max_pos,persistent",
                         [(hip.EXACT, 40, 24, 96, True), (hip.KV_F32, 40, 24, 96, True),
                          (hip.EXACT, 440, 60, 512, True), (hip.EXACT, 500, 12, 700, False)])
def test_step_f32_caches(qshape, monkeypatch, flags, prompt, steps, max_pos, persistent):
    """Trit's f32 keys and values on the persistent step (EXACT, or KV_F32
    with Trit's orders), up to 512 positions; past that the per-kernel loop.
    Logits and greedy tokens bit for bit the oracle's, the per-kernel loop's
    tokens, and the caches the steps wrote (one more token through the
    prompt path gives the oracle's logits bit for bit)."""
    print(f"case decoder step, f32 caches (flags {flags}, prompt {prompt}, {steps} steps, {max_pos} positions)",
          flush=True)
    w, ref, lm, _ = qshape
    p = synth.prompt(99, prompt, QS["vocab"])
    s = lm.session(max_pos, flags)
    logits = s.prefill(p)
    got = s.generate(steps)
    assert s.persistent == persistent
    assert len(got) == steps and s.position == prompt + steps - 1
    ref.reset()
    assert same_bits(logits, ref.forward(p))
    check_tokens(got, ref, p, steps)
    if persistent and max_pos <= 96:
        monkeypatch.setenv("TRIT_HIP_STEP", "0")
        k = lm.session(max_pos, flags)
        k.prefill(p)
        kern = k.generate(steps)
        assert not k.persistent
        monkeypatch.delenv("TRIT_HIP_STEP")
        assert got.tolist() == kern.tolist()
    nxt = np.array([int(got[-1])])
    after = s.prefill(nxt)
    ref.reset()
    ref.forward(np.concatenate([p, got[:-1]]))
    assert same_bits(after, ref.forward(nxt))


@pytest.mark.parametrize("window", [-1, 0])
def test_step_norm_rechained(qshape, monkeypatch, window):
    """The step's RMSNorm and softmax sums join segments chained from
    candidate starts; with no candidates (-1) every segment is chained again
    from its true start, and with the estimate alone (0) most are: the same
    bits either way."""
    print(f"case decoder persistent step, RMSNorm and softmax candidates window {window}", flush=True)
    w, ref, lm, ref16 = qshape
    monkeypatch.setenv("TRIT_HIP_NORM_WINDOW", str(window))
    check_generate_default(w, ref16, lm, QS, monkeypatch)


@pytest.mark.parametrize("attention", ["one-pass", "split"])
def test_step_tree(qshape, monkeypatch, attention):
    """The tree-sum persistent step with each attention form: every key in
    one pass (up to 384 positions), or key splits and their combine."""
    print(f"case decoder persistent step (qwen3 shapes, tree sums, {attention} attention)", flush=True)
    w, ref, lm, ref16 = qshape
    if attention == "split":
        monkeypatch.setenv("TRIT_HIP_STEP_SPLIT", "1")
    check_generate_tree(w, ref16, lm, QS, monkeypatch, persistent=True)


@pytest.mark.parametrize("m", [2, 4, 7, 8])
def test_short_prompt(qshape, m):
    """Prompts of 2..8 rows run the few-row products (on Qwen3-0.6B's layer
    shapes: the streaming kernel with the SwiGLU pair and the residual
    epilogue, the rows quantized in the block or by the quantization pass):
    EXACT and the default mode bit for bit against the oracle, tree sums
    within TREE_RTOL."""
    print(f"case decoder short prompt ({m} rows)", flush=True)
    w, ref, lm, ref16 = qshape
    p = synth.prompt(80 + m, m, QS["vocab"])
    ref.reset()
    want = ref.forward(p)
    ref16.reset()
    want16 = ref16.forward(p)
    for flags, target in [(hip.EXACT, want), (0, want16)]:
        s = lm.session(64, flags)
        got = s.prefill(p)
        s.free()
        assert same_bits(got, target), (flags, rel(got, target))
    f = lm.session(64, hip.TREE_SUMS)
    tree = f.prefill(p)
    f.free()
    print(f"tree sums vs oracle {rel(tree, want16):.3g}", flush=True)
    assert rel(tree, want16) < TREE_RTOL


@pytest.mark.parametrize("prompt,steps,max_pos,persistent", [(330, 54, 384, True), (440, 60, 512, True),
                                                               (700, 40, 760, True), (1564, 64, 1630, True),
                                                               (2040, 30, 2100, True), (4000, 24, 4096, True),
                                                               (4100, 8, 4120, False)])
def test_step_long(qshape, prompt, steps, max_pos, persistent):
    """Long sessions in the default mode: up to 512 positions on the
    persistent step with a thread per key, up to 4096 with the keys in
    rounds of 512 (an audio-LLM decode after a 1564-row prompt, a cleanup
    session's 2000 positions, the limit), past that the per-kernel loop;
    tokens and the logits after them bit for bit the f16-cache oracle's."""
    print(f"case decoder long session (prompt {prompt}, {steps} steps, {max_pos} positions)", flush=True)
    w, ref, lm, ref16 = qshape
    p = synth.prompt(97, prompt, QS["vocab"])
    s = lm.session(max_pos, 0)
    logits = s.prefill(p)
    got = s.generate(steps)
    assert s.persistent == persistent
    assert len(got) == steps and s.position == prompt + steps - 1
    ref16.reset()
    assert same_bits(logits, ref16.forward(p))
    check_tokens(got, ref16, p, steps)
    nxt = np.array([int(got[-1])])
    after = s.prefill(nxt)
    ref16.reset()
    ref16.forward(np.concatenate([p, got[:-1]]))
    assert same_bits(after, ref16.forward(nxt))


@pytest.mark.parametrize("prompt,steps,max_pos", [(330, 54, 384), (700, 40, 760)])
def test_step_tree_long(qshape, prompt, steps, max_pos):
    """The tree-sum step at the one-pass attention's limit (384 positions)
    and past it (the split attention): the caches it wrote against the
    prompt path's fed the same tokens."""
    print(f"case decoder tree-sum step long (prompt {prompt}, {steps} steps, {max_pos} positions)", flush=True)
    w, ref, lm, ref16 = qshape
    p = synth.prompt(97, prompt, QS["vocab"])
    s = lm.session(max_pos, hip.TREE_SUMS)
    s.prefill(p)
    got = s.generate(steps)
    assert s.persistent
    assert len(got) == steps and s.position == prompt + steps - 1
    k = lm.session(max_pos, hip.TREE_SUMS)
    k.prefill(np.concatenate([p, got[:-1]]), want_logits=False)
    nxt = np.array([int(got[-1])])
    after_step, after_prompt = s.prefill(nxt), k.prefill(nxt)
    print(f"after the steps: vs the prompt path {rel(after_step, after_prompt):.3g}", flush=True)
    assert rel(after_step, after_prompt) < TREE_RTOL


def test_mid_step_default(mid, monkeypatch):
    """Four KV heads: four dims of one query head a block, Trit's sums."""
    print("case decoder mid persistent step (Trit's sums)", flush=True)
    w, ref, lm, ref16 = mid
    check_generate_default(w, ref16, lm, MID, monkeypatch, layout=1)


@pytest.mark.parametrize("attention", ["one-pass", "split"])
def test_mid_step_tree(mid, monkeypatch, attention):
    """Four KV heads with tree sums: the one-pass attention at four dims a
    block; the split form's combine would poll from too few waves for this
    model, so it runs the per-kernel loop."""
    print(f"case decoder mid tree sums ({attention})", flush=True)
    w, ref, lm, ref16 = mid
    if attention == "split":
        monkeypatch.setenv("TRIT_HIP_STEP_SPLIT", "1")
    check_generate_tree(w, ref16, lm, MID, monkeypatch, persistent=attention == "one-pass")


def test_mid_prompt_paths(mid, monkeypatch):
    """A 300-row prompt: the default mode's exact attention bit for bit the
    f16-cache oracle's, at once and in two parts; with tree sums, the
    matrix-core attention (and the split kernel) within TREE_RTOL."""
    print("case decoder mid prompt paths", flush=True)
    w, ref, lm, ref16 = mid
    p = synth.prompt(99, 300, MID["vocab"])
    ref16.reset()
    want = ref16.forward(p)
    got = lm.session(320, 0).prefill(p)
    parts = lm.session(320, 0)
    parts.prefill(p[:100])
    got_parts = parts.prefill(p[100:])
    assert same_bits(got, want), rel(got, want)
    assert same_bits(got_parts, want)
    flash = lm.session(320, hip.TREE_SUMS).prefill(p)
    monkeypatch.setenv("TRIT_HIP_FLASH", "0")
    split = lm.session(320, hip.TREE_SUMS).prefill(p)
    monkeypatch.delenv("TRIT_HIP_FLASH")
    print(f"tree sums: flash vs oracle {rel(flash, want):.3g}, split vs oracle {rel(split, want):.3g}", flush=True)
    assert rel(flash, want) < TREE_RTOL and rel(split, want) < TREE_RTOL


def test_mid_prompt_long_rows(mid):
    """Prompt attention over long rows (1100 keys), at once and as 700 +
    400: the default mode bit for bit, tree sums within TREE_RTOL, every
    value finite."""
    print("case decoder mid prompt long rows", flush=True)
    w, ref, lm, ref16 = mid
    p = synth.prompt(98, 1100, MID["vocab"])
    ref16.reset()
    want = ref16.forward(p)
    got = lm.session(1152, 0).prefill(p)
    parts = lm.session(1152, 0)
    parts.prefill(p[:700])
    got_parts = parts.prefill(p[700:])
    assert same_bits(got, want) and same_bits(got_parts, want)
    tree = lm.session(1152, hip.TREE_SUMS).prefill(p)
    print(f"tree sums vs oracle {rel(tree, want):.3g}", flush=True)
    assert np.all(np.isfinite(tree)) and rel(tree, want) < TREE_RTOL


def int8_decoder(w, cfg, seed):
    """The same model with Trit's int8 weights (one f32 scale per row and 128
    inputs) for every linear: device layers and the oracle's."""
    d, ffn, hd = cfg["d"], cfg["ffn"], cfg["head_dim"]
    shapes = [((cfg["heads"] + 2 * cfg["kv_heads"]) * hd, d), (d, cfg["heads"] * hd), (2 * ffn, d), (d, ffn)]
    ref = O.Lm(cfg, w)
    ref16 = O.Lm(cfg, w, kv_f16=True)
    linears = []
    for li in range(cfg["layers"]):
        for which, (n, k) in enumerate(shapes):
            t = synth.seed_for(seed, 4 * li + which)
            codes = synth.ints(t, (n, k), -127, 127).astype(np.int8)
            scales = (synth.normal(t ^ 0x77, (n, k // 128)) * 0.2 / 127).astype(np.float32)
            ref.set_linear_int8(li, which, codes, scales)
            ref16.set_linear_int8(li, which, codes, scales)
            linears.append(hip.Dense.int8(codes, scales))
    embed = hip.Dense.f16(w.embed)
    lm = hip.CausalLm(cfg, linears, w.norms_packed(), embed)
    for layer in linears:
        layer.free()
    embed.free()
    return ref, ref16, lm


def test_int8_linears(small):
    """A decoder whose linears are Trit's int8-128 weights (S1-mini's Auto
    precision): EXACT and the default mode bit for bit, greedy tokens
    identical."""
    print("case decoder int8-128 linears", flush=True)
    w, _, _, _ = small
    ref, ref16, lm = int8_decoder(w, SMALL, 88)
    p = synth.prompt(88, 30, SMALL["vocab"])
    for flags, r in [(hip.EXACT, ref), (0, ref16)]:
        want, want_logits = r.generate(p, 16)
        s = lm.session(64, flags)
        logits = s.prefill(p)
        got = s.generate(16)
        assert same_bits(logits, want_logits), (flags, rel(logits, want_logits))
        assert got.tolist() == want.tolist()


def q4_k_decoder(w, cfg, seed):
    """The same model with Q4_K super-blocks for every linear: device layers
    from the blocks, and the oracle with the Q8_0 codes Trit requantizes
    them to (q4_k_expand, then Blocks::quantize)."""
    import types

    d, ffn, hd = cfg["d"], cfg["ffn"], cfg["head_dim"]
    shapes = {"qkv": ((cfg["heads"] + 2 * cfg["kv_heads"]) * hd, d), "o": (d, cfg["heads"] * hd),
              "gate_up": (2 * ffn, d), "down": (d, ffn)}
    layers, linears = [], []
    for li, L in enumerate(w.layers):
        q8 = {}
        for which, (name, (n, k)) in enumerate(shapes.items()):
            blocks = synth.q4_k_blocks(synth.seed_for(seed, 4 * li + which), n, k)
            codes, scales = O.q8_0_quantize(O.q4_k_expand(blocks))
            q8[name] = synth.q8_0_blocks(codes.reshape(n, k), scales.astype(np.float16).view(np.uint16))
            linears.append(hip.Dense.q4_k(n, k, blocks))
        layers.append(types.SimpleNamespace(**{**vars(L), **q8}))
    w4 = synth.LmWeights(cfg, layers, w.embed, w.final_norm)
    embed = hip.Dense.f16(w.embed)
    lm = hip.CausalLm(cfg, linears, w.norms_packed(), embed)
    for layer in linears:
        layer.free()
    embed.free()
    return O.Lm(cfg, w4, O.isa_best()), O.Lm(cfg, w4, O.isa_best(), kv_f16=True), lm


@pytest.mark.parametrize("step", ["0", "1"])
def test_q4_k_linears(qshape, monkeypatch, step):
    """A decoder whose linears are Q4_K blocks (Qwen3-0.6B's layer shapes):
    EXACT and the default mode bit for bit against the oracle on Trit's
    requantized codes, greedy tokens identical. The layers are made with
    TRIT_HIP_Q4K=1: with the per-kernel loop (TRIT_HIP_STEP=0) every decode
    product runs natively on the super-blocks, the RMSNorm prologue and the
    SwiGLU pair included; the persistent step reads the requantized codes."""
    print(f"case decoder Q4_K linears step={step}", flush=True)
    w = qshape[0]
    monkeypatch.setenv("TRIT_HIP_Q4K", "1")  # the layers keep their super-blocks
    ref, ref16, lm = q4_k_decoder(w, QS, 89)
    monkeypatch.setenv("TRIT_HIP_STEP", step)
    p = synth.prompt(89, 24, QS["vocab"])
    for flags, r in [(hip.EXACT, ref), (0, ref16)]:
        want, want_logits = r.generate(p, 12)
        s = lm.session(64, flags)
        logits = s.prefill(p)
        got = s.generate(12)
        assert same_bits(logits, want_logits), (flags, rel(logits, want_logits))
        assert got.tolist() == want.tolist(), flags


def test_step_deadline_abort(qshape, monkeypatch):
    """A decode step that misses its deadline: forced from the host with a
    zero deadline, so that every block gives up at its first wait and the
    launch drains. generate reports it; the session then refuses prefill
    and generate until it is reset, and after the reset gives the tokens of
    a fresh session."""
    print("case decoder step deadline abort", flush=True)
    w, ref, lm, ref16 = qshape
    p = synth.prompt(77, 20, QS["vocab"])
    fresh = lm.session(64, 0)
    fresh.prefill(p)
    want = fresh.generate(8)
    assert fresh.persistent
    s = lm.session(64, 0)
    s.prefill(p)
    monkeypatch.setenv("TRIT_HIP_STEP_DEADLINE_US", "0")
    with pytest.raises(hip.TritError, match="deadline"):
        s.generate(8)
    monkeypatch.delenv("TRIT_HIP_STEP_DEADLINE_US")
    with pytest.raises(hip.TritError, match="reset"):
        s.prefill(p[:1])
    with pytest.raises(hip.TritError, match="reset"):
        s.generate(2)
    s.reset()
    s.prefill(p)
    assert s.generate(8).tolist() == want.tolist()


@pytest.mark.parametrize("weights", ["config", "lively"])
def test_qwen3_06b_full_loop(gpu, weights):
    """The full-loop configuration itself: Qwen3-0.6B's shape (28 layers,
    d 1024, 16/8 heads x 128, ffn 3072, vocab 151936, tied f16 head), a
    256-token prompt, 128 greedy steps on the persistent step in the
    default mode (Trit's sums, f16 caches). "config": the configuration's
    weights (Q8_0 scales N(0, 0.02)/127, unit norms), whose greedy stream
    settles on one token; "lively": scales N(0, 0.1)/127 and norms 1 +- 0.2,
    a stream of different tokens in which any error of the loop would change
    every token after it. Prompt logits and all 128 tokens bit for bit the
    f16-cache oracle's (and, with the configuration's weights, the tokens of
    Trit's f32 caches too); the caches the steps wrote give the oracle's
    logits for one more token, bit for bit."""
    print(f"case decoder qwen3-0.6b full loop ({weights} weights, 28 layers, 256 + 128)", flush=True)
    cfg = dict(synth.QWEN3_06B)
    if weights == "config":
        w = synth.lm_weights(cfg, config=1)
    else:
        w = synth.lm_weights(cfg, config=11, sigma=0.1, norm_jitter=0.2)
    p = synth.prompt(1, 256, cfg["vocab"])
    lm = model.build_decoder(w)
    s = lm.session(256 + 128 + 1, 0)
    logits = s.prefill(p)
    got = s.generate(128)
    assert s.persistent and len(got) == 128
    isa = O.isa_best()
    ref16 = O.Lm(cfg, w, isa, kv_f16=True)
    ref16.reset()
    want16_logits = ref16.forward(p)
    assert same_bits(logits, want16_logits), rel(logits, want16_logits)
    print(f"{len(set(got.tolist()))} distinct tokens", flush=True)
    check_tokens(got, ref16, p, 128)
    nxt = np.array([int(got[-1])])
    after = s.prefill(nxt)
    ref16.reset()
    ref16.forward(np.concatenate([p, got[:-1]]))
    assert same_bits(after, ref16.forward(nxt))
    del ref16
    if weights == "config":
        ref32 = O.Lm(cfg, w, isa)
        want32, _ = ref32.generate(p, 128)
        assert got.tolist() == want32.tolist()
