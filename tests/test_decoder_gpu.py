"""The device token loop against the oracle's CausalLm.

Exact mode must give the oracle's logits bit for bit and its greedy tokens;
fast mode (tree RMSNorm sums, f16 keys and values) must give logits within
1e-3 relative and the same greedy tokens.
"""

import numpy as np
import pytest

from oracle import oracle as O
from trit_amd import hip, model, synth

pytestmark = pytest.mark.gpu

SMALL = dict(d=256, ffn=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=1000, eps=1e-6, rope_base=1e6,
             qk_norm=1)


@pytest.fixture(scope="module")
def small(gpu):
    w = synth.lm_weights(SMALL, config=90, sigma=0.2, norm_jitter=0.2)
    ref = O.Lm(SMALL, w)
    lm = model.build_decoder(w)
    return w, ref, lm


MID = dict(d=1024, ffn=2048, layers=2, heads=8, kv_heads=4, head_dim=128, vocab=2000, eps=1e-6, rope_base=1e6,
           qk_norm=1)


@pytest.fixture(scope="module")
def mid(gpu):
    """d 1024: the one-row decode products (k 1024 and 2048) run here."""
    w = synth.lm_weights(MID, config=96, sigma=0.1, norm_jitter=0.2)
    return w, O.Lm(MID, w, O.isa_best()), model.build_decoder(w)


QS = dict(d=1024, ffn=3072, layers=2, heads=16, kv_heads=8, head_dim=128, vocab=3000, eps=1e-6, rope_base=1e6,
          qk_norm=1)


@pytest.fixture(scope="module")
def qshape(gpu):
    """Qwen3-0.6B's layer shapes with two layers: fits the persistent step."""
    w = synth.lm_weights(QS, config=95, sigma=0.1, norm_jitter=0.2)
    return w, O.Lm(QS, w, O.isa_best()), model.build_decoder(w)


def test_mid_generate_exact(mid):
    print("case decoder mid exact", flush=True)
    w, ref, lm = mid
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


def test_mid_generate_fast(mid):
    print("case decoder mid fast", flush=True)
    w, ref, lm = mid
    p = synth.prompt(97, 40, MID["vocab"])
    s = lm.session(80, hip.KV_F32)
    logits = s.prefill(p)
    got = s.generate(24)
    ref.reset()
    want_logits = ref.forward(p)
    assert rel(logits, want_logits) < 1e-3
    check_fast_tokens(got, ref, p, 24, float(np.max(np.abs(logits - want_logits))))


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


def check_fast_tokens(got, ref, prompt, n, bound, least=5):
    """Fast mode sums in other orders: its tokens must equal the oracle's at
    every step until the first one whose top-2 margin is within the logit
    error bound (where either choice is consistent with that error)."""
    want, margins = oracle_steps(ref, prompt, n)
    checked = 0
    for i, (g, w, m) in enumerate(zip(got.tolist(), want, margins)):
        if m <= 2 * bound:
            break
        assert g == w, f"step {i}: {g} vs {w} (margin {m:.4f}, bound {bound:.4f})"
        checked += 1
    print(f"fast tokens identical for {checked} of {n} steps", flush=True)
    assert checked >= least


def test_prefill_logits_exact(small):
    print("case decoder prefill exact", flush=True)
    w, ref, lm = small
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
    w, ref, lm = small
    p = synth.prompt(91, 20, SMALL["vocab"])
    s = lm.session(64, hip.EXACT)
    s.prefill(p[:7], want_logits=False)
    got = s.prefill(p[7:])
    ref.reset()
    ref.forward(p[:7])
    want = ref.forward(p[7:])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("flags", [hip.EXACT, 0, hip.KV_F32])
def test_generate(small, flags):
    print(f"case decoder generate flags={flags}", flush=True)
    w, ref, lm = small
    p = synth.prompt(92, 25, SMALL["vocab"])
    want, want_logits = ref.generate(p, 30)
    s = lm.session(64, flags)
    logits = s.prefill(p)
    got = s.generate(30)
    print(f"rel {rel(logits, want_logits):.3g} tokens {got.tolist()[:10]} want {want.tolist()[:10]}", flush=True)
    if flags & hip.EXACT:
        assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
        assert got.tolist() == want.tolist()
    else:
        # Tree sums (and f16 keys and values) differ from Trit's order by
        # rounding; the int8 activation codes carry those differences on.
        err = rel(logits, want_logits)
        bound = float(np.max(np.abs(logits - want_logits)))
        if flags & hip.KV_F32:
            # Only the order of the sums differs from Trit's.
            assert err < 1e-3
            check_fast_tokens(got, ref, p, 30, bound)
        else:
            # f16 keys and values, whose rounding the int8 activation codes carry on.
            assert err < 5e-2
            check_fast_tokens(got, ref, p, 30, bound, least=0)
    assert s.position == 25 + 29


def test_generate_stop(small):
    print("case decoder stop", flush=True)
    w, ref, lm = small
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
    w, ref, lm = small
    p = synth.prompt(94, 9, SMALL["vocab"])
    rows = w.embed[p].view(np.float16).astype(np.float32)
    s = lm.session(32, hip.EXACT)
    got = s.prefill_rows(rows)
    ref.reset()
    want = ref.forward(p)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_errors(small):
    w, ref, lm = small
    s = lm.session(8, 0)
    with pytest.raises(hip.TritError, match="exceed"):
        s.prefill(np.arange(9))
    with pytest.raises(hip.TritError, match="out of range"):
        s.prefill(np.array([SMALL["vocab"]]))
    with pytest.raises(hip.TritError, match="prefill a prompt first"):
        s.generate(3)


@pytest.mark.parametrize("flags", [0, hip.EXACT, hip.KV_F32])
def test_generate_long_prompt(small, flags):
    """Prompts over several 64-key attention splits."""
    print(f"case decoder long prompt flags={flags}", flush=True)
    w, ref, lm = small
    p = synth.prompt(95, 150, SMALL["vocab"])
    want, want_logits = ref.generate(p, 20)
    s = lm.session(200, flags)
    logits = s.prefill(p)
    got = s.generate(20)
    print(f"rel {rel(logits, want_logits):.3g}", flush=True)
    if flags & hip.EXACT:
        assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
        assert got.tolist() == want.tolist()
    else:
        err = rel(logits, want_logits)
        assert err < 5e-2
        check_fast_tokens(got, ref, p, 20, float(np.max(np.abs(logits - want_logits))), least=0 if flags == 0 else 5)


def check_generate_fast(w, ref, lm, cfg, monkeypatch, persistent):
    """Fast-mode greedy tokens (f16 caches, the default) against the
    oracle's and the per-kernel loop's, positions, a stop token, a second
    generate call that continues the first, and the caches the steps
    wrote."""
    p = synth.prompt(98, 40, cfg["vocab"])
    s = lm.session(96, 0)
    logits = s.prefill(p)
    got = s.generate(24)
    assert s.persistent == persistent
    assert len(got) == 24
    assert s.position == 40 + 23
    ref.reset()
    want_logits = ref.forward(p)
    assert rel(logits, want_logits) < 5e-2
    bound = float(np.max(np.abs(logits - want_logits)))
    check_fast_tokens(got, ref, p, 24, bound, least=0)

    # The per-kernel loop with the same f16 caches: the two differ only in
    # the order of the attention sums (rounding), so the greedy tokens agree.
    monkeypatch.setenv("TRIT_HIP_STEP", "0")
    k = lm.session(96, 0)
    k.prefill(p)
    kern = k.generate(24)
    assert not k.persistent
    monkeypatch.delenv("TRIT_HIP_STEP")
    print(f"step {got.tolist()}\nkernel {kern.tolist()}", flush=True)
    assert got.tolist() == kern.tolist()

    # The caches the steps wrote (every layer's keys and values of the 23
    # forwarded tokens carry the steps' activations): one more token through
    # the prompt path over them, against the per-kernel loop's caches and
    # the oracle fed the same tokens.
    nxt = np.array([int(got[-1])])
    after_step = s.prefill(nxt)
    after_kern = k.prefill(nxt)
    ref.reset()
    ref.forward(np.concatenate([p, got[:-1]]))
    want_after = ref.forward(nxt)
    print(f"after the steps: vs the per-kernel loop {rel(after_step, after_kern):.3g}, "
          f"vs the oracle {rel(after_step, want_after):.3g} (loop vs oracle {rel(after_kern, want_after):.3g})",
          flush=True)
    assert rel(after_step, after_kern) < 2e-2
    assert rel(after_step, want_after) < 5e-2

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


@pytest.mark.parametrize("attention", ["one-pass", "split"])
def test_step_fast(qshape, monkeypatch, attention):
    """The persistent decode step on Qwen3-0.6B's layer shapes, with each
    attention form: every key in one pass (up to 384 positions), or key
    splits and their combine."""
    print(f"case decoder persistent step (qwen3 shapes, {attention} attention)", flush=True)
    w, ref, lm = qshape
    if attention == "split":
        monkeypatch.setenv("TRIT_HIP_STEP_SPLIT", "1")
    check_generate_fast(w, ref, lm, QS, monkeypatch, persistent=True)


@pytest.mark.parametrize("m", [2, 4, 7])
def test_short_prompt(qshape, m):
    """Prompts of 2..8 rows run the few-row products (on Qwen3-0.6B's layer
    shapes: the streaming kernel with the SwiGLU pair and the residual
    epilogue, the rows quantized in the block or by the quantization pass):
    exact mode bit for bit against the oracle, fast mode within its bound."""
    print(f"case decoder short prompt ({m} rows)", flush=True)
    w, ref, lm = qshape
    p = synth.prompt(80 + m, m, QS["vocab"])
    ref.reset()
    want = ref.forward(p)
    s = lm.session(64, hip.EXACT)
    got = s.prefill(p)
    s.free()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rel(got, want)
    f = lm.session(64, 0)
    fast = f.prefill(p)
    f.free()
    print(f"fast vs oracle {rel(fast, want):.3g}", flush=True)
    assert rel(fast, want) < 5e-2


@pytest.mark.parametrize("prompt,steps,max_pos", [(330, 54, 384), (700, 40, 760)])
def test_step_fast_long(qshape, prompt, steps, max_pos):
    """Sessions at the one-pass attention's limit (384 positions: all 12
    chunks of 32 keys) and past it (the split attention takes over): the
    step's tokens against the oracle's up to the first near-tie, and the
    caches it wrote against the prompt path's fed the same tokens (so that
    a near-tie choice cannot make the two diverge)."""
    print(f"case decoder persistent step long (prompt {prompt}, {steps} steps, {max_pos} positions)", flush=True)
    w, ref, lm = qshape
    p = synth.prompt(97, prompt, QS["vocab"])
    s = lm.session(max_pos, 0)
    logits = s.prefill(p)
    got = s.generate(steps)
    assert s.persistent
    assert len(got) == steps and s.position == prompt + steps - 1
    ref.reset()
    want_logits = ref.forward(p)
    assert rel(logits, want_logits) < 5e-2
    check_fast_tokens(got, ref, p, steps, float(np.max(np.abs(logits - want_logits))), least=0)
    k = lm.session(max_pos, 0)
    k.prefill(np.concatenate([p, got[:-1]]), want_logits=False)
    nxt = np.array([int(got[-1])])
    after_step, after_prompt = s.prefill(nxt), k.prefill(nxt)
    print(f"after the steps: vs the prompt path {rel(after_step, after_prompt):.3g}", flush=True)
    assert rel(after_step, after_prompt) < 2e-2


@pytest.mark.parametrize("attention", ["one-pass", "split"])
def test_mid_step_fast(mid, monkeypatch, attention):
    """Four KV heads: four dims of one query head a block in the one-pass
    attention; the split form's combine would poll from too few waves for
    this model, so it runs the per-kernel loop (with the same checks)."""
    print(f"case decoder mid fast f16 caches ({attention})", flush=True)
    w, ref, lm = mid
    if attention == "split":
        monkeypatch.setenv("TRIT_HIP_STEP_SPLIT", "1")
    check_generate_fast(w, ref, lm, MID, monkeypatch, persistent=attention == "one-pass")


def test_mid_flash_prefill(mid, monkeypatch):
    """Prompt attention on the matrix cores (fast mode, f16 caches): logits
    against the oracle's and the split kernel's, a 300-row prompt (several
    64-key tiles, a partial 32-row query tile) at once and in two parts."""
    print("case decoder mid flash prefill", flush=True)
    w, ref, lm = mid
    p = synth.prompt(99, 300, MID["vocab"])
    ref.reset()
    want = ref.forward(p)
    s = lm.session(320, 0)
    got = s.prefill(p)
    parts = lm.session(320, 0)
    parts.prefill(p[:100])
    got_parts = parts.prefill(p[100:])
    monkeypatch.setenv("TRIT_HIP_FLASH", "0")
    k = lm.session(320, 0)
    split = k.prefill(p)
    monkeypatch.delenv("TRIT_HIP_FLASH")
    print(f"flash vs oracle {rel(got, want):.3g}, vs split {rel(got, split):.3g}, parts {rel(got_parts, got):.3g}, "
          f"split vs oracle {rel(split, want):.3g}", flush=True)
    assert rel(got, want) < 5e-2
    assert rel(got, split) < 2e-2
    assert rel(got_parts, got) < 2e-2
    assert int(np.argmax(got)) == int(np.argmax(split))


def test_mid_flash_prefill_long_rows(mid, monkeypatch):
    """Prompt attention over long rows (up to 1100 keys, 18 key tiles of 64):
    1100 rows at once and as 700 + 400 (a continuation whose query tiles
    start mid-way through the keys), against the oracle and the split
    kernel; every value finite."""
    print("case decoder mid flash prefill long rows", flush=True)
    w, ref, lm = mid
    p = synth.prompt(98, 1100, MID["vocab"])
    ref.reset()
    want = ref.forward(p)
    got = lm.session(1152, 0).prefill(p)
    parts = lm.session(1152, 0)
    parts.prefill(p[:700])
    got_parts = parts.prefill(p[700:])
    monkeypatch.setenv("TRIT_HIP_FLASH", "0")
    split = lm.session(1152, 0).prefill(p)
    monkeypatch.delenv("TRIT_HIP_FLASH")
    print(f"flash vs oracle {rel(got, want):.3g}, vs split {rel(got, split):.3g}, parts {rel(got_parts, got):.3g}",
          flush=True)
    assert np.all(np.isfinite(got)) and np.all(np.isfinite(got_parts))
    assert rel(got, want) < 5e-2
    assert rel(got, split) < 2e-2
    assert rel(got_parts, got) < 2e-2
    assert int(np.argmax(got)) == int(np.argmax(split))