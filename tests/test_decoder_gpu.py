"""The device token loop against the oracle's CausalLm.

Exact mode must give the oracle's logits bit for bit and its greedy tokens.
Fast mode sums norms and attention in other orders and keeps f16 keys and
values: it must give logits within 1e-3 relative of the oracle run with the
same f16 caches (each appended key and value rounded through f16, the
oracle's kv_f16) and the same greedy tokens at every step. KV_F32 sessions
are held to the same bar against Trit's f32 caches.
"""

import numpy as np
import pytest

from oracle import oracle as O
from trit_amd import hip, model, synth

pytestmark = pytest.mark.gpu

RTOL = 1e-3

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


def test_mid_generate_fast(mid):
    print("case decoder mid fast", flush=True)
    w, ref, lm, _ = mid
    p = synth.prompt(97, 40, MID["vocab"])
    s = lm.session(80, hip.KV_F32)
    logits = s.prefill(p)
    got = s.generate(24)
    ref.reset()
    want_logits = ref.forward(p)
    assert rel(logits, want_logits) < RTOL
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


@pytest.mark.parametrize("flags", [hip.EXACT, 0, hip.KV_F32])
def test_generate(small, flags):
    print(f"case decoder generate flags={flags}", flush=True)
    w, ref32, lm, ref16 = small
    ref = ref32 if flags else ref16
    p = synth.prompt(92, 25, SMALL["vocab"])
    want, want_logits = ref.generate(p, 30)
    s = lm.session(64, flags)
    logits = s.prefill(p)
    got = s.generate(30)
    print(f"rel {rel(logits, want_logits):.3g} tokens {got.tolist()[:10]} want {want.tolist()[:10]}", flush=True)
    if flags & hip.EXACT:
        assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
    else:
        # Tree sums in place of Trit's serial ones; f16 caches against the
        # oracle with the same f16 caches.
        assert rel(logits, want_logits) < RTOL
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


@pytest.mark.parametrize("flags", [0, hip.EXACT, hip.KV_F32])
def test_generate_long_prompt(small, flags):
    """Prompts over several 64-key attention splits."""
    print(f"case decoder long prompt flags={flags}", flush=True)
    w, ref32, lm, ref16 = small
    ref = ref32 if flags else ref16
    p = synth.prompt(95, 150, SMALL["vocab"])
    want, want_logits = ref.generate(p, 20)
    s = lm.session(200, flags)
    logits = s.prefill(p)
    got = s.generate(20)
    print(f"rel {rel(logits, want_logits):.3g}", flush=True)
    if flags & hip.EXACT:
        assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
    else:
        assert rel(logits, want_logits) < RTOL
    assert got.tolist() == want.tolist()


def check_generate_fast(w, ref16, lm, cfg, monkeypatch, persistent):
    """Fast-mode greedy tokens (f16 caches, the default) against the
    f16-cache oracle's and the per-kernel loop's, positions, a stop token, a
    second generate call that continues the first, and the caches the steps
    wrote."""
    p = synth.prompt(98, 40, cfg["vocab"])
    s = lm.session(96, 0)
    logits = s.prefill(p)
    got = s.generate(24)
    assert s.persistent == persistent
    assert len(got) == 24
    assert s.position == 40 + 23
    ref16.reset()
    want_logits = ref16.forward(p)
    print(f"prompt logits vs the oracle {rel(logits, want_logits):.3g}", flush=True)
    assert rel(logits, want_logits) < RTOL
    check_tokens(got, ref16, p, 24)

    # The per-kernel loop with the same f16 caches gives the same tokens.
    monkeypatch.setenv("TRIT_HIP_STEP", "0")
    k = lm.session(96, 0)
    k.prefill(p)
    kern = k.generate(24)
    assert not k.persistent
    monkeypatch.delenv("TRIT_HIP_STEP")
    assert got.tolist() == kern.tolist()

    # The caches the steps wrote (every layer's keys and values of the 23
    # forwarded tokens carry the steps' activations): one more token through
    # the prompt path over them, against the per-kernel loop's caches and
    # the oracle fed the same tokens.
    nxt = np.array([int(got[-1])])
    after_step = s.prefill(nxt)
    after_kern = k.prefill(nxt)
    ref16.reset()
    ref16.forward(np.concatenate([p, got[:-1]]))
    want_after = ref16.forward(nxt)
    print(f"after the steps: vs the per-kernel loop {rel(after_step, after_kern):.3g}, "
          f"vs the oracle {rel(after_step, want_after):.3g} (loop vs oracle {rel(after_kern, want_after):.3g})",
          flush=True)
    assert rel(after_step, after_kern) < RTOL
    assert rel(after_step, want_after) < RTOL

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
    w, ref, lm, ref16 = qshape
    if attention == "split":
        monkeypatch.setenv("TRIT_HIP_STEP_SPLIT", "1")
    check_generate_fast(w, ref16, lm, QS, monkeypatch, persistent=True)


@pytest.mark.parametrize("m", [2, 4, 7, 8])
def test_short_prompt(qshape, m):
    """Prompts of 2..8 rows run the few-row products (on Qwen3-0.6B's layer
    shapes: the streaming kernel with the SwiGLU pair and the residual
    epilogue, the rows quantized in the block or by the quantization pass):
    exact mode bit for bit against the oracle, fast mode within 1e-3 of the
    f16-cache oracle."""
    print(f"case decoder short prompt ({m} rows)", flush=True)
    w, ref, lm, ref16 = qshape
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
    ref16.reset()
    want16 = ref16.forward(p)
    print(f"fast vs oracle {rel(fast, want16):.3g}", flush=True)
    assert rel(fast, want16) < RTOL


@pytest.mark.parametrize("prompt,steps,max_pos", [(330, 54, 384), (700, 40, 760)])
def test_step_fast_long(qshape, prompt, steps, max_pos):
    """Sessions at the one-pass attention's limit (384 positions: all 12
    chunks of 32 keys) and past it (the split attention takes over): the
    step's tokens against the f16-cache oracle's at every step, and the
    caches it wrote against the prompt path's fed the same tokens."""
    print(f"case decoder persistent step long (prompt {prompt}, {steps} steps, {max_pos} positions)", flush=True)
    w, ref, lm, ref16 = qshape
    p = synth.prompt(97, prompt, QS["vocab"])
    s = lm.session(max_pos, 0)
    logits = s.prefill(p)
    got = s.generate(steps)
    assert s.persistent
    assert len(got) == steps and s.position == prompt + steps - 1
    ref16.reset()
    want_logits = ref16.forward(p)
    assert rel(logits, want_logits) < RTOL
    check_tokens(got, ref16, p, steps)
    k = lm.session(max_pos, 0)
    k.prefill(np.concatenate([p, got[:-1]]), want_logits=False)
    nxt = np.array([int(got[-1])])
    after_step, after_prompt = s.prefill(nxt), k.prefill(nxt)
    print(f"after the steps: vs the prompt path {rel(after_step, after_prompt):.3g}", flush=True)
    assert rel(after_step, after_prompt) < RTOL


@pytest.mark.parametrize("attention", ["one-pass", "split"])
def test_mid_step_fast(mid, monkeypatch, attention):
    """Four KV heads: four dims of one query head a block in the one-pass
    attention; the split form's combine would poll from too few waves for
    this model, so it runs the per-kernel loop (with the same checks)."""
    print(f"case decoder mid fast f16 caches ({attention})", flush=True)
    w, ref, lm, ref16 = mid
    if attention == "split":
        monkeypatch.setenv("TRIT_HIP_STEP_SPLIT", "1")
    check_generate_fast(w, ref16, lm, MID, monkeypatch, persistent=attention == "one-pass")


def test_mid_flash_prefill(mid, monkeypatch):
    """Prompt attention on the matrix cores (fast mode, f16 caches): logits
    against the f16-cache oracle's and the split kernel's, a 300-row prompt
    (several 64-key tiles, a partial 32-row query tile) at once and in two
    parts."""
    print("case decoder mid flash prefill", flush=True)
    w, ref, lm, ref16 = mid
    p = synth.prompt(99, 300, MID["vocab"])
    ref16.reset()
    want = ref16.forward(p)
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
    assert rel(got, want) < RTOL
    assert rel(split, want) < RTOL
    assert rel(got_parts, want) < RTOL
    assert int(np.argmax(got)) == int(np.argmax(want))


def test_mid_flash_prefill_long_rows(mid, monkeypatch):
    """Prompt attention over long rows (up to 1100 keys, 18 key tiles of 64):
    1100 rows at once and as 700 + 400 (a continuation whose query tiles
    start mid-way through the keys), against the f16-cache oracle and the
    split kernel; every value finite."""
    print("case decoder mid flash prefill long rows", flush=True)
    w, ref, lm, ref16 = mid
    p = synth.prompt(98, 1100, MID["vocab"])
    ref16.reset()
    want = ref16.forward(p)
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
    assert rel(got, want) < RTOL
    assert rel(split, want) < RTOL
    assert rel(got_parts, want) < RTOL


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
    precision): exact mode bit for bit, fast mode within 1e-3 of the
    f16-cache oracle, greedy tokens identical in both."""
    print("case decoder int8-128 linears", flush=True)
    w, _, _, _ = small
    ref, ref16, lm = int8_decoder(w, SMALL, 88)
    p = synth.prompt(88, 30, SMALL["vocab"])
    want, want_logits = ref.generate(p, 16)
    s = lm.session(64, hip.EXACT)
    logits = s.prefill(p)
    got = s.generate(16)
    assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32)), rel(logits, want_logits)
    assert got.tolist() == want.tolist()
    want16, want16_logits = ref16.generate(p, 16)
    f = lm.session(64, 0)
    fl = f.prefill(p)
    fast = f.generate(16)
    print(f"fast vs oracle {rel(fl, want16_logits):.3g}", flush=True)
    assert rel(fl, want16_logits) < RTOL
    assert fast.tolist() == want16.tolist()


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
    256-token prompt, 128 greedy steps on the persistent step (f16 caches).
    "config": the configuration's weights (Q8_0 scales N(0, 0.02)/127, unit
    norms), whose greedy stream settles on one token; "lively": scales
    N(0, 0.1)/127 and norms 1 +- 0.2, a stream of 128 different tokens in
    which any error of the loop would change the tokens that follow.
    Prompt logits within 1e-3 of the f16-cache oracle; all 128 tokens equal
    to its tokens (and, with the configuration's weights, to Trit's with
    f32 caches); the caches the steps wrote give the oracle's logits for one
    more token."""
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
    print(f"prompt logits vs the f16-cache oracle {rel(logits, want16_logits):.3g}", flush=True)
    assert rel(logits, want16_logits) < RTOL
    print(f"{len(set(got.tolist()))} distinct tokens", flush=True)
    check_tokens(got, ref16, p, 128)
    nxt = np.array([int(got[-1])])
    after = s.prefill(nxt)
    ref16.reset()
    ref16.forward(np.concatenate([p, got[:-1]]))
    want_after = ref16.forward(nxt)
    print(f"after the 128 steps vs the oracle {rel(after, want_after):.3g}", flush=True)
    assert rel(after, want_after) < RTOL
    del ref16
    if weights == "config":
        ref32 = O.Lm(cfg, w, isa)
        want32, _ = ref32.generate(p, 128)
        assert got.tolist() == want32.tolist()
