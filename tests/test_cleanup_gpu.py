"""Transcript cleanup end to end (Trit's Cleaner, src/cleanup.rs): the
tokenizer, the system turn as a Prefix, the prompt of each call, the token
loop on the device until <|im_end|>, the decoded text -- against the
oracle's greedy tokens for the same prompt ids (a prefix gives the whole
prompt's keys and values), decoded by the same tokenizer."""

import numpy as np
import pytest

from oracle import oracle as O
from tests.test_tokenizer import corpus, train
from trit_amd import cleanup, hip, model, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup(gpu):
    pytest.importorskip("tokenizers")
    tok = train("qwen")
    bpe = hip.Bpe(text=tok.to_str())
    vocab = tok.get_vocab_size()
    cfg = dict(d=256, ffn=512, layers=2, heads=4, kv_heads=2, head_dim=64, vocab=vocab, eps=1e-6, rope_base=1e6,
               qk_norm=1)
    w = synth.lm_weights(cfg, config=130, sigma=0.2, norm_jitter=0.2)
    return cfg, w, bpe, model.build_decoder(w)


def oracle_clean(ref, bpe, cleaner, transcript, style=(2, 0, 0)):
    """Cleaner::clean_part on the oracle: generate over the whole prompt."""
    ids = bpe.cleanup_prompt(transcript, *style)
    budget = min(len(transcript.encode()) // 2 + 64, 1024)
    out, _ = ref.generate(np.array(ids, np.int32), budget, cleaner.stop)
    return bpe.decode(out.tolist()).strip(), out.tolist()


@pytest.mark.parametrize("flags", [0, hip.EXACT])
def test_cleanup_against_oracle(setup, flags):
    print(f"case cleanup end to end flags={flags}", flush=True)
    cfg, w, bpe, lm = setup
    ref = O.Lm(cfg, w, O.isa_best(), kv_f16=not flags)
    cleaner = cleanup.Cleaner(lm, bpe, flags)
    for i, transcript in enumerate(corpus(140, 3)):
        got = cleaner.clean(transcript)
        want, ids = oracle_clean(ref, bpe, cleaner, transcript.strip())
        print(f"  {len(ids)} tokens: {want[:60]!r}", flush=True)
        assert got == want, i
    # Style settings reach the prompt.
    got = cleaner.clean("so um we meet tomorrow", "formal", "lists", "email")
    want, _ = oracle_clean(ref, bpe, cleaner, "so um we meet tomorrow", (3, 1, 1))
    assert got == want
    assert cleaner.clean("   ") == ""
