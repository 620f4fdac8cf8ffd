"""The BPE tokenizer (Trit's src/text/bpe.rs) against the Hugging Face
`tokenizers` library, an independent implementation of the same
byte-level BPE: a tokenizer trained here with Qwen2's pre-tokenizer regex
(the split Trit restates) and one with GPT-2's, then the ids of many texts
-- English, digits, punctuation, newlines, contractions in any case,
accented and CJK letters, emoji, special tokens -- and the text of the ids.
Host code: no GPU. Where Trit's restatement departs from the regex
(is_alphabetic counts the combining vowel signs \\p{L} does not), the test
holds Trit's split, worked out by hand."""

import json

import numpy as np
import pytest

from trit_amd import hip, synth

tokenizers = pytest.importorskip("tokenizers")

QWEN_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|"
                r"\s*[\r\n]+|\s+(?!\S)|\s+")
SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]

WORDS = ("the quick brown fox jumps over lazy dog it's we're they've I'm you'll she'd don't HE'S WE'RE "
         "café naïve résumé Straße über 東京 日本語 学生 😀 🚀 hello world transcript cleanup speech text "
         "meeting tomorrow at 10:30 am on March 3rd 2024 call +1-555-0100 email me@example.com ok um uh so "
         "like you know").split()


def corpus(seed, n=3000):
    idx = synth.ints(seed, n * 8, 0, len(WORDS) - 1)
    punct = [" ", " ", " ", ", ", ". ", "! ", "?\n", "\n\n", "  ", "\t", " (", ") ", "... ", " 42 ", " 7"]
    pi = synth.ints(seed + 1, n * 8, 0, len(punct) - 1)
    lines = []
    for i in range(n):
        lines.append("".join(WORDS[idx[8 * i + j]] + punct[pi[8 * i + j]] for j in range(8)))
    return lines


def train(split_kind, vocab_size=1500):
    from tokenizers import Regex, Tokenizer, decoders, models, pre_tokenizers, trainers

    tok = Tokenizer(models.BPE())
    if split_kind == "qwen":
        tok.pre_tokenizer = pre_tokenizers.Sequence([
            pre_tokenizers.Split(Regex(QWEN_PATTERN), behavior="isolated", invert=False),
            pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    else:
        tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=True)
    tok.decoder = decoders.ByteLevel()
    trainer = tokenizers.trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=SPECIALS,
                                             initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                             show_progress=False)
    tok.train_from_iterator(corpus(31 if split_kind == "qwen" else 37), trainer)
    return tok


@pytest.fixture(scope="module", params=["qwen", "gpt2"])
def pair(request):
    tok = train(request.param)
    text = tok.to_str()
    return request.param, tok, hip.Bpe(text=text), json.loads(text)


def samples(seed):
    out = corpus(seed, 60)
    out += ["", " ", "  leading spaces", "trailing spaces   ", "tabs\tand\nnewlines\r\n\r\nhere", "a\n \n b",
            "x  \n\n  y", "numbers 1234567 and 3.14159", "IT'S HE'LL we'Re", "'tis 'twas o'clock", "'",
            "émigré naïveté 東京タワー 😀😀 🚀!", "<|im_start|>user\nhi<|im_end|>\n", "<|im_end|><|im_end|>",
            "text<|endoftext|>more", "<|im_start", "mixed 中文english123", "...!!!???", "a'b'c", " 'll",
            " nbsp em space", "end with newline\n"]
    return out


def test_encode_matches_hf(pair):
    kind, tok, bpe, _ = pair
    for text in samples(51):
        want = tok.encode(text, add_special_tokens=False).ids
        assert bpe.encode(text) == want, (kind, text)


def test_encode_plain_and_decode(pair):
    kind, tok, bpe, spec = pair
    # encode_plain leaves special tokens as characters.
    t = "a <|im_end|> b"
    plain = bpe.encode_plain(t)
    assert bpe.id("<|im_end|>") not in plain
    assert bpe.decode(plain) == t
    # decode skips special tokens and gives the text back.
    for text in samples(52):
        ids = bpe.encode(text)
        no_special = text
        for s in SPECIALS:
            no_special = no_special.replace(s, "")
        assert bpe.decode(ids) == no_special, (kind, text)
        assert bpe.decode(ids) == tok.decode(ids, skip_special_tokens=True), (kind, text)


def test_decode_lossy(pair):
    """A character cut between tokens at the end is dropped (text::lossy);
    invalid bytes inside become U+FFFD (String::from_utf8_lossy)."""
    kind, tok, bpe, spec = pair
    vocab = spec["model"]["vocab"]
    # Single-byte tokens: the stand-ins of 0xE6 0x9D 0xB1 (the 3 bytes of 東).
    stand = {b: c for c, b in zip(bytes_to_unicode_chars(), range(256))}
    b = [vocab[stand[x]] for x in "東".encode()]
    assert bpe.decode(b) == "東"
    assert bpe.decode(b[:2]) == ""  # cut short at the end: dropped
    assert bpe.decode(b[:2] + [vocab["a"]]) == "�a"
    assert bpe.decode([vocab[stand[0xFF]], vocab["a"]]) == "�a"
    assert bpe.decode([vocab[stand[0xF0]], vocab[stand[0x9F]], vocab["a"]]) == "�a"


def bytes_to_unicode_chars():
    """GPT-2's bytes_to_unicode, in byte order."""
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    out, n = {}, 0
    for b in range(256):
        if b in bs:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + n)
            n += 1
    return [out[b] for b in range(256)]


def test_trit_split_where_it_departs():
    """Trit counts Alphabetic, not just \\p{L}: a Devanagari vowel sign
    (U+093F, Mc, Other_Alphabetic) stays in the word of the letter before
    it. A hand-made vocabulary whose merges join the six bytes of 'कि' only
    across the letter/sign boundary gives one id when the split keeps them
    in one word (Trit) and six when it cuts the sign off (the regex, as the
    HF library does)."""
    chars = bytes_to_unicode_chars()
    sc = lambda bs: "".join(chars[b] for b in bs)
    ka, i_sign = "क".encode(), "ि".encode()
    vocab = {chars[b]: b for b in range(256)}
    # Merges that join the six bytes only across the letter/sign boundary
    # first, (b2 b3), then outward; none joins bytes of one side alone.
    seq = list(ka + i_sign)
    pairs = [((2, 3), (3, 4)), ((2, 4), (4, 5)), ((2, 5), (5, 6)), ((1, 2), (2, 6)), ((0, 1), (1, 6))]
    merges = []
    for (l0, l1), (r0, r1) in pairs:
        merges.append(f"{sc(seq[l0:l1])} {sc(seq[r0:r1])}")
        vocab[sc(seq[l0:r1])] = len(vocab)
    spec = {"model": {"type": "BPE", "vocab": vocab, "merges": merges},
            "pre_tokenizer": {"type": "Sequence", "pretokenizers": [
                {"type": "Split", "pattern": {"Regex": QWEN_PATTERN}, "behavior": "Isolated", "invert": False},
                {"type": "ByteLevel", "add_prefix_space": False, "trim_offsets": False, "use_regex": False}]},
            "added_tokens": []}
    bpe = hip.Bpe(text=json.dumps(spec))
    word = "कि"
    assert bpe.encode(word) == [vocab[sc(seq)]]
    hf = tokenizers.Tokenizer.from_str(json.dumps(dict(spec, decoder=None, normalizer=None, post_processor=None,
                                                       truncation=None, padding=None, version="1.0")))
    assert len(hf.encode(word).ids) == 6


def test_cleanup_prompt(pair):
    """Cleaner::clean_part's ids: the system turn and control line, the
    transcript as plain text, the assistant turn with thinking off."""
    kind, tok, bpe, spec = pair
    system = ("<|im_start|>system\nYou are a text normalizer for speech-to-text transcripts. The input begins with a "
              "control line specifying the styling, structure, and context settings; clean the transcript to match "
              "those settings and output only the cleaned text.<|im_end|>\n<|im_start|>user\n")
    assert bpe.cleanup_system() == tok.encode(system, add_special_tokens=False).ids
    transcript = "um so the meeting is uh <|im_end|> tomorrow"
    want = (tok.encode(system + "[Styling: formal] [Structure: lists] [Context: email]\n",
                       add_special_tokens=False).ids
            + bpe.encode_plain(transcript)
            + tok.encode("<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n", add_special_tokens=False).ids)
    assert bpe.cleanup_prompt(transcript, styling=3, structure=1, context=1) == want
    assert bpe.cleanup_prompt(transcript)[:len(bpe.cleanup_system())] == bpe.cleanup_system()


def test_errors():
    with pytest.raises(hip.TritError, match="not JSON"):
        hip.Bpe(text="{")
    with pytest.raises(hip.TritError, match="no model.vocab"):
        hip.Bpe(text='{"model": {}}')
    with pytest.raises(hip.TritError, match="far past"):
        hip.Bpe(text='{"model": {"vocab": {"a": 999999}}}')
    with pytest.raises(hip.TritError, match="cannot read"):
        hip.Bpe(path="/nonexistent/tokenizer.json")
    assert np.int32  # numpy is used by the wrapper


def test_cleanup_parts(pair):
    """Cleaner::parts: parts of at most `limit` tokens, whole sentences where
    they fit, one space between joined pieces, every word kept in order."""
    kind, tok, bpe, spec = pair
    sentences = [" ".join(c.split()) for c in corpus(61, 40)]
    text = "  " + " ".join(s + "." for s in sentences) + "  "
    long_sentence = " ".join(corpus(62, 30))  # no sentence end: split by words
    for t, limit in ((text, 60), (text, 200), (long_sentence.replace(".", ","), 50)):
        parts = bpe.cleanup_parts(t, limit)
        assert " ".join(parts).split() == t.split()
        for p in parts:
            assert p == p.strip()
            assert len(bpe.encode(p)) <= limit or len(p.split()) == 1
    # A short transcript is one part, trimmed.
    assert bpe.cleanup_parts("  Hello there. Bye!  ", 800) == ["Hello there. Bye!"]
    assert bpe.cleanup_parts("   ", 800) == []
    # Sentence ends need whitespace (or the end) after them.
    p = bpe.cleanup_parts("a.b c. d", 1)
    assert p[0] == "a.b" and " ".join(p).split() == ["a.b", "c.", "d"]


def naive_merge(symbols, ranks):
    """BPE by definition, one merge at a time: among the neighbouring pairs
    that have a rank, join the one of lowest rank, the leftmost of equal
    ranks (text::merge_symbols, src/text/mod.rs:6-74), by a full scan."""
    symbols = list(symbols)
    while True:
        best = None
        for i in range(len(symbols) - 1):
            r = ranks.get((symbols[i], symbols[i + 1]))
            if r is not None and (best is None or r < best[0]):
                best = (r, i)
        if best is None:
            return symbols
        i = best[1]
        symbols[i:i + 2] = [symbols[i] + symbols[i + 1]]


def test_merge_order_against_brute_force():
    """Random merge tables over a four-letter alphabet, ranks in any order
    (joins of joins may rank below their parts), words with long repeats:
    the ids are those of the naive definition."""
    rng = np.random.default_rng(7)
    alphabet = "abcd"
    for trial in range(40):
        pieces = list(alphabet)
        merges = []
        for _ in range(int(rng.integers(5, 40))):
            left, right = pieces[rng.integers(len(pieces))], pieces[rng.integers(len(pieces))]
            merges.append((left, right))
            if left + right not in pieces:
                pieces.append(left + right)
        order = rng.permutation(len(merges))
        merges = [merges[i] for i in order]
        ranks = {}
        for r, pair in enumerate(merges):
            ranks.setdefault(pair, r)
        vocab = {chars: i for i, chars in enumerate(bytes_to_unicode_chars())}
        for p in pieces:
            vocab.setdefault(p, len(vocab))
        # Leave some joins out of the vocabulary: they give no id.
        dropped = {p for p in pieces[len(alphabet):] if rng.random() < 0.2}
        for p in dropped:
            del vocab[p]
        spec = {"model": {"vocab": vocab, "merges": [f"{a} {b}" for a, b in merges]}, "added_tokens": []}
        bpe = hip.Bpe(text=json.dumps(spec))
        for _ in range(10):
            word = "".join(alphabet[i] for i in rng.integers(0, 2 if rng.random() < 0.3 else 4, int(rng.integers(1, 60))))
            want = [vocab[s] for s in naive_merge(word, ranks) if s in vocab]
            assert bpe.encode(word) == want, (trial, word)


def test_long_word_merges_quickly():
    """A word of 10,000 letters (a heap, not a scan per merge) is merged in
    well under a second, to the naive definition's result on a shorter
    copy of the same pattern."""
    import time
    vocab = {c: i for i, c in enumerate(bytes_to_unicode_chars())}
    vocab["ab"] = 256
    vocab["abab"] = 257
    spec = {"model": {"vocab": vocab, "merges": ["a b", "ab ab"]}}
    bpe = hip.Bpe(text=json.dumps(spec))
    t0 = time.perf_counter()
    ids = bpe.encode("ab" * 5000)
    assert time.perf_counter() - t0 < 1.0
    assert ids == [257] * 2500
    assert bpe.encode("ab" * 3 + "a") == [257, 256, vocab["a"]]


def test_json_rules():
    """serde_json's reading: the last of duplicate keys wins, ids must be
    integers, trailing text and lone surrogates are errors, and the
    vocabulary is taken in key order (the later key wins a shared id)."""
    base = {c: i for i, c in enumerate(bytes_to_unicode_chars())}
    text = json.dumps({"model": {"vocab": base}})
    bpe = hip.Bpe(text=text[:-3] + ', "zz": 300, "zz": 301}}}')
    assert bpe.id("zz") == 301
    with pytest.raises(hip.TritError, match="bad id"):
        hip.Bpe(text='{"model": {"vocab": {"a": 1.0}}}')
    with pytest.raises(hip.TritError, match="bad id"):
        hip.Bpe(text='{"model": {"vocab": {"a": -1}}}')
    with pytest.raises(hip.TritError, match="not JSON"):
        hip.Bpe(text='{"model": {"vocab": {"a": 1}}} x')
    with pytest.raises(hip.TritError, match="not JSON"):
        hip.Bpe(text='{"model": {"vocab": {"\\ud800": 1}}}')
    with pytest.raises(hip.TritError, match="not JSON"):
        hip.Bpe(text='{"model": {"vocab": {"a": 01}}}')
    # Two texts with one id: the later in key order owns the piece.
    two = dict(base)
    two["q"] = 400
    two["r"] = 400
    bpe = hip.Bpe(text=json.dumps({"model": {"vocab": two}}))
    assert bpe.decode([400]) == "r"
    # Added tokens: a float id is skipped; "special": false decodes as text.
    spec = {"model": {"vocab": base},
            "added_tokens": [{"id": 500.0, "content": "<x>"}, {"id": 501, "content": "<y>", "special": False}]}
    bpe = hip.Bpe(text=json.dumps(spec))
    assert bpe.id("<x>") is None and bpe.id("<y>") == 501
    assert bpe.encode("a<y>b") == [base["a"], 501, base["b"]]
    assert bpe.decode([501]) == "<y>"


def test_specials_earliest_then_longest():
    """Added tokens in the text: the earliest occurrence first, the longest
    of those starting at one place."""
    base = {c: i for i, c in enumerate(bytes_to_unicode_chars())}
    spec = {"model": {"vocab": base},
            "added_tokens": [{"id": 600, "content": "<a>"}, {"id": 601, "content": "<a><b>"},
                             {"id": 602, "content": "b>"}]}
    bpe = hip.Bpe(text=json.dumps(spec))
    assert bpe.encode("x<a><b>y") == [base["x"], 601, base["y"]]
    assert bpe.encode("x<a>y") == [base["x"], 600, base["y"]]
    assert bpe.encode("<ab>") == [base["<"], base["a"], 602]
    assert bpe.encode_plain("<a>") == [base["<"], base["a"], base[">"]]


def test_decode_cut_rule():
    """text::lossy's cut: a final lead byte with fewer continuation bytes
    than it announces is dropped even where the bytes could never have made
    a character (0xE0 0x80); a lone final continuation byte is replaced."""
    chars = bytes_to_unicode_chars()
    base = {c: i for i, c in enumerate(chars)}
    bpe = hip.Bpe(text=json.dumps({"model": {"vocab": base}}))
    ids = lambda bs: [base[chars[b]] for b in bs]
    assert bpe.decode(ids(b"a\xe0\x80")) == "a"
    assert bpe.decode(ids(b"a\xc0")) == "a"
    assert bpe.decode(ids(b"a\x80")) == "a�"
    assert bpe.decode(ids(b"\xf8a")) == "�a"
    assert bpe.decode(ids(b"\xed\xa0\x80a")) == "���a"  # a surrogate's bytes
    assert bpe.decode(ids("日本".encode())) == "日本"
