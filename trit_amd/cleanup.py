"""Transcript cleanup with an S1-mini-style decoder, as Trit's Cleaner runs
it (src/cleanup.rs:160-301): the fixed system turn made once as a Prefix,
then per call the control line, the transcript as plain text and the
assistant turn, greedy tokens until <|im_end|> or <|endoftext|>, decoded
and trimmed. A transcript longer than 800 tokens is cleaned in parts.
Everything runs through the C ABI: the tokenizer and the prompt in host
code, the token loop on the device."""

from __future__ import annotations

from . import hip

PART_TOKENS = 800
STYLING = ("casual", "semi-casual", "semi-formal", "formal")
STRUCTURE = ("prose", "lists")
CONTEXT = ("general", "email")


class Cleaner:
    """Cleaner::load_now (src/cleanup.rs:187-215) from a decoder and a
    tokenizer already loaded."""

    def __init__(self, lm: hip.CausalLm, bpe: hip.Bpe, flags: int = 0):
        self.lm, self.bpe, self.flags = lm, bpe, flags
        self.stop = [i for i in (bpe.id("<|im_end|>"), bpe.id("<|endoftext|>")) if i is not None]
        if not self.stop:
            raise hip.TritError("the tokenizer has no <|im_end|> token; it is not a chat model")
        self.system = lm.prefix(bpe.cleanup_system(), flags)

    def clean(self, transcript: str, styling="semi-formal", structure="prose", context="general") -> str:
        """Cleaner::clean (src/cleanup.rs:219-236)."""
        style = (STYLING.index(styling), STRUCTURE.index(structure), CONTEXT.index(context))
        transcript = transcript.strip()
        if not transcript:
            return ""
        if len(self.bpe.encode(transcript)) <= PART_TOKENS:
            return self.clean_part(transcript, style)
        parts = [self.clean_part(p, style) for p in self.bpe.cleanup_parts(transcript, PART_TOKENS)]
        return " ".join(p for p in parts if p)

    def clean_part(self, transcript: str, style) -> str:
        """Cleaner::clean_part (src/cleanup.rs:280-301)."""
        ids = self.bpe.cleanup_prompt(transcript, *style)
        budget = min(len(transcript.encode()) // 2 + 64, 1024)
        out = self.lm.generate(ids, budget, self.stop, flags=self.flags, prefix=self.system)
        return self.bpe.decode(out).strip()
