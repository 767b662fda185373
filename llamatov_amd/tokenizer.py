"""Byte-level BPE tokenizer built from a GGUF file's embedded vocabulary and merge list: the
reference's bpd/lib/qwen_bpe.py (QwenBPE(blob).encode / .decode, :19-66), with the same
behaviour on the same file:

  * text -> UTF-8 bytes -> one printable character per byte (the GPT-2 byte alphabet: the
    188 printable Latin-1 bytes stand for themselves, the other 68 bytes map in byte order to
    U+0100 .. U+0143; qwen_bpe.py:10-17), so a space becomes U+0120;
  * pre-tokenization: a new chunk starts at every U+0120 that follows a non-empty chunk
    (qwen_bpe.py:40-50; the reference's stand-in for the GPT-2 regex);
  * per chunk, merges applied one at a time: the adjacent pair of lowest merge rank, the
    leftmost such pair on equal rank, until no adjacent pair is in the merge list
    (qwen_bpe.py:27-35);
  * each resulting piece becomes its vocabulary id; a piece missing from the vocabulary falls
    back to the ids of its characters, characters missing too are dropped (:51-56);
  * decode joins the token strings and maps each character back to its byte (a character
    outside the byte alphabet stands for its own code point, which raises ValueError above
    255, as the reference's bytes() does), then decodes UTF-8 with replacement (:60-63).

The merge loop keeps a rank per adjacent pair and updates only the two neighbours of each
merge, so a chunk of n symbols costs O(n) rank lookups per merge instead of re-ranking every
pair.
"""
from __future__ import annotations

from .gguf import parse_gguf

_NO_MERGE = 1 << 62


def byte_alphabet() -> dict[int, str]:
    """byte -> character of the GPT-2 byte-level alphabet."""
    keep = [b for b in range(256) if 0x21 <= b <= 0x7E or 0xA1 <= b <= 0xAC or 0xAE <= b <= 0xFF]
    kept = set(keep)
    out = {b: chr(b) for b in keep}
    extra = 0
    for b in range(256):
        if b not in kept:
            out[b] = chr(0x100 + extra)
            extra += 1
    return out


class QwenBPE:
    """QwenBPE(blob): blob is the path of a GGUF file whose metadata holds
    tokenizer.ggml.tokens and tokenizer.ggml.merges."""

    def __init__(self, blob=None, *, tokens=None, merges=None):
        if blob is not None:
            md, _, _ = parse_gguf(blob)
            tokens = md["tokenizer.ggml.tokens"]
            merges = md["tokenizer.ggml.merges"]
        if tokens is None or merges is None:
            raise ValueError("QwenBPE needs a GGUF path or tokens= and merges=")
        self.tokens = list(tokens)
        self.tok2id = {}
        for i, t in enumerate(self.tokens):   # a repeated string keeps its last id
            self.tok2id[t] = i
        self.merge_rank = {}
        for i, m in enumerate(merges):     # "left right" (a key of another arity never matches)
            self.merge_rank[tuple(m.split(" "))] = i
        self.b2u = byte_alphabet()
        self.u2b = {c: b for b, c in self.b2u.items()}

    # -- merging ---------------------------------------------------------------------
    def _rank(self, a: str, b: str) -> int:
        return self.merge_rank.get((a, b), _NO_MERGE)

    def _bpe(self, chunk: str) -> list[str]:
        sym = list(chunk)
        if len(sym) < 2:
            return sym
        ranks = [self._rank(sym[i], sym[i + 1]) for i in range(len(sym) - 1)]
        while ranks:
            best = min(ranks)
            if best == _NO_MERGE:
                break
            i = ranks.index(best)            # leftmost pair of the lowest rank
            sym[i:i + 2] = [sym[i] + sym[i + 1]]
            del ranks[i]
            if i < len(ranks):               # the pair (merged, right neighbour)
                ranks[i] = self._rank(sym[i], sym[i + 1])
            if i > 0:                        # the pair (left neighbour, merged)
                ranks[i - 1] = self._rank(sym[i - 1], sym[i])
        return sym

    # -- the reference interface -----------------------------------------------------
    def chunks(self, text: str) -> list[str]:
        mapped = "".join(self.b2u[b] for b in text.encode("utf-8"))
        out, cur = [], ""
        for ch in mapped:
            if ch == "Ġ" and cur:
                out.append(cur)
                cur = ch
            else:
                cur += ch
        if cur:
            out.append(cur)
        return out

    def encode(self, text: str) -> list[int]:
        ids: list[int] = []
        for chunk in self.chunks(text):
            for piece in self._bpe(chunk):
                tid = self.tok2id.get(piece)
                if tid is not None:
                    ids.append(tid)
                else:
                    ids.extend(self.tok2id[c] for c in piece if c in self.tok2id)
        return ids

    def decode(self, ids) -> str:
        s = "".join(self.tokens[int(i)] for i in ids)
        return bytes(self.u2b.get(c, ord(c)) for c in s).decode("utf-8", errors="replace")
