"""The byte-level BPE tokenizer (llamatov_amd/tokenizer.py, the reference's
bpd/lib/qwen_bpe.py interface): the GPT-2 byte alphabet's closed form, hand-worked merges,
the pre-tokenizer's chunking, the vocabulary fallback, UTF-8 round trips, the GGUF metadata
path, and agreement with the definition (re-rank every pair, take the lowest rank, leftmost
on ties) on random merge lists."""
import random

import pytest

from llamatov_amd import gguf
from llamatov_amd.tokenizer import QwenBPE, byte_alphabet


def base_tokens():
    return [byte_alphabet()[b] for b in range(256)]


def test_byte_alphabet_closed_form():
    m = byte_alphabet()
    assert len(set(m.values())) == 256
    assert m[ord("A")] == "A" and m[ord("~")] == "~" and m[0xE9] == "é"
    assert m[0x20] == "Ġ" and m[0x0A] == "Ċ" and m[0x00] == "Ā"
    assert m[0x7F] == "ġ" and m[0xA0] == "ł" and m[0xAD] == "Ń"
    assert sum(1 for b, c in m.items() if ord(c) == b) == 188


def test_hand_worked_merges():
    merges = ["h e", "l l", "he ll", "hell o", "Ġ w", "o r", "Ġw or", "Ġwor l", "Ġworl d"]
    tokens = base_tokens() + ["he", "ll", "hell", "hello", "Ġw", "or", "Ġwor", "Ġworl", "Ġworld"]
    t = QwenBPE(tokens=tokens, merges=merges)
    assert t.chunks("hello world") == ["hello", "Ġworld"]
    assert t.encode("hello world") == [tokens.index("hello"), tokens.index("Ġworld")]
    assert t.decode(t.encode("hello world")) == "hello world"
    # one merge at a time, leftmost first: "aaa" -> [aa, a]; "aaaa" -> [aa, aa]
    t2 = QwenBPE(tokens=base_tokens() + ["aa"], merges=["a a"])
    assert t2._bpe("aaa") == ["aa", "a"] and t2._bpe("aaaa") == ["aa", "aa"]
    # a merged piece missing from the vocabulary falls back to its characters
    t3 = QwenBPE(tokens=base_tokens(), merges=["a b"])
    assert t3._bpe("ab") == ["ab"] and t3.encode("ab") == [t3.tok2id["a"], t3.tok2id["b"]]
    # leading and repeated spaces: a chunk starts at each space marker after a non-empty chunk
    assert t.chunks("  a b") == ["Ġ", "Ġa", "Ġb"]


def test_utf8_round_trip_and_decode_errors():
    t = QwenBPE(tokens=base_tokens() + ["Ġc", "af"], merges=["Ġ c", "a f"])
    for s in ["naïve café 日本語", "tabs\tand\nnewlines", "", "­ x"]:
        assert t.decode(t.encode(s)) == s
    bad = QwenBPE(tokens=base_tokens() + ["一"], merges=[])
    with pytest.raises(ValueError):
        bad.decode([256])


def test_gguf_metadata_path(tmp_path):
    tokens = base_tokens() + ["he", "hel", "hell", "hello"]
    merges = ["h e", "he l", "hel l", "hell o"]
    p = tmp_path / "tok.gguf"
    gguf.write_gguf(p, {"general.architecture": "qwen2",
                        "tokenizer.ggml.tokens": (gguf.GGUF_ARRAY, gguf.GGUF_STRING, tokens),
                        "tokenizer.ggml.merges": (gguf.GGUF_ARRAY, gguf.GGUF_STRING, merges)}, [])
    t = QwenBPE(str(p))
    assert t.encode("hello hello") == [tokens.index("hello"), t.tok2id["Ġ"], tokens.index("hello")]


def _definition_bpe(t, chunk):
    word = list(chunk)
    while len(word) > 1:
        best = min((t.merge_rank.get((word[i], word[i + 1]), 1 << 62), i) for i in range(len(word) - 1))
        if best[0] == 1 << 62:
            break
        i = best[1]
        word = word[:i] + [word[i] + word[i + 1]] + word[i + 2:]
    return word


def test_agrees_with_the_definition_on_random_merges():
    rng = random.Random(7)
    alphabet = "abcĠ"
    for trial in range(40):
        pieces = list(alphabet)
        merges = []
        for _ in range(rng.randint(3, 25)):
            a, b = rng.choice(pieces), rng.choice(pieces)
            if f"{a} {b}" not in merges and len(a + b) <= 6:
                merges.append(f"{a} {b}")
                pieces.append(a + b)
        t = QwenBPE(tokens=base_tokens() + sorted(set(pieces) - set(alphabet)), merges=merges)
        for _ in range(30):
            s = "".join(rng.choice("abc ") for _ in range(rng.randint(1, 24)))
            for chunk in t.chunks(s):
                assert t._bpe(chunk) == _definition_bpe(t, chunk), (merges, chunk)
