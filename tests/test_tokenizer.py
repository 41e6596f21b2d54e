"""The library's tokenizer (C ABI: mg_tokenizer_*, mg_pretokenize) and the oracle's restatement
(oracle/text.py), both against the reference's own tokenizer tests (internal/tokenizer/pretokenize_test.go,
tokenizer_test.go) and the vocabulary of the reference's trained order-search model (tests/golden/orders.mgn),
then against each other on generated text. No GPU is used."""
import json
import os
import random
import struct

import pytest

from helpers import GOLDEN
from mignon_ai_amd import tokenizer as product
from mignon_ai_amd._lib import MignonError
from oracle import text as oracle

ORDERS = os.path.join(GOLDEN, "orders.mgn")
IMPLS = ["product", "oracle"]


@pytest.fixture(scope="module")
def orders_bytes():
    with open(ORDERS, "rb") as f:
        return f.read()


@pytest.fixture(scope="module")
def toks(orders_bytes):
    return {"product": product.Tokenizer.from_model_file(orders_bytes),
            "oracle": oracle.Tokenizer.from_model_file(orders_bytes)}


def dec(tok, ids) -> str:
    s = tok.decode(ids)
    return s.decode("utf-8") if isinstance(s, bytes) else s


def split(impl, text: str) -> list[str]:
    if impl == "product":
        return product.split_words(text)
    return [w.decode("utf-8") for w in oracle.split_words(text.encode("utf-8"))]


def json_tokenizer(impl, vocab, merges, version=2):
    """A tokenizer from a header-only legacy JSON model file."""
    data = json.dumps({"vocab": vocab, "merges": [{"pair1": a, "pair2": b} for a, b in merges],
                       "metadata": {"tokenizer_version": version}}).encode()
    return (product if impl == "product" else oracle).Tokenizer.from_model_file(data)


# TestSplitWordsGivesSpaceToNextWord (pretokenize_test.go:15-33)
SPLIT_CASES = {
    "git pull --rebase origin": ["git", " pull", " --", "rebase", " origin"],
    "commit -m 'fix: bug'\ngit": ["commit", " -", "m", " '", "fix", ":", " bug", "'", "\n", "git"],
    "two  spaces\n\n tab\tend.": ["two", " ", " spaces", "\n\n", " tab", "\t", "end", "."],
    " leading": [" leading"],
    "trailing ": ["trailing", " "],
    "HEAD~1 && echo done": ["HEAD", "~", "1", " &&", " echo", " done"],
}


@pytest.mark.parametrize("impl", IMPLS)
@pytest.mark.parametrize("text", list(SPLIT_CASES))
def test_split_words_gives_space_to_next_word(impl, text):
    got = split(impl, text)
    assert got == SPLIT_CASES[text]
    assert "".join(got) == text


@pytest.mark.parametrize("impl", IMPLS)
def test_split_words_caps_long_runs(impl):
    """TestSplitWordsCapsLongRuns (pretokenize_test.go:35-47); the cap counts bytes."""
    text = "a" * (3 * oracle.MAX_WORD_BYTES + 5)
    words = split(impl, text)
    assert "".join(words) == text
    assert [len(w) for w in words] == [128, 128, 128, 5]
    words = split(impl, "é" * 130)  # two bytes each: a run closes once it holds 128 bytes
    assert [len(w.encode()) for w in words] == [128, 128, 4]


@pytest.mark.parametrize("impl", IMPLS)
def test_split_words_unicode_classes(impl):
    """classOf (pretokenize.go:19-30): White_Space, P*/S* categories, Nd, everything else a word."""
    assert split(impl, "a b") == ["a", " ", "b"]       # no-break space is a space
    assert split(impl, "x  y") == ["x", " ", " y"]     # only a final ASCII ' ' moves on
    assert split(impl, "$€+→!") == ["$€+→!"]  # Sc, Sm, So group with punctuation
    assert split(impl, "12٣") == ["1", "2", "٣"]       # every Nd digit stands alone
    assert split(impl, "x½y") == ["x½y"]              # No is not a digit
    assert split(impl, "") == []


def test_split_words_invalid_utf8():
    """Go reads an invalid byte as one U+FFFD rune of width 1 (a symbol); pre-tokens keep the raw bytes."""
    for impl_split in (product.split_words, oracle.split_words):
        assert impl_split(b"ab\xffcd") == [b"ab", b"\xff", b"cd"]
        assert impl_split(b"x\xe2\x82 y") == [b"x", b"\xe2\x82", b" y"]   # truncated: two runes
        assert impl_split(b"\xed\xa0\x80z") == [b"\xed\xa0\x80", b"z"]     # encoded surrogate: three
        assert impl_split(b"\xc0\xafz") == [b"\xc0\xaf", b"z"]             # overlong: two
        assert impl_split(b"a\xf0\x9f\x9a\x80b") == [b"a", b"\xf0\x9f\x9a\x80", b"b"]  # a valid 4-byte symbol


def _probe_pieces(c: int) -> list[str]:
    """The pre-tokens of "a" c c "a" for the oracle's class of c."""
    ch = chr(c)
    k = oracle.char_class(c)
    if k == 0:
        return ["a" + ch + ch + "a"]
    if k == 3:
        return ["a", ch, ch, "a"]
    if c == 0x20:
        return ["a", " ", " a"]
    return ["a", ch + ch, "a"]


def test_character_classes_of_every_code_point():
    """The library's class table against the oracle's classOf: every code point of planes 0-2 and a sample
    of the rest, each probed as "a c c a" (a word joins the a's, punctuation pairs up, a digit stands alone,
    a space run sits between them), probes separated by "\\n\\n", a space run of its own."""
    rng = random.Random(3)
    cps = [c for c in range(0x20, 0x32000) if not 0xD800 <= c < 0xE000]
    cps += [rng.randrange(0x32000, 0x110000) for _ in range(20000)]
    text = "\n\n".join("a" + chr(c) + chr(c) + "a" for c in cps)
    want = []
    for i, c in enumerate(cps):
        if i:
            want.append("\n\n")
        want.extend(_probe_pieces(c))
    assert product.split_words(text) == want


@pytest.mark.parametrize("impl", IMPLS)
def test_vocabulary_and_specials(impl, toks, orders_bytes):
    tok = toks[impl]
    n = struct.unpack_from("<I", orders_bytes, 8)[0]
    hdr = json.loads(orders_bytes[12:12 + n])
    assert hdr["metadata"]["tokenizer_version"] == 2
    assert tok.vocab == hdr["vocab"] and len(tok.vocab) == 2048
    assert (tok.pad_id(), tok.user_id(), tok.bot_id(), tok.eos_id()) == (0, 2, 3, 4)


@pytest.mark.parametrize("impl", IMPLS)
def test_chat_template(impl, toks):
    """TestChatTemplate (pretokenize_test.go:66-80) on the trained vocabulary."""
    tok = toks[impl]
    prompt = tok.encode_prompt("push to main")
    assert prompt[0] == tok.user_id() and prompt[-1] == tok.bot_id()
    reply = tok.encode_reply("git push origin main")
    assert reply[-1] == tok.eos_id()
    assert dec(tok, prompt + reply) == "push to maingit push origin main"


@pytest.mark.parametrize("impl", IMPLS)
def test_drop_oldest_turns(impl, toks):
    """TestDropOldestTurns (pretokenize_test.go:82-98)."""
    tok = toks[impl]

    def turn(u, b):
        return tok.encode_prompt(u) + tok.encode_reply(b)
    first, second = turn("hi", "hello"), turn("bye", "bye")
    history = first + second
    assert tok.drop_oldest_turns(history, len(history)) == history
    assert tok.drop_oldest_turns(history, len(second)) == second
    assert tok.drop_oldest_turns(history, 0) == []
    assert tok.drop_oldest_turns(tok.encode_prompt("no reply yet") * 2, 3) == []


@pytest.mark.parametrize("impl", IMPLS)
def test_unknown_characters_decode_to_replacement(impl, toks):
    """TestTokenizerUnkDecoding / TestTokenizerSkipsRareCharacters (tokenizer_test.go:120-156)."""
    tok = toks[impl]
    ids = tok.encode("\U0001F680")
    assert ids == [1]
    assert dec(tok, ids) == "�"
    assert dec(tok, tok.encode("orders find")) == "orders find"


@pytest.mark.parametrize("impl", IMPLS)
def test_special_tokens_are_atomic(impl, toks):
    """TestSpecialTokensAtomicEncoding (tokenizer_test.go:164-205): a registered <...> token is one id,
    anything else between < and > is ordinary text."""
    tok = toks[impl]
    ids = tok.encode("hi<USER>there<BOT>")
    assert ids.count(tok.user_id()) == 1 and ids.count(tok.bot_id()) == 1
    assert dec(tok, ids) == "hithere"
    for text in ["a <b> c", "x<y", "<USER", "a>b<c"]:
        assert dec(tok, tok.encode(text)) == text
    assert tok.encode("<<USER>>") == tok.encode("<") + [tok.user_id()] + tok.encode(">")


@pytest.mark.parametrize("impl", IMPLS)
def test_merge_rank_order(impl):
    """encodeWord (tokenizer.go:179-227): the lowest-ranked pair present merges first, the leftmost on a
    tie, until no ranked pair is left; merging ignores the vocabulary, and a missing piece is <UNK>."""
    vocab = ["<PAD>", "<UNK>", "a", "b", "c", "ab", "bc", "aa", "aaa", "abc"]

    def pieces(merges, text):
        t = json_tokenizer(impl, vocab, merges)
        return [vocab[i] for i in t.encode(text)]
    assert pieces([("b", "c"), ("a", "b")], "abc") == ["a", "bc"]
    assert pieces([("a", "b"), ("b", "c"), ("ab", "c")], "abc") == ["abc"]
    assert pieces([("a", "a")], "aaa") == ["aa", "a"]
    assert pieces([("a", "a"), ("aa", "a")], "aaaa") == ["aa", "aa"]
    # a a a a a -> aa a a a -> aa aa a (rank 0 beats the leftmost rank-1 pair) -> aa aaa
    assert pieces([("a", "a"), ("aa", "a")], "aaaaa") == ["aa", "aaa"]
    assert json_tokenizer(impl, vocab, [("a", "x")]).encode("ax") == [1]
    assert json_tokenizer(impl, vocab, [("a", "x")]).encode("xa") == [1, 2]
    # a repeated pair keeps its last rank (initRanks overwrites)
    assert pieces([("b", "c"), ("a", "b"), ("b", "c")], "abc") == ["ab", "c"]


@pytest.mark.parametrize("impl", IMPLS)
def test_format_version_is_checked(impl, orders_bytes):
    """CheckFormat (internal/tokenizer/format.go:12-17) via quant.Decode (checkpoint.go:201-207)."""
    n = struct.unpack_from("<I", orders_bytes, 8)[0]
    hdr = json.loads(orders_bytes[12:12 + n])
    hdr["metadata"]["tokenizer_version"] = 1
    raw = json.dumps(hdr).encode()
    bad = orders_bytes[:8] + struct.pack("<I", len(raw)) + raw + orders_bytes[12 + n:]
    mod = product if impl == "product" else oracle
    err = MignonError if impl == "product" else oracle.TokenizerError
    with pytest.raises(err, match="version 1 is not supported"):
        mod.Tokenizer.from_model_file(bad)
    hdr["vocab"] = []
    raw = json.dumps(hdr).encode()
    assert mod.Tokenizer.from_model_file(orders_bytes[:8] + struct.pack("<I", len(raw)) + raw + orders_bytes[12 + n:]) is None


def test_token_bytes(toks):
    """TokenBytes (internal/tokenizer/bytes.go:13-22): 0 for markers and padding, 3 for <UNK> (U+FFFD)."""
    tb = toks["product"].token_bytes()
    assert tb == toks["oracle"].token_bytes()
    assert tb[:5] == [0, 3, 0, 0, 0]
    assert all(tb[i] == len(toks["oracle"].vocab[i].encode()) for i in range(5, len(tb)))


def _random_text(rng, n):
    alphabet = ("abcdefghij orders find --status unpaid 0123456789 $€→!?.,;:'\"<>/\\\n\t"
                "é漢字\U0001F680  ٣½")
    parts = []
    for _ in range(n):
        r = rng.random()
        if r < 0.7:
            parts.append(rng.choice(alphabet))
        elif r < 0.8:
            parts.append(rng.choice(["<USER>", "<BOT>", "<EOS>", "<PAD>", "<UNK>", "<x>", "<"]))
        else:
            c = rng.randrange(0x20, 0x3000)
            parts.append(chr(c) if not 0xD800 <= c < 0xE000 else "?")
    return "".join(parts).encode("utf-8")


def test_product_matches_oracle_on_generated_text(toks):
    """Encode, decode and pre-tokenization of the library and the restatement agree on random text mixing
    the vocabulary's words, markers, other scripts, symbols and invalid UTF-8 bytes."""
    rng = random.Random(11)
    p, o = toks["product"], toks["oracle"]
    for i in range(400):
        b = _random_text(rng, rng.randrange(0, 80))
        if i % 5 == 0 and b:
            b = bytearray(b)
            for _ in range(3):
                b[rng.randrange(len(b))] = rng.randrange(0x80, 0x100)
            b = bytes(b)
        assert product.split_words(b) == oracle.split_words(b), b
        ids = p.encode(b)
        assert ids == o.encode(b), b
        assert p.decode_bytes(ids) == o.decode(ids), b
        assert p.encode_prompt(b) == o.encode_prompt(b)
        assert p.encode_reply(b) == o.encode_reply(b)


def test_encode_round_trips_orders_requests(toks):
    """Every request and reply of the order-search set decodes back from its encoding, and no token
    crosses a pre-token boundary."""
    tok = toks["product"]
    with open(os.path.join(GOLDEN, "orders_handwritten.json")) as f:
        pairs = json.load(f)
    for p in pairs:
        for text in (p["instruction"], p["output"]):
            ids = tok.encode(text)
            assert tok.decode(ids) == text
            bounds, pos = set(), 0
            for w in product.split_words(text):
                pos += len(w)
                bounds.add(pos)
            pos = 0
            for i in ids:
                start, pos = pos, pos + len(tok.vocab[i])
                assert not any(start < b < pos for b in bounds), text


# unicode.IsSpace (Go): the Latin-1 spaces and the White_Space property above Latin-1
GO_WHITE_SPACE = "\t\n\v\f\r \x85\xa0\u1680" + "".join(chr(c) for c in range(0x2000, 0x200B)) + \
    "\u2028\u2029\u202f\u205f\u3000"


def test_decode_rows_equals_decode_of_each_row(toks):
    """mg_tokenizer_decode_rows (one call for a batch of replies) gives every row what Decode gives it
    (the restatement's), and with trimming strings.TrimSpace of that: rows of random ids and of encoded
    text with white space at either end, markers, <UNK>, empty and full rows."""
    import numpy as np

    p, o = toks["product"], toks["oracle"]
    rng = random.Random(12)
    V = p.vocab_size()
    rows = []
    for i in range(300):
        if i % 3 == 0:
            rows.append([rng.randrange(V) for _ in range(rng.randrange(0, 40))])
        else:
            pre = "".join(rng.choice(GO_WHITE_SPACE) for _ in range(rng.randrange(0, 3)))
            post = "".join(rng.choice(GO_WHITE_SPACE + "<EOS>") for _ in range(rng.randrange(0, 3)))
            rows.append(p.encode(pre + _random_text(rng, rng.randrange(0, 30)).decode("utf-8") + post))
    rows.append([])
    rows.append(p.encode(" \t\n "))  # white space only
    ld = max(len(r) for r in rows)
    ids = np.zeros((len(rows), ld), np.int32)
    counts = np.array([len(r) for r in rows], np.int32)
    for i, r in enumerate(rows):
        ids[i, :len(r)] = r
        ids[i, len(r):] = rng.randrange(V)  # past the row's end: never read
    want = [o.decode(r).decode("utf-8", errors="replace") for r in rows]
    assert p.decode_rows(ids, counts) == want
    assert p.decode_rows(ids, counts, trim=True) == [w.strip(GO_WHITE_SPACE) for w in want]
    assert p.decode_rows(ids[:0], counts[:0]) == []
