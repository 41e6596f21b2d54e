"""Host-side tokenizer (mignon_ai_amd.tokenizer) against the reference's own tokenizer tests
(internal/tokenizer/pretokenize_test.go, tokenizer_test.go) and the vocabulary of the trained order-search
model (tests/golden/orders.mgn, the reference's examples/order-search/orders.mgn)."""
import json
import os
import struct

import pytest

from helpers import GOLDEN
from mignon_ai_amd.tokenizer import (MAX_WORD_BYTES, Tokenizer, TokenizerError, read_header, split_words)

ORDERS = os.path.join(GOLDEN, "orders.mgn")


@pytest.fixture(scope="module")
def orders_bytes():
    with open(ORDERS, "rb") as f:
        return f.read()


@pytest.fixture(scope="module")
def tok(orders_bytes):
    return Tokenizer.from_model_file(orders_bytes)


# TestSplitWordsGivesSpaceToNextWord (pretokenize_test.go:15-33)
SPLIT_CASES = {
    "git pull --rebase origin": ["git", " pull", " --", "rebase", " origin"],
    "commit -m 'fix: bug'\ngit": ["commit", " -", "m", " '", "fix", ":", " bug", "'", "\n", "git"],
    "two  spaces\n\n tab\tend.": ["two", " ", " spaces", "\n\n", " tab", "\t", "end", "."],
    " leading": [" leading"],
    "trailing ": ["trailing", " "],
    "HEAD~1 && echo done": ["HEAD", "~", "1", " &&", " echo", " done"],
}


@pytest.mark.parametrize("text", list(SPLIT_CASES))
def test_split_words_gives_space_to_next_word(text):
    got = split_words(text)
    assert got == SPLIT_CASES[text]
    assert "".join(got) == text


def test_split_words_caps_long_runs():
    """TestSplitWordsCapsLongRuns (pretokenize_test.go:35-47), plus the cap counted in bytes."""
    text = "a" * (3 * MAX_WORD_BYTES + 5)
    words = split_words(text)
    assert all(len(w.encode()) <= MAX_WORD_BYTES for w in words)
    assert "".join(words) == text
    assert [len(w) for w in words] == [128, 128, 128, 5]
    # two-byte letters: a run stops once it holds 128 bytes (64 characters)
    words = split_words("é" * 130)
    assert [len(w.encode()) for w in words] == [128, 128, 4]


def test_split_words_unicode_classes():
    """classOf (pretokenize.go:19-30) on Go's unicode tables: White_Space, P*/S* categories, Nd."""
    # no-break and em spaces are spaces; a space run only hands a final ASCII " " to the next run
    assert split_words("a\u00a0b") == ["a", "\u00a0", "b"]
    assert split_words("x\u2003 y") == ["x", "\u2003", " y"]
    # symbols (Sc, Sm, So) group with punctuation
    assert split_words("$€+→!") == ["$€+→!"]
    # every decimal digit stands alone, in any script; other numerals (No) are word characters
    assert split_words("12٣") == ["1", "2", "٣"]
    assert split_words("x½y") == ["x½y"]
    assert split_words("") == []


def test_vocabulary_and_specials(tok, orders_bytes):
    hdr = read_header(orders_bytes)
    assert hdr["metadata"]["tokenizer_version"] == 2
    assert tok.vocab_size() == len(hdr["vocab"]) == 2048
    assert tok.vocab[:5] == ["<PAD>", "<UNK>", "<USER>", "<BOT>", "<EOS>"]
    assert (tok.pad_id(), tok.user_id(), tok.bot_id(), tok.eos_id()) == (0, 2, 3, 4)


def test_chat_template(tok):
    """TestChatTemplate (pretokenize_test.go:66-80) on the trained vocabulary."""
    prompt = tok.encode_prompt("push to main")
    assert prompt[0] == tok.user_id() and prompt[-1] == tok.bot_id()
    reply = tok.encode_reply("git push origin main")
    assert reply[-1] == tok.eos_id()
    assert tok.decode(prompt + reply) == "push to maingit push origin main"


def test_drop_oldest_turns(tok):
    """TestDropOldestTurns (pretokenize_test.go:82-98)."""
    def turn(u, b):
        return tok.encode_prompt(u) + tok.encode_reply(b)
    first, second = turn("hi", "hello"), turn("bye", "bye")
    history = first + second
    assert tok.drop_oldest_turns(history, len(history)) == history
    assert tok.drop_oldest_turns(history, len(second)) == second
    assert tok.drop_oldest_turns(history, 0) == []
    assert tok.drop_oldest_turns(tok.encode_prompt("no reply yet") * 2, 3) == []


def test_unknown_characters_decode_to_replacement(tok):
    """TestTokenizerUnkDecoding / TestTokenizerSkipsRareCharacters (tokenizer_test.go:120-156)."""
    ids = tok.encode("🚀")
    assert ids == [tok.token_to_id["<UNK>"]]
    assert tok.decode(ids) == "�"
    assert tok.decode(tok.encode("orders find")) == "orders find"


def test_special_tokens_are_atomic(tok):
    """TestSpecialTokensAtomicEncoding (tokenizer_test.go:164-205): a registered <...> token is one id,
    anything else between < and > is ordinary text."""
    ids = tok.encode("hi<USER>there<BOT>")
    assert ids.count(tok.user_id()) == 1 and ids.count(tok.bot_id()) == 1
    assert tok.decode(ids) == "hithere"
    plain = tok.encode("a <b> c")
    assert tok.decode(plain) == "a <b> c"
    assert tok.decode(tok.encode("x<y")) == "x<y"
    assert tok.decode(tok.encode("<USER")) == "<USER"


def test_encode_round_trips_orders_requests(tok):
    """Every request of the order-search set decodes back from its encoding (all its characters are in
    the vocabulary), and merges never cross a pre-token boundary."""
    with open(os.path.join(GOLDEN, "orders_handwritten.json")) as f:
        pairs = json.load(f)
    for p in pairs:
        for text in (p["instruction"], p["output"]):
            ids = tok.encode(text)
            assert tok.decode(ids) == text
            pieces = [tok.vocab[i] for i in ids]
            bounds = set()
            pos = 0
            for w in split_words(text):
                pos += len(w)
                bounds.add(pos)
            pos = 0
            for pc in pieces:
                start = pos
                pos += len(pc)
                assert not any(start < b < pos for b in bounds), (text, pieces)


def test_merge_rank_order():
    """encodeWord (tokenizer.go:180-232): the lowest-ranked pair present merges first, the leftmost one
    on a tie, and merges repeat until no ranked pair is left; missing pieces become <UNK>."""
    vocab = ["<PAD>", "<UNK>", "a", "b", "c", "ab", "bc", "aa", "aaa", "abc"]
    t1 = Tokenizer(vocab, [("b", "c"), ("a", "b")])
    assert [t1.vocab[i] for i in t1.encode("abc")] == ["a", "bc"]
    t2 = Tokenizer(vocab, [("a", "b"), ("b", "c"), ("ab", "c")])
    assert [t2.vocab[i] for i in t2.encode("abc")] == ["abc"]
    t3 = Tokenizer(vocab, [("a", "a")])
    assert [t3.vocab[i] for i in t3.encode("aaa")] == ["aa", "a"]
    t4 = Tokenizer(vocab, [("a", "a"), ("aa", "a")])
    assert [t4.vocab[i] for i in t4.encode("aaaa")] == ["aa", "aa"]
    # a a a a a -> aa a a a -> aa aa a (rank 0 beats the leftmost rank-1 pair) -> aa aaa
    assert [t4.vocab[i] for i in t4.encode("aaaaa")] == ["aa", "aaa"]
    # merging does not consult the vocabulary; a piece missing from it is <UNK> after merging
    t5 = Tokenizer(vocab, [("a", "x")])
    assert t5.encode("ax") == [1]
    assert t5.encode("xa") == [1, 2]


def test_format_version_is_checked(orders_bytes):
    """CheckFormat (internal/tokenizer/format.go:12-17) via quant.Decode (checkpoint.go:201-207)."""
    n = struct.unpack_from("<I", orders_bytes, 8)[0]
    hdr = json.loads(orders_bytes[12:12 + n])
    hdr["metadata"]["tokenizer_version"] = 1
    raw = json.dumps(hdr).encode()
    bad = orders_bytes[:8] + struct.pack("<I", len(raw)) + raw + orders_bytes[12 + n:]
    with pytest.raises(TokenizerError, match="version 1 is not supported"):
        Tokenizer.from_model_file(bad)
    with pytest.raises(TokenizerError):
        read_header(b"JUNK" + orders_bytes[4:])
    hdr["vocab"] = []
    raw = json.dumps(hdr).encode()
    empty = orders_bytes[:8] + struct.pack("<I", len(raw)) + raw + orders_bytes[12 + n:]
    assert Tokenizer.from_model_file(empty) is None
