"""GPT-2 byte-level BPE tokenizer (host code): the library against the CPU
oracle (oracle/bpe_tokenizer.py), and the oracle pinned.

The reference holds no tokenizer test or vocabulary file (python/export_gpt2.py
downloads GPT-2's at export time, and there is no network here), so the
vocabularies are made here: a byte-level BPE trained by the `tokenizers`
library on seeded synthetic text (its merges are ordered as training learned
them, as GPT-2's are), and hand-written tables for the known answers.  Bar:
identical ids and bytes.
"""
import ctypes
import json
import os
import random

import pytest

from oracle.bpe_tokenizer import EOS, TABLE_IDS, OracleBPE, byte_table, reference_scan_vocab

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "ie_tokenizer.h")


def write_tables(d, vocab, merges):
    """vocab {str: id} as JSON (ensure_ascii, like GPT-2's file), merges as
    "a b" lines after a version header."""
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "vocab.json"), "w") as f:
        json.dump(vocab, f)
    with open(os.path.join(d, "merges.txt"), "w", encoding="utf-8") as f:
        f.write("#version: 0.2\n" + "".join(f"{a} {b}\n" for a, b in merges))
    return d


@pytest.fixture(scope="module")
def trained_dir(tmp_path_factory):
    tokenizers = pytest.importorskip("tokenizers")
    rng = random.Random(5)
    words = ["".join(rng.choice("abcdefghijklmnop") for _ in range(rng.randint(1, 9))) for _ in range(400)]
    corpus = [" ".join(rng.choice(words) for _ in range(24)) for _ in range(600)]
    t = tokenizers.ByteLevelBPETokenizer()
    t.train_from_iterator(corpus, vocab_size=900, min_frequency=1, show_progress=False)
    d = str(tmp_path_factory.mktemp("bpe_trained"))
    t.save_model(d)
    return d, t, words


def random_text(rng, words):
    """Words, punctuation, UTF-8 (2-4 byte characters), lone high bytes and
    every whitespace byte, including leading and trailing runs."""
    parts = []
    for _ in range(rng.randint(0, 14)):
        k = rng.random()
        if k < 0.5:
            w = rng.choice(words).encode()
        elif k < 0.6:
            w = rng.choice(["é", "中文", "😀x", "naïve", "Ж"]).encode()
        elif k < 0.7:
            w = bytes(rng.randrange(128, 256) for _ in range(rng.randint(1, 3)))
        elif k < 0.8:
            w = bytes(rng.randrange(33, 127) for _ in range(rng.randint(1, 4)))
        else:
            w = rng.choice(words).encode() + rng.choice([b",", b".", b"!", b"'s", b"\x00"])
        parts.append(w)
        parts.append(bytes(rng.choice(b" \t\n\v\f\r") for _ in range(rng.randint(1, 3))))
    if rng.random() < 0.5:
        parts.insert(0, b"  \n")
    return b"".join(parts)


# ------------------------------------------------------------- oracle pins
def test_byte_table_pinned():
    from transformers.convert_slow_tokenizer import bytes_to_unicode

    t = byte_table()
    assert t == bytes_to_unicode()
    assert len(set(t.values())) == 256
    assert all(t[b] == chr(b) for b in range(33, 127))
    assert t[0x20] == "Ġ" and t[0x0A] == "Ċ" and t[0xAD] == "Ń" and t[0] == "Ā"


def test_merge_known_answers():
    # Ranks are list order.  "a b" first, then "ab c": abc in two passes.
    o = OracleBPE(vocab={}, merges=[b"a b", b"ab c", b"b c"])
    assert o.merge([b"a", b"b", b"c"]) == [b"abc"]
    # Equal ranks: the leftmost pair merges first (a a a -> aa a).
    o = OracleBPE(vocab={}, merges=[b"a a"])
    assert o.merge([b"a", b"a", b"a"]) == [b"aa", b"a"]
    # One pair per pass: b c merges at the left, then the new "bc b" (rank 0)
    # outranks the second "b c"; merging every "b c" at once would give bc bc.
    o = OracleBPE(vocab={}, merges=[b"bc b", b"b c"])
    assert o.merge([b"b", b"c", b"b", b"c"]) == [b"bcb", b"c"]
    # Comment and blank lines take no rank; the split is at the first space;
    # a repeated pair keeps its later rank.
    o = OracleBPE(vocab={}, merges=[b"#x y", b"", b"x y", b"y z", b"x y"])
    assert o.rank == {(b"y", b"z"): 1, (b"x", b"y"): 2}
    assert o.merge([b"x", b"y", b"z"]) == [b"x", b"yz"]


def test_oracle_matches_tokenizers_bpe(trained_dir):
    """Lower-case words separated by single spaces are pre-tokenized alike by
    both (the space symbol before every word after the first), so the ids pin
    the merge loop on a trained merge list."""
    d, hf, words = trained_dir
    o = OracleBPE(d)
    rng = random.Random(1)
    for _ in range(300):
        text = " ".join(rng.choice(words) for _ in range(rng.randint(1, 12)))
        assert o.encode(text.encode()) == hf.encode(text).ids, text


def test_oracle_round_trip(trained_dir):
    o = OracleBPE(trained_dir[0])
    rng = random.Random(2)
    for _ in range(200):
        t = random_text(rng, trained_dir[2])
        assert o.decode(o.encode(t)) == b" ".join(t.split())


def test_reference_scan_agrees_except_backslash_keys(trained_dir):
    raw = open(os.path.join(trained_dir[0], "vocab.json"), "rb").read()
    o = OracleBPE(trained_dir[0])
    ref = reference_scan_vocab(raw)
    # Every byte-level vocabulary (GPT-2's too) holds "\\" as id 59 and "]" as
    # id 60; the reference's scan loses both and files 60 under a garbled key.
    assert {k: v for k, v in ref.items() if o.tok2id.get(k) != v} == {b'\\":59,': 60}
    assert {k: v for k, v in o.tok2id.items() if ref.get(k) != v} == {b"\\": 59, b"]": 60}
    # A key that closes on an escaped backslash: the reference's scan takes
    # the next key's opening quote as its end, so "\" is lost and id 60 is
    # filed under a garbled key; JSON gives both.
    raw = b'{"!": 0, "\\\\": 59, "]": 60, "a": 61}'
    assert reference_scan_vocab(raw) == {b"!": 0, b'\\": 59, ': 60, b"a": 61}
    assert json.loads(raw) == {"!": 0, "\\": 59, "]": 60, "a": 61}


# ------------------------------------------------------------ library parity
def test_symbols_exported(ie):
    import re

    names = re.findall(r"^\s*int\s+(ie_tokenizer_\w+)\s*\(", open(HDR).read(), re.M)
    assert len(names) == 6
    lib = ctypes.CDLL(ie.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n


def test_library_matches_oracle(ie, trained_dir):
    d, _, words = trained_dir
    tok, o = ie.Tokenizer(d), OracleBPE(d)
    assert tok.vocab_size == TABLE_IDS and tok.eos_token == EOS
    rng = random.Random(3)
    for _ in range(400):
        t = random_text(rng, words)
        ids = tok.encode(t)
        assert ids == o.encode(t), t
        assert tok.decode(ids) == o.decode(ids)
    assert tok.encode("") == [] and tok.encode(" \t\n") == [] and tok.decode([]) == b""
    for _ in range(100):
        ids = [rng.choice([-1, TABLE_IDS, 10**6, rng.randrange(0, 1000)]) for _ in range(rng.randint(1, 20))]
        assert tok.decode(ids) == o.decode(ids)
    assert tok.decode(7) == o.decode([7])


def test_library_known_answers(ie, tmp_path):
    sym = byte_table()
    sp = sym[0x20]
    vocab = {sym[b]: b for b in range(256)}
    vocab.update({"He": 256, "ll": 257, "Hell": 258, "Hello": 259, sp + "w": 260, sp + "wor": 261,
                  sp + "world": 262, "or": 263, "ld": 264, "\\": 300, "x\\": 301, "\U0001F600": 302,
                  "<|endoftext|>": 50256, "beyond": 60000})
    merges = [("H", "e"), ("l", "l"), ("He", "ll"), ("Hell", "o"), (sp, "w"), ("o", "r"), (sp + "w", "or"),
              ("l", "d"), (sp + "wor", "ld"), ("x", "\\"), ("b", "e"), ("be", "y"), ("bey", "o"),
              ("beyo", "n"), ("beyon", "d")]
    d = write_tables(str(tmp_path / "known"), vocab, merges)
    tok, o = ie.Tokenizer(d), OracleBPE(d)
    # Hello world  /  tabs and newlines act as the single space; leading
    # whitespace gives no space symbol to the first word
    assert tok.encode("Hello world") == [259, 262] == o.encode(b"Hello world")
    assert tok.encode("\n\tHello \n world ") == [259, 262]
    assert tok.encode("Hello, world!") == [259, ord(","), 262, ord("!")]
    # keys ending in a backslash, and a surrogate-pair escape, parse as JSON
    assert tok.encode("x\\ \\") == [301, 32, 300] == o.encode(b"x\\ \\")
    assert tok.decode([300, 301]) == b"\\x\\"
    assert tok.decode([302]) == "\U0001F600".encode()
    # ids past the 50257-entry table decode to nothing but still encode
    assert tok.encode("beyond") == [60000] and tok.decode([60000, 50256]) == b"<|endoftext|>"
    assert tok.decode(ie.Tokenizer(d).encode("Hello world")) == b"Hello world"


def test_errors(ie, tmp_path):
    with pytest.raises(ie.IeError, match="cannot open"):
        ie.Tokenizer(str(tmp_path / "missing"))
    d = tmp_path / "bad"
    d.mkdir()
    (d / "merges.txt").write_text("")
    for bad in ['["a"]', '{"a": x}', '{"a": -1}', '{"a": 1,', '{"a\\q": 1}']:
        (d / "vocab.json").write_text(bad)
        with pytest.raises(ie.IeError, match="vocab.json"):
            ie.Tokenizer(str(d))
    (d / "vocab.json").write_text("{}")
    (d / "merges.txt").unlink()
    with pytest.raises(ie.IeError, match="merges.txt"):
        ie.Tokenizer(str(d))
    lib = ie.load()
    assert lib.ie_tokenizer_create(None, b"x") == ie.IE_ERR_INVALID
    assert lib.ie_tokenizer_vocab_size(None) == -1


def test_cpp_class_drop_in(ie, trained_dir, tmp_path):
    """src/main.cpp's use of BPETokenizer (src/main.cpp:224-230, 355-367),
    compiled against include/ie_bpe_tokenizer.h and linked with libie_amd.so:
    the ids and text match the oracle's, and a missing directory throws."""
    import subprocess

    d, _, words = trained_dir
    text = " ".join(words[:40]) + " \\ ] x"
    src = r"""
#include "ie_bpe_tokenizer.h"
#include <cstdio>
#include <stdexcept>
int main(int argc, char** argv) {
    BPETokenizer tokenizer(argv[1]);
    std::vector<int> ids = tokenizer.encode(argv[2]);
    for (int id : ids) printf("%d ", id);
    printf("\n%s\n%d %d\n", tokenizer.decode(ids).c_str(), tokenizer.vocab_size(), tokenizer.eos_token());
    try { BPETokenizer missing(std::string(argv[1]) + "/nowhere"); } catch (const std::runtime_error&) { return 0; }
    return 3;
}
"""
    cpp, exe = str(tmp_path / "t.cpp"), str(tmp_path / "t")
    open(cpp, "w").write(src)
    subprocess.run(["g++", "-std=c++17", "-I", os.path.join(ROOT, "include"), cpp, "-o", exe, ie.LIB_PATH,
                    f"-Wl,-rpath,{os.path.dirname(ie.LIB_PATH)}"], check=True)
    r = subprocess.run([exe, d, text], capture_output=True)
    assert r.returncode == 0, (r.returncode, r.stderr)
    lines = r.stdout.split(b"\n")
    o = OracleBPE(d)
    want = o.encode(text.encode())
    assert [int(x) for x in lines[0].split()] == want and 59 in want and 60 in want
    assert lines[1] == o.decode(want) == text.encode()
    assert lines[2] == f"{TABLE_IDS} {EOS}".encode()
