"""CPU oracle of the GPT-2 byte-level BPE tokenizer (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this; the product's tokenizer is cuda-llm-inference-engine_amd/host/tokenizer.cpp.

Restates the reference's BPETokenizer (/root/reference/src/tokenizer.cpp):
  * byte_table          tokenizer.cpp:11-48   GPT-2's byte -> character table
  * reference_scan_vocab tokenizer.cpp:61-116 the reference's quote scanner,
                        kept to show where it and a JSON parse differ
  * load                tokenizer.cpp:55-131  vocab.json (here: json.loads) and merges.txt
  * merge               tokenizer.cpp:134-167 greedy lowest-rank merge, leftmost
                        pair first among equal ranks, one pair per pass
  * encode              tokenizer.cpp:169-189 whitespace words, the space symbol
                        before every word after the first, unknown pieces dropped
  * decode              tokenizer.cpp:191-217 characters back to bytes, others
                        copied, ids outside the 50257-entry table give nothing
Pins (tests/test_tokenizer.py): byte_table against transformers'
convert_slow_tokenizer.bytes_to_unicode and the table's closed-form
properties; merge against hand-derived answers (including a merge list where
one pair per pass and all pairs per pass differ) and against the `tokenizers`
library's BPE on trained merges; encode/decode by the decode(encode(t)) round
trip.
"""
import json
import os

TABLE_IDS = 50257
EOS = 50256
_SPACE = b" \t\n\v\f\r"


def byte_table():
    """Byte -> one-character str: printable Latin-1 bytes map to themselves,
    the other 68 to chr(256), chr(257), ... in byte order (tokenizer.cpp:13-28)."""
    out, nxt = {}, 256
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255:
            out[b] = chr(b)
        else:
            out[b] = chr(nxt)
            nxt += 1
    return out


def _char_len(c):
    """Bytes of the character with lead byte c, counted as tokenizer.cpp:140-143 does."""
    return 4 if c >= 0xF0 else 3 if c >= 0xE0 else 2 if c >= 0xC0 else 1


def reference_scan_vocab(raw: bytes):
    """The reference's vocab.json scan (tokenizer.cpp:61-116) as a pure-Python
    loop: a key ends at the first quote not preceded by a backslash; escapes
    \\" \\\\ \\n \\t \\uXXXX are decoded (each \\u as its own character of up to
    3 UTF-8 bytes), any other backslash kept; the id is the first run of digits
    after the next ':'.  Returns {token bytes: id}."""
    s = raw
    out = {}
    pos = 1
    while pos < len(s):
        ks = s.find(b'"', pos)
        if ks < 0:
            break
        ke = s.find(b'"', ks + 1)
        while ke >= 0 and s[ke - 1:ke] == b"\\":
            ke = s.find(b'"', ke + 1)
        key = s[ks + 1:ke]
        clean = bytearray()
        i = 0
        while i < len(key):
            c = key[i:i + 1]
            if c == b"\\" and i + 1 < len(key):
                n = key[i + 1:i + 2]
                if n in (b'"', b"\\"):
                    clean += n
                    i += 1
                elif n == b"n":
                    clean += b"\n"
                    i += 1
                elif n == b"t":
                    clean += b"\t"
                    i += 1
                elif n == b"u":
                    cp = 0
                    for j in range(4):
                        if i + 2 + j >= len(key):
                            break
                        cp = (cp << 4) | int(chr(key[i + 2 + j]), 16)
                    if cp < 0x80:
                        clean.append(cp)
                    elif cp < 0x800:
                        clean += bytes([0xC0 | cp >> 6, 0x80 | cp & 0x3F])
                    else:
                        clean += bytes([0xE0 | cp >> 12, 0x80 | (cp >> 6) & 0x3F, 0x80 | cp & 0x3F])
                    i += 5
                else:
                    clean += c
            else:
                clean += c
            i += 1
        cs = s.find(b":", ke)
        vs = cs
        while vs < len(s) and not (48 <= s[vs] <= 57):
            vs += 1
        ve = vs
        while ve < len(s) and 48 <= s[ve] <= 57:
            ve += 1
        out[bytes(clean)] = int(s[vs:ve])
        pos = ve
        nxt = min([p for p in (s.find(b",", pos), s.find(b"}", pos)) if p >= 0], default=-1)
        if nxt < 0 or s[nxt:nxt + 1] == b"}":
            break
        pos = nxt + 1
    return out


class OracleBPE:
    """Tables and operations of BPETokenizer(model_dir); token strings are UTF-8 bytes."""

    def __init__(self, model_dir=None, vocab=None, merges=None):
        if model_dir is not None:
            with open(os.path.join(model_dir, "vocab.json"), "rb") as f:
                vocab = {k.encode("utf-8", "surrogatepass"): v for k, v in json.loads(f.read()).items()}
            with open(os.path.join(model_dir, "merges.txt"), "rb") as f:
                merges = f.read().split(b"\n")
            if merges and merges[-1] == b"":
                merges.pop()
        self.sym = {b: c.encode("utf-8") for b, c in byte_table().items()}
        self.unsym = {v: k for k, v in self.sym.items()}
        self.tok2id = dict(vocab)
        self.id2tok = [b""] * TABLE_IDS
        for t, i in vocab.items():
            if 0 <= i < TABLE_IDS:
                self.id2tok[i] = t
        self.rank = {}
        r = 0
        for line in merges:  # tokenizer.cpp:122-131
            if not line or line[:1] == b"#" or b" " not in line:
                continue
            a, b = line.split(b" ", 1)
            self.rank[(a, b)] = r
            r += 1

    def merge(self, syms):
        syms = list(syms)
        while len(syms) > 1:
            best, at = None, -1
            for j in range(len(syms) - 1):
                r = self.rank.get((syms[j], syms[j + 1]))
                if r is not None and (best is None or r < best):
                    best, at = r, j
            if at < 0:
                break
            syms[at:at + 2] = [syms[at] + syms[at + 1]]
        return syms

    def encode(self, text: bytes):
        ids = []
        words = [w for w in _split_ws(text)]
        for n, w in enumerate(words):
            syms = ([self.sym[0x20]] if n else []) + [self.sym[b] for b in w]
            for piece in self.merge(syms):
                if piece in self.tok2id:
                    ids.append(self.tok2id[piece])
        return ids

    def decode(self, ids):
        out = bytearray()
        for i in ids:
            if not 0 <= i < TABLE_IDS:
                continue
            t = self.id2tok[i]
            p = 0
            while p < len(t):
                ch = t[p:p + _char_len(t[p])]
                out += bytes([self.unsym[ch]]) if ch in self.unsym else ch
                p += len(ch)
        return bytes(out)


def _split_ws(text: bytes):
    word = bytearray()
    for b in text:
        if b in _SPACE:
            if word:
                yield bytes(word)
                word = bytearray()
        else:
            word.append(b)
    if word:
        yield bytes(word)
