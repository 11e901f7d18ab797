"""Byte-level BPE tokenizer of a Qwen2 GGUF vocabulary (the reference's
LlamaCppTokenizer, runtime/adapters/llama_cpp_tokenizer.cpp:50-137, over
llama.cpp's llama_vocab), on the CPU.

llama.cpp is not vendored in the reference and no vocabulary ships with it,
so agreement with llama.cpp itself is unpinned. What is pinned: the same
algorithm in HuggingFace `tokenizers` (the library Qwen2's own tokenizer runs
on): a byte-level BPE vocabulary is trained with it over the Qwen2
pre-tokenizer regex (written as llama.cpp writes it: ASCII case classes for
the contractions), stored as GGUF metadata, and every string — fixed cases
and random strings over letters, digits, white space, CR/LF, punctuation and
apostrophes of many scripts — must give the same ids. Pieces must spell the
text back byte for byte; end-of-generation ids follow llama.cpp's rules (EOS
/ EOT / EOM ids, the end and fill-in-the-middle texts); a package imported
from a GGUF file keeps the vocabulary in its metadata.gguf.
"""
from __future__ import annotations

import functools
import os
import random
import struct
import unicodedata

import pytest

import jetsonfabric_amd as jf
from tests.test_gguf_import import gguf_file, tensor_infos

tokenizers = pytest.importorskip("tokenizers")

QWEN2_PATTERN = (r"(?:'[sS]|'[tT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD])|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}"
                 r"| ?[^\s\p{L}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")
SPECIALS = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<|fim_pad|>"]

CORPUS = [
    "The quick brown fox jumps over the lazy dog. It's 10:45, and we'll leave at 11.",
    "def forward(self, x):\n    return self.proj(x) + 1234567890\n\n\tpass  # TODO",
    "Speculative decoding proposes k draft tokens; the target model verifies them in one pass.",
    "Ünïcödé façade — naïve café, São Paulo, Zürich, Kraków, Ærøskøbing.",
    "Ελληνικά κείμενα και Кириллица тоже: привет, мир! Добро пожаловать.",
    "中文字符测试：你好，世界。日本語のテキスト、カタカナとひらがな。한국어 문장입니다.",
    "emoji 😀👍🏽🚀 and symbols ©®™ ∑∫√∞ ≤≥ ← → ★☆ ₿ €100 ¥200 £3",
    "I'm sure THEY'RE right; don't you think we'D've known? 'Tis the 'Ll case.",
    "   leading spaces, trailing spaces   \r\n\r\nwindows lines\nunix lines\n\n\n",
    "numbers: 3.14159 2.71828 6.022e23 0x7fff 1,000,000 ٣٤٥ ⅫⅣ ½ ²³",
    "<html><body class=\"x\">a &amp; b</body></html> {\"key\": [1, 2, 3]}",
    "tabs\tand\tvertical\x0bfeeds\x0cand non breaking spaces　here",
]
FIXED = CORPUS + [
    " x", "x ", "  x", "x  ", "\n", " \n ", "\t\t", "a\r\nb", "'s", "'S'", "don't", "''", "'",
    "1", "12345", "a1b2c3", "...", " ...\n\n", "!!!?", " !", "😀", "a😀b", "́", "é",
    "<|im_start|>user\nReply with OK only.<|im_end|>\n<|im_start|>assistant\n",
    "x<|endoftext|>y", "<|endoftext|><|endoftext|>", "<|im_end", "im_end|>", " <|im_start|> ",
]


def _pool():
    rng = random.Random(7)
    chars = []
    for lo, hi, k in ((0x20, 0x7E, 60), (0xA0, 0x24F, 25), (0x370, 0x52F, 20), (0x590, 0x6FF, 10),
                      (0x900, 0xDFF, 10), (0x1E00, 0x1FFF, 10), (0x2000, 0x2BFF, 20), (0x3000, 0x30FF, 15),
                      (0x4E00, 0x9FFF, 15), (0xAC00, 0xD7A3, 10), (0xFF00, 0xFFEF, 10), (0x1F300, 0x1FAFF, 15)):
        cand = [chr(c) for c in range(lo, hi + 1) if unicodedata.category(chr(c)) not in ("Cn", "Cs", "Co")]
        chars += rng.sample(cand, min(k, len(cand)))
    chars += list("    \t\n\n\r\x0b\x0c  　''''0123456789") + ["'s", "'LL", "'re", "'d"]
    return chars


@functools.lru_cache(maxsize=1)
def train_vocab():
    """A byte-level BPE vocabulary of 1500 tokens trained over the Qwen2 pre-tokenizer."""
    from tokenizers import Regex, Tokenizer, decoders, models, pre_tokenizers, trainers
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(QWEN2_PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False),
    ])
    tok.decoder = decoders.ByteLevel()
    rng = random.Random(1)
    pool = _pool()
    corpus = CORPUS * 20 + ["".join(rng.choice(pool) for _ in range(rng.randint(5, 60))) for _ in range(400)]
    trainer = trainers.BpeTrainer(vocab_size=1500, special_tokens=SPECIALS,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet(), show_progress=False)
    tok.train_from_iterator(corpus, trainer)
    return tok


@pytest.fixture(scope="module")
def hf():
    return train_vocab()


def _kv(key: str, value) -> bytes:
    k = key.encode()
    out = struct.pack("<Q", len(k)) + k

    def s(x: str) -> bytes:
        b = x.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if isinstance(value, bool):
        return out + struct.pack("<IB", 7, int(value))
    if isinstance(value, int):
        return out + struct.pack("<II", 4, value)
    if isinstance(value, str):
        return out + struct.pack("<I", 8) + s(value)
    kind, items = value
    if kind == "str":
        return out + struct.pack("<IIQ", 9, 8, len(items)) + b"".join(s(x) for x in items)
    return out + struct.pack("<IIQ", 9, 5, len(items)) + b"".join(struct.pack("<i", x) for x in items)


def _vocab_kv(hf_tok, eos="<|endoftext|>", extra=()):
    import json
    model = json.loads(hf_tok.to_str())["model"]
    vocab = model["vocab"]
    tokens = [None] * len(vocab)
    for text, i in vocab.items():
        tokens[i] = text
    merges = [m if isinstance(m, str) else " ".join(m) for m in model["merges"]]
    types = [3 if t in SPECIALS else 1 for t in tokens]
    kv = [("tokenizer.ggml.model", "gpt2"), ("tokenizer.ggml.pre", "qwen2"),
          ("tokenizer.ggml.tokens", ("str", tokens)), ("tokenizer.ggml.token_type", ("i32", types)),
          ("tokenizer.ggml.merges", ("str", merges)), ("tokenizer.ggml.eos_token_id", vocab[eos]),
          ("tokenizer.ggml.add_bos_token", False), *extra]
    return kv, vocab


def _metadata(kv) -> bytes:
    body = b"".join(_kv(k, v) for k, v in kv)
    return b"GGUF" + struct.pack("<IQQ", 3, 0, len(kv)) + body


@pytest.fixture(scope="module")
def tok(hf, tmp_path_factory):
    kv, _ = _vocab_kv(hf)
    pkg = tmp_path_factory.mktemp("tokpkg")
    (pkg / "metadata.gguf").write_bytes(_metadata(kv))
    t = jf.Tokenizer(str(pkg))
    yield t
    t.close()


def test_fixed_strings_match_the_bpe_library(tok, hf):
    assert tok.vocab_size == hf.get_vocab_size()
    for s in FIXED:
        assert tok.tokenize(s) == hf.encode(s).ids, repr(s)


def test_random_strings_match_the_bpe_library(tok, hf):
    rng = random.Random(2024)
    pool = _pool()
    for _ in range(1500):
        s = "".join(rng.choice(pool) for _ in range(rng.randint(1, 40)))
        assert tok.tokenize(s) == hf.encode(s).ids, repr(s)


def test_long_runs(tok, hf):
    for s in (" " * 3000 + "x", "\n" * 500 + "a", "a" * 2000, "1" * 300, "😀" * 200, "ab " * 700):
        assert tok.tokenize(s) == hf.encode(s).ids


def test_pieces_spell_the_text(tok):
    rng = random.Random(5)
    pool = _pool()
    for s in FIXED + ["".join(rng.choice(pool) for _ in range(30)) for _ in range(200)]:
        assert tok.detokenize(tok.tokenize(s)) == s.encode("utf-8"), repr(s)
    # invalid UTF-8 bytes are read as U+FFFD, one per byte
    assert tok.detokenize(tok.tokenize(b"a\xffb\xc3")) == "a�b�".encode()


def test_special_tokens_and_end_tokens(tok, hf):
    ids = {t: hf.token_to_id(t) for t in SPECIALS}
    assert tok.tokenize("<|im_start|>hi<|im_end|>")[0] == ids["<|im_start|>"]
    assert tok.tokenize("<|im_start|>hi<|im_end|>")[-1] == ids["<|im_end|>"]
    assert tok.token_piece(ids["<|im_end|>"]) == b"<|im_end|>"
    # EOS plus the end and fill-in-the-middle texts llama.cpp marks as end of generation
    assert tok.end_tokens() == sorted([ids["<|endoftext|>"], ids["<|im_end|>"], ids["<|fim_pad|>"]])
    assert tok.is_end_token(-1) and tok.is_end_token(ids["<|im_end|>"])
    assert not tok.is_end_token(ids["<|im_start|>"]) and not tok.is_end_token(hf.token_to_id("a"))
    with pytest.raises(jf.InvalidArgument):
        tok.tokenize("")
    with pytest.raises(jf.InvalidArgument):
        tok.token_piece(tok.vocab_size)


def test_bos_eos_from_metadata(hf, tmp_path):
    kv, vocab = _vocab_kv(hf, extra=[("tokenizer.ggml.bos_token_id", 1), ("tokenizer.ggml.add_eos_token", True)])
    kv = [(k, True if k == "tokenizer.ggml.add_bos_token" else v) for k, v in kv]
    (tmp_path / "metadata.gguf").write_bytes(_metadata(kv))
    t = jf.Tokenizer(str(tmp_path))
    ids = t.tokenize("hello")
    assert ids[0] == 1 and ids[-1] == vocab["<|endoftext|>"] and ids[1:-1] == hf.encode("hello").ids
    t.close()


def test_duplicate_and_empty_token_texts(hf, tmp_path):
    """As llama.cpp loads a vocabulary: a text listed twice maps to its last id
    (the merges and byte tokens then produce that id), and an empty text is
    spelled "[EMPTY_<id>]". Parity with llama.cpp itself is unpinned (no
    llama.cpp in this environment); this pins the rule as restated."""
    kv, vocab = _vocab_kv(hf)
    tokens = list(dict(kv)["tokenizer.ggml.tokens"][1])
    types = list(dict(kv)["tokenizer.ggml.token_type"][1])
    h_id = vocab["h"]
    tokens += ["h", ""]  # a second "h" and an empty text at the end
    types += [1, 1]
    kv = [(k, ("str", tokens) if k == "tokenizer.ggml.tokens" else ("i32", types) if k == "tokenizer.ggml.token_type"
           else v) for k, v in kv]
    (tmp_path / "metadata.gguf").write_bytes(_metadata(kv))
    t = jf.Tokenizer(str(tmp_path))
    dup, empty = len(tokens) - 2, len(tokens) - 1
    try:
        assert t.vocab_size == len(tokens)
        ids = t.tokenize("h")
        assert ids == [dup] and h_id != dup
        assert t.token_piece(dup) == b"h" and t.token_piece(h_id) == b"h"
        assert t.token_piece(empty) == f"[EMPTY_{empty}]".encode()
    finally:
        t.close()


def test_open_errors(tmp_path):
    with pytest.raises(jf.JfhError) as e:
        jf.Tokenizer(str(tmp_path))
    assert e.value.code == 4  # not found: a package directory without metadata.gguf
    # metadata without a vocabulary (a synthesized model's package)
    model = jf.Model.synthesize(jf.ModelConfig(n_layer=1, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=512,
                                               n_ctx=64), seed=1)
    model.write_package(str(tmp_path / "pkg"))
    with pytest.raises(jf.JfhError) as e:
        jf.Tokenizer(str(tmp_path / "pkg"))
    assert e.value.code == 3


def gguf_with_vocab(model, hf_tok, path) -> None:
    """Writes `model` as a GGUF file whose metadata also holds `hf_tok`'s vocabulary."""
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        model.write_package(d)
        with open(os.path.join(d, "metadata.gguf"), "rb") as f:
            header = f.read()
    kv, _ = _vocab_kv(hf_tok)
    # the vocabulary's key/values appended to the header's KV section
    n_tensors, n_kv = struct.unpack_from("<QQ", header, 8)
    c = 24
    for _ in range(n_kv):
        (n,) = struct.unpack_from("<Q", header, c)
        c += 8 + n
        (t,) = struct.unpack_from("<I", header, c)
        c += 4
        c += struct.unpack_from("<Q", header, c)[0] + 8 if t == 8 else 4
    extra = b"".join(_kv(k, v) for k, v in kv)
    infos, _ = tensor_infos(header)
    infos_end = infos[-1][3] + 12  # after the last tensor info's type and offset
    new_header = header[:16] + struct.pack("<Q", n_kv + len(kv)) + header[24:c] + extra + header[c:infos_end]
    new_header += b"\0" * (-len(new_header) % 32)
    with open(path, "wb") as f:
        f.write(bytes(gguf_file(new_header, model.tensor_bytes)))


def test_imported_gguf_keeps_the_vocabulary(hf, tmp_path):
    """A GGUF file with a vocabulary: the imported package's metadata.gguf
    serves the same tokenizer as the file itself."""
    cfg = jf.ModelConfig(n_layer=1, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, n_vocab=hf.get_vocab_size(), n_ctx=64)
    model = jf.Model.synthesize(cfg, seed=2)
    path = tmp_path / "with_vocab.gguf"
    gguf_with_vocab(model, hf, str(path))
    imported = jf.Model.open_gguf(str(path))
    imported.write_package(str(tmp_path / "imported"))
    a, b = jf.Tokenizer(str(path)), jf.Tokenizer(str(tmp_path / "imported"))
    for s in FIXED[:12]:
        assert a.tokenize(s) == b.tokenize(s) == hf.encode(s).ids
    a.close()
    b.close()
