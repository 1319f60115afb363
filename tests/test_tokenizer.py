"""Tokenizer (include/toyinfer_tokenizer.h, host C++) against the oracle's
restatement of src/tokenizer.cpp (oracle/bpe.py), on files written by
toyinfer_amd.export from a byte-level BPE trained here with the
`tokenizers` library.  Host code only: these run without a GPU.

Bars: token ids identical to the oracle's (exact); decode of the ids gives
back the input bytes; the oracle itself agrees with the `tokenizers` BPE
model on single words (where its pre-tokeniser splits nothing) and with
hand-worked merge sequences; the rendered prompt equals the string the
reference's own test expects (tests/test_tokenizer.cpp:11-14).
"""
import json
import os
import struct

import numpy as np
import pytest

from oracle import bpe
from toyinfer_amd import attn, export
from toyinfer_amd.tokenizer import Tokenizer

SPECIAL = ["<|im_start|>", "<|im_end|>", "<think>", "</think>"]
# A chat template of Qwen3's shape for the four exported variants.
CHAT = ("{% for m in messages %}<|im_start|>{{ m.role }}\n{{ m.content }}<|im_end|>\n{% endfor %}"
        "{% if add_generation_prompt %}<|im_start|>assistant\n"
        "{% if not enable_thinking %}<think>\n\n</think>\n\n{% endif %}{% endif %}")
WORDS = ("the quick brown fox jumps over lazy dog attention kernel prefill decode wavefront "
         "memory bandwidth tensor matrix core cache token sample merge byte pair encoding "
         "über naïve café 東京 日本語 テスト").split()


def corpus(n=400, seed=0):
    rng = np.random.default_rng(seed)
    return [" ".join(rng.choice(WORDS, size=rng.integers(3, 12))) + rng.choice([".", "!", "?", ""])
            for _ in range(n)]


@pytest.fixture(scope="module")
def hf_tok():
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import models, pre_tokenizers, trainers
    tok = tokenizers.Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    trainer = trainers.BpeTrainer(vocab_size=600, special_tokens=SPECIAL, show_progress=False,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(corpus(), trainer)
    return tok


@pytest.fixture(scope="module")
def model_dir(hf_tok, tmp_path_factory):
    d = str(tmp_path_factory.mktemp("tok"))
    export.export_tokenizer(json.loads(hf_tok.to_str()), d)
    export.export_templates(CHAT, d)
    return d


def padded(hf_tok):
    return (hf_tok.get_vocab_size() + 127) // 128 * 128   # vocab padded as the reference notes


def test_files_load_and_decode(hf_tok, model_dir):
    V = padded(hf_tok)
    t = Tokenizer(model_dir, V)
    o = bpe.Tokenizer(model_dir, V)
    assert t.vocab_size == V
    assert t.num_merges == len(json.loads(hf_tok.to_str())["model"]["merges"])
    for i in range(V):
        assert t.decode(i) == o.vocab[i], i
    assert t.decode(V - 1) == b""                      # padding ids are empty
    assert t.decode(V) is None
    alpha = export.byte_alphabet()
    assert sorted(set(alpha.values())) == sorted(pre_alphabet())
    for b in range(256):                               # every byte has its own token
        assert bytes([b]) in o.index


def pre_alphabet():
    from tokenizers import pre_tokenizers
    return pre_tokenizers.ByteLevel.alphabet()


def texts(seed=1):
    rng = np.random.default_rng(seed)
    out = ["", "a", "<", "<>", "<|im_start|>", "<|im_start|>user\nhello<|im_end|>\n",
           "x <think>\n\n</think> y", "<notatoken> <|im_end", "a<b>c<|im_end|>>",
           "100% sure", "tab\tand\nnewline", "mixed 東京 naïve über café"]
    for _ in range(40):
        words = list(rng.choice(WORDS + SPECIAL + ["<", ">", "  ", "\n"], size=rng.integers(1, 20)))
        out.append("".join(w + rng.choice(["", " ", "  "]) for w in words))
    out.append(bytes(rng.integers(1, 256, size=200).astype(np.uint8)))   # arbitrary bytes
    return out


def test_encode_matches_oracle(hf_tok, model_dir):
    V = padded(hf_tok)
    t = Tokenizer(model_dir, V)
    o = bpe.Tokenizer(model_dir, V)
    for s in texts():
        b = s if isinstance(s, bytes) else s.encode("utf-8")
        ids = t.encode(b)
        assert ids == o.encode(b), b
        assert o.decode(ids) == b
        assert b"".join(t.decode(i) for i in ids) == b


def test_special_tokens_kept_whole(hf_tok, model_dir):
    t = Tokenizer(model_dir, padded(hf_tok))
    vocab = hf_tok.get_vocab()
    ids = t.encode("<|im_start|>user\nhi<|im_end|>")
    assert ids[0] == vocab["<|im_start|>"] and ids[-1] == vocab["<|im_end|>"]
    # "<not>" is no token: '<' and 'n' ... merge like any other bytes
    ids = t.encode("<not>")
    assert vocab["<|im_start|>"] not in ids and len(ids) >= 2


def test_oracle_matches_library_bpe_on_words(hf_tok, model_dir):
    """On a single word the library's byte-level pre-tokeniser splits
    nothing, so its BPE merges the same byte sequence by the same rule
    (lowest rank, then leftmost)."""
    o = bpe.Tokenizer(model_dir, padded(hf_tok))
    rng = np.random.default_rng(2)
    letters = list("abcdefghijklmnopqrstuvwxyz")
    words = [w for w in WORDS if w.isascii()] + \
            ["".join(rng.choice(letters, size=rng.integers(2, 14))) for _ in range(200)]
    for w in words:
        assert o.encode(w.encode()) == hf_tok.encode(w).ids, w


def write_files(d, vocab, merges, user_tmpl="U:%s", system_tmpl="S:%s U:%s"):
    with open(os.path.join(d, "tokenizer.bin"), "wb") as f:
        f.write(struct.pack("<I", len(vocab)))
        for t in vocab:
            f.write(struct.pack("<I", len(t)) + t)
    with open(os.path.join(d, "merges.bin"), "wb") as f:
        f.write(struct.pack("<I", len(merges)))
        for m in merges:
            f.write(struct.pack("<III", *m))
    for sfx in (".txt", "_thinking.txt"):
        open(os.path.join(d, "template_user" + sfx), "w").write(user_tmpl)
        open(os.path.join(d, "template_system" + sfx), "w").write(system_tmpl)


def test_hand_worked_merges(tmp_path):
    """Vocabulary a b c ab bc abc <x>; merges rank 0 (b,c), 1 (a,b), 2 (a,bc).
    "abc": (b,c) merges first, the queued (a,b) goes stale, then (a,bc).
    "abab": both (a,b) at rank 1, left first.  "<x>ab": special token whole."""
    d = str(tmp_path)
    vocab = [b"a", b"b", b"c", b"ab", b"bc", b"abc", b"<x>", b"<", b"x", b">"]
    write_files(d, vocab, [(1, 2, 4), (0, 1, 3), (0, 4, 5)])
    t, o = Tokenizer(d, 12), bpe.Tokenizer(d, 12)
    cases = {"abc": [5], "abab": [3, 3], "cab": [2, 3], "bcbc": [4, 4], "<x>ab": [6, 3],
             "<x": [7, 8], "ab<x>>": [3, 6, 9], "": []}
    for s, exp in cases.items():
        assert t.encode(s) == exp == o.encode(s.encode()), s


def test_render_prompt(hf_tok, model_dir):
    """tests/test_tokenizer.cpp:11-14: the non-thinking user prompt."""
    t = Tokenizer(model_dir, padded(hf_tok))
    for user in ("aaa", "aaaaa"):
        exp = ("<|im_start|>user\n" + user +
               "<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n").encode()
        assert t.render_prompt(user) == exp
        assert t.encode(t.render_prompt(user))[0] == hf_tok.get_vocab()["<|im_start|>"]
    o = bpe.Tokenizer(model_dir, padded(hf_tok))
    assert t.render_prompt("hi", "be brief") == o.render_prompt(b"hi", b"be brief")
    assert t.render_prompt("hi", "be brief").startswith(b"<|im_start|>system\nbe brief<|im_end|>")
    th = Tokenizer(model_dir, padded(hf_tok), thinking=True)
    assert th.render_prompt("q").endswith(b"<|im_start|>assistant\n")


def test_render_percent_forms(tmp_path):
    d = str(tmp_path)
    write_files(d, [b"a"], [], user_tmpl="100%% of %s")
    assert Tokenizer(d, 1).render_prompt("x") == b"100% of x"
    write_files(d, [b"a"], [], user_tmpl="%d %s")
    with pytest.raises(attn.ToyInferError):
        Tokenizer(d, 1).render_prompt("x")


def test_errors(tmp_path):
    d = str(tmp_path)
    with pytest.raises(attn.ToyInferError) as e:
        Tokenizer(d, 10)                                   # no files
    assert e.value.status == attn.ERR_IO
    write_files(d, [b"a", b"b"], [(0, 1, 7)])               # merged id outside the vocabulary
    with pytest.raises(attn.ToyInferError):
        Tokenizer(d, 4)
    write_files(d, [b"a", b"b", b"ab"], [(0, 1, 2)])
    with pytest.raises(attn.ToyInferError):
        Tokenizer(d, 2)                                    # count above vocab_size
    t = Tokenizer(d, 3)
    with pytest.raises(attn.ToyInferError) as e:
        t.encode("abc")                                    # no token for 'c'
    assert e.value.status == attn.ERR_INVALID_ARGUMENT
    import ctypes
    n = ctypes.c_uint32()
    ids = (ctypes.c_uint32 * 1)()
    st = attn.LIB.toyinfer_tokenizer_encode(t.h, b"aba", ids, 1, ctypes.byref(n))
    assert st == attn.ERR_WORKSPACE and n.value == 2 and ids[0] == 2


def test_header_functions_exported_and_bound():
    import re
    import subprocess
    from toyinfer_amd import tokenizer
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(root, "include", "toyinfer_tokenizer.h")).read(),
                  flags=re.S)
    names = set(re.findall(r"\b(toyinfer_\w+)\s*\(", text))
    assert len(names) == 7
    out = subprocess.run(["nm", "-D", "--defined-only", attn.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    assert names <= set(re.findall(r"\bT (toyinfer_\w+)", out))
    assert names == set(tokenizer._SIGS)


def test_special_token_scan_limits(tmp_path):
    """src/tokenizer.cpp:177-197: the '>' must come within the longest token
    length (counted from the '<'), and only the first '>' is tried."""
    d = str(tmp_path)
    vocab = [b"<", b">", b"a", b"b", b"<ab>", b"<a>"]          # longest token: 4 bytes
    write_files(d, vocab, [])
    t, o = Tokenizer(d, 8), bpe.Tokenizer(d, 8)
    cases = {"<ab>": [4], "<a>": [5], "<a>>": [5, 1],
             "<abb>": [0, 2, 3, 3, 1],        # '>' at offset 4: beyond the scan window
             "<a<ab>": [0, 2, 4],             # no '>' in the first window; the second '<' starts "<ab>"
             "<": [0], "<ab": [0, 2, 3]}
    for s, exp in cases.items():
        assert t.encode(s) == exp == o.encode(s.encode()), s
