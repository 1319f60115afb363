"""CPU restatement of the reference tokenizer's encode and prompt rendering.

TEST INFRASTRUCTURE ONLY: the checker for toyinfer_amd's tokenizer
(toyinfer_amd/csrc/tokenizer.cpp); never imported by the product.

Follows src/tokenizer.cpp step by step, in plain Python loops (small inputs):
  * files: tokenizer.bin (:74-124), merges.bin (:22-39), templates (:126-167);
  * encode (:169-325): special tokens "<...>" up to the first '>' within the
    longest token length, else single bytes; then merges from a priority
    queue ordered by (rank, left position), skipping stale entries;
  * render_prompt (:335-369): snprintf of the template with (system, user)
    or (user).

Pinned in tests/test_tokenizer.py by: hand-worked merge sequences, a
library cross-check (the `tokenizers` BPE model on single words, where no
pre-tokenisation split applies), the decode(encode(x)) == x round trip, and
the prompt string the reference's own test expects (tests/test_tokenizer.cpp:11-14).
"""
import heapq
import os
import struct


class Tokenizer:
    def __init__(self, model_dir, vocab_size, thinking=False):
        with open(os.path.join(model_dir, "tokenizer.bin"), "rb") as f:
            b = f.read()
        count = struct.unpack_from("<I", b, 0)[0]
        if count > vocab_size:
            raise ValueError("token count above vocab_size")
        self.vocab = [b""] * vocab_size
        off = 4
        for i in range(vocab_size):
            if off >= len(b):
                break
            n = struct.unpack_from("<I", b, off)[0]
            off += 4
            self.vocab[i] = b[off:off + n]
            off += n
        self.max_len = max(len(t) for t in self.vocab)
        self.index = {}
        for i, t in enumerate(self.vocab):
            self.index.setdefault(t, i)
        with open(os.path.join(model_dir, "merges.bin"), "rb") as f:
            m = f.read()
        n = struct.unpack_from("<I", m, 0)[0]
        self.merges = {}
        for r in range(n):
            a, c, z = struct.unpack_from("<III", m, 4 + 12 * r)
            self.merges[(a, c)] = (z, r)
        sfx = "_thinking.txt" if thinking else ".txt"
        with open(os.path.join(model_dir, "template_system" + sfx), "rb") as f:
            self.system_template = f.read()
        with open(os.path.join(model_dir, "template_user" + sfx), "rb") as f:
            self.user_template = f.read()

    def encode(self, text: bytes):
        toks = []
        i = 0
        while i < len(text):
            found = False
            if text[i:i + 1] == b"<":
                for j in range(self.max_len):
                    if i + j >= len(text):
                        break
                    if text[i + j:i + j + 1] == b">":
                        cand = text[i:i + j + 1]
                        if cand in self.index:
                            toks.append(self.index[cand])
                            i += j
                            found = True
                        break
            if not found:
                ch = text[i:i + 1]
                if ch not in self.index:
                    raise ValueError(f"unknown byte {ch!r}")
                toks.append(self.index[ch])
            i += 1
        n = len(toks)
        prev = list(range(-1, n - 1))
        nxt = list(range(1, n)) + [-1] if n else []
        valid = [True] * n
        heap = []
        for i in range(n - 1):
            if (toks[i], toks[i + 1]) in self.merges:
                heapq.heappush(heap, (self.merges[(toks[i], toks[i + 1])][1], i, toks[i], toks[i + 1]))
        while heap:
            _, c, left, right = heapq.heappop(heap)
            if not valid[c] or nxt[c] == -1:
                continue
            r = nxt[c]
            if toks[r] != right or toks[c] != left:
                continue
            toks[c] = self.merges[(left, right)][0]
            valid[r] = False
            nxt[c] = nxt[r]
            if nxt[r] != -1:
                prev[nxt[r]] = c
            p = prev[c]
            if p != -1 and (toks[p], toks[c]) in self.merges:
                heapq.heappush(heap, (self.merges[(toks[p], toks[c])][1], p, toks[p], toks[c]))
            q = nxt[c]
            if q != -1 and (toks[c], toks[q]) in self.merges:
                heapq.heappush(heap, (self.merges[(toks[c], toks[q])][1], c, toks[c], toks[q]))
        out = []
        i = 0 if n else -1
        while i != -1:
            out.append(toks[i])
            i = nxt[i]
        return out

    def decode(self, ids):
        return b"".join(self.vocab[i] for i in ids)

    def render_prompt(self, user: bytes, system: bytes = None) -> bytes:
        if system is not None:
            return self.system_template.replace(b"%s", b"\x00", 2).replace(
                b"\x00", system, 1).replace(b"\x00", user, 1)
        return self.user_template.replace(b"%s", user, 1)
