"""Write the tokenizer files the runtime reads, from a Hugging Face model
directory, without loading the model: the tokenizer part of the reference's
export.py (export.py:49-188).

  tokenizer.bin   u32 count, then per id 0..count-1: u32 length + raw bytes
                  (the byte-level BPE alphabet mapped back to bytes);
  merges.bin      u32 count, then per merge rank: u32 left, right, merged id;
  template_{user,system}[_thinking].txt
                  the chat template rendered around "%s" placeholders
                  (needs jinja2).

Differences from the reference's script: tokenizer.json is read directly
(no transformers import), and ids missing from a non-contiguous vocabulary
are written as empty tokens so that every id keeps its position (the
reference packs the sorted ids, which shifts later ids in that case).
Weights need no export step here: the loader reads the safetensors headers
itself (toyinfer_qwen3_load_weights).

Usage: python -m toyinfer_amd.export MODEL_DIR [OUT_DIR]
"""
import json
import os
import struct
import sys
from typing import Dict, List


def byte_alphabet() -> Dict[int, str]:
    """GPT-2's byte -> printable character table used by byte-level BPE:
    bytes in '!'..'~', U+00A1..U+00AC and U+00AE..U+00FF stand for
    themselves; the other 68 bytes take U+0100 onwards in byte order."""
    keep = set(range(0x21, 0x7F)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    table, extra = {}, 0
    for b in range(256):
        if b in keep:
            table[b] = chr(b)
        else:
            table[b] = chr(0x100 + extra)
            extra += 1
    return table


def token_bytes(token: str, char_to_byte: Dict[str, int]) -> bytes:
    """Alphabet characters back to their bytes; any other character (added
    tokens) as UTF-8 (export.py:43-46)."""
    return b"".join(bytes([char_to_byte[c]]) if c in char_to_byte else c.encode("utf-8")
                    for c in token)


def _merge_pair(m) -> List[str]:
    if isinstance(m, str):
        parts = m.split(" ")
        if len(parts) != 2:
            raise ValueError(f"malformed merge {m!r}")
        return parts
    if isinstance(m, list) and len(m) == 2:
        return m
    raise ValueError(f"malformed merge {m!r}")


def export_tokenizer(tokenizer_json: dict, out_dir: str) -> None:
    """tokenizer.bin and merges.bin from a parsed tokenizer.json."""
    model = tokenizer_json["model"]
    vocab: Dict[str, int] = dict(model["vocab"])
    full = dict(vocab)
    for t in tokenizer_json.get("added_tokens", []):
        full[t["content"]] = t["id"]
    by_id: Dict[int, str] = {i: t for t, i in full.items()}
    n = max(by_id) + 1
    char_to_byte = {c: b for b, c in byte_alphabet().items()}
    with open(os.path.join(out_dir, "tokenizer.bin"), "wb") as f:
        f.write(struct.pack("<I", n))
        for i in range(n):
            b = token_bytes(by_id[i], char_to_byte) if i in by_id else b""
            f.write(struct.pack("<I", len(b)))
            f.write(b)
    rows = []
    for m in model["merges"]:
        a, c = _merge_pair(m)
        for t in (a, c, a + c):
            if t not in vocab:
                raise ValueError(f"merge token {t!r} not in the vocabulary")
        rows.append((vocab[a], vocab[c], vocab[a + c]))
    with open(os.path.join(out_dir, "merges.bin"), "wb") as f:
        f.write(struct.pack("<I", len(rows)))
        for r in rows:
            f.write(struct.pack("<III", *r))


def export_templates(chat_template: str, out_dir: str) -> None:
    """The four prompt templates (export.py:138-188): user / system+user,
    each without and with thinking, rendered with "%s" as the content."""
    import jinja2

    tmpl = jinja2.Environment().from_string(chat_template)
    user = [{"role": "user", "content": "%s"}]
    system = [{"role": "system", "content": "%s"}, {"role": "user", "content": "%s"}]
    for name, msgs, think in (("template_user.txt", user, False),
                              ("template_user_thinking.txt", user, True),
                              ("template_system.txt", system, False),
                              ("template_system_thinking.txt", system, True)):
        text = tmpl.render(messages=msgs, add_generation_prompt=True, enable_thinking=think)
        with open(os.path.join(out_dir, name), "w", encoding="utf-8", newline="") as f:
            f.write(text)


def export_model_dir(model_dir: str, out_dir: str = None) -> None:
    out_dir = out_dir or model_dir
    with open(os.path.join(model_dir, "tokenizer.json"), encoding="utf-8") as f:
        export_tokenizer(json.load(f), out_dir)
    cfg_path = os.path.join(model_dir, "tokenizer_config.json")
    if os.path.exists(cfg_path):
        with open(cfg_path, encoding="utf-8") as f:
            chat = json.load(f).get("chat_template")
        if chat:
            export_templates(chat, out_dir)


if __name__ == "__main__":
    export_model_dir(sys.argv[1], sys.argv[2] if len(sys.argv) > 2 else None)
