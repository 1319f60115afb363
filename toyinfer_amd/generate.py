"""Prompt-to-text generation over the model harness: the request path of the
reference's engine (src/engine.cpp:420-480): render the chat prompt, encode
it, prefill, then sample tokens until the end-of-sequence id or the token
budget, and turn the ids back into bytes.

Differences by design: the pick runs on the device inside the decode graph
(toyinfer_qwen3_set_sampling), so the host reads the generated ids back in
blocks of `block` steps instead of copying the logits every step; steps run
past an end-of-sequence id inside the last block are discarded.
"""
from typing import List, Optional, Tuple

import numpy as np
import torch

from toyinfer_amd.qwen3 import Qwen3
from toyinfer_amd.tokenizer import Tokenizer


def generate(model: Qwen3, tokenizer: Tokenizer, user_prompt, system_prompt=None,
             max_new_tokens: int = 64, temperature: float = 0.6, top_k: int = 20,
             top_p: float = 0.95, seed: int = 0, eos_token_id: Optional[int] = None,
             use_graph: bool = True, block: int = 16) -> Tuple[List[int], bytes]:
    """(generated ids, their text) for one request; the end-of-sequence id,
    when met, is the last id and contributes no text."""
    prompt = tokenizer.render_prompt(user_prompt, system_prompt)
    ids = np.asarray(tokenizer.encode(prompt), dtype=np.uint32)
    n = len(ids)
    cfg = model.cfg
    if n == 0 or n > cfg.max_prefill_tokens:
        raise ValueError(f"prompt of {n} tokens (1..{cfg.max_prefill_tokens} allowed)")
    budget = min(max_new_tokens, cfg.max_seq_len - n)
    if budget < 1:
        raise ValueError("no room left in max_seq_len for a generated token")
    model.set_sampling(temperature, top_k, top_p, seed)
    # The prefill copies the ids on the model's own stream: keep the device
    # tensor alive until that stream has passed it.
    ids_d = torch.from_numpy(ids.view(np.int32)).to("cuda")
    model.prefill(ids_d, n)
    model.synchronize()
    del ids_d
    out: List[int] = []
    done = 1  # the prefill's pick is generated token 1
    while True:
        toks = model.tokens_host(n + done)[n:]
        for t in toks[len(out):]:
            out.append(int(t))
            if eos_token_id is not None and int(t) == eos_token_id:
                return out, _text(tokenizer, out[:-1])
            if len(out) == budget:
                return out, _text(tokenizer, out)
        steps = min(block, budget - done)
        model.decode(steps, use_graph)
        done += steps


def _text(tokenizer: Tokenizer, ids: List[int]) -> bytes:
    return b"".join(tokenizer.decode(i) or b"" for i in ids)
