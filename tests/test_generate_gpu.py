"""Prompt to text on one model directory holding both the exported tokenizer
files and safetensors weights: Qwen3.from_pretrained + Tokenizer +
generate().  The generated ids must equal a step-by-step run of the same
model (prefill, then one directly launched decode step at a time) with the
same sampling settings, stop at the end-of-sequence id, and decode to the
concatenated token bytes."""
import json

import numpy as np
import pytest
import torch

from tests.test_tokenizer import CHAT, SPECIAL, corpus
from tests.test_weights import TINY, random_tensors, write_model
from toyinfer_amd import export, qwen3
from toyinfer_amd.generate import generate
from toyinfer_amd.tokenizer import Tokenizer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model_dir(tmp_path_factory):
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import models, pre_tokenizers, trainers
    d = str(tmp_path_factory.mktemp("model"))
    tok = tokenizers.Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.train_from_iterator(corpus(), trainers.BpeTrainer(
        vocab_size=600, special_tokens=SPECIAL, show_progress=False,
        initial_alphabet=pre_tokenizers.ByteLevel.alphabet()))
    export.export_tokenizer(json.loads(tok.to_str()), d)
    export.export_templates(CHAT, d)
    write_model(d, TINY, random_tensors(TINY, seed=62), 2, True)
    return d


def stepwise(model, ids, steps, settings):
    model.set_sampling(*settings)
    model.prefill(torch.from_numpy(ids.astype(np.int32)).to("cuda"), len(ids))
    for _ in range(steps - 1):
        model.decode(1, False)
    return [int(t) for t in model.tokens_host(len(ids) + steps)[len(ids):]]


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_generate_matches_stepwise(model_dir, temperature):
    print(f"[step] generate T={temperature}", flush=True)
    m = qwen3.Qwen3.from_pretrained(model_dir, 128, 64)
    tk = Tokenizer(model_dir, m.cfg.vocab_size)
    settings = (temperature, 20, 0.95, 11)
    ids, text = generate(m, tk, "the quick brown fox", max_new_tokens=40, temperature=temperature,
                         top_k=20, top_p=0.95, seed=11, block=7)
    assert len(ids) == 40
    assert text == b"".join(tk.decode(i) for i in ids)
    prompt = np.asarray(tk.encode(tk.render_prompt("the quick brown fox")), np.uint32)
    assert stepwise(m, prompt, 40, settings) == ids
    # End of sequence: the id generated fifth stops the next request there.
    eos = ids[4]
    first = ids.index(eos)
    ids2, text2 = generate(m, tk, "the quick brown fox", max_new_tokens=40,
                           temperature=temperature, top_k=20, top_p=0.95, seed=11,
                           eos_token_id=eos, block=3)
    assert ids2 == ids[:first + 1]
    assert text2 == b"".join(tk.decode(i) for i in ids[:first])
    m.close()
