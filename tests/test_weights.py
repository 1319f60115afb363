"""Checkpoint loading (include/toyinfer_qwen3.h: toyinfer_qwen3_read_config,
_check_weights, _load_weights) against files written by the `safetensors`
library from a small random model.

CPU tests: config.json fields, the header walk (index file or a directory
of shards), and every rejection (missing tensor, wrong dtype, wrong shape,
bytes outside the file, malformed JSON).  GPU tests: every uploaded tensor
is byte-identical to its source, and a model created from the loaded
weights produces bit-identical logits and tokens to one created from the
same tensors uploaded directly.
"""
import json
import os

import numpy as np
import pytest
import torch

from toyinfer_amd import attn, qwen3

TINY = dict(num_layers=2, hidden_size=256, num_q_heads=4, num_kv_heads=2, head_dim=64,
            intermediate_size=512, vocab_size=1000, max_seq_len=64, max_prefill_tokens=32,
            rms_norm_eps=1e-6, rope_theta=1e6)
HF_NAMES = {"input_layernorm": "input_layernorm", "q_proj": "self_attn.q_proj",
            "k_proj": "self_attn.k_proj", "v_proj": "self_attn.v_proj",
            "q_norm": "self_attn.q_norm", "k_norm": "self_attn.k_norm",
            "o_proj": "self_attn.o_proj", "post_attention_layernorm": "post_attention_layernorm",
            "gate_proj": "mlp.gate_proj", "up_proj": "mlp.up_proj", "down_proj": "mlp.down_proj"}


def hf_config(cfg, tie):
    return {"architectures": ["Qwen3ForCausalLM"], "num_hidden_layers": cfg["num_layers"],
            "hidden_size": cfg["hidden_size"], "num_attention_heads": cfg["num_q_heads"],
            "num_key_value_heads": cfg["num_kv_heads"], "head_dim": cfg["head_dim"],
            "intermediate_size": cfg["intermediate_size"], "vocab_size": cfg["vocab_size"],
            "rms_norm_eps": cfg["rms_norm_eps"], "rope_theta": cfg["rope_theta"],
            "max_position_embeddings": 40960, "bos_token_id": 151643, "eos_token_id": 151645,
            "tie_word_embeddings": tie, "torch_dtype": "bfloat16", "rope_scaling": None}


def random_tensors(cfg, seed=60, tie=False):
    """name -> bf16 CPU tensor, HF Qwen3 names."""
    g = torch.Generator().manual_seed(seed)
    shapes = qwen3.layer_shapes(qwen3.Config(**cfg))
    out = {}
    for l in range(cfg["num_layers"]):
        for n, shp in shapes.items():
            t = torch.randn(*shp, generator=g) * (0.05 if len(shp) == 2 else 0.1) + (len(shp) == 1)
            out[f"model.layers.{l}.{HF_NAMES[n]}.weight"] = t.to(torch.bfloat16)
    V, H = cfg["vocab_size"], cfg["hidden_size"]
    out["model.embed_tokens.weight"] = torch.randn(V, H, generator=g).to(torch.bfloat16)
    out["model.norm.weight"] = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    if not tie:
        out["lm_head.weight"] = (0.05 * torch.randn(V, H, generator=g)).to(torch.bfloat16)
    return out


def write_model(d, cfg, tensors, shards=2, index=True, tie=False):
    from safetensors.torch import save_file
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(hf_config(cfg, tie), f)
    names = sorted(tensors)
    parts = [names[i::shards] for i in range(shards)]
    weight_map = {}
    for i, part in enumerate(parts):
        fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        save_file({n: tensors[n] for n in part}, os.path.join(d, fn), metadata={"format": "pt"})
        weight_map.update({n: fn for n in part})
    if index:
        with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {"total_size": 0}, "weight_map": weight_map}, f)


def cfg_of(d):
    return qwen3.read_config(d, 64, 32)


def test_read_config(tmp_path):
    d = str(tmp_path)
    write_model(d, TINY, random_tensors(TINY))
    cfg, info = qwen3.read_config(d, 0, 32)
    for k, v in TINY.items():
        if k == "max_seq_len":
            assert cfg.max_seq_len == 40960                 # 0 takes max_position_embeddings
        elif isinstance(v, float):
            assert getattr(cfg, k) == pytest.approx(v, rel=1e-7), k
        else:
            assert getattr(cfg, k) == v, k
    assert (info.bos_token_id, info.eos_token_id, info.tie_word_embeddings) == (151643, 151645, 0)
    c = json.load(open(os.path.join(d, "config.json")))
    del c["head_dim"]                                      # default hidden / heads
    c["eos_token_id"] = [7, 8]
    json.dump(c, open(os.path.join(d, "config.json"), "w"))
    cfg, info = qwen3.read_config(d, 64, 32)
    assert cfg.head_dim == 64 and info.eos_token_id == 7
    for bad in ('{"hidden_size": 256', '{"hidden_size": -1}', "[]"):
        open(os.path.join(d, "config.json"), "w").write(bad)
        with pytest.raises(attn.ToyInferError) as e:
            qwen3.read_config(d, 64, 32)
        assert e.value.status == attn.ERR_IO


@pytest.mark.parametrize("shards,index,tie", [(1, False, False), (3, True, False), (2, False, True)])
def test_check_weights_layouts(tmp_path, shards, index, tie):
    d = str(tmp_path)
    t = random_tensors(TINY, tie=tie)
    write_model(d, TINY, t, shards, index, tie)
    cfg, info = cfg_of(d)
    n = qwen3.check_weights(d, cfg, bool(info.tie_word_embeddings))
    exp = sum((v.numel() * 2 + 255) // 256 * 256 for v in t.values())
    assert n == exp


def expect_io(d, cfg, status=attn.ERR_IO, tie=False):
    with pytest.raises(attn.ToyInferError) as e:
        qwen3.check_weights(d, cfg, tie)
    assert e.value.status == status


def test_check_weights_rejects(tmp_path):
    base = random_tensors(TINY)
    cfg = qwen3.Config(**TINY)
    d = str(tmp_path / "missing")
    t = dict(base)
    del t["model.layers.1.mlp.up_proj.weight"]
    write_model(d, TINY, t, 2, False)
    expect_io(d, cfg)
    d = str(tmp_path / "dtype")
    t = dict(base)
    t["model.norm.weight"] = t["model.norm.weight"].float()
    write_model(d, TINY, t, 2, False)
    expect_io(d, cfg, attn.ERR_UNSUPPORTED)
    d = str(tmp_path / "shape")
    t = dict(base)
    t["model.layers.0.self_attn.k_proj.weight"] = t["model.layers.0.self_attn.q_proj.weight"]
    write_model(d, TINY, t, 2, False)
    expect_io(d, cfg)
    d = str(tmp_path / "truncated")
    write_model(d, TINY, base, 1, False)
    fn = os.path.join(d, "model-00001-of-00001.safetensors")
    os.truncate(fn, os.path.getsize(fn) - 64)
    expect_io(d, cfg)
    d = str(tmp_path / "badjson")
    write_model(d, TINY, base, 1, False)
    with open(fn := os.path.join(d, "model-00001-of-00001.safetensors"), "r+b") as f:
        f.seek(8)
        f.write(b"}")
    expect_io(d, cfg)
    d = str(tmp_path / "index_names_absent_file")
    write_model(d, TINY, base, 2, True)
    os.remove(os.path.join(d, "model-00002-of-00002.safetensors"))
    expect_io(d, cfg)
    expect_io(str(tmp_path / "nothing_here"), cfg)
    d = str(tmp_path / "good")
    write_model(d, TINY, base, 2, True)
    assert qwen3.check_weights(d, cfg, False) > 0
    expect_io(d, qwen3.Config(**dict(TINY, intermediate_size=640)))  # config and files disagree
    expect_io(d, qwen3.Config(**dict(TINY, num_layers=3)))


@pytest.mark.gpu
@pytest.mark.parametrize("tie", [False, True])
def test_load_weights_bytes_and_model(dev, tmp_path, tie):
    print(f"[step] load weights tie={tie}", flush=True)
    d = str(tmp_path)
    t = random_tensors(TINY, seed=61, tie=tie)
    write_model(d, TINY, t, 3, True, tie)
    cfg, info = cfg_of(d)
    lw = qwen3.LoadedWeights(d, cfg, bool(info.tie_word_embeddings))
    w = lw.as_dict()
    bits = lambda x: x.view(torch.int16).numpy()

    def dev_bits(addr, ref):
        out = np.empty(ref.numel(), np.int16)
        qwen3._hip_memcpy_d2h(out, addr.data_ptr())
        return out.reshape(tuple(ref.shape))
    assert np.array_equal(dev_bits(w["embed_tokens"], t["model.embed_tokens.weight"]),
                          bits(t["model.embed_tokens.weight"]))
    assert np.array_equal(dev_bits(w["norm"], t["model.norm.weight"]), bits(t["model.norm.weight"]))
    head = t["model.embed_tokens.weight"] if tie else t["lm_head.weight"]
    assert np.array_equal(dev_bits(w["lm_head"], head), bits(head))
    for l in range(TINY["num_layers"]):
        for n, hf in HF_NAMES.items():
            ref = t[f"model.layers.{l}.{hf}.weight"]
            assert np.array_equal(dev_bits(w["layers"][l][n], ref), bits(ref)), (l, n)
            assert w["layers"][l][n].data_ptr() % 256 == 0
    # The same model from directly uploaded tensors: identical logits and tokens.
    direct = {"embed_tokens": t["model.embed_tokens.weight"].to(dev),
              "norm": t["model.norm.weight"].to(dev),
              "lm_head": head.to(dev),
              "layers": [{n: t[f"model.layers.{l}.{hf}.weight"].to(dev) for n, hf in HF_NAMES.items()}
                         for l in range(TINY["num_layers"])]}
    a = qwen3.Qwen3.from_pretrained(d, 64, 32)
    b = qwen3.Qwen3(qwen3.Config(**TINY), direct)
    torch.cuda.synchronize()
    ids = torch.from_numpy(np.arange(5, 17, dtype=np.int32) * 37 % 1000).to(dev)
    for m in (a, b):
        m.prefill(ids, 12)
        m.decode(4, True)
    assert np.array_equal(a.logits_host().view(np.uint32), b.logits_host().view(np.uint32))
    assert np.array_equal(a.tokens_host(17), b.tokens_host(17))
    a.close()
    b.close()
    lw.close()


def test_config_json_forms(tmp_path):
    """The loader's JSON reader on valid forms real configs use (nested
    objects, escapes, surrogate pairs, exponents, null) and on malformed ones."""
    d = str(tmp_path)
    good = ('{"architectures": ["Qwen3ForCausalLM"], "name": "caf\\u00e9 \\ud83d\\ude00 \\"q\\" \\\\ \\/",'
            ' "rope_scaling": {"type": "yarn", "factor": 4.0, "deep": [[[1, 2], {"a": null}]]},'
            ' "num_hidden_layers": 2, "hidden_size": 256, "num_attention_heads": 4,'
            ' "num_key_value_heads": 2, "head_dim": 64, "intermediate_size": 512,'
            ' "vocab_size": 1000, "rms_norm_eps": 1e-06, "rope_theta": 1000000.0,'
            ' "max_position_embeddings": 40960, "bos_token_id": null, "eos_token_id": [151645, 151643],'
            ' "tie_word_embeddings": true, "torch_dtype": "bfloat16", "use_cache": false}')
    open(os.path.join(d, "config.json"), "w").write(good)
    cfg, info = qwen3.read_config(d, 0, 16)
    assert cfg.rms_norm_eps == pytest.approx(1e-6) and cfg.rope_theta == 1e6
    assert (info.bos_token_id, info.eos_token_id, info.tie_word_embeddings) == (0, 151645, 1)
    bad = [good[:-1],                                           # unterminated object
           good.replace('"use_cache": false}', '"use_cache": false,}'),   # trailing comma
           good.replace("\\u00e9", "\\u00g9"),                  # bad hex digit
           good.replace("\\ud83d\\ude00", "\\ud83d"),           # lone high surrogate
           good.replace("4.0", "4."),                           # digits must follow '.'
           good.replace('"hidden_size": 256', '"hidden_size": 256.5'),   # not an integer
           '[' * 100 + ']' * 100,                               # nesting too deep
           good + " x"]                                         # trailing garbage
    for b in bad:
        open(os.path.join(d, "config.json"), "w").write(b)
        with pytest.raises(attn.ToyInferError) as e:
            qwen3.read_config(d, 0, 16)
        assert e.value.status == attn.ERR_IO, b[:60]


def test_lm_head_choice(tmp_path):
    """lm_head.weight is loaded only when present and the embeddings are not
    tied; otherwise the embeddings serve as the lm-head (the reference always
    uses them, src/qwen.cpp:482-483)."""
    d = str(tmp_path)
    t = random_tensors(TINY)                       # has lm_head.weight
    write_model(d, TINY, t, 2, True)
    cfg = qwen3.Config(**TINY)
    head = (t["lm_head.weight"].numel() * 2 + 255) // 256 * 256
    untied = qwen3.check_weights(d, cfg, False)
    assert qwen3.check_weights(d, cfg, True) == untied - head
    d2 = str(tmp_path / "nohead")
    t2 = dict(t)
    del t2["lm_head.weight"]
    write_model(d2, TINY, t2, 2, True)
    assert qwen3.check_weights(d2, cfg, False) == untied - head
