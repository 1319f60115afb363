"""ctypes binding of the Qwen3 model harness (include/toyinfer_qwen3.h).

The model reads the caller's device weights (torch tensors here, kept alive by
the object) and owns its state; `prefill`, `decode` enqueue on the model's own
stream, `synchronize` waits for it, and the `*_host` readers copy state to the
host after synchronising.
"""
from __future__ import annotations

import ctypes
from typing import Dict, Sequence

import numpy as np

from . import attn

_vp, _u32, _f32, _i32, _sz = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_float, ctypes.c_int,
                              ctypes.c_size_t)

LAYER_FIELDS = ("input_layernorm", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "o_proj",
                "post_attention_layernorm", "gate_proj", "up_proj", "down_proj")


class Config(ctypes.Structure):
    _fields_ = [("num_layers", _u32), ("hidden_size", _u32), ("num_q_heads", _u32),
                ("num_kv_heads", _u32), ("head_dim", _u32), ("intermediate_size", _u32),
                ("vocab_size", _u32), ("max_seq_len", _u32), ("max_prefill_tokens", _u32),
                ("rms_norm_eps", _f32), ("rope_theta", _f32)]


class Layer(ctypes.Structure):
    _fields_ = [(n, _vp) for n in LAYER_FIELDS]


class ModelInfo(ctypes.Structure):
    _fields_ = [("bos_token_id", _u32), ("eos_token_id", _u32),
                ("max_position_embeddings", _u32), ("tie_word_embeddings", ctypes.c_int32)]


class Weights(ctypes.Structure):
    _fields_ = [("device", _vp), ("device_bytes", _sz), ("embed_tokens", _vp),
                ("final_norm", _vp), ("lm_head", _vp), ("layers", ctypes.POINTER(Layer)),
                ("num_layers", _u32)]


_SIGS = {
    "toyinfer_qwen3_read_config": (_i32, [ctypes.c_char_p, _u32, _u32, ctypes.POINTER(Config),
                                          ctypes.POINTER(ModelInfo)]),
    "toyinfer_qwen3_check_weights": (_i32, [ctypes.c_char_p, ctypes.POINTER(Config), _i32,
                                            ctypes.POINTER(_sz)]),
    "toyinfer_qwen3_load_weights": (_i32, [ctypes.c_char_p, ctypes.POINTER(Config), _i32, _vp,
                                           ctypes.POINTER(Weights)]),
    "toyinfer_qwen3_free_weights": (None, [ctypes.POINTER(Weights)]),
    "toyinfer_qwen3_state_bytes": (_sz, [ctypes.POINTER(Config)]),
    "toyinfer_qwen3_create": (_i32, [ctypes.POINTER(Config), _vp, _vp, _vp, ctypes.POINTER(Layer),
                                     ctypes.POINTER(_vp)]),
    "toyinfer_qwen3_destroy": (None, [_vp]),
    "toyinfer_qwen3_prefill": (_i32, [_vp, _vp, _u32]),
    "toyinfer_qwen3_decode": (_i32, [_vp, _u32, _i32]),
    "toyinfer_qwen3_set_sampling": (_i32, [_vp, ctypes.c_float, _u32, ctypes.c_float,
                                           ctypes.c_uint64]),
    "toyinfer_qwen3_synchronize": (_i32, [_vp]),
    "toyinfer_qwen3_logits": (_vp, [_vp]),
    "toyinfer_qwen3_tokens": (_vp, [_vp]),
    "toyinfer_qwen3_position": (_vp, [_vp]),
    "toyinfer_qwen3_stream": (_vp, [_vp]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(attn.LIB, _name)
    _fn.restype, _fn.argtypes = _res, _args

_hip = None


def _hip_memcpy_d2h(dst: np.ndarray, src_ptr: int) -> None:
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipMemcpy.argtypes = [_vp, _vp, _sz, ctypes.c_int]
    err = _hip.hipMemcpy(dst.ctypes.data, src_ptr, dst.nbytes, 2)  # hipMemcpyDeviceToHost
    if err != 0:
        raise RuntimeError(f"hipMemcpy failed: {err}")


def make_config(**kw) -> Config:
    return Config(**kw)


def read_config(model_dir: str, max_seq_len: int = 0, max_prefill_tokens: int = 4096):
    """(Config, ModelInfo) from model_dir/config.json (src/config.cpp:10-40)."""
    cfg, info = Config(), ModelInfo()
    attn._check("qwen3_read_config", attn.LIB.toyinfer_qwen3_read_config(
        model_dir.encode(), max_seq_len, max_prefill_tokens, ctypes.byref(cfg), ctypes.byref(info)))
    return cfg, info


def check_weights(model_dir: str, cfg: Config, tie: bool) -> int:
    """Device bytes the load needs; raises if the checkpoint does not match cfg."""
    n = _sz()
    attn._check("qwen3_check_weights", attn.LIB.toyinfer_qwen3_check_weights(
        model_dir.encode(), ctypes.byref(cfg), int(tie), ctypes.byref(n)))
    return n.value


class _Addr:
    """A device address standing in for a tensor (data_ptr only)."""

    def __init__(self, p: int):
        self.p = int(p)

    def data_ptr(self) -> int:
        return self.p


class LoadedWeights:
    """Checkpoint weights uploaded by toyinfer_qwen3_load_weights; the dict
    form (`as_dict`) is what Qwen3 takes."""

    def __init__(self, model_dir: str, cfg: Config, tie: bool, stream=None):
        self.w = Weights()
        attn._check("qwen3_load_weights", attn.LIB.toyinfer_qwen3_load_weights(
            model_dir.encode(), ctypes.byref(cfg), int(tie), stream, ctypes.byref(self.w)))

    def as_dict(self) -> Dict:
        w = self.w
        layers = [{n: _Addr(getattr(w.layers[i], n)) for n in LAYER_FIELDS}
                  for i in range(w.num_layers)]
        return {"embed_tokens": _Addr(w.embed_tokens), "norm": _Addr(w.final_norm),
                "lm_head": _Addr(w.lm_head), "layers": layers, "_owner": self}

    def close(self) -> None:
        if self.w.device:
            attn.LIB.toyinfer_qwen3_free_weights(ctypes.byref(self.w))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Qwen3:
    """weights: dict with embed_tokens, norm, lm_head (may be embed_tokens) and
    layers: a list of dicts keyed by LAYER_FIELDS; all bf16 CUDA tensors."""

    def __init__(self, cfg: Config, weights: Dict):
        self.cfg = cfg
        self._keep = weights
        self._held = []  # device ids whose copy may still be queued (prefill)
        layers = (Layer * cfg.num_layers)()
        for i, lw in enumerate(weights["layers"]):
            for n in LAYER_FIELDS:
                setattr(layers[i], n, lw[n].data_ptr())
        self._layers = layers
        handle = _vp()
        attn._check("qwen3_create", attn.LIB.toyinfer_qwen3_create(
            ctypes.byref(cfg), weights["embed_tokens"].data_ptr(), weights["norm"].data_ptr(),
            weights["lm_head"].data_ptr(), layers, ctypes.byref(handle)))
        self.h = handle

    @classmethod
    def from_pretrained(cls, model_dir: str, max_seq_len: int = 0,
                        max_prefill_tokens: int = 4096) -> "Qwen3":
        """config.json + safetensors shards of model_dir (the reference's
        LLMConfig and Qwen3::load_weights, src/config.cpp, src/qwen.cpp)."""
        cfg, info = read_config(model_dir, max_seq_len, max_prefill_tokens)
        weights = LoadedWeights(model_dir, cfg, bool(info.tie_word_embeddings))
        m = cls(cfg, weights.as_dict())
        m.info = info
        return m

    def close(self):
        if self.h:
            attn.LIB.toyinfer_qwen3_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def state_bytes(cfg: Config) -> int:
        return attn.LIB.toyinfer_qwen3_state_bytes(ctypes.byref(cfg))

    def prefill(self, ids_dev, n: int) -> None:
        """The ids are copied on the model's stream after this returns, so
        the tensor is held here until the next synchronize(): a caller's
        temporary is not handed back to torch's allocator before the copy."""
        attn._check("qwen3_prefill", attn.LIB.toyinfer_qwen3_prefill(self.h, ids_dev.data_ptr(), n))
        self._held.append(ids_dev)

    def decode(self, steps: int, graph: bool) -> None:
        attn._check("qwen3_decode", attn.LIB.toyinfer_qwen3_decode(self.h, steps, int(graph)))

    def set_sampling(self, temperature: float, top_k: int, top_p: float, seed: int) -> None:
        attn._check("qwen3_set_sampling",
                    attn.LIB.toyinfer_qwen3_set_sampling(self.h, temperature, top_k, top_p, seed))

    def synchronize(self) -> None:
        attn._check("qwen3_synchronize", attn.LIB.toyinfer_qwen3_synchronize(self.h))
        self._held.clear()

    def logits_host(self) -> np.ndarray:
        self.synchronize()
        out = np.empty(self.cfg.vocab_size, np.float32)
        _hip_memcpy_d2h(out, attn.LIB.toyinfer_qwen3_logits(self.h))
        return out

    def tokens_host(self, n: int) -> np.ndarray:
        self.synchronize()
        out = np.empty(n, np.uint32)
        _hip_memcpy_d2h(out, attn.LIB.toyinfer_qwen3_tokens(self.h))
        return out

    def position_host(self) -> int:
        self.synchronize()
        out = np.empty(1, np.uint32)
        _hip_memcpy_d2h(out, attn.LIB.toyinfer_qwen3_position(self.h))
        return int(out[0])

    @property
    def stream_ptr(self) -> int:
        return attn.LIB.toyinfer_qwen3_stream(self.h)


def layer_shapes(cfg: Config) -> Dict[str, Sequence[int]]:
    qd, kv = cfg.num_q_heads * cfg.head_dim, cfg.num_kv_heads * cfg.head_dim
    H, F = cfg.hidden_size, cfg.intermediate_size
    return {"input_layernorm": (H,), "q_proj": (qd, H), "k_proj": (kv, H), "v_proj": (kv, H),
            "q_norm": (cfg.head_dim,), "k_norm": (cfg.head_dim,), "o_proj": (H, qd),
            "post_attention_layernorm": (H,), "gate_proj": (F, H), "up_proj": (F, H),
            "down_proj": (H, F)}
