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


_SIGS = {
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


class Qwen3:
    """weights: dict with embed_tokens, norm, lm_head (may be embed_tokens) and
    layers: a list of dicts keyed by LAYER_FIELDS; all bf16 CUDA tensors."""

    def __init__(self, cfg: Config, weights: Dict):
        self.cfg = cfg
        self._keep = weights
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
        attn._check("qwen3_prefill", attn.LIB.toyinfer_qwen3_prefill(self.h, ids_dev.data_ptr(), n))

    def decode(self, steps: int, graph: bool) -> None:
        attn._check("qwen3_decode", attn.LIB.toyinfer_qwen3_decode(self.h, steps, int(graph)))

    def set_sampling(self, temperature: float, top_k: int, top_p: float, seed: int) -> None:
        attn._check("qwen3_set_sampling",
                    attn.LIB.toyinfer_qwen3_set_sampling(self.h, temperature, top_k, top_p, seed))

    def synchronize(self) -> None:
        attn._check("qwen3_synchronize", attn.LIB.toyinfer_qwen3_synchronize(self.h))

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
