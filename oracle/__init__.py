"""Python view of the CPU oracle (``oracle/attn_oracle.c``).

TEST INFRASTRUCTURE ONLY: the checker for the HIP attention path.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module.  Nothing under ``toyinfer_amd/`` uses it.

Every function restates one host reference of the reference's tests; the
C file's header lists them with file:line citations, and
``tests/test_oracle.py`` pins each against fixtures, closed forms and
invariants.  Arrays are numpy: bf16 tensors travel as ``uint16`` bit
patterns, everything else as ``float32``.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u32 = ctypes.c_uint32
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_f32 = ctypes.c_float
_vp = ctypes.c_void_p


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(
            f"{_LIB_PATH} is missing: build it with `make -C oracle` "
            "(or __graft_entry__.build())")
    lib = ctypes.CDLL(_LIB_PATH)
    sig = {
        "or_f32_to_bf16_array": (None, [_f32p, _u16p, ctypes.c_int64]),
        "or_bf16_to_f32_array": (None, [_u16p, _f32p, ctypes.c_int64]),
        "or_make_flash_case": (None, [_u32, _u32, _u32, _u32, _f32, _f32, _f32, _f32, _f32,
                                      _f32p, _f32p, _f32p]),
        "or_make_causal_focus_case": (None, [_f32p, _f32p, _f32p]),
        "or_make_attention_case": (None, [_u32, _u32, _u32, _u32, _f32, _f32,
                                          _f32p, _f32p, _f32p]),
        "or_make_rmsnorm_case": (None, [_u32, _u32, _u32, _f32, _f32, _f32p, _f32p]),
        "or_make_batch_rmsnorm_case": (None, [_u32, _u32, _u32, _f32, _f32, _f32p, _f32p]),
        "or_make_rope_case": (None, [_u32, _u32, _u32, _f32, _f32, _f32p, _f32p]),
        "or_flash_reference_f32": (None, [_f32p, _f32p, _f32p, _f32p, _u32, _u32, _u32, _u32,
                                          _vp, _u32, ctypes.c_int]),
        "or_flash_reference_bf16": (None, [_u16p, _u16p, _u16p, _f32p, _u32, _u32, _u32, _u32,
                                           _vp, _u32, ctypes.c_int]),
        "or_decode_qk_scores": (None, [_f32p, _f32p, _f32p, _u32, _u32, _u32, _u32, _u32]),
        "or_decode_softmax": (None, [_f32p, _u32, _u32, _u32]),
        "or_decode_apply": (None, [_f32p, _f32p, _f32p, _u32, _u32, _u32, _u32, _u32]),
        "or_decode_attention_f32": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _vp, _u32, _u32,
                                           _u32, _u32, _u32]),
        "or_decode_batched_bf16": (None, [_u16p, _u16p, _u16p, _f32p, _u32, _u32, _u32, _u32,
                                          _vp, ctypes.c_int64, ctypes.c_int]),
        "or_multi_rmsnorm": (None, [_f32p, _f32p, _f32p, _u32, _u32, _f32]),
        "or_rope": (None, [_f32p, _f32p, _u32, _u32, _u32, _u32]),
        "or_inv_freq": (None, [_f32p, ctypes.c_int, _f32]),
        "or_qk_norm_rope": (None, [_f32p, _f32p, _f32p, _u32, _u32, _u32, _f32]),
        "or_make_gemv_case": (None, [_u32, _u32, _f32, _f32, _f32p, _f32p]),
        "or_make_batch_gemv_case": (None, [_u32, _u32, _u32, _f32, _f32, _f32p, _f32p]),
        "or_gemv": (None, [_f32p, _f32p, _f32p, _u32, _u32, _u32, ctypes.c_int]),
        "or_make_rmsnorm_row_case": (None, [_u32, _u32, _f32, _f32, _f32p, _f32p]),
        "or_make_batch_row_rmsnorm_case": (None, [_u32, _u32, _f32, _f32, _f32p, _f32p]),
        "or_make_swiglu_case": (None, [_u32, _u32, _f32, _f32, _f32p, _f32p]),
        "or_make_add_case": (None, [_u32, _u32, _f32, _f32, _f32, _f32p, _f32p]),
        "or_residual_add": (None, [_f32p, _f32p, _f32p, ctypes.c_int64]),
        "or_swiglu": (None, [_f32p, _f32p, _f32p, ctypes.c_int64]),
        "or_argmax": (_u32, [_f32p, _u32]),
        "or_sample_topk_topp": (_u32, [_f32p, _u32, _f32, _u32, _f32, _f32, _u32p, _f32p,
                                       _u32p]),
        "or_sample_coin": (_f32, [ctypes.c_uint64, _u32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------ bf16

def f32_to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bit patterns (RNE, quiet NaN)."""
    x = _c32(x)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_bf16_to_f32_array(h.reshape(-1), out.reshape(-1), h.size)
    return out


def round_bf16(x) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(x))


# ------------------------------------------------------- case generators

def make_flash_case(hq, hkv, d, s, q_phase, kv_phase, q_scale=1.0, k_scale=1.0, v_scale=1.0):
    """tests/flash_attention_test_common.h:25-85 -> float (q, k, v)."""
    q = np.empty((s, hq, d), np.float32)
    k = np.empty((s, hkv, d), np.float32)
    v = np.empty((s, hkv, d), np.float32)
    lib().or_make_flash_case(hq, hkv, d, s, q_phase, kv_phase, q_scale, k_scale, v_scale,
                             q.reshape(-1), k.reshape(-1), v.reshape(-1))
    return q, k, v


def make_causal_focus_case():
    """tests/test_flash_attention_v1_bf16.cu:11-45 -> (q, k, v), Hq2 Hkv1 D64 S6."""
    q = np.empty((6, 2, 64), np.float32)
    k = np.empty((6, 1, 64), np.float32)
    v = np.empty((6, 1, 64), np.float32)
    lib().or_make_causal_focus_case(q.reshape(-1), k.reshape(-1), v.reshape(-1))
    return q, k, v


def make_attention_case(hq, hkv, d, max_seq_len, q_phase, kv_phase):
    """tests/attention_test_common.h:40-85 -> float (q [Hq][D], k, v [MSL][Hkv][D])."""
    q = np.empty((hq, d), np.float32)
    k = np.empty((max_seq_len, hkv, d), np.float32)
    v = np.empty((max_seq_len, hkv, d), np.float32)
    lib().or_make_attention_case(hq, hkv, d, max_seq_len, q_phase, kv_phase,
                                 q.reshape(-1), k.reshape(-1), v.reshape(-1))
    return q, k, v


def make_rmsnorm_case(num_heads, d, buffer_size, input_phase, weight_phase):
    x = np.empty(buffer_size, np.float32)
    w = np.empty(d, np.float32)
    lib().or_make_rmsnorm_case(num_heads, d, buffer_size, input_phase, weight_phase, x, w)
    return x, w


def make_batch_rmsnorm_case(batch, num_heads, d, input_phase, weight_phase):
    x = np.empty((batch, num_heads, d), np.float32)
    w = np.empty(d, np.float32)
    lib().or_make_batch_rmsnorm_case(batch, num_heads, d, input_phase, weight_phase,
                                     x.reshape(-1), w)
    return x, w


def make_rope_case(num_heads, d, buffer_size, qk_phase, freq_scale):
    qk = np.empty(buffer_size, np.float32)
    f = np.empty(d // 2, np.float32)
    lib().or_make_rope_case(num_heads, d, buffer_size, qk_phase, freq_scale, qk, f)
    return qk, f


# ----------------------------------------------------------- references

def _rows_arg(rows):
    if rows is None:
        return None, 0, None
    r = np.ascontiguousarray(rows, dtype=np.uint32)
    return r.ctypes.data_as(_vp), r.size, r


def flash_reference(q, k, v, rows: Optional[Sequence[int]] = None, nthreads: int = 0):
    """Causal GQA prefill reference (flash_attention_test_common.h:87-136).

    q [S][Hq][D], k/v [S][Hkv][D]: uint16 bf16 bits or float32 (already
    bf16-valued).  Returns float32 [S][Hq][D] before the final bf16 rounding;
    rows not in ``rows`` are NaN.
    """
    s, hq, d = q.shape
    hkv = k.shape[1]
    out = np.full((s, hq, d), np.nan, np.float32)
    rp, nr, keep = _rows_arg(rows)
    if q.dtype == np.uint16:
        lib().or_flash_reference_bf16(np.ascontiguousarray(q).reshape(-1),
                                      np.ascontiguousarray(k).reshape(-1),
                                      np.ascontiguousarray(v).reshape(-1), out.reshape(-1),
                                      hq, hkv, d, s, rp, nr, nthreads)
    else:
        lib().or_flash_reference_f32(_c32(q).reshape(-1), _c32(k).reshape(-1),
                                     _c32(v).reshape(-1), out.reshape(-1),
                                     hq, hkv, d, s, rp, nr, nthreads)
    del keep
    return out


def decode_qk_scores(q, k, init_score, pos, max_seq_len):
    hq, d = q.shape
    hkv = k.shape[1]
    sc = _c32(init_score).copy().reshape(-1)
    lib().or_decode_qk_scores(_c32(q).reshape(-1), _c32(k).reshape(-1), sc, hq, hkv, d, pos,
                              max_seq_len)
    return sc.reshape(hq, max_seq_len)


def decode_softmax(score, pos):
    hq, msl = score.shape
    sc = _c32(score).copy()
    lib().or_decode_softmax(sc.reshape(-1), hq, pos, msl)
    return sc


def decode_apply(score, v, init_o, pos):
    hq, msl = score.shape
    hkv, d = v.shape[1], v.shape[2]
    o = _c32(init_o).copy()
    lib().or_decode_apply(_c32(score).reshape(-1), _c32(v).reshape(-1), o.reshape(-1), hq, hkv,
                          d, pos, msl)
    return o


def decode_attention(q, k, v, pos, max_seq_len):
    """Single-sequence decode reference -> (score [Hq][MSL], o_buffer [Hq][D] f32,
    o [Hq][D] bf16 bits).  q/k/v float32, already bf16-valued."""
    hq, d = q.shape
    hkv = k.shape[1]
    score = np.empty((hq, max_seq_len), np.float32)
    ob = np.empty((hq, d), np.float32)
    o = np.empty((hq, d), np.uint16)
    lib().or_decode_attention_f32(_c32(q).reshape(-1), _c32(k).reshape(-1), _c32(v).reshape(-1),
                                  score.reshape(-1), ob.reshape(-1),
                                  o.ctypes.data_as(_vp), hq, hkv, d, pos, max_seq_len)
    return score, ob, o


def decode_batched(q, k, v, lens, nthreads: int = 0):
    """Batched decode on bf16 bits: q [B][Hq][D], k/v [B][Lcap][Hkv][D]
    -> o_buffer float32 [B][Hq][D]."""
    b, hq, d = q.shape
    hkv = k.shape[2]
    stride = k.shape[1] * hkv * d
    lens_a = np.ascontiguousarray(lens, dtype=np.uint32)
    out = np.empty((b, hq, d), np.float32)
    lib().or_decode_batched_bf16(np.ascontiguousarray(q).reshape(-1),
                                 np.ascontiguousarray(k).reshape(-1),
                                 np.ascontiguousarray(v).reshape(-1), out.reshape(-1),
                                 b, hq, hkv, d, lens_a.ctypes.data_as(_vp), stride, nthreads)
    return out


def multi_rmsnorm(x, w, d, eps):
    """Per-head RMSNorm of x (float, rows of D) -> float holding bf16 values."""
    x = _c32(x)
    out = np.empty_like(x)
    rows = x.size // d
    lib().or_multi_rmsnorm(x.reshape(-1), _c32(w), out.reshape(-1), rows, d, eps)
    return out


def rope(qk, inv_freq, num_tokens, num_heads, d, pos0=0):
    out = _c32(qk).copy()
    lib().or_rope(out.reshape(-1), _c32(inv_freq), num_tokens, num_heads, d, pos0)
    return out


def inv_freq(d, theta):
    out = np.empty(d // 2, np.float32)
    lib().or_inv_freq(out, d, theta)
    return out


def qk_norm_rope(x, gamma, inv_freq_arr, eps):
    """x float [T][H][D] -> norm -> bf16 -> RoPE(pos = token) -> bf16."""
    t, h, d = x.shape
    out = _c32(x).copy()
    lib().or_qk_norm_rope(out.reshape(-1), _c32(gamma), _c32(inv_freq_arr), t, h, d, eps)
    return out


# ----------------------------------------------------------- projections

def make_gemv_case(M, N, x_phase, w_phase):
    """tests/gemv_test_common.h:24-50 -> (x [N], w [M][N]) float."""
    x = np.empty(N, np.float32)
    w = np.empty((M, N), np.float32)
    lib().or_make_gemv_case(M, N, x_phase, w_phase, x, w.reshape(-1))
    return x, w


def make_batch_gemv_case(batch, M, N, hidden_phase, w_phase):
    """tests/test_batch_gemv_proj_bf16.cu:20-50 -> (hidden [B][N], w [M][N])."""
    x = np.empty((batch, N), np.float32)
    w = np.empty((M, N), np.float32)
    lib().or_make_batch_gemv_case(batch, M, N, hidden_phase, w_phase, x.reshape(-1),
                                  w.reshape(-1))
    return x, w


def gemv(w, x, nthreads: int = 0):
    """y[t][m] = sum_n w[m][n] x[t][n] in float, in n order; x [N] or [T][N]."""
    w = _c32(w)
    x = _c32(x)
    M, N = w.shape
    tokens = x.size // N
    y = np.empty(tokens * M, np.float32)
    lib().or_gemv(w.reshape(-1), x.reshape(-1), y, tokens, M, N, nthreads)
    return y.reshape(x.shape[:-1] + (M,)) if x.ndim > 1 else y


# ------------------------------------------------- rest of a decoder layer

def make_rmsnorm_row_case(size, buffer_size, input_phase, weight_phase):
    """tests/rmsnorm_test_common.h:24-42 -> (input, weight), buffer_size each."""
    x = np.empty(buffer_size, np.float32)
    w = np.empty(buffer_size, np.float32)
    lib().or_make_rmsnorm_row_case(size, buffer_size, input_phase, weight_phase, x, w)
    return x, w


def make_batch_row_rmsnorm_case(batch, size, input_phase, weight_phase):
    """tests/test_batch_rmsnorm_bf16.cu:20-46 -> (input [B][size], weight [size])."""
    x = np.empty((batch, size), np.float32)
    w = np.empty(size, np.float32)
    lib().or_make_batch_row_rmsnorm_case(batch, size, input_phase, weight_phase, x.reshape(-1),
                                         w)
    return x, w


def make_swiglu_case(size, buffer_size, gate_phase, up_phase):
    g = np.empty(buffer_size, np.float32)
    u = np.empty(buffer_size, np.float32)
    lib().or_make_swiglu_case(size, buffer_size, gate_phase, up_phase, g, u)
    return g, u


def make_add_case(size, buffer_size, residual_phase, hidden_phase, tail_bias):
    r = np.empty(buffer_size, np.float32)
    h = np.empty(buffer_size, np.float32)
    lib().or_make_add_case(size, buffer_size, residual_phase, hidden_phase, tail_bias, r, h)
    return r, h


def rmsnorm_rows(x, w, eps):
    """Full-row RMSNorm of every row of x ([..., size]); bf16-valued float32."""
    x = _c32(x)
    size = x.shape[-1]
    out = np.empty_like(x)
    lib().or_multi_rmsnorm(x.reshape(-1), _c32(w), out.reshape(-1), x.size // size, size, eps)
    return out


def residual_add(hidden, residual):
    h, r = _c32(hidden), _c32(residual)
    out = np.empty_like(h)
    lib().or_residual_add(h.reshape(-1), r.reshape(-1), out.reshape(-1), h.size)
    return out


def swiglu(gate, up):
    g, u = _c32(gate), _c32(up)
    out = np.empty_like(g)
    lib().or_swiglu(g.reshape(-1), u.reshape(-1), out.reshape(-1), g.size)
    return out


def argmax(logits):
    x = _c32(logits).reshape(-1)
    return int(lib().or_argmax(x, x.size))


def sample_topk_topp(logits, temperature, top_k, top_p, u):
    """src/sampler.cpp:18-67 with the uniform draw u given: (token, order,
    probs, kept) where order/probs are the sorted top-k ids and probabilities
    (empty on the greedy path) and kept is the top-p prefix length."""
    x = _c32(logits).reshape(-1)
    greedy = abs(temperature) < 1e-3 or top_k == 1
    k = 0 if greedy else min(top_k, x.size)
    order = np.zeros(max(k, 1), np.uint32)
    probs = np.zeros(max(k, 1), np.float32)
    kept = np.zeros(1, np.uint32)
    tok = lib().or_sample_topk_topp(x, x.size, temperature, top_k, top_p, u, order, probs, kept)
    return int(tok), order[:k], probs[:k], int(kept[0])


def sample_coin(seed, pos):
    """The harness's per-position uniform draw (SplitMix64 output function)."""
    return float(lib().or_sample_coin(seed, pos))


# ------------------------------------------------------------ Qwen3 forward

class Qwen3Reference:
    """The reference's Qwen3 forward (src/transformer.cpp:320-470 prefill,
    :483-628 decode body, :625-630 final norm + lm-head) composed from the
    restated kernels above, with the same rounding points: every projection,
    norm, RoPE, attention, residual add and SwiGLU output rounded to bf16;
    logits fp32.  Weights are float32 arrays holding bf16 values (dict as in
    toyinfer_amd.qwen3, plus "inv_freq").  Caches [layers][max_seq_len][Hkv][D]."""

    def __init__(self, cfg: dict, weights: dict, nthreads: int = 0):
        self.cfg = cfg
        self.w = weights
        # OpenMP threads of the projections and the prefill attention (0: this
        # process's CPUs, at most 16); the results do not depend on it.
        self.nt = nthreads if nthreads > 0 else max(1, min(16, len(os.sched_getaffinity(0))))
        L, msl = cfg["num_layers"], cfg["max_seq_len"]
        shape = (L, msl, cfg["num_kv_heads"], cfg["head_dim"])
        self.kc = np.zeros(shape, np.float32)
        self.vc = np.zeros(shape, np.float32)

    def _layer(self, l, x, pos0):
        c, W = self.cfg, self.w["layers"][l]
        T = x.shape[0]
        hq, hkv, d, eps = c["num_q_heads"], c["num_kv_heads"], c["head_dim"], c["rms_norm_eps"]
        xn = rmsnorm_rows(x, W["input_layernorm"], eps)
        q = round_bf16(gemv(W["q_proj"], xn, self.nt))
        k = round_bf16(gemv(W["k_proj"], xn, self.nt))
        v = round_bf16(gemv(W["v_proj"], xn, self.nt))
        q = rope(multi_rmsnorm(q, W["q_norm"], d, eps), self.w["inv_freq"], T, hq, d, pos0)
        k = rope(multi_rmsnorm(k, W["k_norm"], d, eps), self.w["inv_freq"], T, hkv, d, pos0)
        self.kc[l, pos0:pos0 + T] = k.reshape(T, hkv, d)
        self.vc[l, pos0:pos0 + T] = v.reshape(T, hkv, d)
        if T > 1:
            assert pos0 == 0
            o = round_bf16(flash_reference(q.reshape(T, hq, d), k.reshape(T, hkv, d),
                                           v.reshape(T, hkv, d), nthreads=self.nt))
        else:
            _, _, ob = decode_attention(q.reshape(hq, d), self.kc[l], self.vc[l], pos0,
                                        c["max_seq_len"])
            o = bf16_to_f32(ob)
        a = round_bf16(gemv(W["o_proj"], o.reshape(T, hq * d), self.nt))
        x = residual_add(x, a)
        xn = rmsnorm_rows(x, W["post_attention_layernorm"], eps)
        g = round_bf16(gemv(W["gate_proj"], xn, self.nt))
        u = round_bf16(gemv(W["up_proj"], xn, self.nt))
        dn = round_bf16(gemv(W["down_proj"], swiglu(g, u), self.nt))
        return residual_add(x, dn)

    def _logits(self, x_last):
        xn = rmsnorm_rows(x_last[None, :], self.w["norm"], self.cfg["rms_norm_eps"])
        return gemv(self.w["lm_head"], xn, self.nt)[0]

    def forward(self, token_ids, pos0):
        """Tokens at positions pos0.. (a prompt from 0, or one decode token)
        -> fp32 logits of the last one."""
        x = self.w["embed_tokens"][np.asarray(token_ids, np.int64)]
        for l in range(self.cfg["num_layers"]):
            x = self._layer(l, x, pos0)
        return self._logits(x[-1])

