"""Python binding of the byte-level BPE tokenizer (include/toyinfer_tokenizer.h):
the reference's toyinfer::Tokenizer (include/tokenizer.h:30-57) over the files
export.py writes.  Host code in libtoyinfer_attn.so; no GPU involved."""
import ctypes
from typing import List, Optional

from toyinfer_amd import attn

_vp, _u32, _sz, _i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_int
_SIGS = {
    "toyinfer_tokenizer_create": (_i32, [ctypes.c_char_p, _u32, _i32, ctypes.POINTER(_vp)]),
    "toyinfer_tokenizer_destroy": (None, [_vp]),
    "toyinfer_tokenizer_encode": (_i32, [_vp, ctypes.c_char_p, ctypes.POINTER(_u32), _u32,
                                         ctypes.POINTER(_u32)]),
    "toyinfer_tokenizer_decode": (ctypes.POINTER(ctypes.c_char), [_vp, _u32, ctypes.POINTER(_u32)]),
    "toyinfer_tokenizer_render_prompt": (_i32, [_vp, ctypes.c_char_p, ctypes.c_char_p,
                                                ctypes.c_char_p, _sz, ctypes.POINTER(_sz)]),
    "toyinfer_tokenizer_vocab_size": (_u32, [_vp]),
    "toyinfer_tokenizer_num_merges": (_u32, [_vp]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(attn.LIB, _name)
    _fn.restype, _fn.argtypes = _res, _args


def _bytes(s) -> bytes:
    return s.encode("utf-8") if isinstance(s, str) else bytes(s)


class Tokenizer:
    def __init__(self, model_dir: str, vocab_size: int, thinking: bool = False):
        self.h = _vp()
        attn._check("tokenizer_create", attn.LIB.toyinfer_tokenizer_create(
            _bytes(model_dir), vocab_size, int(thinking), ctypes.byref(self.h)))

    def close(self) -> None:
        if self.h:
            attn.LIB.toyinfer_tokenizer_destroy(self.h)
            self.h = _vp()

    def __del__(self):
        self.close()

    @property
    def vocab_size(self) -> int:
        return int(attn.LIB.toyinfer_tokenizer_vocab_size(self.h))

    @property
    def num_merges(self) -> int:
        return int(attn.LIB.toyinfer_tokenizer_num_merges(self.h))

    def encode(self, text) -> List[int]:
        b = _bytes(text)
        cap = len(b)
        ids = (_u32 * max(cap, 1))()
        n = _u32()
        attn._check("tokenizer_encode", attn.LIB.toyinfer_tokenizer_encode(
            self.h, b, ids, cap, ctypes.byref(n)))
        return list(ids[:n.value])

    def decode(self, token_id: int) -> Optional[bytes]:
        n = _u32()
        p = attn.LIB.toyinfer_tokenizer_decode(self.h, token_id, ctypes.byref(n))
        return ctypes.string_at(p, n.value) if p else None

    def render_prompt(self, user, system=None) -> bytes:
        u = _bytes(user)
        s = None if system is None else _bytes(system)
        need = _sz()
        st = attn.LIB.toyinfer_tokenizer_render_prompt(self.h, u, s, None, 0, ctypes.byref(need))
        if st != attn.ERR_WORKSPACE:
            attn._check("tokenizer_render_prompt", st)
        buf = ctypes.create_string_buffer(need.value + 1)
        attn._check("tokenizer_render_prompt", attn.LIB.toyinfer_tokenizer_render_prompt(
            self.h, u, s, buf, need.value + 1, ctypes.byref(need)))
        return buf.raw[:need.value]
