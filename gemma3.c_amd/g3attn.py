"""ctypes binding of libg3attn.so, the MI355X attention path of gemma3.c.

Mirrors include/g3attn.h one to one, so Python tests and the benchmark call
the same C-ABI a C caller (the reference transformer built with -DUSE_HIP)
would.  Host-pointer entry points take numpy arrays; ``*_device`` entry
points take raw device addresses (ints), e.g. ``torch_tensor.data_ptr()``.

The library is loaded from ``gemma3.c_amd/lib/libg3attn.so`` (built in tree
by ``__graft_entry__.build()``); a missing library raises, there is no CPU
fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("G3ATTN_LIB") or os.path.join(HERE, "lib", "libg3attn.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "g3attn.h")

# gemma3_error (gemma3.h:57-67) codes returned by the entry points
OK = 0
ERR_INVALID_ARG = -1
ERR_OUT_OF_MEMORY = -4
ERR_CONTEXT_OVERFLOW = -8

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_vp = C.c_void_p


class Config(C.Structure):
    """g3attn_config == gemma3_config (gemma3.h:82-95), field for field."""
    _fields_ = [
        ("vocab_size", C.c_int), ("hidden_size", C.c_int), ("intermediate_size", C.c_int),
        ("num_layers", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int), ("max_context", C.c_int), ("sliding_window", C.c_int),
        ("rmsnorm_eps", C.c_float), ("rope_theta_local", C.c_float),
        ("rope_theta_global", C.c_float),
    ]


class G3AttnError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"rc={rc}: {msg}")
        self.rc = rc


_lib = None


def declared_functions() -> list[str]:
    """Names of the functions declared in include/g3attn.h."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(g3attn_\w+)\s*\(", text)))


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libg3attn.so not built: {LIB_PATH} (run __graft_entry__.build())")
    L = C.CDLL(LIB_PATH)
    L.g3attn_default_config.argtypes = [C.POINTER(Config)]
    L.g3attn_is_global_layer.argtypes = [C.c_int]
    L.g3attn_is_global_layer.restype = C.c_int
    L.g3attn_rope_precompute.argtypes = [_f32p, C.c_int, C.c_int, C.c_float]
    L.g3attn_create.argtypes = [C.POINTER(Config), C.c_int, C.c_void_p, C.c_void_p]
    L.g3attn_create.restype = _vp
    L.g3attn_destroy.argtypes = [_vp]
    L.g3attn_reset.argtypes = [_vp]
    L.g3attn_decode.argtypes = [_vp, C.c_int, C.c_int, _f32p, _f32p, _f32p, _vp, _vp, _f32p]
    L.g3attn_prefill.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _f32p, _f32p, _f32p, _vp, _vp,
                                 _f32p]
    L.g3attn_decode_device.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp, _vp]
    L.g3attn_prefill_device.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp,
                                        _vp]
    L.g3attn_kv_append.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _f32p, _f32p, _vp]
    L.g3attn_kv_append_device.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp, _vp]
    L.g3attn_kv_write.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
    L.g3attn_kv_read.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _f32p, _f32p]
    L.g3attn_gqa.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                             C.c_float, _vp, _vp]
    L.g3attn_gqa.restype = None
    L.g3attn_gqa_noalloc.argtypes = [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int,
                                     C.c_float, _vp, _vp]
    L.g3attn_stream.argtypes = [_vp]
    L.g3attn_stream.restype = _vp
    L.g3attn_synchronize.argtypes = [_vp]
    L.g3attn_last_error.restype = C.c_char_p
    L.g3attn_profile_enable.argtypes = [_vp, C.c_int]
    L.g3attn_profile_read.argtypes = [_vp, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_int)]
    L.g3attn_last_splits.argtypes = [_vp, C.c_int, C.POINTER(C.c_int)]
    L.g3attn_matvec_bf16.argtypes = [_f32p, _vp, _f32p, C.c_int, C.c_int, _vp]
    L.g3attn_matvec_bf16.restype = None
    L.g3attn_matvec_bf16_device.argtypes = [_vp, _vp, _vp, _vp, C.c_int, C.c_int]
    L.g3attn_qkv_proj_device.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
    L.g3attn_layer_attention_device.argtypes = [_vp, C.c_int, C.c_int, _vp, _vp, _vp, _vp, _vp,
                                                _vp, _vp, _vp]
    L.g3attn_forward_device.argtypes = [_vp, C.c_void_p, C.c_int, C.c_int, _vp, C.c_int, _vp]
    L.g3attn_upload_weights.argtypes = [_vp, C.c_void_p]
    L.g3attn_upload_rope.argtypes = [_vp, _f32p, _f32p, C.c_int, C.c_int]
    L.g3attn_device_weights.argtypes = [_vp]
    L.g3attn_device_weights.restype = C.c_void_p
    L.g3attn_forward_token.argtypes = [_vp, C.c_int, C.c_int, C.c_void_p, C.c_int]
    L.g3attn_prefill_tokens.argtypes = [_vp, _i32p, C.c_int, C.c_int, C.c_void_p]
    L.g3attn_matmul_bf16_device.argtypes = [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int]
    L.g3attn_forward_token_device.argtypes = [_vp, C.c_int, C.c_int, _vp]
    L.g3attn_prefill_forward_device.argtypes = [_vp, C.c_void_p, _i32p, C.c_int, C.c_int, _vp]
    for name in ("g3attn_decode", "g3attn_prefill", "g3attn_decode_device",
                 "g3attn_prefill_device", "g3attn_kv_append", "g3attn_kv_append_device",
                 "g3attn_kv_write", "g3attn_kv_read", "g3attn_synchronize",
                 "g3attn_profile_enable", "g3attn_profile_read", "g3attn_matvec_bf16_device",
                 "g3attn_qkv_proj_device", "g3attn_layer_attention_device",
                 "g3attn_forward_device", "g3attn_upload_weights", "g3attn_forward_token",
                 "g3attn_prefill_tokens", "g3attn_matmul_bf16_device",
                 "g3attn_prefill_forward_device", "g3attn_forward_token_device",
                 "g3attn_gqa_noalloc", "g3attn_upload_rope", "g3attn_last_splits"):
        getattr(L, name).restype = C.c_int
    _lib = L
    return L


def last_error() -> str:
    return lib().g3attn_last_error().decode()


def default_config(**overrides) -> Config:
    c = Config()
    lib().g3attn_default_config(C.byref(c))
    for k, v in overrides.items():
        setattr(c, k, v)
    return c


def is_global_layer(layer: int) -> bool:
    return bool(lib().g3attn_is_global_layer(layer))


def rope_precompute(max_pos: int, theta: float, head_dim: int = 256) -> np.ndarray:
    t = np.empty(max_pos * head_dim, dtype=np.float32)
    lib().g3attn_rope_precompute(t, max_pos, head_dim, theta)
    return t


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def _check(rc: int):
    if rc != OK:
        raise G3AttnError(rc, last_error())


def gqa(q, k_cache, v_cache, n_heads, n_kv_heads, seq_len, head_dim=256, scale=0.0625,
        mask=None) -> np.ndarray:
    """gemma3_gqa-shaped call (gemma3_kernels.h:188-191) on the GPU."""
    out = np.full(n_heads * head_dim, np.nan, dtype=np.float32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32)
    lib().g3attn_gqa(out, np.ascontiguousarray(q, dtype=np.float32),
                     np.ascontiguousarray(k_cache, dtype=np.float32),
                     np.ascontiguousarray(v_cache, dtype=np.float32), n_heads, n_kv_heads,
                     seq_len, head_dim, scale, _p(m), None)
    err = last_error()
    if err:
        raise G3AttnError(ERR_INVALID_ARG, err)
    return out


NOALLOC_MAX_HEADS = 16   # G3ATTN_NOALLOC_MAX_HEADS


def gqa_noalloc(out_ptr, q_ptr, k_ptr, v_ptr, n_heads, n_kv_heads, seq_len, head_dim=256,
                scale=0.0625, mask_ptr=None, stream=None) -> None:
    """g3attn_gqa_noalloc on device addresses (ints); enqueues and returns."""
    _check(lib().g3attn_gqa_noalloc(out_ptr, q_ptr, k_ptr, v_ptr, n_heads, n_kv_heads, seq_len,
                                    head_dim, scale, mask_ptr, stream))


def matvec_bf16(A, x) -> np.ndarray:
    """gemma3_matvec_bf16-shaped call (gemma3_kernels.h:217-218) on the GPU:
    A [M][K] bf16 bit patterns (uint16), x [K] fp32 -> y [M] fp32."""
    A = np.ascontiguousarray(A, dtype=np.uint16)
    M, K = A.shape
    y = np.full(M, np.nan, dtype=np.float32)
    lib().g3attn_matvec_bf16(y, A.ctypes.data_as(_vp), np.ascontiguousarray(x, dtype=np.float32),
                             M, K, None)
    err = last_error()
    if err:
        raise G3AttnError(ERR_INVALID_ARG, err)
    return y


class LayerWeights(C.Structure):
    """g3attn_layer_weights: device addresses of one layer's bf16 tensors."""
    _fields_ = [(n, C.c_void_p) for n in (
        "input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
        "post_attention_layernorm", "gate_proj", "up_proj", "down_proj",
        "pre_feedforward_layernorm", "post_feedforward_layernorm")]


MAX_LAYERS = 34


class Weights(C.Structure):
    """g3attn_weights (the layout of the reference's gemma3_weights_t)."""
    _fields_ = [("embed_tokens", C.c_void_p), ("layers", LayerWeights * MAX_LAYERS),
                ("norm", C.c_void_p)]


LAYER_TENSORS = tuple(n for n, _ in LayerWeights._fields_)


def host_weights(embed: np.ndarray, layers, norm: np.ndarray):
    """A Weights of host addresses for upload_weights: ``layers`` is a list of
    dicts keyed by LAYER_TENSORS (uint16 bf16 arrays, None where absent).
    Returns (weights, arrays) - keep ``arrays`` alive until the upload returns."""
    keep = []

    def ptr(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=np.uint16)
        keep.append(a)
        return a.ctypes.data
    W = Weights()
    W.embed_tokens, W.norm = ptr(embed), ptr(norm)
    for l, lw in enumerate(layers):
        for name in LAYER_TENSORS:
            setattr(W.layers[l], name, ptr(lw.get(name)))
    return W, keep


class Context:
    """A device context: the per-layer KV cache, RoPE tables and stream."""

    def __init__(self, cfg: Config | None = None, max_context: int | None = None,
                 rope_local: np.ndarray | None = None, rope_global: np.ndarray | None = None,
                 defer_rope: bool = False):
        """Tables default to g3attn_rope_precompute's; defer_rope creates the
        context without tables (NULL), for a later upload_rope."""
        self.cfg = cfg if cfg is not None else default_config()
        self.max_context = int(max_context if max_context is not None else self.cfg.max_context)
        if defer_rope:
            rope_local = rope_global = None
        else:
            if rope_local is None:
                rope_local = rope_precompute(self.max_context, self.cfg.rope_theta_local)
            if rope_global is None:
                rope_global = rope_precompute(self.max_context, self.cfg.rope_theta_global)
            rope_local = np.ascontiguousarray(rope_local, dtype=np.float32)
            rope_global = np.ascontiguousarray(rope_global, dtype=np.float32)
        self.rope_local, self.rope_global = rope_local, rope_global
        self._h = lib().g3attn_create(C.byref(self.cfg), self.max_context,
                                      None if rope_local is None else rope_local.ctypes.data,
                                      None if rope_global is None else rope_global.ctypes.data)
        if not self._h:
            raise G3AttnError(ERR_INVALID_ARG, last_error())

    def upload_rope(self, rope_local: np.ndarray, rope_global: np.ndarray, max_context: int | None = None,
                    head_dim: int = 256):
        """g3attn_upload_rope (gemma3_metal_upload_rope): replace both tables."""
        n = self.max_context if max_context is None else int(max_context)
        _check(lib().g3attn_upload_rope(self._h, np.ascontiguousarray(rope_local, dtype=np.float32),
                                        np.ascontiguousarray(rope_global, dtype=np.float32), n, head_dim))

    @property
    def handle(self):
        return self._h

    def close(self):
        if self._h:
            lib().g3attn_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def qs(self):
        return self.cfg.num_heads * self.cfg.head_dim

    @property
    def ks(self):
        return self.cfg.num_kv_heads * self.cfg.head_dim

    def rows(self, layer: int) -> int:
        return self.max_context if is_global_layer(layer) else self.cfg.sliding_window

    def reset(self):
        lib().g3attn_reset(self._h)

    def stream(self) -> int:
        return lib().g3attn_stream(self._h) or 0

    def synchronize(self):
        _check(lib().g3attn_synchronize(self._h))

    def profile(self, enable: bool = True):
        """Bracket the main attention kernel of every call with HIP events."""
        _check(lib().g3attn_profile_enable(self._h, int(enable)))

    def profile_read(self, kind: int):
        """(summed ms, launches) of kind 0 (decode kernel) or 1 (prefill kernel) since the
        last read."""
        ms, n = C.c_double(), C.c_int()
        _check(lib().g3attn_profile_read(self._h, kind, C.byref(ms), C.byref(n)))
        return ms.value, n.value

    def last_splits(self, kind: int) -> int:
        """Key splits the last call of kind 0 (decode) or 1 (prefill) chose;
        kind 2: query heads per workgroup of the last decode's one-launch
        form (0: decode + combine launches, or one split)."""
        n = C.c_int()
        _check(lib().g3attn_last_splits(self._h, kind, C.byref(n)))
        return n.value

    def decode(self, layer, pos, q, k, v, q_norm=None, k_norm=None) -> np.ndarray:
        out = np.empty(self.qs, dtype=np.float32)
        _check(lib().g3attn_decode(self._h, layer, pos, np.ascontiguousarray(q, np.float32),
                                   np.ascontiguousarray(k, np.float32),
                                   np.ascontiguousarray(v, np.float32), _p(q_norm), _p(k_norm),
                                   out))
        return out

    def decode_rc(self, layer, pos, q, k, v, q_norm=None, k_norm=None) -> int:
        out = np.empty(self.qs, dtype=np.float32)
        return lib().g3attn_decode(self._h, layer, pos, np.ascontiguousarray(q, np.float32),
                                   np.ascontiguousarray(k, np.float32),
                                   np.ascontiguousarray(v, np.float32), _p(q_norm), _p(k_norm),
                                   out)

    def prefill(self, layer, start_pos, Q, K, V, q_norm=None, k_norm=None) -> np.ndarray:
        Q = np.ascontiguousarray(Q, np.float32)
        n = Q.shape[0]
        out = np.empty((n, self.qs), dtype=np.float32)
        _check(lib().g3attn_prefill(self._h, layer, start_pos, n, Q,
                                    np.ascontiguousarray(K, np.float32),
                                    np.ascontiguousarray(V, np.float32), _p(q_norm), _p(k_norm),
                                    out))
        return out

    def decode_device(self, layer, pos, q, k, v, q_norm, k_norm, out):
        _check(lib().g3attn_decode_device(self._h, layer, pos, q, k, v, q_norm, k_norm, out))

    def prefill_device(self, layer, start_pos, n, Q, K, V, q_norm, k_norm, out):
        _check(lib().g3attn_prefill_device(self._h, layer, start_pos, n, Q, K, V, q_norm, k_norm,
                                           out))

    def matvec_bf16_device(self, y, A, x, M, K):
        _check(lib().g3attn_matvec_bf16_device(self._h, y, A, x, M, K))

    def qkv_proj_device(self, x, wq, wk, wv, q, k, v):
        _check(lib().g3attn_qkv_proj_device(self._h, x, wq, wk, wv, q, k, v))

    def forward_device(self, weights: "Weights", token, pos, logits, compute_logits=True,
                       hidden_out=None):
        _check(lib().g3attn_forward_device(self._h, C.byref(weights), token, pos, logits,
                                           int(compute_logits), hidden_out))

    def upload_weights(self, weights: "Weights"):
        """weights: a Weights of HOST addresses (the gemma3_weights_t the
        safetensors loader fills); see host_weights()."""
        _check(lib().g3attn_upload_weights(self._h, C.byref(weights)))

    def device_weights(self) -> "Weights | None":
        p = lib().g3attn_device_weights(self._h)
        return None if not p else Weights.from_address(p)

    def forward_token(self, token, pos, compute_logits=True) -> np.ndarray | None:
        """gemma3_metal_forward_token: logits [vocab] on the host, or None."""
        out = np.empty(self.cfg.vocab_size, np.float32) if compute_logits else None
        _check(lib().g3attn_forward_token(self._h, int(token), int(pos),
                                          None if out is None else out.ctypes.data,
                                          int(compute_logits)))
        return out

    def forward_token_device(self, token, pos, logits=None):
        """The uploaded model's token forward, enqueued; logits: device address or None."""
        _check(lib().g3attn_forward_token_device(self._h, int(token), int(pos), logits))

    def prefill_tokens(self, tokens, start_pos=0, logits=True) -> np.ndarray | None:
        """gemma3_metal_prefill: the last token's logits, or None."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.cfg.vocab_size, np.float32) if logits else None
        _check(lib().g3attn_prefill_tokens(self._h, tokens, tokens.size, int(start_pos),
                                           None if out is None else out.ctypes.data))
        return out

    def matmul_bf16_device(self, C, W, X, N, M, K):
        """C [N][M] = X [N][K] . W [M][K]^T (device pointers)."""
        _check(lib().g3attn_matmul_bf16_device(self._h, C, W, X, N, M, K))

    def prefill_forward_device(self, weights: "Weights", tokens, start_pos=0, logits=None):
        """The batched prefill of host tokens on device weights; logits: a
        device address or None."""
        tokens = np.ascontiguousarray(tokens, np.int32)
        _check(lib().g3attn_prefill_forward_device(self._h, C.byref(weights), tokens, tokens.size,
                                                   int(start_pos), logits))

    def layer_attention_device(self, layer, pos, x, wq, wk, wv, wo, q_norm, k_norm, out):
        _check(lib().g3attn_layer_attention_device(self._h, layer, pos, x, wq, wk, wv, wo, q_norm,
                                                   k_norm, out))

    def kv_append(self, layer, start_pos, K, V, k_norm=None):
        K = np.ascontiguousarray(K, np.float32)
        _check(lib().g3attn_kv_append(self._h, layer, start_pos, K.shape[0], K,
                                      np.ascontiguousarray(V, np.float32), _p(k_norm)))

    def kv_append_device(self, layer, start_pos, n, K, V, k_norm):
        _check(lib().g3attn_kv_append_device(self._h, layer, start_pos, n, K, V, k_norm))

    def kv_write(self, layer, slot, k_rows, v_rows):
        k_rows = np.ascontiguousarray(k_rows, np.float32).reshape(-1, self.ks)
        _check(lib().g3attn_kv_write(self._h, layer, slot, k_rows.shape[0], k_rows,
                                     np.ascontiguousarray(v_rows, np.float32).reshape(-1, self.ks)))

    def kv_read(self, layer, slot, n):
        k = np.empty((n, self.ks), dtype=np.float32)
        v = np.empty((n, self.ks), dtype=np.float32)
        _check(lib().g3attn_kv_read(self._h, layer, slot, n, k, v))
        return k, v
