"""ctypes binding of the CPU checker libraries (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg import
this module.  It loads

* ``oracle/lib/libg3oracle.so`` - the C11 restatement of the reference path
  (g3_oracle.c; reference lines cited there), and
* ``oracle/_ref/libg3ref.so`` - the real reference sources compiled in place
  (ref_harness.c), present only where ``/root/reference`` was available at
  build time, and ``libg3ref_v4.so``, the same at -march=x86-64-v4 (AVX-512),
  which ``ref_timing()`` picks for bench.py's CPU baseline on hosts that run it.

Arrays are numpy float32 / uint16, C-contiguous; shapes follow the reference:
q [H_q*d], k/v [H_kv*d], caches [rows][H_kv][d].
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "lib", "libg3oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libg3ref.so")
REF_V4_SO = os.path.join(HERE, "_ref", "libg3ref_v4.so")
# x86-64-v4: AVX-512 F, BW, CD, DQ and VL on top of x86-64-v3
_V4_FLAGS = ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


class _Cfg(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int), ("max_context", C.c_int), ("sliding_window", C.c_int),
        ("rmsnorm_eps", C.c_float), ("rope_theta_local", C.c_float),
        ("rope_theta_global", C.c_float),
    ]


class _Model(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_int), ("hidden_size", C.c_int), ("intermediate_size", C.c_int),
        ("num_layers", C.c_int), ("num_heads", C.c_int), ("num_kv_heads", C.c_int),
        ("head_dim", C.c_int), ("max_context", C.c_int), ("sliding_window", C.c_int),
        ("rmsnorm_eps", C.c_float), ("rope_theta_local", C.c_float),
        ("rope_theta_global", C.c_float),
    ]


@dataclass
class Config:
    """gemma3_config subset (gemma3.h:82-95) read by the attention path."""
    num_layers: int = 34
    num_heads: int = 8
    num_kv_heads: int = 4
    head_dim: int = 256
    max_context: int = 8192
    sliding_window: int = 1024
    rmsnorm_eps: float = 1e-6
    rope_theta_local: float = 10000.0
    rope_theta_global: float = 1000000.0

    def c(self) -> _Cfg:
        return _Cfg(self.num_layers, self.num_heads, self.num_kv_heads, self.head_dim,
                    self.max_context, self.sliding_window, self.rmsnorm_eps,
                    self.rope_theta_local, self.rope_theta_global)

    def theta(self, layer: int) -> float:
        return self.rope_theta_global if is_global_layer(layer) else self.rope_theta_local

    def cache_rows(self, layer: int) -> int:
        return self.max_context if is_global_layer(layer) else self.sliding_window


def is_global_layer(layer: int) -> bool:
    """gemma3.h:347-350."""
    return (layer + 1) % 6 == 0


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle library missing: {ORACLE_SO} (run __graft_entry__.build())")
        L = C.CDLL(ORACLE_SO)
        L.g3o_rope_precompute.argtypes = [_f32p, C.c_int, C.c_int, C.c_float]
        L.g3o_rope_apply.argtypes = [_f32p, _f32p, C.c_int, C.c_int]
        L.g3o_rmsnorm_bf16.argtypes = [_f32p, _f32p, _u16p, C.c_int, C.c_float]
        L.g3o_softmax.argtypes = [_f32p, C.c_int]
        L.g3o_causal_mask.argtypes = [_f32p, C.c_int, C.c_int]
        L.g3o_gqa.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                              C.c_float, C.c_void_p, C.c_void_p]
        L.g3o_gqa_rows.argtypes = [_f32p, _f32p, _f32p, _f32p, _i32p, C.c_int, C.c_int, C.c_int,
                                   C.c_int, C.c_float, C.c_void_p, C.c_void_p]
        L.g3o_cache_kv.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.g3o_layer_decode.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_void_p, C.c_void_p,
                                       _f32p, _f32p, _f32p, C.POINTER(_Cfg), C.c_int, C.c_int,
                                       _f32p]
        L.g3o_layer_decode.restype = C.c_int
        L.g3o_prefill.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_void_p, C.c_void_p, _f32p, _f32p,
                                  _f32p, C.POINTER(_Cfg), C.c_int, C.c_int, C.c_int, _f32p]
        L.g3o_prefill.restype = C.c_int
        L.g3o_prefill_mt.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_void_p, C.c_void_p, _f32p,
                                     _f32p, _f32p, C.POINTER(_Cfg), C.c_int, C.c_int, C.c_int,
                                     C.c_int]
        L.g3o_prefill_mt.restype = C.c_int
        L.g3o_prefill_rows.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_void_p, C.c_void_p, _f32p,
                                       _f32p, _f32p, C.POINTER(_Cfg), C.c_int, C.c_int, C.c_int,
                                       _i32p, C.c_int, C.c_int]
        L.g3o_prefill_rows.restype = C.c_int
        L.g3o_norm_rope_batch.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_void_p, _f32p,
                                          C.c_int, C.c_float, C.c_int]
        L.g3o_gen_normal_bf16.argtypes = [_f32p, C.c_size_t, C.c_uint64, C.c_size_t, C.c_int]
        L.g3o_matvec_bf16.argtypes = [_f32p, _u16p, _f32p, C.c_int, C.c_int]
        L.g3o_gelu_tanh.argtypes = [_f32p, C.c_int]
        L.g3o_forward_seq.argtypes = [_f32p, _f32p, _i32p, C.c_int, _u16p, C.c_void_p, _u16p,
                                      C.POINTER(_Model)]
        L.g3o_forward_seq.restype = C.c_int
        L.g3o_forward_cached.argtypes = [_f32p, C.c_int, C.c_void_p, _i32p, C.c_int, C.c_int, _u16p, C.c_void_p,
                                         _u16p, C.POINTER(_Model), C.c_void_p, C.c_void_p, C.c_int]
        L.g3o_forward_cached.restype = C.c_int
        L.g3o_splitmix64.argtypes = [C.c_uint64, C.c_uint64]
        L.g3o_splitmix64.restype = C.c_uint64
        L.g3o_fnv1a64.argtypes = [C.c_void_p, C.c_size_t]
        L.g3o_fnv1a64.restype = C.c_uint64
        L.g3o_bf16_to_f32.argtypes = [C.c_uint16]
        L.g3o_bf16_to_f32.restype = C.c_float
        L.g3o_f32_to_bf16_trunc.argtypes = [C.c_float]
        L.g3o_f32_to_bf16_trunc.restype = C.c_uint16
        L.g3o_f32_to_bf16_rne.argtypes = [C.c_float]
        L.g3o_f32_to_bf16_rne.restype = C.c_uint16
        _lib = L
    return _lib


def have_ref() -> bool:
    return os.path.exists(REF_SO)


def _host_has_v4() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return all(x in flags for x in _V4_FLAGS)
    except OSError:
        pass
    return False


def ref_timing_build() -> str:
    """Which reference build ref_timing() loads: "x86-64-v4" where this host
    runs AVX-512 and the build exists, else "x86-64-v3"."""
    return "x86-64-v4" if os.path.exists(REF_V4_SO) and _host_has_v4() else "x86-64-v3"


_ref_v4 = None


def ref_timing():
    """The reference build for timing on this host: the x86-64-v4 one (the
    vector width the reference's -march=native gives on an AVX-512 host)
    where it runs, else ref().  Parity checks use ref()."""
    global _ref_v4
    if ref_timing_build() == "x86-64-v3":
        return ref()
    if _ref_v4 is None:
        _ref_v4 = _bind_ref(C.CDLL(REF_V4_SO))
    return _ref_v4


def ref():
    """The real reference kernels (oracle/_ref); raises if not built here."""
    global _ref
    if _ref is None:
        if not have_ref():
            raise RuntimeError(f"reference harness not built: {REF_SO}")
        _ref = _bind_ref(C.CDLL(REF_SO))
    return _ref


def _bind_ref(R):
    """Declares the harness entry points on a loaded reference build."""
    R.ref_rope_precompute.argtypes = [_f32p, C.c_int, C.c_int, C.c_float]
    R.ref_rope_apply.argtypes = [_f32p, _f32p, C.c_int, C.c_int]
    R.ref_rmsnorm_bf16.argtypes = [_f32p, _f32p, _u16p, C.c_int, C.c_float]
    R.ref_softmax.argtypes = [_f32p, C.c_int]
    R.ref_causal_mask.argtypes = [_f32p, C.c_int, C.c_int]
    R.ref_gqa.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                          C.c_float, C.c_void_p, C.c_void_p]
    R.ref_layer_decode.argtypes = [_f32p, C.c_void_p, C.c_void_p, _f32p, _f32p, _f32p,
                                   C.c_void_p, C.c_void_p, _f32p, _f32p, _f32p, C.c_int,
                                   C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
    R.ref_layer_decode.restype = C.c_int
    R.ref_prefill_loop.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_void_p, C.c_void_p, _f32p,
                                   _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                   C.c_int, C.c_int]
    R.ref_prefill_loop.restype = C.c_int
    R.ref_time_decode.argtypes = [_f32p, _f32p, _f32p, C.c_void_p, C.c_void_p, _f32p, _f32p,
                                  _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                  C.c_int, C.c_int]
    R.ref_time_decode.restype = C.c_double
    R.ref_matvec_bf16.argtypes = [_f32p, _u16p, _f32p, C.c_int, C.c_int]
    R.ref_layer_attention.argtypes = [_f32p, _f32p, _u16p, _u16p, _u16p, _u16p, C.c_void_p,
                                      C.c_void_p, _f32p, _f32p, _f32p, C.c_int, C.c_int,
                                      C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
    R.ref_layer_attention.restype = C.c_int
    R.ref_forward_seq.argtypes = [_f32p, _f32p, _i32p, C.c_int, _u16p, C.c_void_p, _u16p,
                                  C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                  C.c_int, C.c_int]
    R.ref_forward_seq.restype = C.c_int
    R.ref_time_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                   C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]
    R.ref_time_forward.restype = C.c_double
    return R


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- generator

def gen_normal_bf16(n: int, seed: int, first: int = 0, threads: int = 0) -> np.ndarray:
    """Seeded N(0,1) values rounded to bf16 (stored as float32)."""
    out = np.empty(int(n), dtype=np.float32)
    lib().g3o_gen_normal_bf16(out, out.size, seed & (2**64 - 1), first, threads)
    return out


def seed_for(config: int, tensor: int, layer: int = 0) -> int:
    """Per-tensor seed: 0x5EED0000 + 16*config + tensor (+256*layer for the stack)."""
    return 0x5EED0000 + 16 * config + tensor + 256 * layer


def fnv1a64(a: np.ndarray) -> int:
    a = np.ascontiguousarray(a)
    return int(lib().g3o_fnv1a64(a.ctypes.data_as(C.c_void_p), a.nbytes))


def zero_norm(d: int = 256) -> np.ndarray:
    """bf16 weight 0 = unit gain under the (1 + w) RMSNorm."""
    return np.zeros(d, dtype=np.uint16)


# ---------------------------------------------------------------- restatement

def rope_table(max_pos: int, theta: float, d: int = 256, use_ref: bool = False) -> np.ndarray:
    t = np.empty(max_pos * d, dtype=np.float32)
    (ref().ref_rope_precompute if use_ref else lib().g3o_rope_precompute)(t, max_pos, d, theta)
    return t


def norm_rope_batch(X: np.ndarray, table: np.ndarray, start_pos: int, w=None, eps=1e-6,
                    threads: int = 0) -> np.ndarray:
    """In-place QK-norm + RoPE of X [n][heads][256] (token i at start_pos + i)."""
    assert X.dtype == np.float32 and X.flags.c_contiguous
    n, heads = X.shape[0], X.shape[1] if X.ndim == 3 else X.shape[1] // 256
    lib().g3o_norm_rope_batch(X.reshape(-1), n, heads, 256, _ptr(w), table, start_pos, eps, threads)
    return X


def rmsnorm_bf16(x: np.ndarray, w: np.ndarray, eps: float = 1e-6, use_ref=False) -> np.ndarray:
    y = np.empty_like(x)
    (ref().ref_rmsnorm_bf16 if use_ref else lib().g3o_rmsnorm_bf16)(y, np.ascontiguousarray(x), w, x.size, eps)
    return y


def rope_apply(x: np.ndarray, table: np.ndarray, pos: int, use_ref=False) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    (ref().ref_rope_apply if use_ref else lib().g3o_rope_apply)(y, table, y.size, pos)
    return y


def softmax(x: np.ndarray, use_ref=False) -> np.ndarray:
    y = np.array(x, dtype=np.float32, copy=True)
    (ref().ref_softmax if use_ref else lib().g3o_softmax)(y, y.size)
    return y


def gqa(q, k, v, n_heads, n_kv, seq_len, d=256, scale=0.0625, mask=None, use_ref=False):
    out = np.empty(n_heads * d, dtype=np.float32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32)
    f = ref().ref_gqa if use_ref else lib().g3o_gqa
    f(out, np.ascontiguousarray(q), np.ascontiguousarray(k), np.ascontiguousarray(v),
      n_heads, n_kv, seq_len, d, scale, _ptr(m), None)
    return out


def matvec_bf16(A: np.ndarray, x: np.ndarray, use_ref=False) -> np.ndarray:
    """gemma3_matvec_bf16 (gemma3_kernels.c:188-238): A [M][K] bf16 bits (uint16),
    x [K] fp32 -> y [M] fp32, in the reference AVX2 build's summation order."""
    A = np.ascontiguousarray(A, dtype=np.uint16)
    M, K = A.shape
    y = np.empty(M, dtype=np.float32)
    (ref().ref_matvec_bf16 if use_ref else lib().g3o_matvec_bf16)(
        y, A, np.ascontiguousarray(x, dtype=np.float32), M, K)
    return y


def layer_attention(cfg: Config, layer: int, pos: int, x, wq, wk, wv, wo, k_cache, v_cache,
                    table, q_norm=None, k_norm=None, use_ref=False):
    """The whole of layer_attention (gemma3_transformer.c:258-356) for one token:
    x [hidden] -> Q/K/V GEMVs -> attention section -> o_proj GEMV -> [hidden].
    The caches are updated in place."""
    hidden = x.size
    if use_ref:
        out = np.empty(hidden, dtype=np.float32)
        rc = ref().ref_layer_attention(out, np.ascontiguousarray(x, np.float32), wq, wk, wv, wo,
                                       _ptr(q_norm), _ptr(k_norm), k_cache, v_cache, table,
                                       cfg.num_heads, cfg.num_kv_heads, hidden, layer, pos,
                                       cfg.max_context, cfg.sliding_window)
        if rc:
            raise RuntimeError(f"ref_layer_attention rc={rc}")
        return out
    q, k, v = matvec_bf16(wq, x), matvec_bf16(wk, x), matvec_bf16(wv, x)
    attn, _, _ = layer_decode(cfg, layer, pos, q, k, v, k_cache, v_cache, table, q_norm, k_norm)
    return matvec_bf16(wo, attn)


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """gemma3_gelu_tanh_inplace (gemma3_kernels.c:348-357) on a copy of x."""
    y = np.array(x, dtype=np.float32, copy=True)
    lib().g3o_gelu_tanh(y, y.size)
    return y


# the 13 per-layer tensors in gemma3_weights_t order (gemma3.h)
LAYER_TENSORS = ("input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
                 "post_attention_layernorm", "gate_proj", "up_proj", "down_proj",
                 "pre_feedforward_layernorm", "post_feedforward_layernorm")


def forward_cached(cfg: Config, hidden: int, inter: int, tokens, pos0: int, embed: np.ndarray, layers,
                   norm: np.ndarray, kc=None, vc=None, n_logits: int = 1, threads: int = 1):
    """gemma3_transformer_forward for tokens at positions pos0.. on the given
    caches (lists of cfg.num_layers float32 arrays [rows][kv heads x 256],
    the reference layout, updated in place; None: empty caches).  Returns
    (logits of the last n_logits tokens [n_logits][vocab], hidden state
    after the last token).  The GEMVs split over `threads` threads (same
    bits for any count)."""
    tokens = np.ascontiguousarray(tokens, dtype=np.int32)
    vocab = embed.size // hidden
    ks = cfg.num_kv_heads * cfg.head_dim
    if kc is None:
        kc = [np.zeros((cfg.cache_rows(l), ks), np.float32) for l in range(cfg.num_layers)]
        vc = [np.zeros((cfg.cache_rows(l), ks), np.float32) for l in range(cfg.num_layers)]
    for l in range(cfg.num_layers):
        assert kc[l].dtype == np.float32 and kc[l].flags.c_contiguous and kc[l].shape == (cfg.cache_rows(l), ks)
        assert vc[l].dtype == np.float32 and vc[l].flags.c_contiguous and vc[l].shape == kc[l].shape
    keep = []
    ptrs = (C.c_void_p * (13 * cfg.num_layers))()
    for l, lw in enumerate(layers):
        for j, name in enumerate(LAYER_TENSORS):
            a = lw.get(name)
            if a is not None:
                a = np.ascontiguousarray(a, dtype=np.uint16)
                keep.append(a)
                ptrs[13 * l + j] = a.ctypes.data
    kp = (C.c_void_p * cfg.num_layers)(*[a.ctypes.data for a in kc])
    vp = (C.c_void_p * cfg.num_layers)(*[a.ctypes.data for a in vc])
    logits = np.empty((n_logits, vocab), dtype=np.float32)
    hid = np.empty(hidden, dtype=np.float32)
    m = _Model(vocab, hidden, inter, cfg.num_layers, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim,
               cfg.max_context, cfg.sliding_window, cfg.rmsnorm_eps, cfg.rope_theta_local, cfg.rope_theta_global)
    rc = lib().g3o_forward_cached(logits, n_logits, hid.ctypes.data, tokens, tokens.size, pos0,
                                  np.ascontiguousarray(embed, np.uint16), ptrs, np.ascontiguousarray(norm, np.uint16),
                                  C.byref(m), kp, vp, threads)
    if rc:
        raise RuntimeError(f"g3o_forward_cached -> {rc}")
    return logits, hid


GQA_ENGINE_SO = os.path.join(HERE, "_ref", "libg3gqa.so")
_gqa_engine = None


def gqa_engine():
    """The reference harness compiled with -Dgemma3_gqa=g3attn_gqa
    (oracle/_ref/libg3gqa.so): the engine's attention on the GPU through the
    drop-in.  Raises if not built here."""
    global _gqa_engine
    if _gqa_engine is None:
        if not os.path.exists(GQA_ENGINE_SO):
            raise RuntimeError(f"drop-in engine harness not built: {GQA_ENGINE_SO}")
        _gqa_engine = _bind_ref(C.CDLL(GQA_ENGINE_SO))
    return _gqa_engine


def forward_seq(cfg: Config, hidden: int, inter: int, tokens, embed: np.ndarray, layers,
                norm: np.ndarray, use_ref=False, ref_lib=None):
    """gemma3_transformer_forward (gemma3_transformer.c:396-512) for tokens at
    positions 0..n-1 from an empty cache.  ``layers`` is a list of
    cfg.num_layers dicts keyed by LAYER_TENSORS (bf16 uint16 arrays; the
    norms other than input_layernorm may be None).  ``embed`` is
    [vocab][hidden] bf16 (tied with the logits).  Returns (logits [n][vocab]
    fp32, hidden state after the last token [hidden])."""
    tokens = np.ascontiguousarray(tokens, dtype=np.int32)
    vocab = embed.size // hidden
    assert embed.size == vocab * hidden and len(layers) == cfg.num_layers
    keep = []
    ptrs = (C.c_void_p * (13 * cfg.num_layers))()
    for l, lw in enumerate(layers):
        for j, name in enumerate(LAYER_TENSORS):
            a = lw.get(name)
            if a is not None:
                a = np.ascontiguousarray(a, dtype=np.uint16)
                keep.append(a)
                ptrs[13 * l + j] = a.ctypes.data
    logits = np.empty((tokens.size, vocab), dtype=np.float32)
    hid = np.empty(hidden, dtype=np.float32)
    if use_ref or ref_lib is not None:
        rc = (ref_lib or ref()).ref_forward_seq(logits, hid, tokens, tokens.size, embed, ptrs, norm, vocab,
                                   hidden, inter, cfg.num_layers, cfg.num_heads, cfg.num_kv_heads,
                                   cfg.max_context, cfg.sliding_window)
    else:
        m = _Model(vocab, hidden, inter, cfg.num_layers, cfg.num_heads, cfg.num_kv_heads,
                   cfg.head_dim, cfg.max_context, cfg.sliding_window, cfg.rmsnorm_eps,
                   cfg.rope_theta_local, cfg.rope_theta_global)
        rc = lib().g3o_forward_seq(logits, hid, tokens, tokens.size, embed, ptrs, norm, C.byref(m))
    if rc:
        raise RuntimeError(f"forward_seq rc={rc}")
    return logits, hid


def layer_decode(cfg: Config, layer: int, pos: int, q, k, v, k_cache, v_cache, table,
                 q_norm=None, k_norm=None):
    """One decode step (gemma3_transformer.c:294-352).  Returns (attn_out, q_rot, k_rot);
    k_cache / v_cache are updated in place."""
    q = np.array(q, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    out = np.empty(cfg.num_heads * cfg.head_dim, dtype=np.float32)
    cap = max(cfg.max_context, cfg.sliding_window)
    work = np.empty(2 * cap, dtype=np.float32)
    c = cfg.c()
    rc = lib().g3o_layer_decode(out, q, k, np.ascontiguousarray(v, dtype=np.float32),
                                _ptr(q_norm), _ptr(k_norm), k_cache, v_cache, table,
                                C.byref(c), layer, pos, work)
    if rc:
        raise RuntimeError(f"g3o_layer_decode rc={rc}")
    return out, q, k


def prefill(cfg: Config, layer: int, start_pos: int, Q, K, V, k_cache, v_cache, table,
            q_norm=None, k_norm=None, threads: int = 1):
    """Prefill attention loop (gemma3_transformer.c:641-692).  Returns attn_out [n][H_q*d];
    Q/K copies are normed + RoPE'd, k_cache / v_cache updated in place."""
    Q = np.array(Q, dtype=np.float32, copy=True)
    K = np.array(K, dtype=np.float32, copy=True)
    V = np.ascontiguousarray(V, dtype=np.float32)
    n = Q.shape[0]
    out = np.empty((n, cfg.num_heads * cfg.head_dim), dtype=np.float32)
    c = cfg.c()
    if threads == 1:
        cap = max(cfg.max_context, cfg.sliding_window)
        work = np.empty(2 * cap, dtype=np.float32)
        rc = lib().g3o_prefill(out, Q, K, V, _ptr(q_norm), _ptr(k_norm), k_cache, v_cache, table,
                               C.byref(c), layer, start_pos, n, work)
    else:
        rc = lib().g3o_prefill_mt(out, Q, K, V, _ptr(q_norm), _ptr(k_norm), k_cache, v_cache,
                                  table, C.byref(c), layer, start_pos, n, threads)
    if rc:
        raise RuntimeError(f"g3o_prefill rc={rc}")
    return out, Q, K


def prefill_rows(cfg: Config, layer: int, start_pos: int, Q, K, V, k_cache, v_cache, table,
                 rows, q_norm=None, k_norm=None, threads: int = 0):
    """Prefill (gemma3_transformer.c:641-692) evaluated only for batch tokens `rows`.
    Returns attn_out [len(rows)][H_q*d]; k_cache / v_cache end as after the full loop."""
    Q = np.array(Q, dtype=np.float32, copy=True)
    K = np.array(K, dtype=np.float32, copy=True)
    V = np.ascontiguousarray(V, dtype=np.float32)
    sel = np.ascontiguousarray(rows, dtype=np.int32)
    out = np.empty((sel.size, cfg.num_heads * cfg.head_dim), dtype=np.float32)
    c = cfg.c()
    rc = lib().g3o_prefill_rows(out, Q, K, V, _ptr(q_norm), _ptr(k_norm), k_cache, v_cache, table,
                                C.byref(c), layer, start_pos, Q.shape[0], sel, sel.size, threads)
    if rc:
        raise RuntimeError(f"g3o_prefill_rows rc={rc}")
    return out


# ---------------------------------------------------------------- reference harness

def ref_layer_decode(cfg: Config, layer: int, pos: int, q, k, v, k_cache, v_cache, table,
                     q_norm=None, k_norm=None):
    """The reference's own layer_attention (via oracle/_ref).  Returns (attn_out, q_rot, k_rot)."""
    out = np.empty(cfg.num_heads * cfg.head_dim, dtype=np.float32)
    q_rot = np.empty_like(out)
    k_rot = np.empty(cfg.num_kv_heads * cfg.head_dim, dtype=np.float32)
    rc = ref().ref_layer_decode(out, _ptr(q_rot), _ptr(k_rot),
                                np.ascontiguousarray(q, dtype=np.float32),
                                np.ascontiguousarray(k, dtype=np.float32),
                                np.ascontiguousarray(v, dtype=np.float32),
                                _ptr(q_norm), _ptr(k_norm), k_cache, v_cache, table,
                                cfg.num_heads, cfg.num_kv_heads, layer, pos, cfg.max_context,
                                cfg.sliding_window)
    if rc:
        raise RuntimeError(f"ref_layer_decode rc={rc}")
    return out, q_rot, k_rot


def ref_prefill(cfg: Config, layer: int, start_pos: int, Q, K, V, k_cache, v_cache, table,
                q_norm=None, k_norm=None, lib=None):
    """The reference's prefill loop; lib: a loaded reference build (default
    ref(); bench.py passes ref_timing())."""
    Q = np.array(Q, dtype=np.float32, copy=True)
    K = np.array(K, dtype=np.float32, copy=True)
    V = np.ascontiguousarray(V, dtype=np.float32)
    n = Q.shape[0]
    out = np.empty((n, cfg.num_heads * cfg.head_dim), dtype=np.float32)
    rc = (lib or ref()).ref_prefill_loop(out, Q, K, V, _ptr(q_norm), _ptr(k_norm), k_cache, v_cache, table,
                                cfg.num_heads, cfg.num_kv_heads, layer, start_pos, n,
                                cfg.max_context, cfg.sliding_window)
    if rc:
        raise RuntimeError(f"ref_prefill_loop rc={rc}")
    return out, Q, K
