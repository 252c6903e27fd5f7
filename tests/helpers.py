"""Shared helpers for the test suite: module loading and seeded workloads.

Every workload is generated on the host by the oracle's seeded generator
(splitmix64 + Box-Muller, bf16-exact values), so the HIP path and the CPU
oracle consume byte-identical inputs.  Cache rows are built the way the
reference builds them: row p holds K_p QK-normed and RoPE'd at position p,
and V_p raw (gemma3_transformer.c:294-316).
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "oracle"))

import g3_oracle as O  # noqa: E402

D = 256
HQ, HKV = 8, 4
QS, KS = HQ * D, HKV * D
TOL = 2e-3  # max-abs error / output RMS, the bar the path is judged by

_g3 = None


def g3attn():
    """The product binding (gemma3.c_amd/g3attn.py; the package dir has a dot)."""
    global _g3
    if _g3 is None:
        path = os.path.join(REPO, "gemma3.c_amd", "g3attn.py")
        spec = importlib.util.spec_from_file_location("g3attn", path)
        mod = importlib.util.module_from_spec(spec)
        sys.modules["g3attn"] = mod
        spec.loader.exec_module(mod)
        _g3 = mod
    return _g3


class DeviceBuffer:
    """Device memory for the _device entry points, allocated through the HIP
    runtime the product library itself links (no torch in the test process,
    so exactly one HIP runtime is loaded)."""

    _hip = None

    @classmethod
    def hip(cls):
        if cls._hip is None:
            import ctypes as C
            g3attn().lib()                     # the library's runtime is loaded first
            h = C.CDLL("libamdhip64.so.7")
            h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
            h.hipFree.argtypes = [C.c_void_p]
            h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
            h.hipDeviceSynchronize.argtypes = []
            cls._hip = h
        return cls._hip

    def __init__(self, nbytes: int):
        import ctypes as C
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        rc = self.hip().hipMalloc(C.byref(p), max(self.nbytes, 1))
        assert rc == 0, f"hipMalloc({self.nbytes}) -> {rc}"
        self.ptr = int(p.value)

    @classmethod
    def of(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        assert self.hip().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, 1) == 0

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        assert self.hip().hipDeviceSynchronize() == 0
        assert self.hip().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes, 2) == 0
        return out

    def free(self):
        if self.ptr:
            self.hip().hipFree(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / RMS(ref)."""
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    return float(np.max(np.abs(np.asarray(got, dtype=np.float64) - ref)) / rms)


def tensor(config: int, tensor_id: int, n: int, first: int = 0, layer: int = 0) -> np.ndarray:
    return O.gen_normal_bf16(n, O.seed_for(config, tensor_id, layer), first)


class DecodeCase:
    """One decode step of one layer at position `pos`, cache holding 0..pos-1.

    Inputs: q from stream (config, 1); token p's k and v are rows p of
    streams (config, 2) and (config, 3), so the new token is row `pos`.
    """

    def __init__(self, config: int, layer: int, pos: int, max_context: int,
                 window: int = 1024, norm: bool = True, layer_seed: int = 0,
                 n_heads: int = HQ, n_kv: int = HKV):
        self.config, self.layer, self.pos = config, layer, pos
        self.cfg = O.Config(max_context=max_context, sliding_window=window, num_heads=n_heads,
                            num_kv_heads=n_kv)
        self.is_global = O.is_global_layer(layer)
        self.table = O.rope_table(max_context, self.cfg.theta(layer))
        QS, KS, HKV = n_heads * D, n_kv * D, n_kv
        self.q = tensor(config, 1, QS, layer=layer_seed)
        # oldest position still visible to the new token (ring keeps `window` slots)
        self.lo = 0 if self.is_global else max(0, pos - window)
        n_hist = pos - self.lo
        self.k_hist = tensor(config, 2, n_hist * KS, self.lo * KS, layer_seed).reshape(n_hist, KS)
        self.v_hist = tensor(config, 3, n_hist * KS, self.lo * KS, layer_seed).reshape(n_hist, KS)
        self.k = tensor(config, 2, KS, pos * KS, layer_seed)
        self.v = tensor(config, 3, KS, pos * KS, layer_seed)
        self.norm = O.zero_norm() if norm else None
        # cached rows are normed + RoPE'd at their own positions
        self.k_rows = self.k_hist.copy()
        if n_hist:
            O.norm_rope_batch(self.k_rows.reshape(n_hist, HKV, D), self.table, self.lo, self.norm)
        self.rows = self.cfg.cache_rows(layer)

    def slots(self) -> np.ndarray:
        p = np.arange(self.lo, self.pos)
        return p if self.is_global else p % self.cfg.sliding_window

    def oracle_cache(self):
        ks = self.cfg.num_kv_heads * D
        Kc = np.zeros((self.rows, ks), dtype=np.float32)
        Vc = np.zeros((self.rows, ks), dtype=np.float32)
        s = self.slots()
        Kc[s] = self.k_rows
        Vc[s] = self.v_hist
        return Kc, Vc

    def oracle(self):
        """(attn_out, k_cache, v_cache) from the CPU restatement."""
        Kc, Vc = self.oracle_cache()
        out, _, _ = O.layer_decode(self.cfg, self.layer, self.pos, self.q, self.k, self.v, Kc, Vc,
                                   self.table, self.norm, self.norm)
        return out, Kc, Vc

    def load_gpu(self, ctx):
        """Write the history rows into a g3attn context's cache (reference layout)."""
        s = self.slots()
        if s.size == 0:
            return
        # contiguous runs of slots (a ring may wrap once)
        breaks = np.nonzero(np.diff(s) != 1)[0] + 1
        for chunk in np.split(np.arange(s.size), breaks):
            ctx.kv_write(self.layer, int(s[chunk[0]]), self.k_rows[chunk], self.v_hist[chunk])

    def gpu(self, ctx):
        return ctx.decode(self.layer, self.pos, self.q, self.k, self.v, self.norm, self.norm)
