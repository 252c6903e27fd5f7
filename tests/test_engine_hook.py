"""The reference engine, unmodified, running on libg3attn through its own GPU
backend hook.

oracle/_ref/libg3engine.so is gemma3_transformer.c + gemma3_kernels.c
compiled in place with -DUSE_MPS and linked against libg3backend.so, which
defines the eight backend functions the engine declares
(gemma3_transformer.c:17-31).  So these tests exercise the engine's own
create / upload / fallback logic (:889-905), its forward_token and
prefill_tokens branches (:931-935, :954-958) and its reset (:974-978)
against the reference's real types, with no patch.

The model is the 6-layer forward fixture (tests/golden/make_golden.py
FORWARD; tests/golden/forward.npz holds the reference CPU engine's logits).
On the GPU the bar is the token forward's, 1e-4 x RMS per logits row, and the
argmax of every decoded row.  When the backend is unavailable or fails to
upload (G3ATTN_FAULT), the engine must fall back to its CPU path, whose logits
are the fixture's own (1e-5: the same code, possibly another host CPU).
"""
import ctypes as C
import importlib.util
import os

import numpy as np
import pytest

from helpers import O, REPO, g3attn, rel_err

GOLD = os.path.join(REPO, "tests", "golden")
ENGINE_SO = os.path.join(REPO, "oracle", "_ref", "libg3engine.so")
BACKEND_SO = os.path.join(REPO, "gemma3.c_amd", "lib", "libg3backend.so")
HOOKS = ("gemma3_metal_available", "gemma3_metal_init", "gemma3_metal_free", "gemma3_metal_upload_weights",
         "gemma3_metal_upload_rope", "gemma3_metal_forward_token", "gemma3_metal_prefill",
         "gemma3_metal_reset_cache")

_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLD, "make_golden.py"))
MG = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(MG)

needs_engine = pytest.mark.skipif(not os.path.exists(ENGINE_SO),
                                  reason="oracle/_ref/libg3engine.so not built (needs /root/reference at build time)")


def _engine():
    lib = C.CDLL(ENGINE_SO)
    f = lib.eng_run
    f.restype = C.c_int
    f.argtypes = [np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS"), C.POINTER(C.c_int),
                  np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS"), C.c_int, C.c_int, C.c_int,
                  np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS"), C.c_void_p,
                  np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")] + [C.c_int] * 8
    return f


def run_engine(n_prefill, passes=1):
    """(rc, on_gpu, logits [passes][n][vocab]) of the engine on the fixture
    model; rows the engine does not return stay NaN."""
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    keep = []
    ptrs = (C.c_void_p * (13 * cfg.num_layers))()
    for l, lw in enumerate(layers):
        for j, name in enumerate(O.LAYER_TENSORS):
            a = lw.get(name)
            if a is not None:
                a = np.ascontiguousarray(a, dtype=np.uint16)
                keep.append(a)
                ptrs[13 * l + j] = a.ctypes.data
    n = len(tokens)
    logits = np.full((passes, n, f["vocab"]), np.nan, np.float32)
    on_gpu = C.c_int(-1)
    rc = _engine()(logits, C.byref(on_gpu), np.ascontiguousarray(tokens, np.int32), n, n_prefill, passes,
                   np.ascontiguousarray(embed, np.uint16), C.cast(ptrs, C.c_void_p),
                   np.ascontiguousarray(norm, np.uint16), f["vocab"], f["hidden"], f["inter"], cfg.num_layers,
                   cfg.num_heads, cfg.num_kv_heads, f["max_context"], f["window"])
    return rc, on_gpu.value, logits


def _golden():
    return np.load(os.path.join(GOLD, "forward.npz"), allow_pickle=False)


def _check_rows(logits, first_row, tol):
    """Every fixture row from first_row on, and the argmax of every row from
    first_row on, against the reference CPU engine."""
    g = _golden()
    rows = [int(r) for r in g["rows"]]
    errs = []
    for k, r in enumerate(rows):
        if r >= first_row:
            errs.append(rel_err(logits[r], g["logits"][k]))
            assert errs[-1] < tol, (r, errs[-1])
    assert np.array_equal(logits[first_row:].argmax(axis=1), g["argmax"][first_row:])
    return max(errs)


# ---------------------------------------------------------------- CPU

@needs_engine
def test_engine_links_the_backend_hook():
    """The engine library resolves the backend functions from libg3backend.so,
    which defines all eight that gemma3_transformer.c declares."""
    lib = C.CDLL(BACKEND_SO)
    for name in HOOKS:
        assert hasattr(lib, name), name
    assert hasattr(C.CDLL(ENGINE_SO), "eng_run")


@needs_engine
def test_engine_falls_back_when_create_fails(monkeypatch):
    """G3ATTN_FAULT=create: gemma3_metal_init returns NULL, the engine keeps
    its CPU path (gemma3_transformer.c:889-905) and produces the reference's
    logits; the injected cause is in g3attn_last_error."""
    monkeypatch.setenv("G3ATTN_FAULT", "create")
    rc, on_gpu, logits = run_engine(n_prefill=16)
    assert rc == 0 and on_gpu == 0
    assert "injected" in g3attn().last_error()
    _check_rows(logits[0], 15, 1e-5)


@needs_engine
def test_engine_without_a_device_uses_the_cpu():
    """No GPU visible (this container): init fails on the device check and the
    engine's CPU path runs every token.  Whether a device is visible is
    decided by the backend library itself (gemma3_metal_available: its own
    hipGetDeviceCount through the HIP runtime libg3attn links), not by
    another runtime's view of the machine."""
    if C.CDLL(BACKEND_SO).gemma3_metal_available():
        pytest.skip("the backend library sees a HIP device")
    rc, on_gpu, logits = run_engine(n_prefill=0)
    assert rc == 0 and on_gpu == 0
    assert "no HIP device" in g3attn().last_error()
    _check_rows(logits[0], 0, 1e-5)


# ---------------------------------------------------------------- GPU

@needs_engine
@pytest.mark.gpu
def test_engine_hook_runs_on_the_gpu():
    """Backend on: 16 prompt tokens through gemma3_metal_prefill (the batched
    MFMA prefill), then 24 decoded tokens through gemma3_metal_forward_token,
    against the reference CPU engine; a second pass after
    gemma3_transformer_reset repeats the first bit for bit."""
    rc, on_gpu, logits = run_engine(n_prefill=16, passes=2)
    assert rc == 0 and on_gpu == 1, g3attn().last_error()
    err = _check_rows(logits[0], 15, 1e-4)
    print(f"[engine hook] prefill 16 + decode 24: worst logits rel_err={err:.3e}", flush=True)
    assert np.array_equal(logits[0][15:], logits[1][15:])


@needs_engine
@pytest.mark.gpu
def test_engine_hook_token_loop_on_the_gpu():
    """Backend on, every token through gemma3_metal_forward_token (the engine's
    decode of a prompt in non-BLAS builds)."""
    rc, on_gpu, logits = run_engine(n_prefill=0)
    assert rc == 0 and on_gpu == 1, g3attn().last_error()
    err = _check_rows(logits[0], 0, 1e-4)
    print(f"[engine hook] 40 tokens: worst logits rel_err={err:.3e}", flush=True)


@needs_engine
@pytest.mark.gpu
def test_engine_falls_back_when_upload_fails(monkeypatch):
    """G3ATTN_FAULT=upload: gemma3_metal_upload_weights returns -4 on a live
    GPU context; the engine frees it and answers on the CPU
    (gemma3_transformer.c:892-898)."""
    monkeypatch.setenv("G3ATTN_FAULT", "upload")
    rc, on_gpu, logits = run_engine(n_prefill=16)
    assert rc == 0 and on_gpu == 0
    assert "injected" in g3attn().last_error()
    _check_rows(logits[0], 15, 1e-5)


@needs_engine
@pytest.mark.gpu
def test_engine_returns_a_forward_failure(monkeypatch):
    """G3ATTN_FAULT=forward: the GPU forward returns -1 and the engine passes
    it to its caller (gemma3_transformer.c:931-935, 954-958) rather than
    answering from a CPU cache that never saw the prompt."""
    monkeypatch.setenv("G3ATTN_FAULT", "forward")
    rc, on_gpu, _ = run_engine(n_prefill=16)
    assert on_gpu == 1 and rc == -1
    rc, on_gpu, _ = run_engine(n_prefill=0)
    assert on_gpu == 1 and rc == -1


@pytest.mark.skipif(not os.path.exists(O.GQA_ENGINE_SO), reason="oracle/_ref/libg3gqa.so not built")
def test_engine_attention_call_is_the_dropin():
    """oracle/_ref/libg3gqa.so (the engine compiled with
    -Dgemma3_gqa=g3attn_gqa) resolves its attention call to libg3attn: with no
    device visible, the engine's gemma3_gqa call (through the harness's
    ref_gqa) leaves the output untouched and libg3attn reports the missing
    device, where the CPU reference would have computed it."""
    if C.CDLL(BACKEND_SO).gemma3_metal_available():
        pytest.skip("the backend library sees a HIP device")
    eng = O.gqa_engine()
    q = np.ones(8 * 256, np.float32)
    k = v = np.ones(4 * 4 * 256, np.float32)
    out = np.full(8 * 256, np.nan, np.float32)
    eng.ref_gqa(out, q, k, v, 8, 4, 4, 256, 0.0625, None, None)
    assert np.isnan(out).all()
    assert "device" in g3attn().last_error()
