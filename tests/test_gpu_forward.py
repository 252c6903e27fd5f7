"""The whole token forward on the GPU (g3attn_forward_device, replacing
gemma3_transformer_forward, gemma3_transformer.c:396-512) against the
reference's own output on a small model of Gemma 3's structure.

The model (tests/golden/make_golden.py FORWARD): 6 layers with layer 5
global, 8 query / 4 KV heads of 256, hidden 512, intermediate 1536, vocab
1024, a 16-row sliding window that the 40-token sequence wraps, and a layer
without its optional norms.  Every kernel on the path runs: embedding, the
RMSNorm / residual steps, the fused Q/K/V GEMV, QK-norm + RoPE + cache write
+ split-K attention, o_proj, the GEGLU gate/up GEMV, down_proj and the tied
logits.  The bar is 1e-4 x RMS on logits and hidden state (fp32 throughout;
only summation orders differ), and every step's argmax must agree.
"""
import importlib.util
import os

import numpy as np
import pytest

from helpers import O, REPO, DeviceBuffer, g3attn, rel_err

pytestmark = pytest.mark.gpu

G = g3attn()
GOLD = os.path.join(REPO, "tests", "golden")
_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLD, "make_golden.py"))
MG = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(MG)


def _gpu_config(f):
    return G.default_config(num_layers=f["layers"], max_context=f["max_context"],
                            sliding_window=f["window"], hidden_size=f["hidden"],
                            intermediate_size=f["inter"], vocab_size=f["vocab"])


def _upload(embed, layers, norm):
    """Device copies of the weights in a g3attn_weights; the buffers must
    outlive the calls that read them."""
    bufs = []

    def up(a):
        if a is None:
            return None
        b = DeviceBuffer.of(a)
        bufs.append(b)
        return b.ptr

    W = G.Weights()
    W.embed_tokens, W.norm = up(embed), up(norm)
    for l, lw in enumerate(layers):
        for name in O.LAYER_TENSORS:
            setattr(W.layers[l], name, up(lw[name]))
    return W, bufs


def _run(ctx, W, tokens, f, logits_at=None):
    """One forward_device call per token; returns every computed logits row
    (None where compute_logits was off) and the final hidden state."""
    dl, dh = DeviceBuffer(f["vocab"] * 4), DeviceBuffer(f["hidden"] * 4)
    rows = []
    for i, t in enumerate(tokens):
        want = logits_at is None or i in logits_at
        last = i == len(tokens) - 1
        ctx.forward_device(W, int(t), i, dl.ptr if want else None, want, dh.ptr if last else None)
        rows.append(dl.download(np.float32, f["vocab"]) if want else None)
    return rows, dh.download(np.float32, f["hidden"])


def test_forward_matches_reference_golden():
    g = np.load(os.path.join(GOLD, "forward.npz"), allow_pickle=False)
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    assert list(MG.forward_hash(embed, layers, norm, tokens)) == list(g["in_hash"])
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        W, bufs = _upload(embed, layers, norm)
        rows, hid = _run(ctx, W, tokens, f)
    logits = np.stack(rows)
    err_l = rel_err(logits[list(g["rows"])], g["logits"])
    err_h = rel_err(hid, g["hidden"])
    print(f"[forward golden] n={len(tokens)} logits rel={err_l:.3e} hidden rel={err_h:.3e}", flush=True)
    assert err_l < 1e-4 and err_h < 1e-4
    assert np.array_equal(logits.argmax(axis=1), g["argmax"])
    # every step, not only the kept rows, against the oracle
    want, _ = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm)
    for i in range(len(tokens)):
        assert rel_err(logits[i], want[i]) < 1e-4, i


@pytest.mark.parametrize("fold", [0, 1, 3])
def test_forward_fold_modes(fold, monkeypatch):
    """The residual step between two GEMVs (post-norm, residual add, next
    pre-norm) as the one-workgroup kernel (G3ATTN_FORWARD_FOLD=0), in the
    prologue of the next layer's Q/K/V launch (1, the default), or also in
    the gate/up launch's (3): every step's logits and the final hidden state
    against the oracle.  Layer 2's input norm sits 2 bytes past an 8-byte
    boundary, so the fold into layer 2's Q/K/V launch falls back to the
    kernel for that step, and the residual stream still comes out right."""
    monkeypatch.setenv("G3ATTN_FORWARD_FOLD", str(fold))
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        W, bufs = _upload(embed, layers, norm)
        gain = layers[2]["input_layernorm"]
        odd = DeviceBuffer(gain.nbytes + 16)
        odd.upload(gain, offset=2)
        W.layers[2].input_layernorm = odd.ptr + 2
        rows, hid = _run(ctx, W, tokens, f)
    want, want_h = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm)
    errs = [rel_err(rows[i], want[i]) for i in range(len(tokens))]
    err_h = rel_err(hid, want_h)
    print(f"[forward fold={fold}] worst logits rel={max(errs):.3e} hidden rel={err_h:.3e}", flush=True)
    assert max(errs) < 1e-4 and err_h < 1e-4
    assert np.array_equal(np.stack(rows).argmax(axis=1), want.argmax(axis=1))


def test_forward_without_logits_is_identical():
    """compute_logits = 0 skips the final norm and vocab GEMV only: the state
    the next step reads is bit-identical, so the last step's logits are too."""
    cfg, f, embed, layers, norm, tokens = MG.forward_case(n=20)
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        W, bufs = _upload(embed, layers, norm)
        full, hid_a = _run(ctx, W, tokens, f)
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        W, bufs = _upload(embed, layers, norm)
        sparse, hid_b = _run(ctx, W, tokens, f, logits_at={len(tokens) - 1})
    print("[forward no-logits] steps=20", flush=True)
    assert np.array_equal(full[-1], sparse[-1])
    assert np.array_equal(hid_a, hid_b)


def test_forward_argument_errors():
    cfg, f, embed, layers, norm, tokens = MG.forward_case(n=1)
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        W, bufs = _upload(embed, layers, norm)
        dl = DeviceBuffer(f["vocab"] * 4)
        with pytest.raises(G.G3AttnError):
            ctx.forward_device(W, f["vocab"], 0, dl.ptr)            # token outside the vocabulary
        with pytest.raises(G.G3AttnError) as e:
            ctx.forward_device(W, 1, f["max_context"], dl.ptr)      # past the cache
        assert e.value.rc == G.ERR_CONTEXT_OVERFLOW
        with pytest.raises(G.G3AttnError):
            ctx.forward_device(W, 1, 0, None, True)                 # logits requested, no buffer
        q = W.layers[2].q_proj
        W.layers[2].q_proj = None
        with pytest.raises(G.G3AttnError):
            ctx.forward_device(W, 1, 0, dl.ptr)
        W.layers[2].q_proj = q
        ctx.forward_device(W, 1, 0, dl.ptr)
        assert np.all(np.isfinite(dl.download(np.float32, f["vocab"])))


# ---------------------------------------------------------------- uploaded model
# g3attn_upload_weights / g3attn_forward_token / g3attn_prefill_tokens: the
# backend hook's calls (gemma3_metal_upload_weights, _forward_token, _prefill;
# gemma3_metal.m:560-601, 620-971, 977-987).

def test_upload_and_forward_token_match_reference_golden():
    """Host weights -> upload -> forward_token (host logits) reproduces the
    reference's logits, and equals forward_device on the same device copies
    bit for bit (same kernels, same order)."""
    g = np.load(os.path.join(GOLD, "forward.npz"), allow_pickle=False)
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    HW, keep = G.host_weights(embed, layers, norm)
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        assert ctx.device_weights() is None
        ctx.upload_weights(HW)
        rows = [ctx.forward_token(int(t), i) for i, t in enumerate(tokens)]
        DW = ctx.device_weights()
        assert DW is not None and DW.layers[3].q_norm is None and DW.layers[2].q_norm is not None
    logits = np.stack(rows)
    err = rel_err(logits[list(g["rows"])], g["logits"])
    print(f"[forward_token golden] rel={err:.3e}", flush=True)
    assert err < 1e-4
    assert np.array_equal(logits.argmax(axis=1), g["argmax"])
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        W, bufs = _upload(embed, layers, norm)
        dev_rows, _ = _run(ctx, W, tokens, f)
    assert np.array_equal(logits, np.stack(dev_rows))


def test_forward_token_device_matches_forward_device():
    """g3attn_forward_token_device (the uploaded model, device logits, no
    wait) equals g3attn_forward_device of the same token bit for bit, with
    the two contexts' launches interleaved and only occasional host waits; a
    re-upload takes effect at the next token."""
    cfg, f, embed, layers, norm, tokens = MG.forward_case(n=24)
    HW, keep = G.host_weights(embed, layers, norm)
    with G.Context(_gpu_config(f), f["max_context"]) as gr, G.Context(_gpu_config(f), f["max_context"]) as eg:
        gr.upload_weights(HW)
        W, bufs = _upload(embed, layers, norm)
        dlg, dle = DeviceBuffer(f["vocab"] * 4), DeviceBuffer(f["vocab"] * 4)
        for i, t in enumerate(tokens):
            with_logits = i % 3 != 1                   # tokens without logits in between
            gr.forward_token_device(int(t), i, dlg.ptr if with_logits else None)
            eg.forward_device(W, int(t), i, dle.ptr, True)
            if i % 4 == 0:
                gr.synchronize()
            if with_logits:
                a, b = dlg.download(np.float32, f["vocab"]), dle.download(np.float32, f["vocab"])
                assert np.array_equal(a, b), i
        # a new model
        other = [dict(lw) for lw in layers]
        other[1]["up_proj"] = MG.weights_bf16(f["inter"], f["hidden"], 0xD1D1)
        HW2, keep2 = G.host_weights(embed, other, norm)
        gr.upload_weights(HW2)
        W2, bufs2 = _upload(embed, other, norm)
        t = int(tokens[0])
        gr.forward_token_device(t, len(tokens), dlg.ptr)
        eg.forward_device(W2, t, len(tokens), dle.ptr, True)
        assert np.array_equal(dlg.download(np.float32, f["vocab"]), dle.download(np.float32, f["vocab"]))
    print("[forward_token_device] ok", flush=True)


def test_upload_from_a_file_mapping(tmp_path):
    """The loader's case: tensors packed in one mapped file at 2-byte-aligned
    offsets (as in a safetensors blob), uploaded straight from the mapping."""
    g = np.load(os.path.join(GOLD, "forward.npz"), allow_pickle=False)
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    arrays = [embed, norm] + [lw[n] for lw in layers for n in G.LAYER_TENSORS if lw[n] is not None]
    path = tmp_path / "weights.bin"
    offs, off = [], 2                       # start 2 bytes in: nothing is 16-byte aligned by luck
    with open(path, "wb") as fh:
        fh.write(b"\0\0")
        for a in arrays:
            offs.append(off)
            fh.write(np.ascontiguousarray(a, np.uint16).tobytes())
            off += a.nbytes + 2
            fh.write(b"\0\0")
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    views = iter([mm[o:o + a.nbytes].view(np.uint16) for o, a in zip(offs, arrays)])
    HW = G.Weights()
    HW.embed_tokens, HW.norm = next(views).ctypes.data, next(views).ctypes.data
    for l, lw in enumerate(layers):
        for n in G.LAYER_TENSORS:
            if lw[n] is not None:
                setattr(HW.layers[l], n, next(views).ctypes.data)
    assert HW.embed_tokens % 16 == 2
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        ctx.upload_weights(HW)
        del mm
        last = None
        for i, t in enumerate(tokens):
            last = ctx.forward_token(int(t), i, compute_logits=(i == len(tokens) - 1))
    print("[upload mmap] ok", flush=True)
    assert rel_err(last, g["logits"][-1]) < 1e-4


def test_prefill_tokens_equals_the_token_loop():
    """A batch shorter than G3ATTN_PREFILL_BATCH_MIN: prefill_tokens enqueues
    the tokens back to back and returns the last token's logits, bit-identical
    to forward_token one by one, and decoding continues from it identically.
    (Longer batches take the batched path: tests/test_gpu_gemm.py.)"""
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    HW, keep = G.host_weights(embed, layers, norm)
    n = 12
    with G.Context(_gpu_config(f), f["max_context"]) as a, G.Context(_gpu_config(f), f["max_context"]) as b:
        a.upload_weights(HW)
        b.upload_weights(HW)
        want = [a.forward_token(int(t), i) for i, t in enumerate(tokens[:n + 3])]
        got = b.prefill_tokens(tokens[:n])
        assert np.array_equal(got, want[n - 1])
        assert b.prefill_tokens(tokens[n:n + 2], start_pos=n, logits=False) is None
        assert np.array_equal(b.forward_token(int(tokens[n + 2]), n + 2), want[n + 2])
    print("[prefill_tokens] ok", flush=True)


def test_uploaded_model_errors():
    cfg, f, embed, layers, norm, tokens = MG.forward_case(n=4)
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        with pytest.raises(G.G3AttnError):
            ctx.forward_token(1, 0)                              # nothing uploaded
        HW, keep = G.host_weights(embed, layers, None)
        with pytest.raises(G.G3AttnError):
            ctx.upload_weights(HW)                               # no final norm
        HW, keep = G.host_weights(embed, layers, norm)
        ctx.upload_weights(HW)
        with pytest.raises(G.G3AttnError):
            ctx.prefill_tokens([1, 2, f["vocab"], 3])            # checked before any work
        with pytest.raises(G.G3AttnError) as e:
            ctx.prefill_tokens([1] * 5, start_pos=f["max_context"] - 4)
        assert e.value.rc == G.ERR_CONTEXT_OVERFLOW
        first = ctx.forward_token(int(tokens[0]), 0)
        # a second upload replaces the model
        other = [dict(lw) for lw in layers]
        other[0]["down_proj"] = MG.weights_bf16(f["hidden"], f["inter"], 0xD0D0)
        HW2, keep2 = G.host_weights(embed, other, norm)
        ctx.upload_weights(HW2)
        assert not np.array_equal(ctx.forward_token(int(tokens[0]), 0), first)
