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
