"""The gemma3_gqa drop-in at its own call sites, on the GPU.

oracle/_ref/libg3gqa.so is the reference harness with its translation unit
that #includes gemma3_transformer.c compiled with -Dgemma3_gqa=g3attn_gqa
(oracle/Makefile): the engine's own layer_attention (gemma3_transformer.c:
294-352) and gemma3_transformer_forward (:396-512) call g3attn_gqa for every
token, with no source change; gemma3_kernels.c keeps its CPU gemma3_gqa.

- The forward fixture's model (8 query / 4 KV heads of 256: the split-K decode
  kernels) against the reference CPU engine's logits in tests/golden/
  forward.npz, and a model of the same structure with 6 query / 2 KV heads
  (group 3: the general kernel) against the unmodified reference engine
  (oracle/_ref/libg3ref.so) on the same weights.  Bar: the token forward's
  1e-4 x RMS per logits row, and every argmax.
- g3attn_gqa itself on shapes outside the model's (head_dim 40 to 512, groups
  1 to 8, masked and not) against the oracle's gemma3_gqa (1e-4 x RMS, the
  fp32 decode bar), and g3attn_gqa_noalloc bit for bit against it.
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

needs_engine = pytest.mark.skipif(not os.path.exists(O.GQA_ENGINE_SO) or not O.have_ref(),
                                  reason="oracle/_ref drop-in harness not built (needs /root/reference at build time)")


@needs_engine
def test_engine_forward_through_the_gqa_dropin():
    """The engine's forward over 40 tokens (local ring wrapped, one global
    layer) with its attention on the GPU through g3attn_gqa, against the
    reference CPU engine's logits."""
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    logits, _ = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm, ref_lib=O.gqa_engine())
    g = np.load(os.path.join(GOLD, "forward.npz"), allow_pickle=False)
    errs = [rel_err(logits[int(r)], g["logits"][k]) for k, r in enumerate(g["rows"])]
    print(f"[gqa drop-in engine] 8/4 heads: worst logits rel_err={max(errs):.3e}", flush=True)
    assert max(errs) < 1e-4
    assert np.array_equal(logits.argmax(axis=1), g["argmax"])


@needs_engine
def test_engine_forward_through_the_gqa_dropin_group3():
    """The same with 6 query heads over 2 KV heads (group 3, the general
    kernel), against the unmodified reference engine on the same weights."""
    cfg, f, embed, layers, norm, tokens = MG.forward_case(heads=6, kv_heads=2, n=24)
    got, _ = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm, ref_lib=O.gqa_engine())
    want, _ = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm, use_ref=True)
    errs = [rel_err(got[i], want[i]) for i in range(len(tokens))]
    print(f"[gqa drop-in engine] 6/2 heads: worst logits rel_err={max(errs):.3e}", flush=True)
    assert max(errs) < 1e-4
    assert np.array_equal(got.argmax(axis=1), want.argmax(axis=1))


SHAPES = [(6, 2, 64), (3, 1, 96), (8, 1, 512), (16, 4, 128), (2, 2, 40), (12, 3, 256), (4, 4, 1)]


@pytest.mark.parametrize("heads,kv_heads,d", SHAPES)
def test_gqa_general_shapes(heads, kv_heads, d):
    rng = np.random.default_rng(heads * 1000 + kv_heads * 10 + d)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    for seq, masked in ((1, False), (37, True), (2000, False), (5000, True)):
        q = rng.standard_normal(heads * d).astype(np.float32)
        k = rng.standard_normal(seq * kv_heads * d).astype(np.float32)
        v = rng.standard_normal(seq * kv_heads * d).astype(np.float32)
        mask = None
        if masked:
            mask = (rng.standard_normal(seq) * 2).astype(np.float32)
            mask[rng.random(seq) < 0.3] = -np.inf
            mask[0] = 0.0
        got = G.gqa(q, k, v, heads, kv_heads, seq, head_dim=d, scale=scale, mask=mask)
        want = O.gqa(q, k, v, heads, kv_heads, seq, d=d, scale=scale, mask=mask)
        err = rel_err(got, want)
        print(f"[gqa {heads}/{kv_heads} d={d} seq={seq} mask={masked}] rel_err={err:.3e}", flush=True)
        assert err < 1e-4, (seq, err)
        if heads <= G.NOALLOC_MAX_HEADS:
            bufs = [DeviceBuffer.of(x) for x in (q, k, v)]
            dm = DeviceBuffer.of(mask) if mask is not None else None
            out = DeviceBuffer(heads * d * 4)
            try:
                G.gqa_noalloc(out.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, heads, kv_heads, seq, head_dim=d,
                              scale=scale, mask_ptr=dm.ptr if dm else None)
                DeviceBuffer.hip().hipDeviceSynchronize()
                na = out.download(np.float32, heads * d)
            finally:
                for b in bufs + [out] + ([dm] if dm else []):
                    b.free()
            assert rel_err(na, want) < 1e-4, (seq, "noalloc")


def test_gqa_rejects_out_of_range_shapes():
    """Shapes the reference would read out of bounds with (n_kv_heads not
    dividing n_heads) or beyond the general kernel (head_dim > 512) leave the
    output untouched and set the error."""
    q = np.ones(6 * 64, np.float32)
    k = v = np.ones(10 * 4 * 64, np.float32)
    with pytest.raises(G.G3AttnError):
        G.gqa(q, k, v, 6, 4, 10, head_dim=64)
    with pytest.raises(G.G3AttnError):
        G.gqa(np.ones(2 * 640, np.float32), np.ones(640, np.float32), np.ones(640, np.float32), 2, 1, 1,
              head_dim=640)
