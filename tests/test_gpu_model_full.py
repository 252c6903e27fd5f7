"""The whole-model rows at Gemma3-4B shapes (34 layers, hidden 2560,
intermediate 10240, vocab 262208, 8 / 4 heads of 256, window 1024), with
random bf16 weights: the shapes the bench measures, checked for values.

- Token forward (g3attn_upload_weights + g3attn_forward_token, replacing
  gemma3_transformer_forward, gemma3_transformer.c:396-512) for three tokens
  against the oracle's restatement of the same forward (g3o_forward_seq) on
  the same host weights.  fp32 throughout on both sides; the bar is 1e-4 x
  RMS per logits row, as for the small-model golden.
- Token forward at a long position (pos 1100: the local layers' 1024-row
  rings are full and the global layers attend 1101 keys) on caches
  pre-filled through g3attn_kv_write, against the oracle's forward
  (g3o_forward_cached) on the same cache contents; bar 1e-4 x RMS.
- Batched prefill (g3attn_prefill_tokens for 192 tokens: MFMA GEMM
  projections + the prefill attention kernel, replacing
  gemma3_transformer_prefill_batched, :526-787) and one decode step after it,
  against the oracle's sequential forward over the same 193 tokens.  The GEMMs
  take x as bf16 hi + lo (16 significant bits) where the GEMV reads fp32 x;
  the bar is 1e-3 x RMS of the logits row, with the measured figure printed.
- The same batched prefill at 2048 tokens against the token forward looped
  over the same tokens on the GPU (the engine's non-BLAS prefill, :814-821),
  then one decode step after each: the bench's shape, beyond what the
  one-core oracle covers in a test's time.

The oracle's GEMVs split their rows over up to 16 host threads (the same bits
as one thread).

Weights: bf16 N(0,1) x 2^-6 (norm gains N(0,1) x 2^-3) tiled from a seeded
pool of 2^24 + 43 values, each tensor from its own offset (the odd pool length
keeps rows of one tensor, and tensors, from repeating one another at any
aligned stride).  Both sides read the same bits.  About 7.8 GB of host and
device memory.  No torch in the process (the tests drive the library's own
HIP runtime only).
"""
import os

import numpy as np
import pytest

from helpers import O, g3attn, rel_err

pytestmark = pytest.mark.gpu

G = g3attn()
H, I, V, L = 2560, 10240, 262208, 34
QS, KS = 8 * 256, 4 * 256
MAXCTX = 4096


POOL = (1 << 24) + 43
THREADS = max(1, min(16, os.cpu_count() or 1))
OCFG = O.Config(num_layers=L, max_context=MAXCTX)


@pytest.fixture(scope="module")
def model():
    rng = np.random.default_rng(0x6A33)
    base = rng.standard_normal(POOL).astype(np.float32)
    pools = {sh: ((base * np.float32(2.0 ** -sh)).view(np.uint32) >> 16).astype(np.uint16) for sh in (3, 6)}
    count = [0]

    def w(n, shift=6):
        pool = pools[shift]
        off = (count[0] * 7919 * 1031 + 17) % POOL
        count[0] += 1
        out = np.empty(n, np.uint16)
        first = min(n, POOL - off)
        out[:first] = pool[off:off + first]
        o = first
        while o < n:
            k = min(POOL, n - o)
            out[o:o + k] = pool[:k]
            o += k
        return out

    embed = w(V * H)
    layers = []
    for _ in range(L):
        layers.append(dict(input_layernorm=w(H, 3), q_proj=w(QS * H), k_proj=w(KS * H), v_proj=w(KS * H),
                           o_proj=w(H * QS), q_norm=w(256, 3), k_norm=w(256, 3),
                           post_attention_layernorm=w(H, 3), gate_proj=w(I * H), up_proj=w(I * H),
                           down_proj=w(H * I), pre_feedforward_layernorm=w(H, 3),
                           post_feedforward_layernorm=w(H, 3)))
    norm = w(H, 3)
    print("[full model] weights generated", flush=True)
    cfg = G.default_config(max_context=MAXCTX)
    assert (cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.num_layers) == (H, I, V, L)
    ctx = G.Context(cfg, MAXCTX)
    HW, keep = G.host_weights(embed, layers, norm)
    ctx.upload_weights(HW)
    del keep
    print("[full model] uploaded", flush=True)
    yield ctx, embed, layers, norm
    ctx.close()


def test_forward_full_shapes_vs_oracle(model):
    ctx, embed, layers, norm = model
    tokens = np.array([5, 70001, 262207], np.int32)
    ctx.reset()
    got = np.stack([ctx.forward_token(int(t), i) for i, t in enumerate(tokens)])
    print("[full model] gpu forward done; oracle forward (one core)", flush=True)
    want, _ = O.forward_seq(O.Config(num_layers=L, max_context=64), H, I, tokens, embed, layers, norm)
    for i in range(len(tokens)):
        err = rel_err(got[i], want[i])
        print(f"[full forward] token {i} (pos {i}): logits rel_err={err:.3e}", flush=True)
        assert err < 1e-4, (i, err)
    assert np.array_equal(got.argmax(axis=1), want.argmax(axis=1))


def test_forward_long_position_vs_oracle(model):
    """One token at pos 1100 on caches whose rows (every slot of the local
    rings, positions 0..1099 of the global layers) were written through
    g3attn_kv_write, against the oracle given the same cache contents."""
    ctx, embed, layers, norm = model
    pos = 1100
    rng = np.random.default_rng(0x1100)
    ctx.reset()
    kc, vc = [], []
    for l in range(L):
        rows = OCFG.cache_rows(l)
        n = min(rows, pos)
        k = np.zeros((rows, KS), np.float32)
        v = np.zeros((rows, KS), np.float32)
        k[:n] = rng.standard_normal((n, KS), dtype=np.float32)
        v[:n] = rng.standard_normal((n, KS), dtype=np.float32)
        ctx.kv_write(l, 0, k[:n], v[:n])
        kc.append(k)
        vc.append(v)
    token = 123457
    got = ctx.forward_token(token, pos)
    print("[full model] gpu forward at pos 1100 done; oracle forward", flush=True)
    want, _ = O.forward_cached(OCFG, H, I, [token], pos, embed, layers, norm, kc, vc, threads=THREADS)
    err = rel_err(got, want[0])
    print(f"[full forward] pos {pos} on a pre-filled cache: logits rel_err={err:.3e}", flush=True)
    assert err < 1e-4
    assert int(np.argmax(got)) == int(np.argmax(want[0]))


def test_batched_prefill_vs_oracle(model):
    """g3attn_prefill_tokens over 192 tokens (the batched path) and the
    decode step after it, against the oracle's sequential forward."""
    ctx, embed, layers, norm = model
    n = 192
    tokens = (np.arange(n + 1, dtype=np.int64) * 104729 % (V - 2) + 2).astype(np.int32)
    ctx.reset()
    batched = ctx.prefill_tokens(tokens[:n])
    batched_next = ctx.forward_token(int(tokens[n]), n)
    print("[full model] gpu batched prefill done; oracle forward over 193 tokens", flush=True)
    want, _ = O.forward_cached(OCFG, H, I, tokens, 0, embed, layers, norm, n_logits=2, threads=THREADS)
    e1, e2 = rel_err(batched, want[0]), rel_err(batched_next, want[1])
    print(f"[full prefill] N={n} vs oracle: last logits rel_err={e1:.3e}; next decode rel_err={e2:.3e}",
          flush=True)
    assert e1 < 1e-3 and e2 < 1e-3
    assert int(np.argmax(batched)) == int(np.argmax(want[0]))
    assert int(np.argmax(batched_next)) == int(np.argmax(want[1]))


def test_batched_prefill_2048_vs_token_loop(model):
    ctx, _, _, _ = model
    n = 2048
    tokens = (np.arange(n + 1, dtype=np.int64) * 7919 % (V - 2) + 2).astype(np.int32)
    ctx.reset()
    loop = None
    for i in range(n):
        last = ctx.forward_token(int(tokens[i]), i, compute_logits=(i == n - 1))
        if i == n - 1:
            loop = last
    loop_next = ctx.forward_token(int(tokens[n]), n)
    ctx.reset()
    batched = ctx.prefill_tokens(tokens[:n])
    batched_next = ctx.forward_token(int(tokens[n]), n)
    e1, e2 = rel_err(batched, loop), rel_err(batched_next, loop_next)
    print(f"[full prefill] N={n}: last logits rel_err={e1:.3e}; next decode rel_err={e2:.3e}", flush=True)
    assert e1 < 1e-3 and e2 < 1e-3
    assert int(np.argmax(batched)) == int(np.argmax(loop))
    assert int(np.argmax(batched_next)) == int(np.argmax(loop_next))
