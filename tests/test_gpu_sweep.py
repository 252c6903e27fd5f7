"""Randomised sessions on the GPU against the oracle: breadth over the
combinations the targeted tests pick one at a time.

Each seed draws a head layout (GQA group 1, 2 or 4), a sliding window (1, 7,
32, 64, 100 or 1024), a max_context (1536, or 1000: not a multiple of the
64-key staging grain), and, for half the seeds, the library's own RoPE tables
instead of the oracle's, and then drives one local and one global layer of a
context
through a random sequence of calls from position 0: prefill chunks of 1 to
200 tokens (chunks longer than the window, chunks whose history wraps the
ring) and runs of 1 to 3 decode steps.  Every call draws bf16-valued or
fp32 inputs and non-unit bf16 QK-norm gains or none.  The oracle's caches
carry the same state from call to call (g3o_prefill / g3o_layer_decode,
restating gemma3_transformer.c:641-692 and :294-352), every output is
compared (prefill: 2e-3 x RMS, the path's bar; decode: 1e-4 x RMS), and at
the end so is every cache row (cache_kv, :236-251: K within 1e-5 x RMS,
V exact).  The seeds are fixed, so a failure names its case.
"""
import numpy as np
import pytest

from helpers import O, TOL, g3attn, rel_err

pytestmark = pytest.mark.gpu

G = g3attn()
D = 256


def _bf16(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).view(np.float32)


def _gain(rng):
    return (_bf16(rng.standard_normal(D) * 0.3).view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("seed", range(40))
def test_random_session(seed):
    rng = np.random.default_rng(0x5EED00 + seed)
    heads, kv_heads = [(8, 4), (4, 4), (8, 2)][seed % 3]
    window = [32, 64, 1024, 1, 7, 100][(seed // 3) % 6]
    MAXC = 1000 if seed % 2 else 1536
    cfg_o = O.Config(max_context=MAXC, sliding_window=window, num_heads=heads, num_kv_heads=kv_heads)
    tables = {False: O.rope_table(MAXC, 10000.0), True: O.rope_table(MAXC, 1e6)}
    cfg = G.default_config(max_context=MAXC, sliding_window=window, num_layers=6, num_heads=heads,
                           num_kv_heads=kv_heads)
    qs, ks = heads * D, kv_heads * D
    worst = {"prefill": 0.0, "decode": 0.0}
    n_calls = 0
    # half the seeds run on the library's own RoPE tables
    # (g3attn_rope_precompute, built with the reference's fast-mode flags);
    # the oracle keeps its restatement of gemma3_rope_precompute
    own_tables = seed % 4 >= 2
    with (G.Context(cfg, MAXC) if own_tables else G.Context(cfg, MAXC, tables[False], tables[True])) as ctx:
        for layer in (1, 5):
            is_global = O.is_global_layer(layer)
            table = tables[is_global]
            rows = cfg_o.cache_rows(layer)
            Kc = np.zeros((rows, ks), np.float32)
            Vc = np.zeros((rows, ks), np.float32)
            pos = 0
            limit = int(rng.integers(300, 900))   # < MAXC
            while pos < limit:
                fp32 = rng.random() < 0.3
                conv = (lambda a: a.astype(np.float32)) if fp32 else _bf16
                gq, gk = (_gain(rng), _gain(rng)) if rng.random() < 0.7 else (None, None)
                if rng.random() < 0.5:
                    n = int(min(rng.integers(1, 201), MAXC - pos))
                    Q = conv(rng.standard_normal((n, qs)))
                    K = conv(rng.standard_normal((n, ks)))
                    V = conv(rng.standard_normal((n, ks)))
                    got = ctx.prefill(layer, pos, Q, K, V, gq, gk)
                    want, _, _ = O.prefill(cfg_o, layer, pos, Q, K, V, Kc, Vc, table, gq, gk, threads=16)
                    err = rel_err(got, want)
                    label = f"prefill layer={layer} start={pos} n={n} fp32={fp32} norm={gq is not None}"
                    assert err <= TOL, (seed, label, err)
                    worst["prefill"] = max(worst["prefill"], err)
                    pos += n
                    n_calls += 1
                else:
                    for _ in range(int(rng.integers(1, 4))):
                        q = conv(rng.standard_normal(qs))
                        k = conv(rng.standard_normal(ks))
                        v = conv(rng.standard_normal(ks))
                        got = ctx.decode(layer, pos, q, k, v, gq, gk)
                        want, _, _ = O.layer_decode(cfg_o, layer, pos, q, k, v, Kc, Vc, table, gq, gk)
                        err = rel_err(got, want)
                        label = f"decode layer={layer} pos={pos} fp32={fp32} norm={gq is not None}"
                        assert err <= 1e-4, (seed, label, err)
                        worst["decode"] = max(worst["decode"], err)
                        pos += 1
                        n_calls += 1
            # every cache row the session wrote
            used = min(pos, rows)
            k_got, v_got = ctx.kv_read(layer, 0, used)
            assert rel_err(k_got, Kc[:used]) < 1e-5, (seed, layer)
            assert np.array_equal(v_got, Vc[:used]), (seed, layer)
    print(f"[sweep seed={seed}] heads={heads}/{kv_heads} window={window} max_context={MAXC} own_tables={own_tables} calls={n_calls} "
          f"worst prefill={worst['prefill']:.2e} decode={worst['decode']:.2e}", flush=True)
