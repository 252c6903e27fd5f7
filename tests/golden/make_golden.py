#!/usr/bin/env python3
"""Writes the golden fixtures of tests/golden/ from the REAL reference code.

Runs only where oracle/_ref/libg3ref.so was built, i.e. where the reference
sources (robitec97/gemma3.c: gemma3_kernels.c, gemma3_transformer.c) were
present at build time; that library is the reference's own code compiled in
place by oracle/Makefile (never copied).  Inputs come from the oracle's
seeded generator; each fixture stores the FNV-1a hashes of its inputs so
generator drift on another machine is caught before outputs are compared.

    python tests/golden/make_golden.py            # all fixtures
    python tests/golden/make_golden.py --no-big   # skip the configs[3] run (~1-2 min)
    python tests/golden/make_golden.py --only matvec

Fixtures (numpy .npz, allow_pickle=False):
  rope.npz        RoPE table bits: full-table hashes + sampled rows
                  (gemma3_rope_precompute, gemma3_kernels.c:455-468)
  kernels.npz     rmsnorm / rope_apply / softmax / gqa on seeded vectors
                  (gemma3_kernels.c:289-304, 470-484, 396-415, 527-597)
  decode.npz      layer_attention attention section (gemma3_transformer.c:294-352)
                  at configs[0] (local, pos 511) and configs[1] (global, pos 8191)
  prefill.npz     the prefill attention loop (gemma3_transformer.c:641-692):
                  small / chunked / ring-wrap cases, configs[2] and configs[3]:
                  sampled rows + (sum, sum of squares) of every row, and the
                  hashes of the final cache
  matvec.npz      gemma3_matvec_bf16 (gemma3_kernels.c:188-238) at the Q / K /
                  O projection shapes and ragged ones, and the whole of
                  layer_attention (gemma3_transformer.c:258-356, x -> Q/K/V
                  GEMVs -> attention -> o_proj) on seeded bf16 weights
"""
from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
import g3_oracle as O  # noqa: E402

QS, KS = 2048, 1024


def h64(a) -> np.uint64:
    return np.uint64(O.fnv1a64(np.ascontiguousarray(a)))


def rope_fixture():
    out = {}
    for L in (8192, 131072):
        for theta in (10000.0, 1e6):
            t = O.rope_table(L, theta, use_ref=True)
            tag = f"{L}_{int(theta)}"
            out[f"hash_{tag}"] = h64(t)
            rows = [p for p in (0, 1, 2, 511, 1023, 4097, 8191, 65536, 131071) if p < L]
            out[f"rows_{tag}"] = np.array(rows, np.int32)
            out[f"bits_{tag}"] = t.reshape(L, 256)[rows].view(np.uint32).copy()
    return out


def kernels_fixture():
    out = {}
    x = O.gen_normal_bf16(4 * 256, 0x60D1).reshape(4, 256)   # small enough to store
    w = np.stack([np.zeros(256, np.uint16),
                  (np.arange(256) * 37 % 200 + 0x3C00).astype(np.uint16)])
    out["rms_x"], out["rms_w"] = x, w
    out["rms_y"] = np.stack([O.rmsnorm_bf16(x[i], w[j], use_ref=True) for i in range(4) for j in range(2)])
    t = O.rope_table(8192, 1e6, use_ref=True)
    pos = np.array([0, 1, 300, 8191], np.int32)
    out["rope_pos"] = pos
    out["rope_y"] = np.stack([O.rope_apply(x[i], t, int(pos[i]), use_ref=True) for i in range(4)])
    sm = [O.gen_normal_bf16(n, 0x60D2 + n) * 4 for n in (1, 17, 1000)]
    for i, v in enumerate(sm):
        out[f"softmax_x{i}"] = v
        out[f"softmax_y{i}"] = O.softmax(v, use_ref=True)
    for name, (hq, hkv, L, masked) in {"g1": (8, 4, 1, False), "g2": (8, 4, 17, False),
                                       "g3": (8, 4, 300, True), "g4": (4, 4, 129, False),
                                       "g5": (8, 2, 64, True)}.items():
        q = O.gen_normal_bf16(hq * 256, 0x6100 + L)
        k = O.gen_normal_bf16(L * hkv * 256, 0x6200 + L)
        v = O.gen_normal_bf16(L * hkv * 256, 0x6300 + L)
        mask = None
        if masked:
            mask = np.zeros(L, np.float32)
            mask[::5] = -np.inf
            mask[1::3] = -1.5
        # inputs are regenerated from the seeds (0x6100 / 0x6200 / 0x6300 + L)
        out[f"gqa_{name}_shape"] = np.array([hq, hkv, L, int(masked)], np.int32)
        out[f"gqa_{name}_in_hash"] = np.array([h64(q), h64(k), h64(v)], np.uint64)
        out[f"gqa_{name}_y"] = O.gqa(q, k, v, hq, hkv, L, mask=mask, use_ref=True)
    return out


def decode_case(config, layer, pos, max_context):
    """Inputs of one decode step; the cache holds normed + RoPE'd keys of the
    earlier positions the layer keeps (reference cache layout)."""
    cfg = O.Config(max_context=max_context)
    table = O.rope_table(max_context, cfg.theta(layer), use_ref=True)
    is_g = O.is_global_layer(layer)
    lo = 0 if is_g else max(0, pos - cfg.sliding_window)
    n = pos - lo
    K = O.gen_normal_bf16(n * KS, O.seed_for(config, 2), lo * KS).reshape(n, KS)
    V = O.gen_normal_bf16(n * KS, O.seed_for(config, 3), lo * KS).reshape(n, KS)
    zn = O.zero_norm()
    O.norm_rope_batch(K.reshape(n, 4, 256), table, lo, zn)
    rows = cfg.cache_rows(layer)
    Kc = np.zeros((rows, KS), np.float32)
    Vc = np.zeros((rows, KS), np.float32)
    slots = np.arange(lo, pos) if is_g else np.arange(lo, pos) % cfg.sliding_window
    Kc[slots], Vc[slots] = K, V
    q = O.gen_normal_bf16(QS, O.seed_for(config, 1))
    k = O.gen_normal_bf16(KS, O.seed_for(config, 2), pos * KS)
    v = O.gen_normal_bf16(KS, O.seed_for(config, 3), pos * KS)
    return cfg, table, q, k, v, Kc, Vc, zn


def decode_fixture():
    out = {}
    for name, (config, layer, pos, mc) in {"c1": (1, 0, 511, 8192), "c2": (2, 5, 8191, 8192),
                                           "ring": (8, 0, 1500, 8192)}.items():
        cfg, table, q, k, v, Kc, Vc, zn = decode_case(config, layer, pos, mc)
        out[f"{name}_in_hash"] = np.array([h64(q), h64(k), h64(v), h64(Kc), h64(Vc)], np.uint64)
        out[f"{name}_meta"] = np.array([config, layer, pos, mc], np.int32)
        o, q_rot, k_rot = O.ref_layer_decode(cfg, layer, pos, q, k, v, Kc, Vc, table, zn, zn)
        out[f"{name}_out"], out[f"{name}_q_rot"], out[f"{name}_k_rot"] = o, q_rot, k_rot
    return out


def prefill_inputs(config, start, n, layer, max_context=8192):
    cfg = O.Config(max_context=max_context)
    table = O.rope_table(max_context, cfg.theta(layer), use_ref=True)
    s = lambda t: O.seed_for(config, t)
    Q = O.gen_normal_bf16(n * QS, s(1), start * QS).reshape(n, QS)
    K = O.gen_normal_bf16(n * KS, s(2), start * KS).reshape(n, KS)
    V = O.gen_normal_bf16(n * KS, s(3), start * KS).reshape(n, KS)
    rows = cfg.cache_rows(layer)
    Kc = np.zeros((rows, KS), np.float32)
    Vc = np.zeros((rows, KS), np.float32)
    is_g = O.is_global_layer(layer)
    lo = 0 if is_g else max(0, start - cfg.sliding_window)
    if start > lo:
        hK = O.gen_normal_bf16((start - lo) * KS, s(2), lo * KS).reshape(-1, KS)
        hV = O.gen_normal_bf16((start - lo) * KS, s(3), lo * KS).reshape(-1, KS)
        O.norm_rope_batch(hK.reshape(-1, 4, 256), table, lo, O.zero_norm())
        p = np.arange(lo, start)
        sl = p if is_g else p % cfg.sliding_window
        Kc[sl], Vc[sl] = hK, hV
    return cfg, table, Q, K, V, Kc, Vc


def row_sums(out):
    o = out.astype(np.float64)
    return np.stack([o.sum(1), (o * o).sum(1)], 1)


def prefill_fixture(big: bool):
    out = {}
    cases = {"small_g": (40, 0, 64, 5), "chunk_g": (41, 100, 50, 11),
             "chunk_l": (42, 1000, 80, 0), "wrap_l": (43, 1500, 40, 3),
             "c3": (3, 0, 2048, 0)}
    if big:
        cases["c4"] = (4, 0, 8192, 5)
    for name, (config, start, n, layer) in cases.items():
        t0 = time.time()
        cfg, table, Q, K, V, Kc, Vc = prefill_inputs(config, start, n, layer)
        out[f"{name}_meta"] = np.array([config, start, n, layer], np.int32)
        out[f"{name}_in_hash"] = np.array([h64(Q), h64(K), h64(V), h64(Kc), h64(Vc)], np.uint64)
        zn = O.zero_norm()
        o, _, _ = O.ref_prefill(cfg, layer, start, Q, K, V, Kc, Vc, table, zn, zn)
        rows = np.unique(np.concatenate([np.arange(0, min(n, 3)),
                                         np.linspace(0, n - 1, 6).astype(int)]))
        out[f"{name}_rows"] = rows.astype(np.int32)
        out[f"{name}_out_rows"] = o[rows]
        out[f"{name}_row_sums"] = row_sums(o)
        out[f"{name}_cache_hash"] = np.array([h64(Kc), h64(Vc)], np.uint64)
        print(f"  prefill {name}: {time.time() - t0:.1f} s", flush=True)
    return out


def weights_bf16(M, K, seed):
    """Seeded N(0,1) bf16 weights scaled by 2^-6 (exact in bf16), as uint16 bits."""
    a = (O.gen_normal_bf16(M * K, seed) * np.float32(2.0 ** -6)).astype(np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16).reshape(M, K)


MATVEC_SHAPES = {"q": (2048, 2560), "kv": (1024, 2560), "o": (2560, 2048),
                 "r1": (37, 1000), "r2": (5, 2565), "r3": (1, 1)}


def matvec_case(name):
    M, K = MATVEC_SHAPES[name]
    return weights_bf16(M, K, 0x9000 + M + 7 * K), O.gen_normal_bf16(K, 0x9800 + K)


def layer_attention_case(layer, pos, hidden=2560):
    """Inputs of one full layer_attention call: x, the four projection
    matrices and a cache holding positions the layer keeps before pos."""
    cfg = O.Config(max_context=8192)
    wq, wk, wv = (weights_bf16(r, hidden, s) for r, s in ((2048, 0x9100), (1024, 0x9200), (1024, 0x9300)))
    wo = weights_bf16(hidden, 2048, 0x9400)
    x = O.gen_normal_bf16(hidden, 0x9500 + pos)
    table = O.rope_table(8192, cfg.theta(layer), use_ref=True)
    is_g = O.is_global_layer(layer)
    lo = 0 if is_g else max(0, pos - cfg.sliding_window)
    n = pos - lo
    K = O.gen_normal_bf16(n * KS, 0x9600, lo * KS).reshape(n, KS)
    V = O.gen_normal_bf16(n * KS, 0x9700, lo * KS).reshape(n, KS)
    O.norm_rope_batch(K.reshape(n, 4, 256), table, lo, O.zero_norm())
    rows = cfg.cache_rows(layer)
    Kc = np.zeros((rows, KS), np.float32)
    Vc = np.zeros((rows, KS), np.float32)
    slots = np.arange(lo, pos) if is_g else np.arange(lo, pos) % cfg.sliding_window
    Kc[slots], Vc[slots] = K, V
    return cfg, table, x, wq, wk, wv, wo, Kc, Vc


def matvec_fixture():
    out = {}
    for name in MATVEC_SHAPES:
        A, x = matvec_case(name)
        out[f"{name}_in_hash"] = np.array([h64(A), h64(x)], np.uint64)
        out[f"{name}_y"] = O.matvec_bf16(A, x, use_ref=True)
    for name, (layer, pos) in {"la_g": (5, 1000), "la_l": (0, 1500)}.items():
        cfg, table, x, wq, wk, wv, wo, Kc, Vc = layer_attention_case(layer, pos)
        out[f"{name}_meta"] = np.array([layer, pos], np.int32)
        out[f"{name}_in_hash"] = np.array([h64(x), h64(wq), h64(wk), h64(wv), h64(wo), h64(Vc)], np.uint64)
        zn = O.zero_norm()
        out[f"{name}_y"] = O.layer_attention(cfg, layer, pos, x, wq, wk, wv, wo, Kc, Vc, table, zn, zn,
                                             use_ref=True)
    return out


# A small model of Gemma 3's structure for the whole-token forward: 6 layers
# (layer 5 global), 8 query / 4 KV heads of 256, a 16-row sliding window that
# the 40-token sequence wraps.  Layer 3 drops its optional norms (q_norm,
# k_norm, post-attention, pre- and post-feedforward), which the reference
# skips when NULL.
FORWARD = dict(hidden=512, inter=1536, vocab=1024, n=40, layers=6, max_context=64, window=16)
FORWARD_ROWS = (0, 5, 15, 16, 17, 31, 39)   # the logits rows kept in the fixture


def norm_bf16(n, seed):
    """Small per-channel RMSNorm weights w (gain 1 + w): N(0,1) * 2^-3 in bf16."""
    a = (O.gen_normal_bf16(n, seed) * np.float32(0.125)).astype(np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def forward_case(heads=8, kv_heads=4, **over):
    """The forward fixture's model (FORWARD, with overrides); other head
    counts give a model of the same structure for shape tests (the fixture
    itself is the default 8 / 4)."""
    f = dict(FORWARD, **over)
    H, I, V, L = f["hidden"], f["inter"], f["vocab"], f["layers"]
    cfg = O.Config(num_layers=L, max_context=f["max_context"], sliding_window=f["window"], num_heads=heads,
                   num_kv_heads=kv_heads)
    qs, ks = cfg.num_heads * 256, cfg.num_kv_heads * 256
    embed = weights_bf16(V, H, 0xF000)
    layers = []
    for l in range(L):
        s = 0xF100 + 32 * l
        lw = dict(input_layernorm=norm_bf16(H, s), q_proj=weights_bf16(qs, H, s + 1),
                  k_proj=weights_bf16(ks, H, s + 2), v_proj=weights_bf16(ks, H, s + 3),
                  o_proj=weights_bf16(H, qs, s + 4), q_norm=norm_bf16(256, s + 5),
                  k_norm=norm_bf16(256, s + 6), post_attention_layernorm=norm_bf16(H, s + 7),
                  gate_proj=weights_bf16(I, H, s + 8), up_proj=weights_bf16(I, H, s + 9),
                  down_proj=weights_bf16(H, I, s + 10), pre_feedforward_layernorm=norm_bf16(H, s + 11),
                  post_feedforward_layernorm=norm_bf16(H, s + 12))
        if l == 3:
            for k in ("q_norm", "k_norm", "post_attention_layernorm", "pre_feedforward_layernorm",
                      "post_feedforward_layernorm"):
                lw[k] = None
        layers.append(lw)
    norm = norm_bf16(H, 0xFF00)
    tokens = np.random.default_rng(0xF0F0).integers(0, V, f["n"]).astype(np.int32)
    return cfg, f, embed, layers, norm, tokens


def forward_hash(embed, layers, norm, tokens):
    parts = [h64(embed), h64(norm), h64(tokens)]
    for lw in layers:
        parts += [h64(a) if a is not None else np.uint64(0) for a in (lw[k] for k in O.LAYER_TENSORS)]
    return np.array(parts, np.uint64)


def forward_fixture():
    cfg, f, embed, layers, norm, tokens = forward_case()
    logits, hid = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm, use_ref=True)
    return {"in_hash": forward_hash(embed, layers, norm, tokens),
            "rows": np.array(FORWARD_ROWS, np.int32), "logits": logits[list(FORWARD_ROWS)],
            "argmax": logits.argmax(axis=1).astype(np.int32), "hidden": hid}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--no-big", action="store_true")
    ap.add_argument("--only", default="", help="comma list of fixtures to write (default: all)")
    args = ap.parse_args()
    if not O.have_ref():
        sys.exit("oracle/_ref/libg3ref.so is not built (needs /root/reference at build time)")
    ap_only = set(filter(None, args.only.split(",")))
    for name, fn in (("rope", rope_fixture), ("kernels", kernels_fixture), ("decode", decode_fixture),
                     ("prefill", lambda: prefill_fixture(not args.no_big)), ("matvec", matvec_fixture),
                     ("forward", forward_fixture)):
        if ap_only and name not in ap_only:
            continue
        t0 = time.time()
        data = fn()
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **data)
        print(f"{name}.npz: {len(data)} arrays, {time.time() - t0:.1f} s", flush=True)


if __name__ == "__main__":
    main()
