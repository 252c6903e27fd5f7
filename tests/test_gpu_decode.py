"""Decode parity on the GPU: libg3attn.so (C-ABI) against the CPU oracle.

Each case builds the same seeded inputs for both sides (tests/helpers.py),
runs one decode step of one layer through g3attn_decode and compares with
the oracle's restatement of layer_attention (gemma3_transformer.c:294-352).
Bar: max-abs error <= 2e-3 x output RMS; decode is
fp32 end to end, so it is also held to 1e-4.
"""
import numpy as np
import pytest

from helpers import HKV, KS, QS, TOL, DecodeCase, O, g3attn, rel_err

pytestmark = pytest.mark.gpu

G = g3attn()
FP32_BAR = 1e-4


def _ctx(max_context, window=1024, num_layers=34, n_heads=8, n_kv=4):
    cfg = G.default_config(max_context=max_context, sliding_window=window, num_layers=num_layers,
                           num_heads=n_heads, num_kv_heads=n_kv)
    return G.Context(cfg, max_context,
                     O.rope_table(max_context, 10000.0), O.rope_table(max_context, 1e6))


@pytest.fixture(scope="module")
def ctx8k():
    c = _ctx(8192)
    yield c
    c.close()


def _check(case, ctx, label):
    want, Kc, Vc = case.oracle()
    case.load_gpu(ctx)
    got = case.gpu(ctx)
    err = rel_err(got, want)
    print(f"[{label}] layer={case.layer} pos={case.pos} rel_err={err:.3e}", flush=True)
    assert np.all(np.isfinite(got))
    assert err <= TOL and err <= FP32_BAR, err
    # the new row landed in the right slot, normed + RoPE'd like the oracle's
    slot = case.pos if case.is_global else case.pos % case.cfg.sliding_window
    k_gpu, v_gpu = ctx.kv_read(case.layer, slot, 1)
    assert rel_err(k_gpu[0], Kc[slot]) < 1e-5
    assert np.array_equal(v_gpu[0], Vc[slot])
    return err


def test_config1_local_decode(ctx8k):
    """local layer, pos 511, L = 512 inside the window."""
    _check(DecodeCase(1, layer=0, pos=511, max_context=8192), ctx8k, "config1")


def test_cache_rewritten_by_copy(ctx8k):
    """Cache rows that a decode has read, then rewritten through
    g3attn_kv_write (a host -> device copy into staging, then the scatter
    kernel into the cache), are read back fresh by the next decode: two
    different histories in the same slots, each against its own oracle."""
    for layer_seed in (0, 7, 0):
        _check(DecodeCase(1, layer=11, pos=700, max_context=8192, layer_seed=layer_seed), ctx8k,
               f"rewrite-{layer_seed}")


def test_config2_global_decode(ctx8k):
    """global layer, pos 8191, L = 8192."""
    _check(DecodeCase(2, layer=5, pos=8191, max_context=8192), ctx8k, "config2")


@pytest.mark.timeout(600)   # ~1 minute, mostly the host building 5 GiB of seeded history
def test_config5_stack_128k():
    """configs[4] in full: one decode step at pos 131071 through all 34 layers
    of one context (29 local layers over their 1024-slot rings, 5 global
    layers over 131072 cached positions, 5 GiB of fp32 K/V), each layer with
    its own data, against the oracle."""
    ctx = _ctx(131072)
    try:
        worst = 0.0
        for layer in range(34):
            case = DecodeCase(5, layer=layer, pos=131071, max_context=131072, layer_seed=layer + 1)
            worst = max(worst, _check(case, ctx, f"stack-{layer}"))
            del case
        print(f"[stack128k] 34 layers, worst rel_err={worst:.3e}", flush=True)
    finally:
        ctx.close()


def test_global_decode_128k():
    """configs[4]'s global layer at full size: pos 131071 over 131072 cached
    positions (1 GiB of fp32 K/V; 1024-row splits), against the oracle."""
    ctx = _ctx(131072, num_layers=6)
    try:
        _check(DecodeCase(5, layer=5, pos=131071, max_context=131072), ctx, "128k")
    finally:
        ctx.close()


@pytest.mark.parametrize("pos", [0, 1, 63, 64, 65, 1023])
def test_short_positions(ctx8k, pos):
    _check(DecodeCase(7, layer=5, pos=pos, max_context=8192), ctx8k, "short-global")
    _check(DecodeCase(7, layer=2, pos=pos, max_context=8192), ctx8k, "short-local")


@pytest.mark.parametrize("pos", [1024, 1025, 1500, 2047, 5000])
def test_local_ring_wrap(ctx8k, pos):
    """pos >= window: the ring holds exactly positions pos-1023..pos."""
    _check(DecodeCase(8, layer=0, pos=pos, max_context=8192), ctx8k, "ring")


@pytest.mark.parametrize("n_heads,n_kv", [(4, 4), (8, 2)])
def test_decode_gqa_groups(n_heads, n_kv):
    """The fused decode at GQA groups 1 and 4 (the configs use 2): a local
    layer inside the window and across the ring wrap, a global layer, with
    and without QK-norm."""
    ctx = _ctx(4096, num_layers=6, n_heads=n_heads, n_kv=n_kv)
    try:
        for layer, pos, norm in ((0, 700, True), (1, 2500, True), (5, 3000, True), (5, 999, False)):
            case = DecodeCase(12, layer=layer, pos=pos, max_context=4096, norm=norm,
                              n_heads=n_heads, n_kv=n_kv)
            _check(case, ctx, f"group{n_heads // n_kv}")
    finally:
        ctx.close()


def test_load_forms_agree(monkeypatch):
    """The cache-policy modes of the fused decode (G3ATTN_DECODE_NT: 0 plain
    loads, 1 non-temporal buffer loads on every layer, 2 the default, plain
    on local layers) change how K/V rows are fetched, never what is
    computed: outputs and cache rows are bit-identical across the modes, and
    each matches the oracle.  Local layers inside the window and across the
    ring wrap, a global layer, groups 2 and 4."""
    for n_heads, n_kv in ((8, 4), (8, 2)):
        outs = {}
        for mode in (0, 1, 2):
            monkeypatch.setenv("G3ATTN_DECODE_NT", str(mode))
            ctx = _ctx(4096, num_layers=6, n_heads=n_heads, n_kv=n_kv)
            try:
                got = []
                for layer, pos in ((0, 700), (1, 2500), (5, 3000)):
                    case = DecodeCase(14, layer=layer, pos=pos, max_context=4096, n_heads=n_heads, n_kv=n_kv)
                    _check(case, ctx, f"nt{mode}")
                    got.append(case.gpu(ctx))   # again, on the cache the first call completed
                    got.append(np.concatenate(ctx.kv_read(layer, 0, 64)))
                outs[mode] = got
            finally:
                ctx.close()
        for mode in (1, 2):
            for a, b in zip(outs[0], outs[mode]):
                assert np.array_equal(a, b), (n_heads, n_kv, mode)


def test_one_launch_merge(monkeypatch):
    """Splits merged inside the decode kernel, on each run's XCD, by the last
    workgroup to arrive (the default for local layers wherever the placement
    probe at create passes, as on MI355X), against the two-launch form
    (G3ATTN_DECODE_XMERGE=0) and the oracle: configs[0]'s 16 splits, full
    rings of 32 splits, a short global layer admitted by
    G3ATTN_DECODE_XMERGE=2 (10 splits), each decoded twice on one context
    (the arrival counters are back at zero after every launch), groups 2 and
    4, and group 2 over 8 KV heads (whole groups per workgroup).  The forms
    differ only in the order of the split merge: fp32 sums of
    up to 32 weighted partials, a few ulp apart (1.2e-6 x RMS seen; bar
    1e-5, against the decode's 1e-4)."""
    for n_heads, n_kv in ((8, 4), (8, 2), (16, 8)):
        outs = {}
        for mode in ("0", "1", "2"):
            monkeypatch.setenv("G3ATTN_DECODE_XMERGE", mode)
            ctx = _ctx(4096, num_layers=6, n_heads=n_heads, n_kv=n_kv)
            try:
                got = []
                for layer, pos in ((0, 511), (1, 2500), (2, 4095), (5, 300)):
                    case = DecodeCase(16, layer=layer, pos=pos, max_context=4096, n_heads=n_heads, n_kv=n_kv)
                    _check(case, ctx, f"xm{mode}")
                    one_launch = mode == "2" or (mode == "1" and not case.is_global)
                    heads_per_wg = 2 if n_kv == 8 else 1
                    assert ctx.last_splits(2) == (heads_per_wg if one_launch else 0), (mode, layer)
                    assert ctx.last_splits(0) > 1
                    got.append(case.gpu(ctx))   # again: the counters were left at zero
                outs[mode] = got
            finally:
                ctx.close()
        for mode in ("1", "2"):
            for a, b in zip(outs["0"], outs[mode]):
                assert rel_err(b, a) < 1e-5, (n_heads, n_kv, mode)


@pytest.mark.parametrize("env", [{"G3ATTN_SPLIT_ROWS": "1000000"}, {"G3ATTN_SPLIT_ROWS": "32"},
                                 {"G3ATTN_SPLIT_ROWS": "100"}, {"G3ATTN_DECODE_WGS": "8"},
                                 {"G3ATTN_DECODE_WGS": "4000"}, {"G3ATTN_SPLIT_MIN_ROWS": "512"}])
def test_split_settings(monkeypatch, env):
    """The decode's split-shape knobs against the oracle: one split for the
    whole stream (the kernel writes the normalised output itself), 32-row
    splits (clamped at the maximum split count for long streams), a length
    off the 32-row grain, very few and very many workgroups, and a long
    minimum split.  Local layers in and across the ring wrap and global
    layers at 3000 and 8191."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    ctx = _ctx(8192, num_layers=6)
    try:
        for layer, pos in ((0, 700), (1, 2500), (5, 3000), (5, 8191)):
            _check(DecodeCase(15, layer=layer, pos=pos, max_context=8192), ctx, ",".join(env.values()))
    finally:
        ctx.close()


def test_tables_uploaded_after_create():
    """A context created without RoPE tables (the backend hook's init, which
    takes none) refuses attention calls until g3attn_upload_rope, then matches
    the oracle on both layer kinds; tables of the wrong size are refused."""
    cfg = G.default_config(max_context=2048, num_layers=6)
    ctx = G.Context(cfg, 2048, defer_rope=True)
    try:
        q = np.zeros(QS, np.float32)
        k = np.zeros(KS, np.float32)
        assert ctx.decode_rc(0, 5, q, k, k) == G.ERR_INVALID_ARG
        assert "RoPE" in G.last_error()
        tl, tg = O.rope_table(2048, 10000.0), O.rope_table(2048, 1e6)
        with pytest.raises(G.G3AttnError):
            ctx.upload_rope(tl[:1024], tg[:1024], max_context=1024)
        ctx.upload_rope(tl, tg)
        for layer, pos in ((0, 700), (5, 1500)):
            _check(DecodeCase(13, layer=layer, pos=pos, max_context=2048), ctx, "rope-upload")
    finally:
        ctx.close()


def test_no_norm(ctx8k):
    """q_norm = k_norm = NULL skips the QK-norm (gemma3_transformer.c:295)."""
    _check(DecodeCase(9, layer=5, pos=300, max_context=8192, norm=False), ctx8k, "no-norm")


def test_nonzero_norm_weights(ctx8k):
    case = DecodeCase(10, layer=5, pos=777, max_context=8192)
    case.norm = (np.arange(256, dtype=np.uint16) * 37 % 200 + 0x3C00).astype(np.uint16)
    # rebuild cache rows with the non-unit gain
    case.k_rows = case.k_hist.copy()
    O.norm_rope_batch(case.k_rows.reshape(-1, HKV, 256), case.table, case.lo, case.norm)
    _check(case, ctx8k, "gain")


def test_sequential_decode_matches_oracle(ctx8k):
    """20 consecutive decode steps on a local layer across the ring wrap."""
    cfg = O.Config(max_context=8192)
    table = O.rope_table(8192, 10000.0)
    layer, pos0, n = 3, 1010, 20
    case = DecodeCase(11, layer=layer, pos=pos0, max_context=8192)
    Kc, Vc = case.oracle_cache()
    case.load_gpu(ctx8k)
    zn = O.zero_norm()
    for i in range(n):
        pos = pos0 + i
        q = O.gen_normal_bf16(QS, 0xABC0 + i)
        k = O.gen_normal_bf16(KS, 0xBBC0 + i)
        v = O.gen_normal_bf16(KS, 0xCBC0 + i)
        want, _, _ = O.layer_decode(cfg, layer, pos, q, k, v, Kc, Vc, table, zn, zn)
        got = ctx8k.decode(layer, pos, q, k, v, zn, zn)
        assert rel_err(got, want) < FP32_BAR


def test_context_overflow(ctx8k):
    q = np.zeros(QS, np.float32)
    k = np.zeros(KS, np.float32)
    rc = ctx8k.decode_rc(5, 8192, q, k, k)
    assert rc == G.ERR_CONTEXT_OVERFLOW
    assert "max_context" in G.last_error()
    assert ctx8k.decode_rc(99, 0, q, k, k) == G.ERR_INVALID_ARG
    assert ctx8k.decode_rc(5, -1, q, k, k) == G.ERR_INVALID_ARG


def test_kv_append_matches_oracle(ctx8k):
    """Batched K-norm + RoPE + cache write against the oracle's per-token calls."""
    for layer, start, n in ((5, 100, 300), (0, 900, 300), (1, 0, 2500)):
        K = O.gen_normal_bf16(n * KS, 0x1111 + layer).reshape(n, KS)
        V = O.gen_normal_bf16(n * KS, 0x2222 + layer).reshape(n, KS)
        zn = O.zero_norm()
        ctx8k.kv_append(layer, start, K, V, zn)
        table = O.rope_table(8192, 1e6 if O.is_global_layer(layer) else 10000.0)
        Kr = K.copy()
        O.norm_rope_batch(Kr.reshape(n, HKV, 256), table, start, zn)
        W = 1024
        keep = range(n) if O.is_global_layer(layer) else range(max(0, n - W), n)
        for i in keep[:: max(1, len(keep) // 50)]:
            pos = start + i
            slot = pos if O.is_global_layer(layer) else pos % W
            kg, vg = ctx8k.kv_read(layer, slot, 1)
            assert rel_err(kg[0], Kr[i]) < 1e-5, (layer, i)
            assert np.array_equal(vg[0], V[i])


def test_kv_write_read_roundtrip(ctx8k):
    rows = O.gen_normal_bf16(37 * KS, 0x3333).reshape(37, KS)
    ctx8k.kv_write(11, 1000, rows, -rows)
    k, v = ctx8k.kv_read(11, 1000, 37)
    assert np.array_equal(k, rows) and np.array_equal(v, -rows)
    with pytest.raises(G.G3AttnError):
        ctx8k.kv_read(0, 1000, 37)  # local layer has only 1024 rows


@pytest.mark.parametrize("seq_len,n_heads,n_kv", [(1, 8, 4), (17, 8, 4), (513, 8, 4),
                                                 (4096, 8, 4), (300, 4, 4), (300, 8, 2)])
def test_gqa_entry_matches_gemma3_gqa(seq_len, n_heads, n_kv):
    """g3attn_gqa (gemma3_gqa signature) against the restated gemma3_gqa."""
    q = O.gen_normal_bf16(n_heads * 256, 0x4444 + seq_len)
    k = O.gen_normal_bf16(seq_len * n_kv * 256, 0x5555 + seq_len)
    v = O.gen_normal_bf16(seq_len * n_kv * 256, 0x6666 + seq_len)
    want = O.gqa(q, k, v, n_heads, n_kv, seq_len)
    got = G.gqa(q, k, v, n_heads, n_kv, seq_len)
    assert rel_err(got, want) < FP32_BAR


def test_gqa_entry_mask():
    seq_len = 700
    q = O.gen_normal_bf16(QS, 0x7777)
    k = O.gen_normal_bf16(seq_len * KS, 0x7778)
    v = O.gen_normal_bf16(seq_len * KS, 0x7779)
    mask = np.zeros(seq_len, np.float32)
    mask[::3] = -np.inf
    mask[1::7] = -2.5
    want = O.gqa(q, k, v, 8, 4, seq_len, mask=mask)
    got = G.gqa(q, k, v, 8, 4, seq_len, mask=mask)
    assert rel_err(got, want) < FP32_BAR
