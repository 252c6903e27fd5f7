"""Pins of the CPU oracle (oracle/g3_oracle.c), the checker of the HIP path.

Three kinds of pin, chosen so that a plausible mistake (a dropped term, a
wrong sign or index, a transposed operand, an off-by-one window) fails one:

* golden vectors written by the reference's own code compiled in place
  (tests/golden/make_golden.py -> *.npz), compared after checking that the
  oracle's generator reproduces the fixture inputs bit for bit;
* known answers and closed forms that need no reference: splitmix64's
  published first output, bf16 rounding, RoPE identity / norm preservation /
  angle additivity, softmax of one dominant key, uniform attention = mean,
  fp64 brute force on tiny inputs, permutation invariance of the ring;
* mutation checks: deliberately wrong restatements (numpy, CPU only) must
  fail the same pins the oracle passes.

The reference has no tests or fixtures of its own (it ships no test suite),
so these are the only pins; the reference-run comparisons against
oracle/_ref are skipped where that library is absent (e.g. the GPU box).
"""
import os

import numpy as np
import pytest

from helpers import O, REPO, g3attn

GOLD = os.path.join(REPO, "tests", "golden")
QS, KS = 2048, 1024


def gold(name):
    return np.load(os.path.join(GOLD, f"{name}.npz"), allow_pickle=False)


def h64(a):
    return np.uint64(O.fnv1a64(np.ascontiguousarray(a)))


def rel(a, b):
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(np.asarray(a, np.float64) - b)) / np.sqrt(np.mean(b * b)))


# ---------------------------------------------------------------- generator

def test_splitmix64_known_answer():
    # first output of SplitMix64 seeded with 0 (Steele, Lea, Flood 2014)
    assert O.lib().g3o_splitmix64(0, 0) == 0xE220A8397B1DCDAF


def test_bf16_conversions():
    L = O.lib()
    assert L.g3o_f32_to_bf16_rne(1.0) == 0x3F80
    assert L.g3o_f32_to_bf16_rne(np.float32(1.0 + 2 ** -8)) == 0x3F80      # tie -> even
    assert L.g3o_f32_to_bf16_rne(np.float32(1.0 + 3 * 2 ** -8)) == 0x3F82  # tie -> even (up)
    assert L.g3o_f32_to_bf16_trunc(np.float32(1.0 + 3 * 2 ** -8)) == 0x3F81  # reference truncates
    assert L.g3o_bf16_to_f32(0xC040) == -3.0


def test_generator_statistics_and_bf16_exactness():
    x = O.gen_normal_bf16(200000, 1234)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01
    bits = x.view(np.uint32)
    assert np.all(bits & 0xFFFF == 0)                       # bf16-valued
    # counter-indexed: any window of the stream equals the same slice
    assert np.array_equal(O.gen_normal_bf16(100, 1234, first=777), x[777:877])


# ---------------------------------------------------------------- RoPE table

@pytest.mark.parametrize("L,theta", [(8192, 10000.0), (8192, 1e6), (131072, 10000.0), (131072, 1e6)])
def test_rope_table_matches_reference_bits(L, theta):
    g = gold("rope")
    tag = f"{L}_{int(theta)}"
    t = O.rope_table(L, theta)
    assert np.array_equal(t.reshape(L, 256)[g[f"rows_{tag}"]].view(np.uint32), g[f"bits_{tag}"])
    assert h64(t) == g[f"hash_{tag}"]
    # the product library's host table is the same bits (it is what gets uploaded)
    assert h64(g3attn().rope_precompute(L, theta)) == g[f"hash_{tag}"]


def test_rope_table_closed_form():
    # cos / sin of pos * theta^(-2i/d).  Only small positions: a 1-ulp powf
    # difference in freq grows into pos * ulp of angle error, which is why the
    # bit-exact check above is against the reference's own table.
    t = O.rope_table(32, 1e6).reshape(32, 128, 2).astype(np.float64)
    i = np.arange(128)
    ang = np.arange(32)[:, None] * np.power(1e6, -2.0 * i / 256)[None]
    assert np.max(np.abs(t[..., 0] - np.cos(ang))) < 4e-6
    assert np.max(np.abs(t[..., 1] - np.sin(ang))) < 4e-6
    assert np.all(t[0, :, 0] == 1.0) and np.all(t[0, :, 1] == 0.0)     # pos 0 is the identity


def test_rope_apply_invariants():
    t = O.rope_table(2048, 1e4)
    x = O.gen_normal_bf16(256, 99)
    assert np.array_equal(O.rope_apply(x, t, 0), x)
    for pos in (1, 77, 2047):
        y = O.rope_apply(x, t, pos).astype(np.float64)
        n0 = x[:128].astype(np.float64) ** 2 + x[128:].astype(np.float64) ** 2
        n1 = y[:128] ** 2 + y[128:] ** 2
        assert np.max(np.abs(n1 - n0) / n0.clip(1e-6)) < 1e-5
    # angle additivity: R(a) R(b) = R(a + b), exact-arithmetic rotation in fp64
    def rot(v, p):
        c, s = t.reshape(-1, 128, 2)[p, :, 0].astype(np.float64), t.reshape(-1, 128, 2)[p, :, 1].astype(np.float64)
        a, b = v[:128], v[128:]
        return np.concatenate([a * c - b * s, a * s + b * c])
    x64 = x.astype(np.float64)
    assert np.max(np.abs(rot(rot(x64, 300), 200) - rot(x64, 500))) < 1e-4
    # NeoX half split: dim i pairs with i + 128 (not i + 1)
    e = np.zeros(256, np.float32)
    e[0] = 1.0
    y = O.rope_apply(e, t, 5)
    assert y[128] != 0 and y[1] == 0


# ---------------------------------------------------------------- small kernels

def test_kernels_match_reference_golden():
    g = gold("kernels")
    x, w = g["rms_x"], g["rms_w"]
    y = np.stack([O.rmsnorm_bf16(x[i], w[j]) for i in range(4) for j in range(2)])
    assert np.max(np.abs(y - g["rms_y"])) < 1e-6
    t = O.rope_table(8192, 1e6)
    y = np.stack([O.rope_apply(x[i], t, int(g["rope_pos"][i])) for i in range(4)])
    assert np.max(np.abs(y - g["rope_y"])) < 1e-6
    for i, n in enumerate((1, 17, 1000)):
        assert np.max(np.abs(O.softmax(g[f"softmax_x{i}"]) - g[f"softmax_y{i}"])) < 1e-7
    for name in ("g1", "g2", "g3", "g4", "g5"):
        hq, hkv, L, masked = (int(v) for v in g[f"gqa_{name}_shape"])
        q = O.gen_normal_bf16(hq * 256, 0x6100 + L)
        k = O.gen_normal_bf16(L * hkv * 256, 0x6200 + L)
        v = O.gen_normal_bf16(L * hkv * 256, 0x6300 + L)
        assert np.array_equal(g[f"gqa_{name}_in_hash"], [h64(q), h64(k), h64(v)])
        mask = None
        if masked:
            mask = np.zeros(L, np.float32)
            mask[::5] = -np.inf
            mask[1::3] = -1.5
        assert rel(O.gqa(q, k, v, hq, hkv, L, mask=mask), g[f"gqa_{name}_y"]) < 1e-6


def test_rmsnorm_closed_form():
    x = O.gen_normal_bf16(256, 5) * 3
    y = O.rmsnorm_bf16(x, O.zero_norm()).astype(np.float64)
    ms = np.mean(x.astype(np.float64) ** 2)
    assert abs(np.sqrt(np.mean(y * y)) - np.sqrt(ms / (ms + 1e-6))) < 1e-6
    assert np.max(np.abs(y - x / np.sqrt(ms + 1e-6))) < 1e-5
    w = np.full(256, 0x3F80, np.uint16)                      # w = 1 -> gain 2
    assert np.max(np.abs(O.rmsnorm_bf16(x, w) - 2 * y)) < 1e-5


def test_softmax_properties():
    x = O.gen_normal_bf16(500, 8) * 5
    p = O.softmax(x).astype(np.float64)
    assert abs(p.sum() - 1) < 1e-5 and np.argmax(p) == np.argmax(x)
    assert np.max(np.abs(O.softmax(x + 100) - p)) < 1e-6      # shift invariance
    e = np.zeros(7, np.float32)
    e[3] = 200
    assert np.allclose(O.softmax(e), np.eye(7)[3])


def _gqa64(q, k, v, hq, hkv, L, scale=0.0625, mask=None):
    q = q.reshape(hq, 256).astype(np.float64)
    k = k.reshape(L, hkv, 256).astype(np.float64)
    v = v.reshape(L, hkv, 256).astype(np.float64)
    out = np.empty((hq, 256))
    for h in range(hq):
        kv = h // (hq // hkv)
        s = k[:, kv] @ q[h] * scale + (0 if mask is None else mask)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[:, kv]
    return out.reshape(-1)


GQA_CASES = [(8, 4, 1), (8, 4, 9), (8, 4, 40), (4, 4, 33), (8, 2, 20)]


def _pin_gqa(gqa_impl):
    """Closed-form pins of gemma3_gqa; returns the list of failed pins."""
    failed = []
    for hq, hkv, L in GQA_CASES:
        q = O.gen_normal_bf16(hq * 256, 11 + L)
        k = O.gen_normal_bf16(L * hkv * 256, 12 + L)
        v = O.gen_normal_bf16(L * hkv * 256, 13 + L)
        if rel(gqa_impl(q, k, v, hq, hkv, L), _gqa64(q, k, v, hq, hkv, L)) > 1e-5:
            failed.append(f"brute-force {hq}/{hkv}/{L}")
        # seq_len 1: output = v_0 of each head's kv head
        o1 = gqa_impl(q, k[: hkv * 256], v[: hkv * 256], hq, hkv, 1).reshape(hq, 256)
        want = v[: hkv * 256].reshape(hkv, 256)[np.arange(hq) // (hq // hkv)]
        if np.max(np.abs(o1 - want)) > 1e-6:
            failed.append("seq_len-1")
        # k = 0: uniform weights -> mean of v
        o0 = gqa_impl(q, np.zeros_like(k), v, hq, hkv, L).reshape(hq, 256)
        mean = v.reshape(L, hkv, 256).mean(0)[np.arange(hq) // (hq // hkv)]
        if np.max(np.abs(o0 - mean)) > 1e-5:
            failed.append("uniform")
        # one dominant key j: output -> v_j
        j = L // 2
        kd = np.zeros_like(k).reshape(L, hkv, 256)
        for h in range(hq):
            kd[j, h // (hq // hkv)] = 40 * q.reshape(hq, 256)[h] / np.linalg.norm(q.reshape(hq, 256)[h])
        if hq == hkv or hq // hkv == 1:
            od = gqa_impl(q, kd.reshape(-1), v, hq, hkv, L).reshape(hq, 256)
            if np.max(np.abs(od - v.reshape(L, hkv, 256)[j][np.arange(hq)])) > 1e-3:
                failed.append("dominant")
        # permutation of keys (ring order) does not change the result
        perm = np.random.default_rng(L).permutation(L)
        kp = k.reshape(L, -1)[perm].reshape(-1)
        vp = v.reshape(L, -1)[perm].reshape(-1)
        if rel(gqa_impl(q, kp, vp, hq, hkv, L), gqa_impl(q, k, v, hq, hkv, L)) > 1e-5:
            failed.append("permutation")
    # query heads 2k and 2k+1 with equal q give equal outputs
    q = O.gen_normal_bf16(4 * 256, 21)
    q2 = np.repeat(q.reshape(4, 256), 2, axis=0).reshape(-1)
    k = O.gen_normal_bf16(30 * 4 * 256, 22)
    v = O.gen_normal_bf16(30 * 4 * 256, 23)
    o = gqa_impl(q2, k, v, 8, 4, 30).reshape(8, 256)
    if np.max(np.abs(o[0::2] - o[1::2])) > 0:
        failed.append("group-pairs")
    return failed


def test_gqa_closed_forms():
    assert _pin_gqa(lambda q, k, v, hq, hkv, L: O.gqa(q, k, v, hq, hkv, L)) == []


# ---------------------------------------------------------------- mutation checks

def _rope_np(x, table, pos, sign=1.0):
    row = table.reshape(-1, 128, 2)[pos]
    a, b = x[:128].astype(np.float64), x[128:].astype(np.float64)
    c, s = row[:, 0], sign * row[:, 1]
    return np.concatenate([a * c - b * s, a * s + b * c]).astype(np.float32)


def test_mutants_fail_the_pins():
    """Plausible mistakes, restated in numpy on the CPU, are caught."""
    # GQA with the kv head taken as h % n_kv instead of h / group
    def gqa_wrong_head(q, k, v, hq, hkv, L):
        out = []
        for h in range(hq):
            kv = h % hkv
            qh = q.reshape(hq, 256)[h].astype(np.float64)
            kk = k.reshape(L, hkv, 256)[:, kv].astype(np.float64)
            vv = v.reshape(L, hkv, 256)[:, kv].astype(np.float64)
            s = kk @ qh * 0.0625
            p = np.exp(s - s.max())
            out.append((p / p.sum()) @ vv)
        return np.concatenate(out).astype(np.float32)
    assert _pin_gqa(gqa_wrong_head)
    # GQA that forgets the 1/sqrt(d) scale
    assert _pin_gqa(lambda q, k, v, hq, hkv, L: _gqa64(q, k, v, hq, hkv, L, scale=1.0).astype(np.float32))
    # RoPE with the sign of sin flipped: fails the reference golden rows
    g = gold("kernels")
    t = O.rope_table(8192, 1e6)
    bad = np.stack([_rope_np(g["rms_x"][i], t, int(g["rope_pos"][i]), sign=-1) for i in range(4)])
    good = np.stack([_rope_np(g["rms_x"][i], t, int(g["rope_pos"][i])) for i in range(4)])
    assert np.max(np.abs(good - g["rope_y"])) < 1e-5
    assert np.max(np.abs(bad - g["rope_y"])) > 1e-2
    # RMSNorm that drops the (1 + w) gain's 1: fails the golden with nonzero w
    x, w = g["rms_x"][0].astype(np.float64), g["rms_w"][1]
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    r = 1 / np.sqrt(np.mean(x * x) + 1e-6)
    assert np.max(np.abs(x * r * (1 + wf) - g["rms_y"][1])) < 1e-5
    assert np.max(np.abs(x * r * wf - g["rms_y"][1])) > 1e-1


def test_window_off_by_one_is_caught():
    """Local layer at pos >= window attends exactly the last `window` positions:
    one key more or less changes the output (the pin the decode test uses)."""
    cfg = O.Config(max_context=2048)
    t = O.rope_table(2048, 1e4)
    W, pos = 1024, 1500
    K = O.gen_normal_bf16((pos + 1) * KS, 31).reshape(pos + 1, KS)
    V = O.gen_normal_bf16((pos + 1) * KS, 32).reshape(pos + 1, KS)
    O.norm_rope_batch(K.reshape(-1, 4, 256), t, 0, O.zero_norm())
    q = O.gen_normal_bf16(QS, 33)
    qr = q.copy()
    O.norm_rope_batch(qr.reshape(1, 8, 256), t, pos, O.zero_norm())
    Kc = np.zeros((W, KS), np.float32)
    Vc = np.zeros((W, KS), np.float32)
    p = np.arange(pos - W + 1, pos)
    Kc[p % W], Vc[p % W] = K[p], V[p]
    raw_k = O.gen_normal_bf16((pos + 1) * KS, 31).reshape(pos + 1, KS)[pos]
    got, _, _ = O.layer_decode(cfg, 0, pos, q, raw_k, V[pos], Kc, Vc, t, O.zero_norm(), O.zero_norm())
    right = O.gqa(qr, K[pos - W + 1: pos + 1], V[pos - W + 1: pos + 1], 8, 4, W)
    one_more = O.gqa(qr, K[pos - W: pos + 1], V[pos - W: pos + 1], 8, 4, W + 1)
    assert rel(got, right) < 1e-5
    assert rel(one_more, right) > 1e-4


# ---------------------------------------------------------------- decode / prefill goldens

def test_layer_decode_matches_reference_golden():
    g = gold("decode")
    import importlib.util, sys
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLD, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    for name in ("c1", "c2", "ring"):
        config, layer, pos, mc = (int(v) for v in g[f"{name}_meta"])
        cfg, table, q, k, v, Kc, Vc, zn = mg.decode_case(config, layer, pos, mc)
        table = O.rope_table(mc, cfg.theta(layer))   # the oracle's own table
        assert np.array_equal(g[f"{name}_in_hash"], [h64(q), h64(k), h64(v), h64(Kc), h64(Vc)])
        out, q_rot, k_rot = O.layer_decode(cfg, layer, pos, q, k, v, Kc, Vc, table, zn, zn)
        assert rel(q_rot, g[f"{name}_q_rot"]) < 1e-6
        assert rel(k_rot, g[f"{name}_k_rot"]) < 1e-6
        assert rel(out, g[f"{name}_out"]) < 1e-5, name


def _prefill_golden_case(name, threads):
    g = gold("prefill")
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLD, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    config, start, n, layer = (int(v) for v in g[f"{name}_meta"])
    cfg, table, Q, K, V, Kc, Vc = mg.prefill_inputs(config, start, n, layer)
    table = O.rope_table(8192, cfg.theta(layer))
    assert np.array_equal(g[f"{name}_in_hash"], [h64(Q), h64(K), h64(V), h64(Kc), h64(Vc)])
    zn = O.zero_norm()
    out, _, _ = O.prefill(cfg, layer, start, Q, K, V, Kc, Vc, table, zn, zn, threads=threads)
    rows = g[f"{name}_rows"]
    assert rel(out[rows], g[f"{name}_out_rows"]) < 1e-5, name
    sums = np.stack([out.astype(np.float64).sum(1), (out.astype(np.float64) ** 2).sum(1)], 1)
    assert np.max(np.abs(sums - g[f"{name}_row_sums"])) < 1e-4, name
    assert np.array_equal(g[f"{name}_cache_hash"], [h64(Kc), h64(Vc)]), name


@pytest.mark.parametrize("name", ["small_g", "chunk_g", "chunk_l", "wrap_l", "c3"])
def test_prefill_matches_reference_golden(name):
    _prefill_golden_case(name, threads=1 if name != "c3" else 0)


@pytest.mark.slow
def test_prefill_config4_matches_reference_golden():
    _prefill_golden_case("c4", threads=0)


def test_parallel_prefill_is_bit_identical_to_sequential():
    cfg = O.Config(max_context=2048)
    for layer, start, n in ((5, 0, 300), (0, 900, 400), (3, 0, 1300)):
        t = O.rope_table(2048, cfg.theta(layer))
        Q = O.gen_normal_bf16(n * QS, 50 + layer).reshape(n, QS)
        K = O.gen_normal_bf16(n * KS, 60 + layer).reshape(n, KS)
        V = O.gen_normal_bf16(n * KS, 70 + layer).reshape(n, KS)
        rows = cfg.cache_rows(layer)
        Hk = O.gen_normal_bf16(rows * KS, 80).reshape(rows, KS)
        Kc1, Vc1 = Hk.copy(), -Hk
        Kc2, Vc2 = Hk.copy(), -Hk
        zn = O.zero_norm()
        a, _, _ = O.prefill(cfg, layer, start, Q, K, V, Kc1, Vc1, t, zn, zn, threads=1)
        b, _, _ = O.prefill(cfg, layer, start, Q, K, V, Kc2, Vc2, t, zn, zn, threads=7)
        assert np.array_equal(a, b) and np.array_equal(Kc1, Kc2) and np.array_equal(Vc1, Vc2)


# ---------------------------------------------------------------- oracle vs reference, live

ref_only = pytest.mark.skipif(not O.have_ref(), reason="oracle/_ref not built on this machine")


@ref_only
def test_restatement_equals_reference_build_random():
    rng = np.random.default_rng(7)
    t_ref = O.rope_table(4096, 1e4, use_ref=True)
    t = O.rope_table(4096, 1e4)
    assert np.array_equal(t.view(np.uint32), t_ref.view(np.uint32))
    for _ in range(5):
        L = int(rng.integers(1, 700))
        q = O.gen_normal_bf16(QS, int(rng.integers(1 << 30)))
        k = O.gen_normal_bf16(L * KS, int(rng.integers(1 << 30)))
        v = O.gen_normal_bf16(L * KS, int(rng.integers(1 << 30)))
        assert rel(O.gqa(q, k, v, 8, 4, L), O.gqa(q, k, v, 8, 4, L, use_ref=True)) < 1e-6
    cfg = O.Config(max_context=2048)
    for layer, start, n in ((5, 0, 50), (2, 1020, 30)):
        tt = O.rope_table(2048, cfg.theta(layer))
        Q = O.gen_normal_bf16(n * QS, 91).reshape(n, QS)
        K = O.gen_normal_bf16(n * KS, 92).reshape(n, KS)
        V = O.gen_normal_bf16(n * KS, 93).reshape(n, KS)
        rows = cfg.cache_rows(layer)
        Kc1 = O.gen_normal_bf16(rows * KS, 94).reshape(rows, KS)
        Vc1 = O.gen_normal_bf16(rows * KS, 95).reshape(rows, KS)
        Kc2, Vc2 = Kc1.copy(), Vc1.copy()
        zn = O.zero_norm()
        a, _, _ = O.prefill(cfg, layer, start, Q, K, V, Kc1, Vc1, tt, zn, zn)
        b, _, _ = O.ref_prefill(cfg, layer, start, Q, K, V, Kc2, Vc2, tt, zn, zn)
        # same operation order; -ffast-math may vectorise the two builds'
        # reductions differently, so agreement is to fp32 rounding, not bits
        assert rel(a, b) < 1e-5
        assert rel(Kc1, Kc2) < 1e-6 and np.array_equal(Vc1, Vc2)


# ---------------------------------------------------------------- GEMV (next row: the projections)

def _mg():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLD, "make_golden.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def _bf16_f64(A):
    return (A.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _matvec_bound(A, x):
    """fp32 accumulation error bound per row: K * 2^-24 * sum |a_k x_k|."""
    K = A.shape[1]
    return K * 2.0 ** -24 * (np.abs(_bf16_f64(A)) @ np.abs(x.astype(np.float64))) + 1e-30


def test_matvec_closed_form_and_mutants():
    """gemma3_matvec_bf16 against an fp64 dot product on every shape class
    (vector blocks of 16, a block of 8, scalar tails); a transposed operand, a
    truncated row or a dropped tail fails the same bound."""
    rng = np.random.default_rng(7)
    for M, K in ((3, 1), (2, 7), (4, 8), (5, 16), (3, 24), (6, 37), (9, 1000), (2, 2565)):
        A = (rng.integers(0x3B00, 0x3F00, size=(M, K)) | (rng.integers(0, 2, size=(M, K)) << 15)).astype(np.uint16)
        x = rng.standard_normal(K).astype(np.float32)
        y = O.matvec_bf16(A, x)
        y64 = _bf16_f64(A) @ x.astype(np.float64)
        assert np.all(np.abs(y - y64) <= _matvec_bound(A, x)), (M, K)
        if K > 1:
            wrong_tail = _bf16_f64(A[:, :-1]) @ x[:-1].astype(np.float64)
            assert np.any(np.abs(y - wrong_tail) > _matvec_bound(A, x)), (M, K)
        if M == K or M > 1:
            shuffled = _bf16_f64(A[::-1]) @ x.astype(np.float64)
            assert np.any(np.abs(y - shuffled) > _matvec_bound(A, x)), (M, K)
    A = (rng.integers(0x3B00, 0x3F00, size=(8, 8))).astype(np.uint16)
    x = rng.standard_normal(8).astype(np.float32)
    assert np.any(np.abs(O.matvec_bf16(A, x) - _bf16_f64(A.T) @ x) > _matvec_bound(A, x))


def test_matvec_matches_reference_golden():
    MG = _mg()
    g = gold("matvec")
    for name in MG.MATVEC_SHAPES:
        A, x = MG.matvec_case(name)
        assert [h64(A), h64(x)] == list(g[f"{name}_in_hash"])
        y = O.matvec_bf16(A, x)
        # the reference's fast build reassociates its lane sums; a few ulps of each row's sum
        assert np.all(np.abs(y - g[f"{name}_y"]) <= 4 * _matvec_bound(A, x) / A.shape[1] * 16), name


def test_layer_attention_matches_reference_golden():
    """The whole of layer_attention (Q/K/V GEMVs, attention section, o_proj)."""
    MG = _mg()
    g = gold("matvec")
    for name in ("la_g", "la_l"):
        layer, pos = (int(v) for v in g[f"{name}_meta"])
        cfg, table, x, wq, wk, wv, wo, Kc, Vc = MG.layer_attention_case(layer, pos)
        hs = g[f"{name}_in_hash"]
        assert [hs[0], hs[1], hs[2], hs[3], hs[4], hs[5]] == [h64(x), h64(wq), h64(wk), h64(wv), h64(wo), h64(Vc)]
        zn = O.zero_norm()
        y = O.layer_attention(cfg, layer, pos, x, wq, wk, wv, wo, Kc, Vc, O.rope_table(8192, cfg.theta(layer)), zn, zn)
        assert rel(y, g[f"{name}_y"]) < 1e-5, name


@pytest.mark.skipif(not O.have_ref(), reason="oracle/_ref not built (no reference sources)")
def test_matvec_restatement_equals_reference_build_random():
    rng = np.random.default_rng(11)
    for M, K in ((7, 2560), (5, 2048), (3, 10240), (4, 33)):
        # random bf16 bit patterns: any sign and mantissa, exponents 2^-20 .. 2^12
        A = ((rng.integers(0, 2, size=(M, K)) << 15) | (rng.integers(107, 140, size=(M, K)) << 7)
             | rng.integers(0, 128, size=(M, K))).astype(np.uint16)
        x = rng.standard_normal(K).astype(np.float32)
        y, yr = O.matvec_bf16(A, x), O.matvec_bf16(A, x, use_ref=True)
        assert np.all(np.abs(y - yr) <= 4 * _matvec_bound(A, x) / K * 16), (M, K)


# ---------------------------------------------------------------- token forward

def _gelu64(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def test_gelu_known_values_and_odd_identity():
    """gemma3_gelu_tanh_inplace: gelu(0) = 0; gelu(x) - gelu(-x) = x exactly in
    real arithmetic (0.5x(1 + t) + 0.5x(1 - t)); the tanh form's published
    values at 1 and -1 (0.8411920, -0.1588080); gelu -> x and -> 0 in the tails."""
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    y = O.gelu_tanh(x).astype(np.float64)
    assert O.gelu_tanh(np.zeros(1, np.float32))[0] == 0.0
    neg = O.gelu_tanh(-x).astype(np.float64)
    assert np.all(np.abs((y - neg) - x) <= 2e-6 * np.maximum(1.0, np.abs(x)))
    g1 = O.gelu_tanh(np.array([1.0, -1.0], np.float32))
    assert abs(g1[0] - 0.8411920) < 1e-6 and abs(g1[1] + 0.1588080) < 1e-6
    assert np.all(np.abs(y - _gelu64(x.astype(np.float64))) <= 1e-6 * np.maximum(1.0, np.abs(x)))
    assert abs(y[-1] - 8.0) < 1e-6 and abs(y[0]) < 1e-6
    # the exact-erf GELU and SiLU differ by far more than the bound above
    silu = x / (1 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(y - silu)) > 1e-2


def _bf64(a):
    return (np.asarray(a).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _forward_pos0_64(cfg, f, embed, layers, norm, token, mutant=None):
    """fp64 forward of the first token (position 0): every attention softmax
    is over one row, so each head's output is its KV head's V row and neither
    RoPE nor the QK norms enter.  What is left pins the embedding scale, the
    (1 + w) norms, the residual structure, the GQA head map, the gelu(gate) *
    up MLP and the tied logits; ``mutant`` names one plausible mistake."""
    H = f["hidden"]
    E = _bf64(embed).reshape(-1, H)

    def rms(x, w):
        gain = _bf64(w) if mutant == "gain_w" else 1.0 + _bf64(w)
        return x / np.sqrt((x * x).mean() + 1e-6) * gain

    x = E[token] * (1.0 if mutant == "no_embed_scale" else np.sqrt(H))
    G = cfg.num_heads // cfg.num_kv_heads
    for lw in layers:
        xn = rms(x, lw["input_layernorm"])
        v = (_bf64(lw["v_proj"]) @ xn).reshape(cfg.num_kv_heads, 256)
        kv = [h % cfg.num_kv_heads if mutant == "head_map" else h // G for h in range(cfg.num_heads)]
        proj = _bf64(lw["o_proj"]) @ v[kv].reshape(-1)
        if lw["post_attention_layernorm"] is not None and mutant != "no_post_attn":
            proj = rms(proj, lw["post_attention_layernorm"])
        x = x + proj
        xn = rms(x, lw["pre_feedforward_layernorm"]) if lw["pre_feedforward_layernorm"] is not None else x
        gate, up = _bf64(lw["gate_proj"]) @ xn, _bf64(lw["up_proj"]) @ xn
        h = gate * _gelu64(up) if mutant == "gelu_on_up" else _gelu64(gate) * up
        mlp = _bf64(lw["down_proj"]) @ h
        if lw["post_feedforward_layernorm"] is not None:
            mlp = rms(mlp, lw["post_feedforward_layernorm"])
        x = x + mlp
    return E @ rms(x, norm), x


def test_forward_first_token_closed_form_and_mutants():
    MG = _mg()
    cfg, f, embed, layers, norm, tokens = MG.forward_case(n=1)
    logits, hid = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm)
    want, xw = _forward_pos0_64(cfg, f, embed, layers, norm, int(tokens[0]))
    scale = np.sqrt((want ** 2).mean())
    bar = 2e-5 * scale
    assert np.max(np.abs(logits[0] - want)) <= bar
    assert np.max(np.abs(hid - xw)) <= 2e-5 * np.sqrt((xw ** 2).mean())
    for m in ("gain_w", "no_embed_scale", "head_map", "no_post_attn", "gelu_on_up"):
        wm, _ = _forward_pos0_64(cfg, f, embed, layers, norm, int(tokens[0]), mutant=m)
        assert np.max(np.abs(logits[0] - wm)) > 100 * bar, m


def test_forward_matches_reference_golden():
    """gemma3_transformer_forward over 40 tokens of a 6-layer model (window 16,
    so the local layers' ring wraps; layer 3 without its optional norms)."""
    MG = _mg()
    g = gold("forward")
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    assert list(MG.forward_hash(embed, layers, norm, tokens)) == list(g["in_hash"])
    logits, hid = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm)
    assert rel(logits[list(g["rows"])], g["logits"]) < 1e-5
    assert rel(hid, g["hidden"]) < 1e-5
    assert np.array_equal(logits.argmax(axis=1), g["argmax"])


@pytest.mark.skipif(not O.have_ref(), reason="oracle/_ref not built (no reference sources)")
def test_forward_restatement_equals_reference_build_random():
    MG = _mg()
    cfg, f, embed, layers, norm, tokens = MG.forward_case(hidden=768, inter=1024, vocab=512, n=21,
                                                          window=8, max_context=32)
    a = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm)
    b = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm, use_ref=True)
    assert rel(a[0], b[0]) < 1e-5 and rel(a[1], b[1]) < 1e-5


def test_forward_cached_is_the_same_forward():
    """g3o_forward_cached (the forward from caller-owned caches, GEMV rows over
    a thread pool) against g3o_forward_seq on the forward fixture's model:
    one call from empty caches with 4 threads gives the same bits for every
    token's logits; 40 tokens as 25 + 15 in two calls on the same caches
    give the same last two logits rows (the cache state carries over, ring
    wrapped), and the caches hold what the sequential run's cache_kv writes."""
    MG = _mg()
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    want, hid = O.forward_seq(cfg, f["hidden"], f["inter"], tokens, embed, layers, norm)
    got, hid2 = O.forward_cached(cfg, f["hidden"], f["inter"], tokens, 0, embed, layers, norm,
                                 n_logits=len(tokens), threads=4)
    assert np.array_equal(got, want) and np.array_equal(hid, hid2)
    ks = cfg.num_kv_heads * 256
    kc = [np.zeros((cfg.cache_rows(l), ks), np.float32) for l in range(cfg.num_layers)]
    vc = [np.zeros_like(a) for a in kc]
    O.forward_cached(cfg, f["hidden"], f["inter"], tokens[:25], 0, embed, layers, norm, kc, vc, threads=3)
    last, _ = O.forward_cached(cfg, f["hidden"], f["inter"], tokens[25:], 25, embed, layers, norm, kc, vc,
                               n_logits=2, threads=2)
    assert np.array_equal(last, want[-2:])
    assert np.any(kc[0] != 0) and np.any(vc[5][: len(tokens)] != 0)
