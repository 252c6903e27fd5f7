"""The bf16 GEMV on the GPU (the projections on either side of the attention
block) against the oracle and the reference's golden vectors.

gemma3_matvec_bf16 (gemma3_kernels.c:188-238) sums in fp32 in its own order;
the GPU sums the same products in a different order, so the bar is an fp32
accumulation bound per row, K * 2^-24 * sum_k |a_k x_k| (the closed-form pin
in test_oracle.py holds the oracle to the same bound against fp64).  The last
test runs the whole of layer_attention (gemma3_transformer.c:258-356) on the
GPU, Q/K/V GEMVs -> attention -> o_proj, against the reference's own output.
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


def _bound(A, x):
    Af = (A.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return A.shape[1] * 2.0 ** -24 * (np.abs(Af) @ np.abs(x.astype(np.float64))) + 1e-30


def _check(y, want, A, x, label):
    err = np.abs(y.astype(np.float64) - want)
    ratio = float(np.max(err / _bound(A, x)))
    print(f"[matvec {label}] M={A.shape[0]} K={A.shape[1]} max err / bound = {ratio:.3f}", flush=True)
    assert np.all(np.isfinite(y))
    assert ratio <= 1.0, label


@pytest.mark.parametrize("name", list(MG.MATVEC_SHAPES))
def test_matvec_matches_reference_golden(name):
    g = np.load(os.path.join(GOLD, "matvec.npz"), allow_pickle=False)
    A, x = MG.matvec_case(name)
    assert [np.uint64(O.fnv1a64(A)), np.uint64(O.fnv1a64(x))] == list(g[f"{name}_in_hash"])
    y = G.matvec_bf16(A, x)
    _check(y, g[f"{name}_y"].astype(np.float64), A, x, name)


@pytest.mark.parametrize("M,K", [(1, 1), (3, 7), (64, 8), (65, 16), (37, 1000), (5, 2565),
                                 (9, 2048), (300, 4096), (2560, 10240), (7, 8200), (3, 16392),
                                 (20000, 512), (16385, 2560)])
def test_matvec_shapes(M, K):
    """Vector path (K % 8 == 0), scalar path (ragged K), one and two rows per
    wave (the launch switches at 16384 rows), one round of 4 chunks (K <=
    2048), long rows with x in LDS (8192 <= K <= 16384, here with a partial
    last round) and past the LDS limit."""
    rng = np.random.default_rng(M * 131 + K)
    A = MG.weights_bf16(M, K, 0xA000 + M + K)
    x = rng.standard_normal(K).astype(np.float32)
    _check(G.matvec_bf16(A, x), O.matvec_bf16(A, x).astype(np.float64), A, x, f"{M}x{K}")


def test_matvec_device_unaligned_and_qkv():
    """Device-pointer entry points: an A that is not 16-byte aligned takes
    the scalar path; the fused Q/K/V launch equals three separate GEMVs."""
    with G.Context(G.default_config(max_context=1024, num_layers=6), 1024) as ctx:
        M, K = 96, 2560
        A = MG.weights_bf16(M + 1, K, 0xB100)
        x = O.gen_normal_bf16(K, 0xB200)
        dA, dx, dy = DeviceBuffer.of(A), DeviceBuffer.of(x), DeviceBuffer(M * 4)
        # element 1 onwards, read as M rows of K - 1: 2 bytes past a 16-byte boundary
        ctx.matvec_bf16_device(dy.ptr, dA.ptr + 2, dx.ptr, M, K - 1)
        ctx.synchronize()
        Au = A.reshape(-1)[1:1 + M * (K - 1)].reshape(M, K - 1)
        _check(dy.download(np.float32, M), O.matvec_bf16(Au, x[:K - 1]).astype(np.float64), Au,
               x[:K - 1], "unaligned")

        cfg = ctx.cfg
        hidden = cfg.hidden_size
        ws = [MG.weights_bf16(cfg.num_heads * 256, hidden, 0x9100),
              MG.weights_bf16(cfg.num_kv_heads * 256, hidden, 0x9200),
              MG.weights_bf16(cfg.num_kv_heads * 256, hidden, 0x9300)]
        xh = O.gen_normal_bf16(hidden, 0xB300)
        dw = [DeviceBuffer.of(w) for w in ws]
        dxh = DeviceBuffer.of(xh)
        outs = [DeviceBuffer(w.shape[0] * 4) for w in ws]
        ctx.qkv_proj_device(dxh.ptr, *[w.ptr for w in dw], *[o.ptr for o in outs])
        ctx.synchronize()
        for w, o, n in zip(ws, outs, "qkv"):
            _check(o.download(np.float32, w.shape[0]), O.matvec_bf16(w, xh).astype(np.float64), w, xh,
                   f"qkv-{n}")


@pytest.mark.parametrize("name", ["la_g", "la_l"])
def test_layer_attention_on_gpu_matches_reference_golden(name):
    """x -> g3attn_qkv_proj_device -> g3attn_decode_device ->
    g3attn_matvec_bf16_device(wo): the whole of layer_attention on the GPU,
    against the reference's layer_attention output (fp32 path, bar 1e-4 x RMS)."""
    g = np.load(os.path.join(GOLD, "matvec.npz"), allow_pickle=False)
    layer, pos = (int(v) for v in g[f"{name}_meta"])
    cfg, table, x, wq, wk, wv, wo, Kc, Vc = MG.layer_attention_case(layer, pos)
    hs = g[f"{name}_in_hash"]
    assert [hs[0], hs[5]] == [np.uint64(O.fnv1a64(x)), np.uint64(O.fnv1a64(Vc))]
    with G.Context(G.default_config(max_context=8192), 8192,
                   O.rope_table(8192, 10000.0), O.rope_table(8192, 1e6)) as ctx:
        ctx.kv_write(layer, 0, Kc, Vc)
        dx, dwq, dwk, dwv, dwo = (DeviceBuffer.of(a) for a in (x, wq, wk, wv, wo))
        zn = DeviceBuffer.of(np.zeros(256, np.uint16))
        q, k, v = DeviceBuffer(2048 * 4), DeviceBuffer(1024 * 4), DeviceBuffer(1024 * 4)
        attn, out = DeviceBuffer(2048 * 4), DeviceBuffer(x.size * 4)
        ctx.qkv_proj_device(dx.ptr, dwq.ptr, dwk.ptr, dwv.ptr, q.ptr, k.ptr, v.ptr)
        ctx.decode_device(layer, pos, q.ptr, k.ptr, v.ptr, zn.ptr, zn.ptr, attn.ptr)
        ctx.matvec_bf16_device(out.ptr, dwo.ptr, attn.ptr, x.size, 2048)
        ctx.synchronize()
        got = out.download(np.float32, x.size)
    err = rel_err(got, g[f"{name}_y"])
    print(f"[layer_attention {name}] layer={layer} pos={pos} rel_err={err:.3e}", flush=True)
    assert err < 1e-4


def test_layer_attention_single_entry_point():
    """g3attn_layer_attention_device (the four launches in one call) equals
    the three-call chain above, bit for bit, and the reference's output."""
    g = np.load(os.path.join(GOLD, "matvec.npz"), allow_pickle=False)
    layer, pos = (int(v) for v in g["la_g_meta"])
    cfg, table, x, wq, wk, wv, wo, Kc, Vc = MG.layer_attention_case(layer, pos)
    with G.Context(G.default_config(max_context=8192), 8192,
                   O.rope_table(8192, 10000.0), O.rope_table(8192, 1e6)) as ctx:
        ctx.kv_write(layer, 0, Kc, Vc)
        dx, dwq, dwk, dwv, dwo = (DeviceBuffer.of(a) for a in (x, wq, wk, wv, wo))
        zn = DeviceBuffer.of(np.zeros(256, np.uint16))
        out = DeviceBuffer(x.size * 4)
        ctx.layer_attention_device(layer, pos, dx.ptr, dwq.ptr, dwk.ptr, dwv.ptr, dwo.ptr, zn.ptr,
                                   zn.ptr, out.ptr)
        got = out.download(np.float32, x.size)
    err = rel_err(got, g["la_g_y"])
    print(f"[layer_attention entry] rel_err={err:.3e}", flush=True)
    assert err < 1e-4


def test_weights_rewritten_by_copy():
    """The GEMV streams A with non-temporal loads.  A matrix read by a GEMV,
    then overwritten in place by a host -> device copy, must be read fresh
    by the next GEMV (several rounds, each against its own reference)."""
    with G.Context(G.default_config(max_context=1024, num_layers=6), 1024) as ctx:
        M, K = 2560, 2560
        dA, dx, dy = DeviceBuffer(M * K * 2), DeviceBuffer(K * 4), DeviceBuffer(M * 4)
        x = O.gen_normal_bf16(K, 0xB400)
        dx.upload(x)
        for rnd in range(4):
            A = MG.weights_bf16(M, K, 0xB500 + rnd)
            dA.upload(A)
            ctx.matvec_bf16_device(dy.ptr, dA.ptr, dx.ptr, M, K)
            ctx.synchronize()
            _check(dy.download(np.float32, M), O.matvec_bf16(A, x).astype(np.float64), A, x,
                   f"rewrite-{rnd}")


def test_matvec_errors():
    A = np.zeros((2, 8), np.uint16)
    with pytest.raises(G.G3AttnError):
        G.matvec_bf16(A[:0], np.zeros(8, np.float32))
    with pytest.raises(G.G3AttnError):
        G.matvec_bf16(np.zeros((3, 0), np.uint16), np.zeros(0, np.float32))
    assert np.array_equal(G.matvec_bf16(A, np.ones(8, np.float32)), np.zeros(2, np.float32))
    # long rows take several load rounds
    A = MG.weights_bf16(3, 40968, 0xC100)
    x = O.gen_normal_bf16(40968, 0xC200)
    _check(G.matvec_bf16(A, x), O.matvec_bf16(A, x).astype(np.float64), A, x, "3x40968")
