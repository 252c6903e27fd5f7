"""The batched-prefill projections on MFMA (g3attn_matmul_bf16_device, the
reference's bf16_matrix_to_f32 + cblas_sgemm pairs, gemma3_transformer.c:
614-639, 694-699, 726-751) and the whole batched prefill
(g3attn_prefill_forward_device, gemma3_transformer_prefill_batched :526-787).

The reference's batched prefill needs cblas.h and cannot be built here; it
computes the same functions as gemma3_transformer_forward token by token (the
same norms, projections, attention and MLP; only the summation order of the
sgemm differs), so its output is pinned by the reference's own forward
(tests/golden/forward.npz).

GEMM bar: fp32 accumulation plus the hi / lo split of X (|x - x_hi - x_lo| <=
2^-17 |x|): |C - C64| <= (2^-16 + K 2^-24) sum_k |w_k x_k| per element, the
split term doubled for margin; and max-abs error <= 5e-5 x the output RMS,
which a dropped x_lo pass (x rounded to bf16 alone: >= 2e-3) fails at every K.
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


def _bf64(a):
    return (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _check_gemm(C, W, X, label):
    Wd, Xd = _bf64(W), X.astype(np.float64)
    want = Xd @ Wd.T
    K = W.shape[1]
    bound = (2.0 ** -16 + K * 2.0 ** -24) * (np.abs(Xd) @ np.abs(Wd).T) + 1e-30
    ratio = float(np.max(np.abs(C - want) / bound))
    print(f"[gemm {label}] N={X.shape[0]} M={W.shape[0]} K={K} max err / bound = {ratio:.3f}", flush=True)
    assert np.all(np.isfinite(C))
    assert ratio <= 1.0, label
    return want


@pytest.mark.parametrize("N,M,K", [(1, 4, 32), (5, 12, 64), (130, 260, 96), (16, 128, 32),
                                   (257, 2048, 2560), (64, 1028, 10240), (300, 4, 32),
                                   (129, 132, 2048), (4096, 4096, 512)])
def test_matmul_matches_fp64(N, M, K):
    """Full and ragged tiles in both dimensions (rows past M or N read zero),
    one K step, the projections' K (hidden 2560, q 2048, intermediate 10240),
    and a launch large enough for the 256-row tiles (>= 512 workgroups).
    Split-K (o_proj, down_proj) runs in the batched-prefill tests below."""
    rng = np.random.default_rng(N * 7 + M * 13 + K)
    W = MG.weights_bf16(M, K, 0xE000 + M + K)
    X = rng.standard_normal((N, K)).astype(np.float32)
    with G.Context(G.default_config(max_context=256, num_layers=6), 256) as ctx:
        dW, dX, dC = DeviceBuffer.of(W), DeviceBuffer.of(X), DeviceBuffer(N * M * 4)
        ctx.matmul_bf16_device(dC.ptr, dW.ptr, dX.ptr, N, M, K)
        C = dC.download(np.float32, (N, M)).astype(np.float64)
    want = _check_gemm(C, W, X, f"{N}x{M}x{K}")
    # relative to the output RMS the GPU stays near 2^-17; dropping the x_lo
    # pass (x rounded to bf16 alone, 2^-9) is 20x further off at every K
    Xh = (X.view(np.uint32) + 0x7FFF + ((X.view(np.uint32) >> 16) & 1)) & 0xFFFF0000
    hi_only = Xh.view(np.float32).astype(np.float64) @ _bf64(W).T
    assert rel_err(C, want) < 5e-5
    if N * M >= 64:
        assert rel_err(hi_only, want) > 1e-3


def test_matmul_errors():
    with G.Context(G.default_config(max_context=256, num_layers=6), 256) as ctx:
        d = DeviceBuffer(4096)
        for N, M, K in ((0, 4, 32), (1, 6, 32), (1, 4, 48), (1, 0, 32)):
            with pytest.raises(G.G3AttnError):
                ctx.matmul_bf16_device(d.ptr, d.ptr, d.ptr, N, M, K)


def _gpu_config(f):
    return G.default_config(num_layers=f["layers"], max_context=f["max_context"],
                            sliding_window=f["window"], hidden_size=f["hidden"],
                            intermediate_size=f["inter"], vocab_size=f["vocab"])


def test_batched_prefill_matches_reference_forward():
    """The whole batched prefill of the 40-token golden sequence (window 16:
    the local layers' ring wraps inside the batch; layer 3 without its
    optional norms) gives the reference's last-token logits, in one batch and
    in two chunks (the second attending the first through the cache)."""
    g = np.load(os.path.join(GOLD, "forward.npz"), allow_pickle=False)
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    rows = list(g["rows"])
    HW, keep = G.host_weights(embed, layers, norm)
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        ctx.upload_weights(HW)
        W = ctx.device_weights()
        dl = DeviceBuffer(f["vocab"] * 4)
        ctx.prefill_forward_device(W, tokens, 0, dl.ptr)
        full = dl.download(np.float32, f["vocab"])
        # the same context continues: a decode step after the prefill
        nxt = ctx.forward_token(int(tokens[0]), len(tokens))
    err = rel_err(full, g["logits"][rows.index(39)])
    print(f"[batched prefill] n=40 logits rel={err:.3e}", flush=True)
    assert err < 1e-4 and int(np.argmax(full)) == int(g["argmax"][39])
    with G.Context(_gpu_config(f), f["max_context"]) as ctx:
        ctx.upload_weights(HW)
        W = ctx.device_weights()
        dl = DeviceBuffer(f["vocab"] * 4)
        ctx.prefill_forward_device(W, tokens[:16], 0, dl.ptr)
        first = dl.download(np.float32, f["vocab"])
        ctx.prefill_forward_device(W, tokens[16:], 16, dl.ptr)
        second = dl.download(np.float32, f["vocab"])
        nxt2 = ctx.forward_token(int(tokens[0]), len(tokens))
    assert rel_err(first, g["logits"][rows.index(15)]) < 1e-4
    assert rel_err(second, g["logits"][rows.index(39)]) < 1e-4
    # the cache the batched prefill wrote serves a decode step like the token loop's
    want, _ = O.forward_seq(cfg, f["hidden"], f["inter"], np.append(tokens, tokens[0]), embed, layers, norm)
    assert rel_err(nxt, want[-1]) < 1e-4 and rel_err(nxt2, want[-1]) < 1e-4


def test_prefill_tokens_takes_the_batched_path():
    """g3attn_prefill_tokens with >= G3ATTN_PREFILL_BATCH_MIN tokens agrees with
    the token loop to the fp32 bar (it is not bit-identical: the GEMMs sum in
    another order and carry x as hi + lo)."""
    cfg, f, embed, layers, norm, tokens = MG.forward_case()
    HW, keep = G.host_weights(embed, layers, norm)
    with G.Context(_gpu_config(f), f["max_context"]) as a, G.Context(_gpu_config(f), f["max_context"]) as b:
        a.upload_weights(HW)
        b.upload_weights(HW)
        loop = [a.forward_token(int(t), i) for i, t in enumerate(tokens[:30])][-1]
        batched = b.prefill_tokens(tokens[:30])
        assert rel_err(batched, loop) < 1e-4
        assert not np.array_equal(batched, loop)   # the batched path really ran
        # and both continue identically enough
        assert rel_err(b.forward_token(int(tokens[30]), 30), a.forward_token(int(tokens[30]), 30)) < 1e-4
    print("[prefill_tokens batched] ok", flush=True)
