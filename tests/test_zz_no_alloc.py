"""The allocation-free gemma3_gqa entry point (g3attn_gqa_noalloc) against
the allocating one (g3attn_gqa), through the C ABI on the GPU.

g3attn_gqa_noalloc keeps its split partials in a fixed static device scratch
instead of allocated workspace; it picks the same splits and runs the same
kernels as g3attn_gqa, so the outputs must agree bit for bit (the decode
path's own bar, 1e-4 x output RMS against the oracle, is also checked).
Two calls in a row share the scratch; the second is smaller, so stale
partials of the first would show.
"""
import numpy as np
import pytest

from helpers import DeviceBuffer, O, g3attn, rel_err

pytestmark = pytest.mark.gpu

G = g3attn()
FP32_BAR = 1e-4


def _call(q, k, v, n_heads, n_kv, seq_len, mask=None):
    bufs = [DeviceBuffer.of(q), DeviceBuffer.of(k), DeviceBuffer.of(v)]
    dm = DeviceBuffer.of(mask) if mask is not None else None
    out = DeviceBuffer(n_heads * 256 * 4)
    try:
        G.gqa_noalloc(out.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, n_heads, n_kv, seq_len,
                      mask_ptr=dm.ptr if dm else None)
        return out.download(np.float32, n_heads * 256)
    finally:
        for b in bufs + [out] + ([dm] if dm else []):
            b.free()


def _inputs(seq_len, n_heads, n_kv, seed):
    q = O.gen_normal_bf16(n_heads * 256, seed)
    k = O.gen_normal_bf16(seq_len * n_kv * 256, seed + 1)
    v = O.gen_normal_bf16(seq_len * n_kv * 256, seed + 2)
    return q, k, v


@pytest.mark.parametrize("shapes", [((8192, 8, 4), (700, 8, 4)), ((4096, 16, 4), (33, 4, 4)),
                                    ((3000, 8, 8), (1, 8, 2))])
def test_noalloc_matches_gqa_twice(shapes):
    for i, (seq_len, n_heads, n_kv) in enumerate(shapes):
        q, k, v = _inputs(seq_len, n_heads, n_kv, 0xA110C + 16 * i + seq_len)
        mask = None
        if i == 1 and seq_len > 3:
            mask = np.zeros(seq_len, np.float32)
            mask[::5] = -np.inf
            mask[2::7] = -1.25
        got = _call(q, k, v, n_heads, n_kv, seq_len, mask)
        ref = G.gqa(q, k, v, n_heads, n_kv, seq_len, mask=mask)
        want = O.gqa(q, k, v, n_heads, n_kv, seq_len, mask=mask)
        print(f"[noalloc] call {i} seq_len={seq_len} heads={n_heads}/{n_kv} "
              f"rel_err={rel_err(got, want):.3e}", flush=True)
        assert np.array_equal(got, ref), (i, seq_len)
        assert rel_err(got, want) < FP32_BAR


def test_noalloc_rejects_oversize():
    q, k, v = _inputs(16, 32, 8, 0xB0B)
    bufs = [DeviceBuffer.of(q), DeviceBuffer.of(k), DeviceBuffer.of(v), DeviceBuffer(32 * 256 * 4)]
    try:
        with pytest.raises(G.G3AttnError) as e:
            G.gqa_noalloc(bufs[3].ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, 32, 8, 16)
        assert "scratch" in str(e.value)
        with pytest.raises(G.G3AttnError):
            G.gqa_noalloc(bufs[3].ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, 8, 4, 0)
    finally:
        for b in bufs:
            b.free()



def test_noalloc_under_graph_capture():
    """g3attn_gqa_noalloc recorded into a HIP graph (stream capture through the
    HIP runtime the library links) and replayed three times.  Before each
    replay a new query is copied into the captured input buffer, and eager
    work (the copy, an allocating g3attn_gqa call) runs between replays; every
    replay matches the eager g3attn_gqa of its query bit for bit.  The call
    records kernel launches only: no allocation, no memset node."""
    import ctypes as C

    hip = DeviceBuffer.hip()
    vp = C.c_void_p
    hip.hipStreamCreate.argtypes = [C.POINTER(vp)]
    hip.hipStreamBeginCapture.argtypes = [vp, C.c_int]
    hip.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
    hip.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
    hip.hipGraphLaunch.argtypes = [vp, vp]
    hip.hipStreamSynchronize.argtypes = [vp]
    for f in ("hipGraphExecDestroy", "hipGraphDestroy", "hipStreamDestroy"):
        getattr(hip, f).argtypes = [vp]

    seq_len, n_heads, n_kv = 2048, 8, 4
    q, k, v = _inputs(seq_len, n_heads, n_kv, 0xC0DE)
    bq, bk, bv = DeviceBuffer.of(q), DeviceBuffer.of(k), DeviceBuffer.of(v)
    out = DeviceBuffer(n_heads * 256 * 4)
    stream, graph, exe = vp(), vp(), vp()
    assert hip.hipStreamCreate(C.byref(stream)) == 0
    try:
        def call():
            G.gqa_noalloc(out.ptr, bq.ptr, bk.ptr, bv.ptr, n_heads, n_kv, seq_len, stream=stream.value)

        # the first call on a device looks its scratch address up: run it eagerly
        call()
        assert hip.hipStreamSynchronize(stream) == 0
        assert hip.hipStreamBeginCapture(stream, 2) == 0     # hipStreamCaptureModeRelaxed
        call()
        assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for rep in range(3):
            qr = O.gen_normal_bf16(n_heads * 256, 0xC0DE + 97 * (rep + 1))
            bq.upload(qr)
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            got = out.download(np.float32, n_heads * 256)
            ref = G.gqa(qr, k, v, n_heads, n_kv, seq_len)
            print(f"[noalloc graph] replay {rep}: max |diff| vs eager = "
                  f"{float(np.max(np.abs(got - ref))):.3e}", flush=True)
            assert np.array_equal(got, ref), rep
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(stream)
        for b in (bq, bk, bv, out):
            b.free()
