"""The decode kernels' own source, run on the CPU under ASan + UBSan.

tests/hostemu/Makefile compiles gemma3.c_amd/csrc/decode.hip (decode_kernel,
combine_kernel and the g3k_decode launcher, unchanged) as host C++ against
stand-in HIP headers that emulate a wave64 machine on host fibers (one
ucontext per GPU thread): cross-lane DPP / permlane-swap / shuffle exchanges
between barriers, __syncthreads over the workgroup, and buffer loads that
abort when they leave their descriptor's range.  The cross-lane lane layouts
were checked against gfx950 with an in-bounds probe of the builtins.  Every input and output is its own exact-size heap allocation.  The
builds stop at the first sanitizer report.

What this shows, for the cases below: no out-of-range access, no undefined
behaviour the sanitizers see, and outputs that match the oracle (the
reference's attention restated, gemma3_transformer.c:294-352 and
gemma3_kernels.c:527-597) to the decode bar.  The same source is run with the
row count per lane-group R forced to 1, 2, 3 and 4 for every group: it is
written generically in R, and the R >= 3 cases pin that on the CPU.

Cases follow the GPU decode tests: configs[0] (local layer, pos 511), a
ring-wrapped local layer (pos 1500, window 1024), one split and many, QK-norm
on and off, non-temporal and plain loads, groups 1 / 2 / 4, and the
gemma3_gqa-shaped path with and without an additive mask.  The one-launch
form (splits merged in the kernel by the last workgroup of each run to
arrive) runs with the workgroups in grid order and in reverse, so the last
split and the first each do the merging, and must leave its arrival
counters zero.
"""
import os
import subprocess

import numpy as np
import pytest

from helpers import O, REPO, D, DecodeCase, rel_err, tensor

EMU = os.path.join(REPO, "tests", "hostemu")
BUILD = os.path.join(EMU, "_build")
LOG2E = 1.4426950408889634
BAR = 1e-4  # max-abs error / output RMS, the fp32 decode bar

pytestmark = pytest.mark.skipif(not os.path.exists("/opt/rocm/lib/llvm/bin/clang++"),
                                reason="ROCm clang not available")


@pytest.fixture(scope="module")
def built():
    r = subprocess.run(["make", "-C", EMU, "-j4"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return True


def _run(exe, tmp, *, fused, group, n_kv, n_heads, kc, vc, row_stride, head_stride, n_stream, skip,
         new_slot, rps, n_splits, q, k_new=None, v_new=None, norm=None, rope_row=None, mask=None,
         nt_loads=0, eps=1e-6, qscale=0.0625 * LOG2E, xm_heads=0, order=None):
    os.makedirs(tmp, exist_ok=True)

    def put(name, a, dtype=np.float32):
        np.ascontiguousarray(a, dtype=dtype).tofile(os.path.join(tmp, name + ".bin"))

    put("q", q)
    put("kc", kc)
    put("vc", vc)
    if fused:
        put("k_new", k_new)
        put("v_new", v_new)
        put("rope_row", rope_row)
    if norm is not None:
        put("q_norm", norm, np.uint16)
        put("k_norm", norm, np.uint16)
    if mask is not None:
        put("mask", mask)
    with open(os.path.join(tmp, "args.txt"), "w") as f:
        f.write(f"{int(fused)} {group} {n_kv} {n_heads} {kc.size} {row_stride} {head_stride} {n_stream} "
                f"{skip} {new_slot} {rps} {n_splits} {nt_loads} {int(norm is not None)} "
                f"{int(mask is not None)} {float(np.float32(eps))!r} {float(np.float32(qscale))!r} {xm_heads}\n")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="print_stacktrace=1")
    if order:
        env["HOSTEMU_WG_ORDER"] = order
    r = subprocess.run([os.path.join(BUILD, exe), tmp], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0 and "decode_emu: ok" in r.stdout, (exe, r.stderr[-4000:])
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]

    def get(name, n):
        return np.fromfile(os.path.join(tmp, name + ".bin"), dtype=np.float32, count=n)

    return get("out", n_heads * D), get("kc_out", kc.size), get("vc_out", vc.size)


def _fused(exe, tmp, case: DecodeCase, rps, n_splits, nt_loads, xm_heads=0, order=None):
    """g3k_decode as g3attn_decode_device sets it up (host/g3attn.c), over a
    head-major cache holding the case's history; checks the output and the
    new token's cache rows against the oracle."""
    cfg, n_kv, n_heads = case.cfg, case.cfg.num_kv_heads, case.cfg.num_heads
    W, pos = cfg.sliding_window, case.pos
    seq_len = pos + 1 if (case.is_global or pos < W) else W
    slot = pos if case.is_global else pos % W
    Kc, Vc = case.oracle_cache()
    hm = lambda c: np.ascontiguousarray(c.reshape(case.rows, n_kv, D).transpose(1, 0, 2))
    want, Kw, Vw = case.oracle()
    got, kc, vc = _run(exe, tmp, fused=True, group=n_heads // n_kv, n_kv=n_kv, n_heads=n_heads,
                       kc=hm(Kc), vc=hm(Vc), row_stride=D, head_stride=case.rows * D, n_stream=seq_len - 1,
                       skip=slot, new_slot=slot, rps=rps, n_splits=n_splits, q=case.q, k_new=case.k,
                       v_new=case.v, norm=case.norm, rope_row=case.table.reshape(-1, D)[pos],
                       nt_loads=nt_loads, xm_heads=xm_heads, order=order)
    kc = kc.reshape(n_kv, case.rows, D)
    vc = vc.reshape(n_kv, case.rows, D)
    # the new token's rows: k normed + rotated (fp32 rounding may differ), v as given
    assert rel_err(kc[:, slot], hm(Kw)[:, slot]) < 1e-5
    assert np.array_equal(vc[:, slot], hm(Vw)[:, slot])
    # every other row untouched
    others = np.ones(case.rows, bool)
    others[slot] = False
    assert np.array_equal(kc[:, others], hm(Kc)[:, others]) and np.array_equal(vc[:, others], hm(Vc)[:, others])
    return rel_err(got, want)


def _splits(n_stream, rps):
    return rps, (n_stream + rps - 1) // rps


EXES = ["decode_emu", "decode_emu_r1", "decode_emu_r2", "decode_emu_r3", "decode_emu_r4"]


@pytest.mark.parametrize("exe", EXES)
def test_config1_local_decode(built, tmp_path, exe):
    """local layer 0, pos 511, 511 cached rows + the new token, 4 KV
    heads x 2 query heads; 64-row splits (8 per head), non-temporal loads."""
    case = DecodeCase(1, layer=0, pos=511, max_context=1024)
    err = _fused(exe, str(tmp_path), case, *_splits(511, 64), nt_loads=1)
    print(f"[hostemu {exe}] configs[0] rel_err={err:.3e}")
    assert err < BAR


@pytest.mark.parametrize("exe", ["decode_emu", "decode_emu_r3", "decode_emu_r4"])
def test_ring_wrap_one_split_plain_loads(built, tmp_path, exe):
    """Local layer past the window (pos 1500: the new slot 476 sits inside the
    streamed ring), one split of all 1023 rows (the single-split emit path),
    plain loads, QK-norm off."""
    case = DecodeCase(1, layer=2, pos=1500, max_context=2048, norm=False)
    err = _fused(exe, str(tmp_path), case, *_splits(1023, 1024), nt_loads=0)
    print(f"[hostemu {exe}] ring wrap rel_err={err:.3e}")
    assert err < BAR


@pytest.mark.parametrize("exe", ["decode_emu", "decode_emu_r4"])
@pytest.mark.parametrize("n_heads,n_kv", [(4, 4), (8, 2)])
def test_other_groups(built, tmp_path, exe, n_heads, n_kv):
    """Groups 1 and 4 (8 query heads over 2 KV heads), global layer pos 300,
    32-row splits."""
    case = DecodeCase(1, layer=5, pos=300, max_context=512, n_heads=n_heads, n_kv=n_kv)
    err = _fused(exe, str(tmp_path), case, *_splits(300, 32), nt_loads=1)
    print(f"[hostemu {exe}] group {n_heads // n_kv} rel_err={err:.3e}")
    assert err < BAR


@pytest.mark.parametrize("exe", ["decode_emu", "decode_emu_r3"])
@pytest.mark.parametrize("masked", [False, True])
def test_gqa_shaped(built, tmp_path, exe, masked):
    """The gemma3_gqa-shaped path (q final, cache in the reference layout
    [seq][H_kv][D], optional additive mask) against the oracle's gemma3_gqa,
    as g3attn_gqa sets it up: 64-row minimum splits."""
    n_heads, n_kv, seq = 8, 4, 333
    q = tensor(7, 1, n_heads * D)
    k = tensor(7, 2, seq * n_kv * D)
    v = tensor(7, 3, seq * n_kv * D)
    mask = None
    if masked:
        mask = np.zeros(seq, np.float32)
        mask[::7] = -1e30
        mask[5:40] = -0.75
    want = O.gqa(q, k, v, n_heads, n_kv, seq, mask=mask)
    got, kc, vc = _run(exe, str(tmp_path), fused=False, group=2, n_kv=n_kv, n_heads=n_heads, kc=k, vc=v,
                       row_stride=n_kv * D, head_stride=D, n_stream=seq, skip=2**31 - 1, new_slot=-1,
                       rps=64, n_splits=6, q=q, mask=mask)
    assert np.array_equal(kc, k) and np.array_equal(vc, v)
    err = rel_err(got, want)
    print(f"[hostemu {exe}] gqa masked={masked} rel_err={err:.3e}")
    assert err < BAR


@pytest.mark.parametrize("order", ["forward", "reverse"])
@pytest.mark.parametrize("n_heads,n_kv,xm,pos,layer,rps", [
    (8, 4, 1, 511, 0, 32),     # configs[0]: 16 splits, one query head per workgroup (8 runs)
    (8, 4, 1, 1500, 2, 32),    # ring-wrapped local layer: 32 splits of 32 rows
    (8, 4, 1, 300, 5, 64),     # a global layer, 5 splits of 64 rows
    (8, 4, 2, 1500, 2, 32),    # whole groups: 4 runs padded to 8 (idle workgroups)
    (16, 8, 2, 700, 1, 32),    # group 2 over 8 KV heads: whole groups per workgroup
    (8, 8, 1, 200, 3, 32),     # group 1
    (8, 2, 1, 400, 4, 32),     # group 4, one query head per workgroup
])
def test_one_launch_merge(built, tmp_path, order, n_heads, n_kv, xm, pos, layer, rps):
    """The one-launch form (xm_heads > 0) against the oracle, with the
    workgroups in grid order and in reverse."""
    case = DecodeCase(1, layer=layer, pos=pos, max_context=2048, n_heads=n_heads, n_kv=n_kv)
    n_stream = (pos + 1 if (case.is_global or pos < 1024) else 1024) - 1
    err = _fused("decode_emu", str(tmp_path), case, *_splits(n_stream, rps), nt_loads=int(case.is_global),
                 xm_heads=xm, order=order)
    print(f"[hostemu xm {order}] H_q {n_heads} H_kv {n_kv} pos {pos} rel_err={err:.3e}")
    assert err < BAR
