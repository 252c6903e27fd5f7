"""The GEMV kernel's own source (csrc/matvec.hip), run on the CPU under ASan +
UBSan on the emulated wave64 machine of tests/hostemu (see
test_decode_hostemu.py for the machine).

Every layout the launcher picks is driven: one row per wave (Q/K/V, K =
2560), rows split over the workgroup's waves (K <= 2048 and K >= 8192), the
GEGLU pair, and the scalar path (K not a multiple of 8, or x unaligned).  The
residual prologue (g3k_matvec_args.pre_*: x = rmsnorm(r + rmsnorm(t, w_post),
w_next), formed by every workgroup, the new residual stored by workgroup 0)
runs with both gains, with the post-norm absent, and on the GEGLU launch.

The expected values come from the oracle: gemma3_matvec_bf16
(gemma3_kernels.c:188-238), gemma3_rmsnorm_bf16 (:289-304) and
gemma3_gelu_tanh_inplace (:348-357) restated; the bar is 1e-5 x RMS (fp32
throughout, summation orders differ).  What this adds to the GPU tests: no
out-of-range access or undefined behaviour in the kernel's indexing, ragged
tails and prologue, under the sanitizers.
"""
import os
import subprocess

import numpy as np
import pytest

from helpers import O, REPO, rel_err

EMU = os.path.join(REPO, "tests", "hostemu")
EXE = os.path.join(EMU, "_build", "matvec_emu")
BAR = 1e-5
GEGLU = 1

pytestmark = pytest.mark.skipif(not os.path.exists("/opt/rocm/lib/llvm/bin/clang++"),
                                reason="ROCm clang not available")


@pytest.fixture(scope="module")
def built():
    r = subprocess.run(["make", "-C", EMU, "-j4"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return True


def _bf16(rng, n, scale):
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def _run(tmp, mats, K, mode=0, x=None, pre=None, x_off=0, eps=1e-6):
    os.makedirs(tmp, exist_ok=True)
    for m, A in enumerate(mats):
        np.ascontiguousarray(A, np.uint16).tofile(os.path.join(tmp, f"A{m}.bin"))
    M = [A.shape[0] for A in mats] + [0] * (3 - len(mats))
    if pre is None:
        np.ascontiguousarray(x, np.float32).tofile(os.path.join(tmp, "x.bin"))
        has_wp = has_wn = 0
    else:
        t, r, wp, wn = pre
        t.astype(np.float32).tofile(os.path.join(tmp, "t.bin"))
        r.astype(np.float32).tofile(os.path.join(tmp, "r.bin"))
        has_wp, has_wn = int(wp is not None), int(wn is not None)
        if has_wp:
            wp.tofile(os.path.join(tmp, "w_post.bin"))
        if has_wn:
            wn.tofile(os.path.join(tmp, "w_next.bin"))
    with open(os.path.join(tmp, "args.txt"), "w") as f:
        f.write(f"{mode} {len(mats)} {K} {M[0]} {M[1]} {M[2]} {int(pre is not None)} {has_wp} {has_wn} "
                f"{x_off} {float(np.float32(eps))!r}\n")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="print_stacktrace=1")
    res = subprocess.run([EXE, tmp], capture_output=True, text=True, timeout=600, env=env)
    assert res.returncode == 0 and "matvec_emu: ok" in res.stdout, res.stderr[-4000:]
    assert "runtime error" not in res.stderr and "AddressSanitizer" not in res.stderr, res.stderr[-4000:]
    n_out = 1 if mode == GEGLU else len(mats)
    ys = [np.fromfile(os.path.join(tmp, f"y{m}.bin"), dtype=np.float32) for m in range(n_out)]
    r_out = np.fromfile(os.path.join(tmp, "r_out.bin"), dtype=np.float32) if pre is not None else None
    return ys, r_out


def _prologue_oracle(t, r, wp, wn, eps=1e-6):
    """s = r + rmsnorm(t, w_post) (r + t without w_post); x = rmsnorm(s, w_next) (s without)."""
    tn = O.rmsnorm_bf16(t, wp, eps) if wp is not None else t
    s = (r + tn).astype(np.float32)
    x = O.rmsnorm_bf16(s, wn, eps) if wn is not None else s
    return s, x


@pytest.mark.parametrize("K,M", [(2560, 70), (512, 40), (10240, 8), (100, 33)])
def test_plain_layouts(built, tmp_path, K, M):
    """One row per wave (K 2560, ragged last workgroup), rows split over the
    waves (K 512 and 10240), and the scalar path (K 100)."""
    rng = np.random.default_rng(K + M)
    A = _bf16(rng, M * K, 0.05).reshape(M, K)
    x = rng.standard_normal(K).astype(np.float32)
    (y,), _ = _run(str(tmp_path), [A], K, x=x)
    err = rel_err(y, O.matvec_bf16(A, x))
    print(f"[hostemu matvec] K={K} M={M} rel_err={err:.3e}")
    assert err < BAR


def test_unaligned_x_takes_the_scalar_path(built, tmp_path):
    rng = np.random.default_rng(7)
    K, M = 2560, 20
    A = _bf16(rng, M * K, 0.05).reshape(M, K)
    x = rng.standard_normal(K).astype(np.float32)
    (y,), _ = _run(str(tmp_path), [A], K, x=x, x_off=1)
    assert rel_err(y, O.matvec_bf16(A, x)) < BAR


@pytest.mark.parametrize("K,post", [(2560, True), (512, False)])
def test_three_matrices_with_residual_prologue(built, tmp_path, K, post):
    """The Q/K/V launch with the residual step in its prologue: three
    matrices sharing x, x formed by every workgroup, the new residual stored
    once.  K 512 without the post-norm takes the split-over-waves layout."""
    rng = np.random.default_rng(K)
    mats = [_bf16(rng, M * K, 0.05).reshape(M, K) for M in (64, 32, 36)]
    t = rng.standard_normal(K).astype(np.float32)
    r = (rng.standard_normal(K) * 3).astype(np.float32)
    wp = _bf16(rng, K, 0.2) if post else None
    wn = _bf16(rng, K, 0.2)
    ys, r_out = _run(str(tmp_path), mats, K, pre=(t, r, wp, wn))
    s, x = _prologue_oracle(t, r, wp, wn)
    assert rel_err(r_out, s) < BAR
    for y, A in zip(ys, mats):
        err = rel_err(y, O.matvec_bf16(A, x))
        print(f"[hostemu matvec prologue] K={K} post={post} M={A.shape[0]} rel_err={err:.3e}")
        assert err < BAR


@pytest.mark.parametrize("K", [100, 12])
def test_residual_prologue_on_the_scalar_path(built, tmp_path, K):
    """K a multiple of 4 but not of 8: the residual prologue forms x in LDS
    and the lane-strided scalar path reads it from there (K = 12: fewer
    elements than one wave's lanes)."""
    rng = np.random.default_rng(K + 5)
    mats = [_bf16(rng, M * K, 0.05).reshape(M, K) for M in (9, 5)]
    t = rng.standard_normal(K).astype(np.float32)
    r = (rng.standard_normal(K) * 2).astype(np.float32)
    wp, wn = _bf16(rng, K, 0.2), _bf16(rng, K, 0.2)
    ys, r_out = _run(str(tmp_path), mats, K, pre=(t, r, wp, wn))
    s, x = _prologue_oracle(t, r, wp, wn)
    assert rel_err(r_out, s) < BAR
    for y, A in zip(ys, mats):
        err = rel_err(y, O.matvec_bf16(A, x))
        print(f"[hostemu matvec prologue scalar] K={K} M={A.shape[0]} rel_err={err:.3e}")
        assert err < BAR


@pytest.mark.parametrize("pre", [False, True])
def test_geglu(built, tmp_path, pre):
    """gelu_tanh(gate . x) * (up . x), plain and with the residual prologue
    (both gains)."""
    rng = np.random.default_rng(11 + pre)
    K, M = 512, 48
    G_, U_ = (_bf16(rng, M * K, 0.05).reshape(M, K) for _ in range(2))
    if pre:
        t = rng.standard_normal(K).astype(np.float32)
        r = rng.standard_normal(K).astype(np.float32)
        wp, wn = _bf16(rng, K, 0.2), _bf16(rng, K, 0.2)
        (y,), r_out = _run(str(tmp_path), [G_, U_], K, mode=GEGLU, pre=(t, r, wp, wn))
        s, x = _prologue_oracle(t, r, wp, wn)
        assert rel_err(r_out, s) < BAR
    else:
        x = rng.standard_normal(K).astype(np.float32)
        (y,), _ = _run(str(tmp_path), [G_, U_], K, mode=GEGLU, x=x)
    want = O.gelu_tanh(O.matvec_bf16(G_, x)) * O.matvec_bf16(U_, x)
    err = rel_err(y, want)
    print(f"[hostemu geglu] pre={pre} rel_err={err:.3e}")
    assert err < BAR
