"""The whole library (gemma3.c_amd/host + every kernel) behind its C ABI, run
on the CPU under ASan + UBSan on the emulated wave64 machine of tests/hostemu.

tests/hostemu/_build/attn_emu executes a script of g3attn calls (create,
kv_write, prefill, decode, kv_read, matmul) against the library compiled for
the host: the host code's staging ranges, key-split choice, ring handling
and buffer sizing run unchanged, and the kernels run from their own source
with MFMA, DPP, permlane swaps and buffer -> LDS loads emulated (see
hostemu/hip/hip_runtime.h).  Each call sequence is mirrored on the oracle,
whose caches carry state from call to call exactly as the library's do:
prefill chunks, the history they stage from the cache, the sliding-window
ring, decode steps after a prefill.

Expected values: the oracle's g3o_prefill / g3o_layer_decode (restating
gemma3_transformer.c:641-692 and :294-352; the bar is the path's 2e-3 x
output RMS, and the emulated kernels land near 1e-5, as on the GPU), the
cache rows the reference's cache_kv leaves (gemma3_transformer.c:236-251),
and an fp64 product for the batched-prefill GEMM.  What this adds to the GPU
tests: no out-of-range access or undefined behaviour in the host code or
the kernels' indexing (LDS rings, ragged tiles, key splits) under the
sanitizers; a barrier or cross-lane operation that some lane misses stops
the run.
"""
import importlib.util
import os
import subprocess

import numpy as np
import pytest

from helpers import O, REPO, TOL, rel_err

EMU = os.path.join(REPO, "tests", "hostemu")
EXE = os.path.join(EMU, "_build", "attn_emu")
D = 256
CLANG = "/opt/rocm/lib/llvm/bin/clang++"

pytestmark = pytest.mark.skipif(not os.path.exists(CLANG), reason="ROCm clang not available")

_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(REPO, "tests", "golden", "make_golden.py"))
MG = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(MG)


@pytest.fixture(scope="module")
def built():
    r = subprocess.run(["make", "-C", EMU, "-j8"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return True


def _bf16_valued(a):
    """Round to the nearest bf16 value (the configs' inputs are bf16-valued)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).view(np.float32)


class Emu:
    """A script of library calls and the same calls on the oracle."""

    def __init__(self, tmp, H=8, Hkv=4, max_context=128, window=16, layers=6, model_dims=None):
        self.dir, self.H, self.Hkv = str(tmp), H, Hkv
        self.cfg = O.Config(max_context=max_context, sliding_window=window, num_heads=H, num_kv_heads=Hkv)
        self.tables = {False: O.rope_table(max_context, 10000.0), True: O.rope_table(max_context, 1e6)}
        self._save("rl.bin", self.tables[False])
        self._save("rg.bin", self.tables[True])
        dims = " ".join(str(x) for x in model_dims) if model_dims else ""
        self.lines = [f"create {H} {Hkv} {max_context} {window} {layers} 1e-6 rl.bin rg.bin {dims}"]
        self.caches = {}
        self.checks = []          # (file, expected, label, bar: x RMS, 0 = exact, or an array bound)
        self.threads = {}
        self.k = 0
        self.rng = np.random.default_rng(1234)

    def _save(self, name, a):
        np.ascontiguousarray(a).tofile(os.path.join(self.dir, name))

    def _name(self, stem):
        self.k += 1
        return f"{stem}{self.k}.bin"

    def _cache(self, layer):
        if layer not in self.caches:
            rows = self.cfg.cache_rows(layer)
            self.caches[layer] = (np.zeros((rows, self.Hkv * D), np.float32),
                                  np.zeros((rows, self.Hkv * D), np.float32))
        return self.caches[layer]

    def inputs(self, n, bf16=True):
        f = _bf16_valued if bf16 else (lambda a: a.astype(np.float32))
        return (f(self.rng.standard_normal((n, self.H * D))), f(self.rng.standard_normal((n, self.Hkv * D))),
                f(self.rng.standard_normal((n, self.Hkv * D))))

    def gains(self, norm):
        """None (no QK-norm), or non-unit bf16 gains for q and k."""
        if not norm:
            return None, None, "-", "-"
        g = [(_bf16_valued(self.rng.standard_normal(D) * 0.3).view(np.uint32) >> 16).astype(np.uint16)
             for _ in range(2)]
        names = [self._name("gq"), self._name("gk")]
        self._save(names[0], g[0])
        self._save(names[1], g[1])
        return g[0], g[1], names[0], names[1]

    def prefill(self, layer, start, n, norm=True, bf16=True, device=False):
        Q, K, V = self.inputs(n, bf16)
        gq, gk, nq, nk = self.gains(norm)
        files = [self._name(s) for s in ("Q", "K", "V", "out")]
        for f, a in zip(files, (Q, K, V)):
            self._save(f, a)
        cmd = "prefill_device" if device else "prefill"
        self.lines.append(f"{cmd} {layer} {start} {n} {files[0]} {files[1]} {files[2]} {nq} {nk} {files[3]}")
        Kc, Vc = self._cache(layer)
        want, _, _ = O.prefill(self.cfg, layer, start, Q, K, V, Kc, Vc,
                               self.tables[O.is_global_layer(layer)], gq, gk)
        self.checks.append((files[3], want, f"prefill layer={layer} start={start} n={n}", TOL))

    def decode(self, layer, pos, norm=True):
        Q, K, V = self.inputs(1)
        gq, gk, nq, nk = self.gains(norm)
        files = [self._name(s) for s in ("q", "k", "v", "o")]
        for f, a in zip(files, (Q, K, V)):
            self._save(f, a)
        self.lines.append(f"decode {layer} {pos} {files[0]} {files[1]} {files[2]} {nq} {nk} {files[3]}")
        Kc, Vc = self._cache(layer)
        want, _, _ = O.layer_decode(self.cfg, layer, pos, Q[0], K[0], V[0], Kc, Vc,
                                    self.tables[O.is_global_layer(layer)], gq, gk)
        self.checks.append((files[3], want, f"decode layer={layer} pos={pos}", TOL))

    def check_cache(self, layer, slot, n):
        """The cache rows [slot, slot + n) as the oracle's cache_kv left them."""
        kf, vf = self._name("kr"), self._name("vr")
        self.lines.append(f"kv_read {layer} {slot} {n} {kf} {vf}")
        Kc, Vc = self._cache(layer)
        self.checks.append((kf, Kc[slot:slot + n].copy(), f"cache k layer={layer} [{slot},{slot + n})", 1e-5))
        self.checks.append((vf, Vc[slot:slot + n].copy(), f"cache v layer={layer} [{slot},{slot + n})", 0.0))

    def matmul(self, N, M, K):
        W = (_bf16_valued(self.rng.standard_normal((M, K)) * 0.05).view(np.uint32) >> 16).astype(np.uint16)
        X = self.rng.standard_normal((N, K)).astype(np.float32)
        files = [self._name(s) for s in ("W", "X", "C")]
        self._save(files[0], W)
        self._save(files[1], X)
        self.lines.append(f"matmul {N} {M} {K} {files[0]} {files[1]} {files[2]}")
        W64 = (W.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        X64 = X.astype(np.float64)
        # elementwise: the hi / lo split of X (2^-17 relative each) and fp32
        # accumulation over K terms
        bound = (2.0 ** -16 + K * 2.0 ** -24) * (np.abs(X64) @ np.abs(W64).T) + 1e-30
        self.checks.append((files[2], X64 @ W64.T, f"matmul N={N} M={M} K={K} (max err / bound)", bound))

    def gqa(self, h, hkv, seq, masked=False, noalloc=False, d=D):
        """g3attn_gqa / _noalloc against the oracle's gemma3_gqa (1e-4 x RMS),
        scale 1 / sqrt(d)."""
        q = self.rng.standard_normal(h * d).astype(np.float32)
        k = self.rng.standard_normal(seq * hkv * d).astype(np.float32)
        v = self.rng.standard_normal(seq * hkv * d).astype(np.float32)
        files = [self._name(s) for s in ("gq", "gk", "gv", "go")]
        for f, a in zip(files, (q, k, v)):
            self._save(f, a)
        mask, mf = None, "-"
        if masked:
            mask = (self.rng.standard_normal(seq) * 2).astype(np.float32)
            mask[self.rng.random(seq) < 0.3] = -1e9
            mf = self._name("gm")
            self._save(mf, mask)
        cmd = "gqa_noalloc" if noalloc else "gqa"
        self.lines.append(f"{cmd} {h} {hkv} {seq} {files[0]} {files[1]} {files[2]} {mf} {files[3]} {d}")
        want = O.gqa(q, k, v, h, hkv, seq, d=d, scale=float(np.float32(1.0) / np.sqrt(np.float32(d))), mask=mask)
        self.checks.append((files[3], want, f"{cmd} {h}/{hkv} d={d} seq={seq} mask={masked}", 1e-4))

    def matvec(self, M, K, device=False):
        """g3attn_matvec_bf16 (host) / _device against gemma3_matvec_bf16 (1e-5 x RMS)."""
        A = (_bf16_valued(self.rng.standard_normal((M, K)) * 0.05).view(np.uint32) >> 16).astype(np.uint16)
        x = self.rng.standard_normal(K).astype(np.float32)
        files = [self._name(s) for s in ("mA", "mx", "my")]
        self._save(files[0], A)
        self._save(files[1], x)
        cmd = "matvec_device" if device else "matvec"
        self.lines.append(f"{cmd} {M} {K} {files[0]} {files[1]} {files[2]}")
        self.checks.append((files[2], O.matvec_bf16(A, x), f"{cmd} M={M} K={K}", 1e-5))

    def kv_append(self, layer, start, n, norm=True):
        """g3attn_kv_append; the oracle's cache gets the K-normed, rotated rows
        in ring order (cache_kv, gemma3_transformer.c:236-251)."""
        _, K, V = self.inputs(n)
        _, gk, _, nk = self.gains(norm)
        kf, vf = self._name("aK"), self._name("aV")
        self._save(kf, K)
        self._save(vf, V)
        self.lines.append(f"kv_append {layer} {start} {n} {kf} {vf} {nk}")
        Kr = K.reshape(n, self.Hkv, D).copy()
        O.norm_rope_batch(Kr, self.tables[O.is_global_layer(layer)], start, gk)
        Kc, Vc = self._cache(layer)
        for i in range(n):
            p = start + i
            slot = p if O.is_global_layer(layer) else p % self.cfg.sliding_window
            Kc[slot] = Kr[i].reshape(-1)
            Vc[slot] = V[i]

    def layer_attention(self, layer, pos, hidden, norm=True):
        """g3attn_layer_attention_device against the oracle's layer_attention
        (gemma3_transformer.c:258-356; 1e-4 x RMS)."""
        qs, ks = self.H * D, self.Hkv * D
        w = [(_bf16_valued(self.rng.standard_normal(r * c) * 0.05).view(np.uint32) >> 16).astype(np.uint16)
             .reshape(r, c) for r, c in ((qs, hidden), (ks, hidden), (ks, hidden), (hidden, qs))]
        x = self.rng.standard_normal(hidden).astype(np.float32)
        gq, gk, nq, nk = self.gains(norm)
        files = [self._name(s) for s in ("lx", "lwq", "lwk", "lwv", "lwo", "lo")]
        for f, a in zip(files, [x] + w):
            self._save(f, a)
        self.lines.append(f"layer_attention {layer} {pos} {hidden} " + " ".join(files[:5]) + f" {nq} {nk} {files[5]}")
        Kc, Vc = self._cache(layer)
        want = O.layer_attention(self.cfg, layer, pos, x, *w, Kc, Vc, self.tables[O.is_global_layer(layer)], gq, gk)
        self.checks.append((files[5], want, f"layer_attention layer={layer} pos={pos}", 1e-4))

    def model(self, embed, layers, norm):
        """The model's tensors as files (absent optional norms: no file)."""
        self._save("m_embed.bin", embed)
        self._save("m_norm.bin", norm)
        for l, lw in enumerate(layers):
            for name in O.LAYER_TENSORS:
                if lw[name] is not None:
                    self._save(f"m_L{l}_{name}.bin", lw[name])
        self.lines.append("model m_")

    def logits(self, cmd, args, want, label):
        f = self._name("lg")
        self.lines.append(f"{cmd} {args} {f}")
        self.checks.append((f, want, label, 1e-4))

    def run(self, **env):
        with open(os.path.join(self.dir, "script.txt"), "w") as f:
            f.write("\n".join(self.lines) + "\n")
        # Stack-use-after-return detection (a fake frame per call on every
        # fiber) doubles the run time and guards against nothing these
        # kernels do: they never pass stack addresses out.  The other checks
        # (heap, globals incl. the LDS arrays, stack bounds, leaks) stay on.
        e = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:detect_stack_use_after_return=0",
                 UBSAN_OPTIONS="print_stacktrace=1")
        e.update({k: str(v) for k, v in env.items()})
        res = subprocess.run([EXE, self.dir], capture_output=True, text=True, timeout=1200, env=e)
        assert res.returncode == 0 and "attn_emu: ok" in res.stdout, res.stdout[-2000:] + res.stderr[-4000:]
        assert "runtime error" not in res.stderr and "AddressSanitizer" not in res.stderr, res.stderr[-4000:]
        for f, want, label, bar in self.checks:
            got = np.fromfile(os.path.join(self.dir, f), dtype=np.float32).reshape(np.shape(want))
            if isinstance(bar, np.ndarray):
                err, bar = float(np.max(np.abs(got - want) / bar)), 1.0
            else:
                err = rel_err(got, want) if bar else float(np.abs(got - want).max())
            print(f"[hostemu attn] {label}: {err:.3e}")
            assert err <= bar, (label, err)
        # "launch <kernel expression> <launches> <workgroups> <threads> <ms>":
        # (launches, workgroups summed over them), keyed by the bare kernel
        # name; self.threads[name]: threads per workgroup of the last launch
        launches = {}
        for ln in res.stdout.splitlines():
            if ln.startswith("launch "):
                expr, count, wgs, threads, _ms = ln[len("launch "):].rsplit(" ", 4)
                name = expr.strip("()").split("<")[0]
                c, w = launches.get(name, (0, 0))
                launches[name] = (c + int(count), w + int(wgs))
                self.threads[name] = int(threads)
        return launches


def test_global_prefill_chunks_then_decode(built, tmp_path):
    """Global layer: a ragged first chunk, a second chunk that stages its
    history from the cache, then two decode steps on the cache it wrote."""
    e = Emu(tmp_path)
    e.prefill(5, 0, 40)
    e.prefill(5, 40, 30)
    e.decode(5, 70)
    e.decode(5, 71)
    e.check_cache(5, 0, 72)
    launches = e.run()
    # the history is staged once by its own launch; each chunk's values are
    # staged inside that chunk's front launch (with K-norm, RoPE, cache write)
    assert launches["stage_kernel"][0] == 1, launches
    assert launches["front_kernel"][0] == 2, launches
    assert "rope_write_kernel" not in launches, launches


def test_local_prefill_ring(built, tmp_path):
    """Local layer, window 16: a 40-token batch (longer than the ring: only
    its last 16 rows are cached), a chunk whose history wraps the ring, and
    a decode step."""
    e = Emu(tmp_path)
    e.prefill(0, 0, 40)
    e.prefill(0, 40, 21)
    e.decode(0, 61)
    e.check_cache(0, 0, 16)
    e.run()


@pytest.mark.parametrize("order", ["forward", "reverse"])
@pytest.mark.parametrize("variant", ["default", "qpw32", "fp32"])
def test_key_splits(built, tmp_path, variant, order):
    """Global prefills long enough for the host's makespan model to split the
    key tiles of every 64-query block over 2 (n = 256: 4 blocks) and 4
    (n = 512: 8 blocks) workgroups (one KV head), merged inside the kernel
    by the split that arrives last: the last split of each block when the
    workgroups run in grid order, split 0 when they run in reverse.  Also
    with the 32-queries-per-wave kernel and with fp32 values (the V_lo pass).
    The prefill is followed by decodes over the same cache, so the arrival
    counters are reused by a second prefill of the same context."""
    env = {"G3ATTN_PREFILL_QPW": 32} if variant == "qpw32" else {}
    if order == "reverse":
        env["HOSTEMU_WG_ORDER"] = "reverse"
    for n, splits in [(256, 2), (512, 4)]:
        d = tmp_path / str(n)
        d.mkdir()
        e = Emu(d, H=2, Hkv=1, max_context=640, window=64)
        e.prefill(5, 0, n, bf16=variant != "fp32")
        e.prefill(5, n, 64, bf16=variant != "fp32")
        launches = e.run(**env)
        # (launches, workgroups over both calls): the first call alone has
        # n / 64 blocks x `splits`, the 64-token second call at least one
        assert launches["prefill_kernel"][0] == 2, launches
        assert launches["prefill_kernel"][1] > n // 64 * splits, launches
        assert "prefill_combine_kernel" not in launches, launches
        assert e.threads["prefill_kernel"] == (256 if variant == "qpw32" else 512)


@pytest.mark.parametrize("splits", [1, 4])
def test_forced_split_counts(built, tmp_path, splits):
    """G3ATTN_PREFILL_SPLITS: a local prefill whose blocks see the window and
    the history before them (four or five tiles each, so four splits leave
    one or two tiles per part), forced to 1 and to 4 key splits, then a
    decode over the same cache."""
    e = Emu(tmp_path, H=2, Hkv=1, max_context=640, window=64)
    e.prefill(0, 0, 100)
    e.prefill(0, 100, 192)
    e.decode(0, 292)
    launches = e.run(G3ATTN_PREFILL_SPLITS=splits)
    # the 192-token call: 3 blocks x splits workgroups; the first call 2 x splits
    assert launches["prefill_kernel"] == (2, 5 * splits), launches


def test_fp32_values_take_the_v_lo_pass(built, tmp_path):
    """Inputs that are not bf16-valued: the staging kernel flags V_lo and the
    kernel adds the P_hi.V_lo pass; also with QK-norm absent."""
    e = Emu(tmp_path)
    e.prefill(5, 0, 70, bf16=False)
    e.prefill(0, 0, 24, bf16=False, norm=False)
    e.run()


@pytest.mark.parametrize("heads,kv_heads", [(4, 4), (8, 2)])
def test_gqa_groups(built, tmp_path, heads, kv_heads):
    """GQA groups 1 and 4 (the configs use 2), prefill and decode."""
    e = Emu(tmp_path, H=heads, Hkv=kv_heads)
    e.prefill(5, 0, 50)
    e.decode(5, 50)
    e.prefill(0, 0, 20)
    e.run()


@pytest.mark.parametrize("env", [{"G3ATTN_PREFILL_QPW": 32}, {"G3ATTN_PREFILL_SCHED": 0},
                                 {"G3ATTN_PREFILL_SCHED": 2}])
def test_prefill_variants(built, tmp_path, env):
    """The selectable prefill forms: 32 queries per wave, and the two other
    SIMD phase schedules."""
    e = Emu(tmp_path)
    e.prefill(5, 0, 70)
    e.prefill(0, 0, 33)
    e.run(**env)
    # the 32-query form runs four waves per workgroup, the others eight
    assert e.threads["prefill_kernel"] == (256 if env.get("G3ATTN_PREFILL_QPW") == 32 else 512)


def test_device_entry_and_matmul(built, tmp_path):
    """g3attn_prefill_device, and the batched-prefill GEMM at ragged N with
    its one-plane (M = 4 multiple) and K = 96 shapes against fp64."""
    e = Emu(tmp_path)
    e.prefill(5, 0, 20, device=True)
    e.matmul(40, 64, 96)
    e.matmul(130, 20, 64)
    launches = e.run()
    assert launches["gemm_kernel"][0] == 2, launches


@pytest.mark.parametrize("heads,kv_heads", [(8, 4), (4, 4), (8, 2)])
def test_gqa_entry_points(built, tmp_path, heads, kv_heads):
    """g3attn_gqa (the gemma3_gqa drop-in, host pointers, a process-wide
    context) with and without an additive mask, and g3attn_gqa_noalloc (device
    buffers, the static scratch) on two calls in a row, the second shorter."""
    e = Emu(tmp_path, H=heads, Hkv=kv_heads)
    e.gqa(heads, kv_heads, 300)
    e.gqa(heads, kv_heads, 77, masked=True)
    e.gqa(heads, kv_heads, 300, masked=True, noalloc=True)
    e.gqa(heads, kv_heads, 40, noalloc=True)
    e.run()


@pytest.mark.parametrize("heads,kv_heads,d", [(6, 2, 64), (3, 1, 96), (8, 1, 512), (2, 2, 40), (5, 5, 1)])
def test_gqa_general_shapes(built, tmp_path, heads, kv_heads, d):
    """g3attn_gqa and g3attn_gqa_noalloc on shapes outside the model's
    (head_dim other than 256, groups other than 1 / 2 / 4): the general
    split-K kernel, with and without a mask, one split and many, against the
    oracle's gemma3_gqa."""
    e = Emu(tmp_path, H=8, Hkv=4)
    e.gqa(heads, kv_heads, 300, d=d)
    e.gqa(heads, kv_heads, 20, masked=True, d=d)
    e.gqa(heads, kv_heads, 700, masked=True, noalloc=True, d=d)
    e.gqa(heads, kv_heads, 9, noalloc=True, d=d)
    launches = e.run()
    assert launches["gqa_generic_kernel"][0] == 4, launches


def test_matvec_entry_points(built, tmp_path):
    """g3attn_matvec_bf16 (the gemma3_matvec_bf16 drop-in, host pointers) and
    the device form, at a Q-projection shape and a ragged one."""
    e = Emu(tmp_path)
    e.matvec(70, 2560)
    e.matvec(33, 100)
    e.matvec(70, 2560, device=True)
    e.matvec(5, 40, device=True)
    e.run()


def test_kv_append_and_layer_attention(built, tmp_path):
    """g3attn_kv_append filling a global and a local layer's cache (the local
    batch longer than its 16-row ring), decode steps over what it wrote, and
    the whole layer_attention on device buffers for three tokens (the
    context's hidden size, 256, sizes x and the projections)."""
    e = Emu(tmp_path, model_dims=(256, 512, 256))
    e.kv_append(5, 0, 50)
    e.decode(5, 50)
    e.kv_append(0, 0, 20, norm=False)
    e.decode(0, 20, norm=False)
    e.check_cache(5, 0, 51)
    e.check_cache(0, 0, 16)
    for pos in range(3):
        e.layer_attention(1, pos, 256)
    e.run()


@pytest.mark.parametrize("seed", range(6))
def test_random_sessions(built, tmp_path, seed):
    """Random sequences of prefill chunks (1-48 tokens) and decode runs on a
    local and a global layer, with odd windows (1, 7, 32) and a max_context
    off the 64-key staging grain (200), bf16 or fp32 inputs, QK-norm or
    none: the host code's ring and staging arithmetic under the sanitizers
    on the combinations the GPU sweep draws at larger sizes."""
    rng = np.random.default_rng(0xE5EED + seed)
    window = [1, 7, 32][seed % 3]
    e = Emu(tmp_path, H=[8, 4, 8][seed % 3], Hkv=[4, 4, 2][seed % 3], max_context=200, window=window)
    for layer in (1, 5):
        pos = 0
        while pos < 90:
            norm, bf16 = bool(rng.random() < 0.7), bool(rng.random() < 0.7)
            if rng.random() < 0.5:
                n = int(rng.integers(1, 49))
                e.prefill(layer, pos, n, norm=norm, bf16=bf16)
                pos += n
            else:
                for _ in range(int(rng.integers(1, 3))):
                    e.decode(layer, pos, norm=norm)
                    pos += 1
        e.check_cache(layer, 0, min(pos, window if layer == 1 else pos))
    e.run()


# A model of Gemma 3's structure small enough to emulate a token in a few
# seconds: 6 layers (layer 5 global), 2 query heads over 1 KV head of 256,
# hidden 128, intermediate 256, vocab 256, an 8-row sliding window, and
# layer 3 without its optional norms (the forward golden's layout, scaled).
SMALL = dict(hidden=128, inter=256, vocab=256, layers=6, max_context=32, window=8, heads=2, kv_heads=1)


def _forward_model(n):
    f = SMALL
    cfg = O.Config(num_layers=f["layers"], max_context=f["max_context"], sliding_window=f["window"],
                   num_heads=f["heads"], num_kv_heads=f["kv_heads"])
    Hd, I, V = f["hidden"], f["inter"], f["vocab"]
    qs, ks = f["heads"] * D, f["kv_heads"] * D
    embed = MG.weights_bf16(V, Hd, 0xE000)
    layers = []
    for l in range(f["layers"]):
        sd = 0xE100 + 32 * l
        lw = dict(input_layernorm=MG.norm_bf16(Hd, sd), q_proj=MG.weights_bf16(qs, Hd, sd + 1),
                  k_proj=MG.weights_bf16(ks, Hd, sd + 2), v_proj=MG.weights_bf16(ks, Hd, sd + 3),
                  o_proj=MG.weights_bf16(Hd, qs, sd + 4), q_norm=MG.norm_bf16(D, sd + 5),
                  k_norm=MG.norm_bf16(D, sd + 6), post_attention_layernorm=MG.norm_bf16(Hd, sd + 7),
                  gate_proj=MG.weights_bf16(I, Hd, sd + 8), up_proj=MG.weights_bf16(I, Hd, sd + 9),
                  down_proj=MG.weights_bf16(Hd, I, sd + 10), pre_feedforward_layernorm=MG.norm_bf16(Hd, sd + 11),
                  post_feedforward_layernorm=MG.norm_bf16(Hd, sd + 12))
        if l == 3:
            for k in ("q_norm", "k_norm", "post_attention_layernorm", "pre_feedforward_layernorm",
                      "post_feedforward_layernorm"):
                lw[k] = None
        layers.append(lw)
    norm = MG.norm_bf16(Hd, 0xEF00)
    tokens = np.random.default_rng(0xE0E0).integers(0, V, n).astype(np.int32)
    logits, _ = O.forward_seq(cfg, Hd, I, tokens, embed, layers, norm)
    return f, embed, layers, norm, tokens, logits


def _emu_for(tmp_path, f):
    return Emu(tmp_path, H=f["heads"], Hkv=f["kv_heads"], max_context=f["max_context"], window=f["window"],
               layers=f["layers"], model_dims=(f["hidden"], f["inter"], f["vocab"]))


# residual_kernel launches per token: fold 0 runs the two steps of every
# layer as kernels; fold 1 moves the step before layers 1-5's Q/K/V launch
# into it; fold 3 also the step before every gate/up launch (the final norm
# after the last layer stays a kernel)
RESIDUAL_PER_TOKEN = {0: 12, 1: 7, 3: 1}


@pytest.mark.parametrize("fold", [0, 1, 3])
def test_token_forward(built, tmp_path, fold):
    """g3attn_forward_device through every token-path kernel (embedding,
    norms, the fused Q/K/V GEMV with or without the residual prologue,
    decode, o_proj, GEGLU, down_proj, tied logits): each token's logits
    against the oracle's gemma3_transformer_forward
    (gemma3_transformer.c:396-512), for each residual-fold mode.  Fold 1
    (the default) runs 11 tokens, wrapping the 8-row window; the others 3.
    Bar 1e-4 x RMS, as on the GPU."""
    n = 11 if fold == 1 else 3
    f, embed, layers, norm, tokens, want = _forward_model(n)
    e = _emu_for(tmp_path, f)
    e.model(embed, layers, norm)
    for i, t in enumerate(tokens):
        e.logits("forward_device", f"{int(t)} {i}", want[i], f"forward_device token {i} fold={fold}")
    launches = e.run(G3ATTN_FORWARD_FOLD=fold)
    assert launches["residual_kernel"][0] == n * RESIDUAL_PER_TOKEN[fold], launches


def test_upload_batched_prefill_then_decode(built, tmp_path):
    """g3attn_upload_weights from host tensors, g3attn_prefill_tokens over 16
    tokens (the batched path: MFMA GEMMs in plain and GEGLU modes, per-row
    kernels, the prefill attention, ring writes past the window) giving the
    last token's logits, then g3attn_forward_token continuing from the cache
    it wrote."""
    n = 17
    f, embed, layers, norm, tokens, want = _forward_model(n)
    e = _emu_for(tmp_path, f)
    e.model(embed, layers, norm)
    e.lines.append("upload")
    e._save("tok.bin", tokens[:n - 1].astype(np.int32))
    e.logits("prefill_tokens", f"{n - 1} tok.bin 0", want[n - 2], f"prefill_tokens n={n - 1} last logits")
    e.logits("forward_token", f"{int(tokens[n - 1])} {n - 1}", want[n - 1], f"forward_token {n - 1}")
    launches = e.run()
    assert launches["gemm_kernel"][0] > 0 and launches["rows_kernel"][0] > 0, launches


def test_front_launch_with_an_empty_batch(built, tmp_path):
    """The prefill front launch (g3k_rope_write_stage) called with an empty
    batch (ra.n = 0) and no cache destination: its staging blocks still stage
    V^T (bf16 hi plane, zero padding to the 64-key grain) and, under the
    sanitizers, write nothing through the absent cache pointers."""
    hkv, nk = 2, 70
    e = Emu(tmp_path, H=4, Hkv=hkv)
    V = _bf16_valued(e.rng.standard_normal((nk, hkv * D)))
    e._save("Vs.bin", V)
    e.lines.append(f"front_stage_only {hkv} {nk} Vs.bin vt.bin")
    e.run()
    ldk = (nk + 63) // 64 * 64
    got = np.fromfile(os.path.join(e.dir, "vt.bin"), dtype=np.uint16).reshape(hkv, D, ldk)
    bits = (V.view(np.uint32) >> 16).astype(np.uint16).reshape(nk, hkv, D)
    want = np.zeros((hkv, D, ldk), np.uint16)
    want[:, :, :nk] = bits.transpose(1, 2, 0)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("order", ["forward", "reverse"])
def test_one_launch_local_decode(built, tmp_path, order):
    """Local-layer decodes at 8 query / 4 KV heads over 95 cached rows (three
    32-row splits) take the one-launch form: the placement probe at create
    passes on the emulated machine (workgroup i on XCD i mod 8), so each
    query head's splits are merged in the kernel by the last to arrive and
    no combine launch follows.  With G3ATTN_DECODE_XMERGE=0 the same script
    runs as decode + combine.  Both against the oracle, over a ring past its
    window, with the workgroups in grid order and in reverse."""
    for xm in (1, 0):
        d = tmp_path / f"xm{xm}"
        d.mkdir()
        e = Emu(d, H=8, Hkv=4, max_context=256, window=96)
        e.prefill(0, 0, 150)
        for pos in (150, 151, 152):
            e.decode(0, pos)
        e.check_cache(0, 0, 96)
        env = {"G3ATTN_DECODE_XMERGE": xm}
        if order == "reverse":
            env["HOSTEMU_WG_ORDER"] = "reverse"
        launches = e.run(**env)
        assert launches["decode_kernel"][0] == 3, launches
        assert ("combine_kernel" in launches) == (xm == 0), launches
