#!/usr/bin/env python3
"""Benchmark of the gemma3.c attention path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME,...]

Headline (the JSON line's `value`): configs[1] of BASELINE.json, global-layer
decode attention at pos 8191 (L = 8192), whole-job HBM GB/s with every input
resident in HBM: one step = one g3attn_decode_device call (QK-norm + RoPE +
cache write + split-K attention + combine, one kernel launch).  Steps rotate
over 10 distinct 64 MiB caches (two 34-layer contexts x 5 global layers,
640 MiB) so the 256 MB Infinity Cache cannot serve them.

Algorithmic bytes per decode call = fp32 K + V rows read (8192 B per
position, 4 KV heads x 256 x 4 B x 2) + q in + out = 8192*L + 16384.

`roofline` is for the decode kernel at the headline config: achieved =
algorithmic bytes / average kernel duration, the duration from paired HIP
events that the library records around every decode_kernel launch on its own
stream (g3attn_profile_*; the small split-combine launch is excluded and
reported separately as part of the per-call time).

Further configs (reported under "extra", not the headline): configs[0] local
decode L=512, 128K global-layer decode, the 34-layer decode stack at
pos 131071 (reference 29 local / 5 global pattern and the config's literal
28 / 6), configs[2] local prefill (N=2048, window 1024) and configs[3]
global prefill (N=8192).  Prefill FLOPs are algorithmic: 4 * H_q * d * P for
P attended (query, key) pairs.  The MFMA kernel issues 2.5x that in FLOPs:
for QK^T one fp16 pass and two fp8 cross-term passes (which run at twice the
fp16 rate), for PV two bf16 passes (three with values off the bf16 grid),
reported as "issued"; in MFMA-pipe time that is 2x the algorithmic work
(2.5x with the third PV pass), reported as "frac_of_mfma_peak_issued".  With
G3ATTN_PREFILL_QK=exact (three fp16 QK^T passes) both are 2.5x (3x).

The rows beyond the attention block, at Gemma3-4B shapes with random bf16
weights (sections `gemv` and `forward`): one layer's Q/K/V + O projection
GEMVs, the whole layer_attention at pos 8191, the model's upload from host
memory, one token through all 34 layers with the tied logits (HBM GB/s over
every weight byte plus the cache rows read), and the batched prefill of 2048
and 8192 tokens through the model (algorithmic TFLOP/s; its projections issue
2x their FLOPs on MFMA, x being carried as bf16 hi + lo).

`cpu_baseline`: the reference's own attention code (oracle/_ref, compiled
from the reference sources with its fast-mode flags, no BLAS) timed on one
host core for the headline workload: median of 20 decode steps.
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib.util
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
METRIC = "decode attn µs/token + HBM GB/s at 8K/128K ctx; prefill attn TFLOP/s at 8K"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2516.6
D, HQ, HKV = 256, 8, 4
QS, KS = HQ * D, HKV * D


def decode_bytes(L: int) -> int:
    return 8192 * L + 16384


def prefill_pairs(n: int, window: int) -> int:
    """Attended (query, key) pairs of a causal prefill from position 0."""
    return sum(min(i + 1, window) for i in range(n))


def prefill_flops(n: int, window: int) -> float:
    return 4.0 * HQ * D * prefill_pairs(n, window)


def measured_traffic(key):
    """HBM bytes per launch of a kernel from the committed rocprofv3 --pmc summary
    (profiles/traffic.json: FETCH_SIZE / WRITE_SIZE scaled by a copy of known
    size); None when absent."""
    try:
        with open(os.path.join(REPO, "profiles", "traffic.json")) as f:
            t = json.load(f)
        e = t[key]
        return round(e["fetch_kib"] * 1024 / t["fetch_scale"] + e["write_kib"] * 1024 / t["write_scale"])
    except (OSError, KeyError, ValueError):
        return None


def load_binding():
    spec = importlib.util.spec_from_file_location("g3attn", os.path.join(REPO, "gemma3.c_amd", "g3attn.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["g3attn"] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Bench:
    def __init__(self, G, torch):
        self.G, self.torch = G, torch
        self.dev = torch.device("cuda", 0)
        self.gen = torch.Generator(device=self.dev)
        self.gen.manual_seed(0x5EED0000)

    def randn_bf16(self, *shape):
        """Seeded N(0,1) rounded to bf16 (RNE), held as fp32 in HBM."""
        t = self.torch.randn(*shape, generator=self.gen, device=self.dev, dtype=self.torch.float32)
        return t.to(self.torch.bfloat16).to(self.torch.float32)

    def randn_f32(self, *shape):
        """Seeded N(0,1) in fp32 (not on the bf16 grid, like a real projection's output)."""
        return self.torch.randn(*shape, generator=self.gen, device=self.dev, dtype=self.torch.float32)

    def context(self, max_context, num_layers=34):
        G = self.G
        cfg = G.default_config(max_context=max_context, num_layers=num_layers)
        return G.Context(cfg, max_context)

    def fill_layer(self, ctx, layer, n_tokens, chunk=16384):
        """Cache rows 0..n-1 of one layer: seeded K (normed + RoPE'd on the GPU
        through g3attn_kv_append_device) and V."""
        zn = self.torch.zeros(D, dtype=self.torch.int16, device=self.dev)
        for s in range(0, n_tokens, chunk):
            n = min(chunk, n_tokens - s)
            K = self.randn_bf16(n, KS)
            V = self.randn_bf16(n, KS)
            self.torch.cuda.synchronize()
            ctx.kv_append_device(layer, s, n, K.data_ptr(), V.data_ptr(), zn.data_ptr())
            ctx.synchronize()

    def token_inputs(self, n=16):
        """n sets of (q, k, v) for one token, and unit-gain norm weights."""
        qkv = [(self.randn_bf16(QS), self.randn_bf16(KS), self.randn_bf16(KS)) for _ in range(n)]
        zn = self.torch.zeros(D, dtype=self.torch.int16, device=self.dev)
        self.torch.cuda.synchronize()
        return qkv, zn

    def time_calls(self, stream_ctx, calls, steps, warmup, prewarm_s=0.0):
        """Run `calls[i % len]` for warmup + steps on the library stream.
        Returns (region seconds, mean per-call seconds, host wall seconds): the
        region is bracketed by two events only, so back-to-back calls run as an
        engine would issue them; per-call times come from a second pass with an
        event pair around every call.  prewarm_s: first run the calls for that
        long (the part's clocks take tens of ms of MFMA load to settle: the
        first prefill calls run 15-25% slower than the settled ones)."""
        torch = self.torch
        s = torch.cuda.ExternalStream(stream_ctx.stream())
        t_end = time.perf_counter() + prewarm_s
        while time.perf_counter() < t_end:
            for f in calls:
                f()
            stream_ctx.synchronize()
        for i in range(warmup):
            calls[i % len(calls)]()
        stream_ctx.synchronize()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(s)
        for i in range(steps):
            calls[(warmup + i) % len(calls)]()
        e1.record(s)
        stream_ctx.synchronize()
        wall = time.perf_counter() - t0
        region = e0.elapsed_time(e1) * 1e-3
        starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
        for i in range(steps):
            starts[i].record(s)
            calls[(warmup + i) % len(calls)]()
            ends[i].record(s)
        stream_ctx.synchronize()
        per = [a.elapsed_time(b) * 1e-3 for a, b in zip(starts, ends)]
        return region, float(np.mean(per)), wall

    def kernel_time(self, ctx, calls, steps, kind):
        """Mean duration of the library's main kernel (kind 0 decode, 1 prefill)
        over `steps` calls, from the event pairs the library records around it."""
        ctx.profile(True)
        for i in range(steps):
            calls[i % len(calls)]()
        ms, n = ctx.profile_read(kind)
        ctx.profile(False)
        return ms * 1e-3 / max(n, 1)

    # ---------------------------------------------------------------- decode
    def decode_calls(self, targets, pos, qkv, zn, out):
        """targets: list of (ctx, layer).  One call per target, inputs rotating."""
        calls = []
        for i, (ctx, layer) in enumerate(targets):
            q, k, v = qkv[i % len(qkv)]

            def f(ctx=ctx, layer=layer, q=q, k=k, v=v):
                ctx.decode_device(layer, pos, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                  zn.data_ptr(), zn.data_ptr(), out.data_ptr())
            calls.append(f)
        return calls


def cpu_baseline(L=8192, reps=20):
    """The reference's attention section on one host core (oracle/_ref)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import g3_oracle as O
    kind = "reference" if O.have_ref() else "port"
    pos = L - 1
    K = O.gen_normal_bf16(L * KS, O.seed_for(2, 2)).reshape(L, KS)
    V = O.gen_normal_bf16(L * KS, O.seed_for(2, 3)).reshape(L, KS)
    zn = O.zero_norm()
    q = O.gen_normal_bf16(QS, O.seed_for(2, 1))
    k, v = K[pos].copy(), V[pos].copy()
    cfg = O.Config(max_context=L)
    if kind == "reference":
        t = O.rope_table(L, 1e6, use_ref=True)
        O.norm_rope_batch(K, t, 0, zn)  # rows as the cache holds them
        zp = zn.ctypes.data_as(C.c_void_p)
        sec = O.ref_timing().ref_time_decode(q, k, v, zp, zp, K, V, t, HQ, HKV, 5, pos, L, 1024, 3, reps)
    else:
        t = O.rope_table(L, 1e6)
        O.norm_rope_batch(K, t, 0, zn)
        ts = []
        for r in range(reps + 3):
            Kc, Vc = K.copy(), V.copy()
            a = time.perf_counter()
            O.layer_decode(cfg, 5, pos, q, k, v, Kc, Vc, t, zn, zn)
            if r >= 3:
                ts.append(time.perf_counter() - a)
        sec = float(np.median(ts))
    try:
        cpu_model = [l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name")][0]
    except Exception:
        cpu_model = "unknown"
    return {
        "value": round(decode_bytes(L) / sec / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": kind,
        "sample": (f"median of {reps} decode steps (configs[1]: L={L}, pos {pos}) after 3 warm-up, "
                   f"{sec * 1e6:.0f} us/step, 1 thread ({cpu_model}; nproc {os.cpu_count()}); "
                   "reference gemma3_kernels.c + gemma3_transformer.c built with "
                   f"-O3 -march={O.ref_timing_build()} -ffast-math (the reference's make fast flags; "
                   "x86-64-v4 is the AVX-512 width its -march=native gives on this host), "
                   "no BLAS (cblas.h absent)"),
    }


def _oracle():
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import g3_oracle as O
    return O


def cpu_gemv_baseline(hid=2560, layers=8, reps=3):
    """The reference's gemma3_matvec_bf16 (oracle/_ref) on one host core for
    one layer's Q, K, V and O projections (the GEMV row's workload), rotating
    over `layers` distinct layers' matrices so that they stream from DRAM."""
    O = _oracle()
    if not O.have_ref():
        return None
    pool = (np.random.default_rng(7).standard_normal(1 << 22) * 2.0 ** -6).astype(np.float32)
    pool = (pool.view(np.uint32) >> 16).astype(np.uint16)
    shapes = ((QS, hid), (KS, hid), (KS, hid), (hid, QS))
    mats = [[np.resize(np.roll(pool, 997 * (4 * l + j)), sh) for j, sh in enumerate(shapes)] for l in range(layers)]
    xs = [np.random.default_rng(8).standard_normal(sh[1]).astype(np.float32) for sh in shapes]
    R = O.ref_timing()
    ys = [np.empty(sh[0], np.float32) for sh in shapes]
    ts = []
    for r in range(reps + 1):
        a = time.perf_counter()
        for lm in mats:
            for m, x, y in zip(lm, xs, ys):
                R.ref_matvec_bf16(y, m, x, m.shape[0], m.shape[1])
        if r:
            ts.append((time.perf_counter() - a) / layers)
    sec = float(np.median(ts))
    byts = sum(m.nbytes for m in mats[0])
    return {"value": round(byts / sec / 1e9, 2), "unit": "GB/s", "cores": 1, "kind": "reference",
            "sample": f"median of {reps} passes over {layers} distinct layers' four projection matrices "
                      f"({layers * byts / 1e6:.0f} MB): {sec * 1e3:.2f} ms per layer, gemma3_matvec_bf16, "
                      f"1 thread, -march={O.ref_timing_build()}"}


def cpu_forward_baseline(HW, cfg, pos, n_tokens=2):
    """The reference's gemma3_transformer_forward (oracle/_ref, one thread, no
    BLAS) on the same host weights: seconds per token at positions pos.."""
    O = _oracle()
    if not O.have_ref():
        return None
    L = cfg.num_layers
    ptrs = (C.c_void_p * (13 * L))()
    names = [n for n, _ in type(HW.layers[0])._fields_]
    for l in range(L):
        for j, n in enumerate(names):
            ptrs[13 * l + j] = getattr(HW.layers[l], n)
    sec = O.ref_timing().ref_time_forward(HW.embed_tokens, ptrs, HW.norm, cfg.vocab_size, cfg.hidden_size,
                                   cfg.intermediate_size, L, cfg.num_heads, cfg.num_kv_heads,
                                   cfg.max_context, cfg.sliding_window, pos, n_tokens)
    return None if sec <= 0 else sec


def cpu_prefill_baseline():
    """The reference's prefill attention loop (gemma3_transformer.c:641-692 order,
    gemma3_gqa per token) on one host core, configs[2] in full (about 2 s)."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import g3_oracle as O
    n, layer = 2048, 0
    cfg = O.Config(max_context=8192)
    kind = "reference" if O.have_ref() else "port"
    t = O.rope_table(8192, cfg.theta(layer), use_ref=kind == "reference")
    s = lambda i: O.seed_for(3, i)
    Q = O.gen_normal_bf16(n * QS, s(1)).reshape(n, QS)
    K = O.gen_normal_bf16(n * KS, s(2)).reshape(n, KS)
    V = O.gen_normal_bf16(n * KS, s(3)).reshape(n, KS)
    Kc = np.zeros((cfg.cache_rows(layer), KS), np.float32)
    Vc = np.zeros_like(Kc)
    zn = O.zero_norm()
    a = time.perf_counter()
    if kind == "reference":
        O.ref_prefill(cfg, layer, 0, Q, K, V, Kc, Vc, t, zn, zn, lib=O.ref_timing())
    else:
        O.prefill(cfg, layer, 0, Q, K, V, Kc, Vc, t, zn, zn, threads=1)
    sec = time.perf_counter() - a
    flops = prefill_flops(n, 1024)
    return {"value": round(flops / sec / 1e12, 6), "unit": "algorithmic TFLOP/s", "cores": 1,
            "kind": kind, "sample": f"configs[2] in full (N={n}, window 1024), one run: {sec:.2f} s"
                                    + (f", -march={O.ref_timing_build()}" if kind == "reference" else "")}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list of sections to run (decode8k = the headline, local512, 128k, "
                         "stack, gemv, forward, prefill, or one prefill line: prefill_local_N2048_w1024, "
                         "prefill_global_N8192, prefill_global_N8192_fp32_values); default: all")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run 5 plain device-to-device copies of this many MiB (the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.copy_probe_mib > 0:
        import torch
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, device="cuda", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_mib": args.copy_probe_mib, "launches": 5,
                          "bytes_read_per_launch": n * 4, "bytes_written_per_launch": n * 4}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard by KV head or by sequence; no multi-GPU figure is "
              "produced)", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    G = load_binding()
    B = Bench(G, torch)
    only = set(filter(None, args.only.split(",")))
    extra = {}

    # ---------------- headline: configs[1] global decode, L = 8192
    value = ms_per_step = achieved = kernel_s = call_s = None
    qkv, zn = B.token_inputs()
    out = torch.empty(QS, device=B.dev, dtype=torch.float32)
    if not only or "decode8k" in only:
        L = 8192
        log("[bench] filling 2 x 34-layer contexts, 10 global layers x 8192 positions")
        ctxs = [B.context(L) for _ in range(2)]
        targets = []
        for ctx in ctxs:
            for layer in (5, 11, 17, 23, 29):
                B.fill_layer(ctx, layer, L - 1)
                targets.append((ctx, layer))
        calls = B.decode_calls(targets, L - 1, qkv, zn, out)
        # all calls go to ctx streams; both contexts are timed through ctx 0's
        # stream only if they share it, so time each context's calls separately
        log(f"[bench] headline decode L={L}: warmup {args.warmup}, steps {args.steps}")
        per_ctx = []
        for ci, ctx in enumerate(ctxs):
            cl = [c for c, (cx, _) in zip(calls, targets) if cx is ctx]
            region, per_call, wall = B.time_calls(ctx, cl, args.steps, args.warmup)
            per_ctx.append((region, per_call, B.kernel_time(ctx, cl, args.steps, 0)))
        region = float(np.mean([r for r, _, _ in per_ctx]))
        call_s = float(np.mean([c for _, c, _ in per_ctx]))
        kernel_s = float(np.mean([k for _, _, k in per_ctx]))
        ms_per_step = region / args.steps * 1e3
        value = decode_bytes(L) / (region / args.steps) / 1e9
        achieved = decode_bytes(L) / kernel_s / 1e9
        log(f"[bench] headline: {ms_per_step * 1e3:.2f} us/step, {value:.1f} GB/s; call {call_s * 1e6:.2f} us; "
            f"decode_kernel {kernel_s * 1e6:.2f} us -> {achieved:.1f} GB/s")
        for c in ctxs:
            c.close()
        del ctxs, targets, calls

    # ---------------- configs[1] through the host-pointer entry point (PCIe-inclusive)
    if not only or "decode8k_host" in only:
        ctx = B.context(8192)
        B.fill_layer(ctx, 5, 8191)
        hq = [np.ascontiguousarray(t.cpu().numpy()) for t in qkv[0]]
        hz = np.zeros(D, np.uint16)
        for _ in range(20):
            ctx.decode(5, 8191, hq[0], hq[1], hq[2], hz, hz)
        ts = []
        for _ in range(200):
            t0 = time.perf_counter()
            ctx.decode(5, 8191, hq[0], hq[1], hq[2], hz, hz)
            ts.append(time.perf_counter() - t0)
        extra["decode_global_L8192_host_pointers"] = {
            "config": "configs[1] through g3attn_decode (host q/k/v in, host attn_out out, blocking)",
            "us_per_call_median": round(float(np.median(ts)) * 1e6, 2),
            "note": "one 64 MiB cache (LLC-warm); adds 16 KiB up + 8 KiB down over PCIe and a host sync",
        }
        log(f"[bench] decode8k host pointers: {extra['decode_global_L8192_host_pointers']}")
        ctx.close()

    # ---------------- local decode at pos 511 (L = 512)
    if not only or "local512" in only:
        ctx = B.context(8192)
        locs = [l for l in range(34) if not G.is_global_layer(l)]
        for l in locs:
            B.fill_layer(ctx, l, 511)
        cl = B.decode_calls([(ctx, l) for l in locs], 511, qkv, zn, out)
        region, per, _ = B.time_calls(ctx, cl, 200, 20)
        ks = B.kernel_time(ctx, cl, 200, 0)
        extra["decode_local_L512"] = {
            "config": "configs[0]: local layer, pos 511, L=512, theta 1e4",
            "us_per_call": round(region / 200 * 1e6, 2),
            "call_us": round(per * 1e6, 2),
            "kernel_us": round(ks * 1e6, 2),
            "GB/s": round(decode_bytes(512) / (region / 200) / 1e9, 1),
            "bytes_per_call": decode_bytes(512),
            # one launch: the splits merged in one XCD's L2 (kernel_us then
            # covers the merge); else decode_kernel + combine_kernel
            "form": "one launch" if ctx.last_splits(2) else "decode + combine",
        }
        log(f"[bench] local512: {extra['decode_local_L512']}")
        ctx.close()

    # ---------------- 128K: single global layer and the 34-layer stack
    if not only or "128k" in only or "stack" in only:
        L = 131072
        log("[bench] filling a 36-layer context at max_context 131072 (6 global layers)")
        ctx = B.context(L, num_layers=36)
        glob = [l for l in range(36) if G.is_global_layer(l)]
        locs = [l for l in range(36) if not G.is_global_layer(l)]
        for l in glob:
            B.fill_layer(ctx, l, L - 1)
        for l in locs:
            B.fill_layer(ctx, l, 1024)
        pos = L - 1
        cl = B.decode_calls([(ctx, l) for l in glob], pos, qkv, zn, out)
        region, per, _ = B.time_calls(ctx, cl, 60, 6)
        ks = B.kernel_time(ctx, cl, 60, 0)
        extra["decode_global_L131072"] = {
            "config": "global layer, pos 131071, L=131072, theta 1e6; 6 distinct 1 GiB caches rotated",
            "us_per_call": round(region / 60 * 1e6, 2),
            "call_us": round(per * 1e6, 2),
            "kernel_us": round(ks * 1e6, 2),
            "GB/s": round(decode_bytes(L) / (region / 60) / 1e9, 1),
            "kernel_GB/s": round(decode_bytes(L) / ks / 1e9, 1),
            "frac_of_hbm_peak": round(decode_bytes(L) / ks / 1e9 / HBM_PEAK_GBS, 4),
            "bytes_per_call": decode_bytes(L),
        }
        log(f"[bench] 128k: {extra['decode_global_L131072']}")
        # 34-layer stack: one token through every layer's attention
        B.decode_calls([(ctx, locs[0])], pos, qkv, zn, out)[0]()
        local_form = "one launch" if ctx.last_splits(2) else "decode + combine"
        for name, layers in (("reference_29local_5global", list(range(34))),
                             ("literal_28local_6global", glob + locs[:28])):
            layers = sorted(layers)
            byts = sum(decode_bytes(L if G.is_global_layer(l) else 1024) for l in layers)
            cl = B.decode_calls([(ctx, l) for l in layers], pos, qkv, zn, out)

            def step(cl=cl):
                for f in cl:
                    f()
            region, per, _ = B.time_calls(ctx, [step], 20, 3)
            extra[f"decode_stack34_L131072_{name}"] = {
                "config": f"configs[4]: 34 layers ({name}), pos 131071",
                "us_per_token": round(region / 20 * 1e6, 1),
                "GB/s": round(byts / (region / 20) / 1e9, 1),
                "frac_of_hbm_peak": round(byts / (region / 20) / 1e9 / HBM_PEAK_GBS, 4),
                "bytes_per_token": byts,
                "local_layer_form": local_form,
            }
            log(f"[bench] stack {name}: {extra[f'decode_stack34_L131072_{name}']}")
        ctx.close()

    # ---------------- next row: the layer's Q/K/V and O projections (bf16 GEMV)
    if not only or "gemv" in only:
        ctx = B.context(8192)
        torch = B.torch
        hid = 2560
        nl = 34   # distinct weights per layer: 34 x 31.5 MB rotate past the 256 MB LLC

        def wbf16(r, c):
            return B.randn_bf16(r, c).mul_(2.0 ** -6).to(torch.bfloat16).view(torch.int16)
        Ws = [(wbf16(QS, hid), wbf16(KS, hid), wbf16(KS, hid), wbf16(hid, QS)) for _ in range(nl)]
        xs = B.randn_bf16(hid)
        qo, ko, vo = (torch.empty(n, device=B.dev) for n in (QS, KS, KS))
        attn_in = B.randn_bf16(QS)
        yo = torch.empty(hid, device=B.dev)
        torch.cuda.synchronize()
        gemv_bytes = 2 * hid * (QS + 2 * KS) + 2 * hid * QS

        def proj_calls():
            cl = []
            for wq, wk, wv, wo in Ws:
                def f(wq=wq, wk=wk, wv=wv, wo=wo):
                    ctx.qkv_proj_device(xs.data_ptr(), wq.data_ptr(), wk.data_ptr(), wv.data_ptr(),
                                        qo.data_ptr(), ko.data_ptr(), vo.data_ptr())
                    ctx.matvec_bf16_device(yo.data_ptr(), wo.data_ptr(), attn_in.data_ptr(), hid, QS)
                cl.append(f)
            return cl
        cl = proj_calls()
        region, per_call, _ = B.time_calls(ctx, cl, 340, 34)
        extra["gemv_qkv_o_projections"] = {
            "config": "one layer's Q/K/V projections (one fused launch) + O projection, Gemma3-4B "
                      "shapes (hidden 2560), bf16 weights, 34 distinct layers rotated (1.07 GB)",
            "us_per_layer": round(region / 340 * 1e6, 2),
            "call_us": round(per_call * 1e6, 2),
            "bytes_per_layer": gemv_bytes,
            "GB/s": round(gemv_bytes / (region / 340) / 1e9, 1),
            "frac_of_hbm_peak": round(gemv_bytes / (region / 340) / 1e9 / HBM_PEAK_GBS, 4),
        }
        if not args.no_cpu:
            extra["gemv_qkv_o_projections"]["cpu_baseline"] = cpu_gemv_baseline(hid)
        log(f"[bench] gemv: {extra['gemv_qkv_o_projections']}")
        # the whole of layer_attention at configs[1]'s position: projections +
        # attention over 8192 cached positions + o_proj, one entry point
        glob = [5, 11, 17, 23, 29]
        for l in glob:
            B.fill_layer(ctx, l, 8191)
        zn16 = torch.zeros(D, dtype=torch.int16, device=B.dev)
        la_out = torch.empty(hid, device=B.dev)
        torch.cuda.synchronize()
        la_calls = []
        for i, l in enumerate(glob):
            wq, wk, wv, wo = Ws[i]

            def f(l=l, wq=wq, wk=wk, wv=wv, wo=wo):
                ctx.layer_attention_device(l, 8191, xs.data_ptr(), wq.data_ptr(), wk.data_ptr(),
                                           wv.data_ptr(), wo.data_ptr(), zn16.data_ptr(),
                                           zn16.data_ptr(), la_out.data_ptr())
            la_calls.append(f)
        region, per_call, _ = B.time_calls(ctx, la_calls, 200, 20)
        la_bytes = gemv_bytes + decode_bytes(8192)
        extra["layer_attention_L8192"] = {
            "config": "the whole of layer_attention for one token at pos 8191 of a global layer: "
                      "Q/K/V projections, attention over 8192 positions, o_proj (5 layers rotated)",
            "us_per_layer": round(region / 200 * 1e6, 2),
            "bytes_per_layer": la_bytes,
            "GB/s": round(la_bytes / (region / 200) / 1e9, 1),
        }
        log(f"[bench] layer_attention 8K: {extra['layer_attention_L8192']}")
        ctx.close()
        del Ws

    # ---------------- next rows: the model uploaded from host memory, then one
    # token through the whole of it (34 layers, tied logits) at configs[1]'s
    # position, Gemma3-4B shapes, random weights
    if not only or "forward" in only:
        torch = B.torch
        ctx = B.context(8192)
        # every buffer is sized from the context's own config: the library reads
        # vocab_size rows of the embedding for the logits and writes vocab_size floats
        cfg = ctx.cfg
        hid, inter, vocab, nl = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size, cfg.num_layers
        assert (hid, inter, vocab, nl) == (2560, 10240, 262208, 34)
        shapes = {"input_layernorm": hid, "q_proj": QS * hid, "k_proj": KS * hid, "v_proj": KS * hid,
                  "o_proj": hid * QS, "q_norm": D, "k_norm": D, "post_attention_layernorm": hid,
                  "gate_proj": inter * hid, "up_proj": inter * hid, "down_proj": hid * inter,
                  "pre_feedforward_layernorm": hid, "post_feedforward_layernorm": hid}
        total = vocab * hid + hid + nl * sum(shapes.values())
        # host model: one pageable buffer (as a file mapping would be) tiled from a
        # 64 MiB pool of seeded N(0,1) * 2^-6 bf16 values
        pool_f = (np.random.default_rng(0x5EED).standard_normal(1 << 25) * 2.0 ** -6).astype(np.float32)
        pool = (pool_f.view(np.uint32) >> 16).astype(np.uint16)
        host = np.empty(total, np.uint16)
        for o in range(0, total, pool.size):
            n = min(pool.size, total - o)
            host[o:o + n] = pool[:n]
        HW, off = G.Weights(), 0

        def take(n):
            nonlocal off
            p = host[off:off + n].ctypes.data
            off += n
            return p
        HW.embed_tokens, HW.norm = take(vocab * hid), take(hid)
        for l in range(nl):
            for name, n in shapes.items():
                setattr(HW.layers[l], name, take(n))
        assert off == total
        t0 = time.perf_counter()
        ctx.upload_weights(HW)
        up_s = time.perf_counter() - t0
        extra["weight_upload"] = {
            "config": "g3attn_upload_weights of the whole Gemma3-4B-shaped model (every bf16 tensor, "
                      "%.2f GB) from pageable host memory through two pinned 32 MiB staging buffers"
                      % (2 * total / 1e9),
            "s": round(up_s, 3),
            "GB/s": round(2 * total / up_s / 1e9, 2),
        }
        log(f"[bench] upload: {extra['weight_upload']}")
        W = ctx.device_weights()
        logits = torch.empty(vocab, device=B.dev)
        torch.cuda.synchronize()
        pos = 8191
        layer_w = 2 * hid * (QS + 2 * KS) + 2 * hid * QS + 3 * 2 * hid * inter
        n_glob = sum(1 for l in range(nl) if G.is_global_layer(l))
        fwd_bytes = (nl * layer_w + 2 * vocab * hid + n_glob * decode_bytes(pos + 1)
                     + (nl - n_glob) * decode_bytes(1024))

        def fwd():
            ctx.forward_device(W, 2, pos, logits.data_ptr(), True)

        steps = 40
        region, per_call, _ = B.time_calls(ctx, [fwd], steps, 5)
        assert bool(torch.isfinite(logits).all())
        t = region / steps
        extra["forward_token_pos8191"] = {
            "config": "one token through all 34 layers + final norm + tied logits at pos 8191 on the "
                      "uploaded model, Gemma3-4B shapes (hidden 2560, intermediate 10240, vocab "
                      "262208), random bf16 weights, cache rows before pos zero; "
                      "g3attn_forward_device, device logits",
            "ms_per_token": round(t * 1e3, 3),
            "tokens_per_s": round(1.0 / t, 1),
            "bytes_per_token": fwd_bytes,
            "GB/s": round(fwd_bytes / t / 1e9, 1),
            "frac_of_hbm_peak": round(fwd_bytes / t / 1e9 / HBM_PEAK_GBS, 4),
        }
        log(f"[bench] forward: {extra['forward_token_pos8191']}")
        # the backend hook's blocking call: host logits, one host round trip per token
        for _ in range(3):
            ctx.forward_token(2, pos)
        t0 = time.perf_counter()
        for _ in range(20):
            lh = ctx.forward_token(2, pos)
        t_host = (time.perf_counter() - t0) / 20
        assert np.all(np.isfinite(lh))
        extra["forward_token_pos8191"]["host_logits_ms_per_token"] = round(t_host * 1e3, 3)
        if not args.no_cpu:
            # the reference's token forward on the same weights (host copy), one thread
            log("[bench] cpu forward baseline (reference, 1 core, 2 tokens at pos 8190-8191 "
                "and 2 at pos 1023-1024)")
            s_hi = cpu_forward_baseline(HW, cfg, pos - 1)
            s_lo = cpu_forward_baseline(HW, cfg, 1023)
            if s_hi:
                extra["forward_token_pos8191"]["cpu_baseline"] = {
                    "value": round(1.0 / s_hi, 3), "unit": "tokens/s", "cores": 1, "kind": "reference",
                    "sample": f"gemma3_transformer_forward, median of 2 tokens at pos 8190-8191 after one "
                              f"warm-up token: {s_hi:.2f} s per token, 1 thread, no BLAS, same weights, "
                              f"-march={_oracle().ref_timing_build()}"}
            if s_lo:
                extra["cpu_prefill_model_token_loop"] = {
                    "value": round(1.0 / s_lo, 3), "unit": "tokens/s", "cores": 1, "kind": "reference",
                    "sample": f"the non-BLAS reference prefill is this token loop "
                              f"(gemma3_transformer.c:814-821): gemma3_transformer_forward at pos "
                              f"1023-1024, {s_lo:.2f} s per token, 1 thread, -march={_oracle().ref_timing_build()} "
                              f"(the BLAS build's batched prefill needs cblas.h, absent)"}
        del host

        # the batched prefill (MFMA projections + the prefill attention kernel)
        # of configs[2]'s length through the whole model
        for ntok in (2048, 8192):
            toks = (np.arange(ntok, dtype=np.int32) * 7919 % (vocab - 2) + 2).astype(np.int32)

            def pf(toks=toks):
                ctx.prefill_forward_device(W, toks, 0, logits.data_ptr())
            steps = 4 if ntok == 2048 else 2
            region, _, _ = B.time_calls(ctx, [pf], steps, 1, prewarm_s=0.2)
            assert bool(torch.isfinite(logits).all())
            t = region / steps
            gemm_flops = 2.0 * ntok * nl * (layer_w // 2)
            attn_flops = sum(prefill_flops(ntok, 1 << 30 if G.is_global_layer(l) else cfg.sliding_window)
                             for l in range(nl))
            extra[f"prefill_model_N{ntok}"] = {
                "config": f"g3attn_prefill_forward_device: {ntok} tokens from position 0 through all 34 "
                          "layers + the last token's logits, Gemma3-4B shapes, random bf16 weights; "
                          "projections as MFMA GEMMs (x as bf16 hi + lo: 2x the algorithmic MFMA work)",
                "ms": round(t * 1e3, 2),
                "tokens_per_s": round(ntok / t, 1),
                "projection_TFLOP": round(gemm_flops / 1e12, 2),
                "attention_TFLOP": round(attn_flops / 1e12, 3),
                "TFLOP/s": round((gemm_flops + attn_flops) / t / 1e12, 1),
                "frac_of_bf16_peak": round((gemm_flops + attn_flops) / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            }
            log(f"[bench] prefill model: {extra[f'prefill_model_N{ntok}']}")
        ctx.close()

    # ---------------- prefill.  The configs' inputs are
    # bf16-valued; the fp32 line feeds values off the bf16 grid, which takes the
    # kernel's extra P_hi.V_lo pass.  Issued FLOPs: QK^T 3x its half of the
    # algorithmic work, PV 2x (3x); MFMA-pipe time: QK^T 2x under the default
    # fp8 cross policy (its two fp8 passes at twice the rate), 3x exact.
    exact_qk = os.environ.get("G3ATTN_PREFILL_QK") == "exact"
    for name, layer, n, window, steps, f32 in (
            ("prefill_local_N2048_w1024", 0, 2048, 1024, 30, False),
            ("prefill_global_N8192", 5, 8192, 1 << 30, 8, False),
            ("prefill_global_N8192_fp32_values", 5, 8192, 1 << 30, 8, True)):
        if only and "prefill" not in only and name not in only:
            continue
        ctx = B.context(8192)
        gen = B.randn_f32 if f32 else B.randn_bf16
        Q, K, V = gen(n, QS), gen(n, KS), gen(n, KS)
        passes = 3.0 if f32 else 2.5                       # issued FLOPs / algorithmic
        pv = 3.0 if f32 else 2.0
        pipe = (3.0 if exact_qk else 2.0) / 2 + pv / 2    # MFMA-pipe time / algorithmic at the bf16 rate
        zn16 = torch.zeros(D, dtype=torch.int16, device=B.dev)
        pout = torch.empty(n, QS, device=B.dev, dtype=torch.float32)
        torch.cuda.synchronize()

        def pf(ctx=ctx, layer=layer, n=n, Q=Q, K=K, V=V, zn16=zn16, pout=pout):
            ctx.prefill_device(layer, 0, n, Q.data_ptr(), K.data_ptr(), V.data_ptr(),
                               zn16.data_ptr(), zn16.data_ptr(), pout.data_ptr())
        region, per_call, _ = B.time_calls(ctx, [pf], steps, 3, prewarm_s=0.2)
        k_s = B.kernel_time(ctx, [pf], steps, 1)
        flops = prefill_flops(n, window)
        extra[name] = {
            "config": (f"configs[{2 if layer == 0 else 3}]: {'local' if layer == 0 else 'global'} "
                       f"prefill, N={n}, start 0" + (f", window {window}" if window < n else "")
                       + (", fp32 inputs off the bf16 grid" if f32 else "")),
            "us_per_call": round(region / steps * 1e6, 1),
            "kernel_us": round(k_s * 1e6, 1),
            "pairs": prefill_pairs(n, window),
            "algorithmic_GFLOP": round(flops / 1e9, 3),
            "algorithmic_TFLOP/s_call": round(flops / (region / steps) / 1e12, 1),
            "algorithmic_TFLOP/s_kernel": round(flops / k_s / 1e12, 1),
            "issued_MFMA_TFLOP/s_kernel": round(passes * flops / k_s / 1e12, 1),
            "frac_of_bf16_peak_algorithmic": round(flops / k_s / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "frac_of_bf16_peak_issued": round(passes * flops / k_s / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "frac_of_mfma_peak_issued": round(pipe * flops / k_s / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "score_policy": "fp16 x3 (exact)" if exact_qk else "fp16 hi + fp8 cross terms",
        }
        log(f"[bench] {name}: {extra[name]}")
        ctx.close()
        del Q, K, V, pout

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (reference code, 1 core)")
        cpu = cpu_baseline()
        log(f"[bench] cpu: {cpu}")
        if not only or "prefill" in only:
            extra["cpu_prefill_local_N2048_w1024"] = cpu_prefill_baseline()
            log(f"[bench] cpu prefill: {extra['cpu_prefill_local_N2048_w1024']}")

    line = {
        "metric": METRIC,
        "value": None if value is None else round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None if ms_per_step is None else round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,1) rounded to bf16, unit-gain QK-norm, RoPE theta 1e6",
        "config": {
            "workload": "configs[1]: global-layer decode attention, batch 1, pos 8191, L=8192, "
                        "8 Q / 4 KV heads, head_dim 256, fp32 KV cache",
            "us_per_token": None if ms_per_step is None else round(ms_per_step * 1e3, 3),
            "bytes_per_step": decode_bytes(8192),
            "llc": "each timed region rotates 5 distinct 64 MiB caches (320 MiB > 256 MB Infinity Cache); two such contexts are timed in turn and averaged",
        },
        "roofline": None if achieved is None else {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic("decode_kernel<2,true,true>@configs[1]"),
            "traffic_source": "profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE, copy-calibrated)",
            "kernel": "decode_kernel<2,true,true>",
            "kernel_us": round(kernel_s * 1e6, 3),
            "call_us": round(call_s * 1e6, 3),
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
