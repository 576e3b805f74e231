"""Decode-throughput benchmark of the MI355X hot path (one GPU).

Workload: one BitNet-b1.58-2B-shaped greedy decode
step at batch 1 and 4096 tokens of context - 30 layers of TL1 ternary
projections (hidden 2560, FFN 6912, 20 q / 5 kv heads of 128), INT8 KV cache
with fp16 scales prefilled with 4096 quantized N(0,1) tokens, int8 LM head over
vocab 128256, RoPE theta 500000. Weights are random-init of that architecture,
generated on the device. A step is the whole token: embedding, 30 layers, LM
head and greedy argmax. The timed run is `--steps` greedy tokens decoded back
to back from position 4096 with each token fed to the next step on the
device (tenzo_hip_engine_decode); the rate of the reference API's per-token
loop (tenzo_generate_step, token returned to the host, cache rewound to 4096
each time) is reported beside it.

Prints ONE JSON line: tok/s, the step's HBM bytes / time against the 8 TB/s
peak, a roofline entry for the dominant kernel (its algorithmic bytes / its
mean launch time, both measured here with HIP events on the stream the kernel
runs on), and the reference CPU path (oracle/_ref, compiled from the
reference's own sources) timed on a bounded sample on the host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--ctx 4096] [--no-cpu]
    python bench.py --prefill N   # prompt prefill throughput instead (own JSON line)
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

# The reference CPU legs (the compiled reference engine in this process, the
# single-kernel configs in a child) run with OpenMP threads placed one per
# core and spread, as the reference's Makefile runs its benchmarks; OpenMP
# reads these once, when its runtime starts, so they are set before anything
# loads it (a caller's own setting wins).
os.environ.setdefault("OMP_PLACES", "cores")
os.environ.setdefault("OMP_PROC_BIND", "spread")

import numpy as np  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
SEED = 2


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-config kernel leg (BASELINE configs 1, 3, 4, 5)")
    ap.add_argument("--configs-only", action="store_true",
                    help="run only the per-config kernel leg (for profiling it)")
    ap.add_argument("--cpu-configs-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--stage-trace", action="store_true",
                    help="print only the persistent kernel's per-stage trace (JSON line)")
    ap.add_argument("--mode", default="persistent", choices=["persistent", "graph", "eager"],
                    help="engine execution mode (one persistent kernel per token, or one "
                         "kernel per stage replayed from a HIP graph / launched eagerly)")
    ap.add_argument("--kv-mode", default="int8_fused",
                    choices=["int8_fused", "tl1_fused", "popcount_fused", "paged_int8"],
                    help="KV cache mode; the ternary modes print their own JSON line (decode on "
                         "the graph path and the ternary attention kernel's roofline)")
    ap.add_argument("--prefill", type=int, default=0, metavar="N",
                    help="instead of the decode benchmark: prefill an N-token prompt with "
                         "tenzo_hip_engine_prefill (--steps timed prompts) beside the "
                         "token-by-token tenzo_prefill_token rate; prints its own JSON line")
    ap.add_argument("--tl1-methods", action="store_true",
                    help="time the masked-v_dot4 TL1 GEMV against the reference's table "
                         "method at 6912x2560 and 65536x8192, print one JSON line, exit")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: one calibration copy of PROBE_COPY_BYTES "
                         "(a plain copy kernel of known size), then --steps chained decode "
                         "steps; prints no JSON line")
    return ap.parse_args()


PROBE_COPY_BYTES = 256 << 20
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_step_hbm_traffic.md")


def measured_traffic():
    """HBM bytes per decode_step_kernel launch as measured by rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration) and
    recorded in profiles/decode_step_hbm_traffic.md, with the source it was
    measured on; None if that file is absent."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


# ---------------------------------------------------------------- synthetic

def tl1_random_dev(torch, n_bytes, gen):
    """TL1 bytes of iid ternary weights (P = 1/3 each) generated on the GPU."""
    v = torch.randint(0, 9, (2, n_bytes), dtype=torch.uint8, device="cuda", generator=gen)
    nib = (v % 3) | ((v // 3) << 2)
    return (nib[0] | (nib[1] << 4)).contiguous()


def tern_rows_dev(torch, shape, planes, gen):
    """Random ternary cache rows (P(-1) = P(+1) = 0.345, P(0) = 0.31) packed on
    the GPU: 2-bit fields (w + 1) four to a byte, or sign bitplanes
    {kp0, kp1, kn0, kn1} when planes."""
    u = torch.rand(shape + (128,), device="cuda", generator=gen)
    w = (u > 0.345).to(torch.int16) + (u > 0.655).to(torch.int16) - 1
    if planes:
        bit = (2 ** torch.arange(8, device="cuda", dtype=torch.int16))
        pos = ((w > 0).to(torch.int16).reshape(shape + (16, 8)) * bit).sum(-1)
        neg = ((w < 0).to(torch.int16).reshape(shape + (16, 8)) * bit).sum(-1)
        return torch.cat([pos, neg], dim=-1).to(torch.uint8).contiguous()
    f = (w + 1).reshape(shape + (32, 4))
    return (f[..., 0] | (f[..., 1] << 2) | (f[..., 2] << 4) | (f[..., 3] << 6)).to(
        torch.uint8).contiguous()


def build_model(torch, cfg, ctx, kv_mode="int8_fused"):
    from tenzo_amd import engine, synth
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED)
    rng = np.random.default_rng(SEED)
    e = engine.Engine(cfg, kv_mode=kv_mode)
    host = {"layers": []}
    for l in range(cfg.n_layers):
        tl1 = {p: tl1_random_dev(torch, n * k // 4, gen)
               for p, (n, k) in ((p, cfg.proj_shape(p)) for p in synth.PROJ)}
        scale = {p: synth.latent_scale(rng) for p in synth.PROJ}
        norms = {f: (1.0 + 0.1 * rng.standard_normal(cfg.ffn if f == "ffn_sub_norm" else
                                                    cfg.hidden)).astype(np.float32)
                 for f in ("in_norm", "attn_sub_norm", "post_norm", "ffn_sub_norm")}
        w = engine.LayerWeights()
        for p, f in zip(synth.PROJ, ["q", "k", "v", "out", "gate", "up", "down"]):
            setattr(w, f + "_w", tl1[p].data_ptr())
            setattr(w, f + "_scale", float(scale[p]))
        for f, a in norms.items():
            setattr(w, f, a.ctypes.data)
        e._check(e.L.tenzo_set_layer_weights(e.h, l, ctypes.byref(w)), "set_layer_weights")
        host["layers"].append((tl1, scale, norms))
    final_norm = (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
    e._check(e.L.tenzo_set_final_norm(e.h, final_norm.ctypes.data), "set_final_norm")
    # LM head / tied embedding: latent N(0, 0.02), per-row int8 (load_model_from_files rule)
    V, H = cfg.vocab, cfg.hidden
    head = torch.empty((V, H), dtype=torch.int8, device="cuda")
    hs = torch.empty(V, dtype=torch.float32, device="cuda")
    for r0 in range(0, V, 16384):
        E = torch.randn((min(16384, V - r0), H), device="cuda", generator=gen) * 0.02
        amax = E.abs().amax(dim=1).clamp_min(1e-8)
        s = amax * (1.0 / 127.0)
        head[r0:r0 + E.shape[0]] = torch.clamp(torch.round(E * (127.0 / amax)[:, None]),
                                               -127, 127).to(torch.int8)
        hs[r0:r0 + E.shape[0]] = s
    e._check(e.L.tenzo_set_lm_head_i8(e.h, head.data_ptr(), hs.data_ptr(), V, H),
             "set_lm_head_i8")
    L, Hkv = cfg.n_layers, cfg.n_kv_heads
    if kv_mode in ("tl1_fused", "popcount_fused"):
        kb = tern_rows_dev(torch, (L, Hkv, ctx), kv_mode == "popcount_fused", gen)
        vb = tern_rows_dev(torch, (L, Hkv, ctx), False, gen)
        ks = torch.rand((L, Hkv, ctx), device="cuda", generator=gen) * 0.6 + 0.9
        vs = torch.rand((L, Hkv, ctx), device="cuda", generator=gen) * 0.6 + 0.9
        if ctx > 0:
            e.set_kv_device(kb.data_ptr(), vb.data_ptr(), ks.data_ptr(), vs.data_ptr(), ctx)
        e.set_rope_theta(cfg.theta)
        torch.cuda.synchronize()
        host.update(final_norm=final_norm, head=head, hs=hs, kc=kb, vc=vb, ks=ks, vs=vs)
        return e, host
    # INT8 KV cache: ctx tokens of N(0,1) per (layer, kv head), quantized per token
    kc = torch.empty((L, Hkv, ctx, 128), dtype=torch.int8, device="cuda")
    vc = torch.empty_like(kc)
    # fp16 scales (BASELINE); paged_int8 keeps the reference's fp32
    sdt = torch.float32 if kv_mode == "paged_int8" else torch.float16
    ks = torch.empty((L, Hkv, ctx), dtype=sdt, device="cuda")
    vs = torch.empty_like(ks)
    for c, s in ((kc, ks), (vc, vs)):
        for l in range(L):
            x = torch.randn((Hkv, ctx, 128), device="cuda", generator=gen)
            amax = x.abs().amax(dim=2).clamp_min(1e-8)
            c[l] = torch.clamp(torch.round(x * (127.0 / amax)[..., None]), -128, 127).to(torch.int8)
            s[l] = (amax * (1.0 / 127.0)).to(sdt)
    if ctx > 0:
        e.set_kv_device(kc.data_ptr(), vc.data_ptr(), ks.data_ptr(), vs.data_ptr(), ctx)
    e.set_rope_theta(cfg.theta)
    torch.cuda.synchronize()
    host.update(final_norm=final_norm, head=head, hs=hs, kc=kc, vc=vc, ks=ks, vs=vs)
    return e, host


# ------------------------------------------------------------------- roofline

def graph_time(torch, fn, reps):
    """Mean duration of one fn() call: fn's launches are captured into a HIP
    graph (no host overhead between them) and the graph is replayed reps times
    between two HIP events on the replay stream."""
    fn()  # first call outside the capture (allocates any library scratch)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    s = torch.cuda.current_stream()
    g.replay()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(s)
    for _ in range(reps):
        g.replay()
    end.record(s)
    end.synchronize()
    return start.elapsed_time(end) / 1e3 / reps


def tl1_roofline(torch, cfg, host):
    """The TL1 GEMV as the engine runs it per token: 4 launches per layer over
    every layer's own weights (521 MB, so the reads come from HBM), replayed
    from a graph and timed with HIP events (the time includes the gaps between
    launches). Algorithmic bytes per launch = packed ternary weights N*K/4 +
    int8 activation codes + fp32 outputs."""
    from tenzo_amd import ops
    H, F, qd, kvd = cfg.hidden, cfg.ffn, cfg.q_dim, cfg.kv_dim
    shapes = [(qd + 2 * kvd, H), (H, H), (2 * F, H), (H, F)]
    packed = []
    for tl1, _, _ in host["layers"]:
        cat_qkv = torch.cat([tl1["q"], tl1["k"], tl1["v"]])
        cat_gu = torch.cat([tl1["gate"], tl1["up"]])
        mats = [cat_qkv, tl1["o"], cat_gu, tl1["down"]]
        packed.append([ops.tl1_repack(m, n, k) for m, (n, k) in zip(mats, shapes)])
    xs = {k: torch.randn(k, device="cuda") for k in (H, F)}
    qs = {k: ops.rmsnorm_quant31(xs[k], None) for k in (H, F)}
    ys = {n: torch.empty(n, device="cuda") for n, _ in shapes}
    def one_token():
        for layer in packed:
            for wp, (n, k) in zip(layer, shapes):
                codes, q, _ = qs[k]
                ops.bitlinear_tl1_into(codes, q, wp, 0.0159, n, k, ys[n])

    t = graph_time(torch, one_token, 5)
    launches = len(packed) * len(shapes)
    alg = sum(n * k // 4 + (k + 63) // 64 * 64 + n * 4 for n, k in shapes) * len(packed)
    return {"kernel": "tl1_gemv_kernel", "launches_per_token": launches,
            "mean_launch_us": t / launches * 1e6, "alg_bytes_per_launch": alg / launches,
            "achieved_gbs": alg / t / 1e9}


def head_roofline(torch, cfg, host):
    """The int8 LM-head GEMV (engine path: fused greedy argmax) over the
    model's 328 MB table. Algorithmic bytes = table + row scales + codes +
    logits."""
    from tenzo_amd import ops
    V, H = cfg.vocab, cfg.hidden
    wp = ops.i8_rows_repack(host["head"], V, H)
    x = torch.randn(H, device="cuda")
    codes, q = ops.actquant127(x)
    logits = torch.empty(V, device="cuda")
    idx = torch.empty(1, dtype=torch.int32, device="cuda")
    t = graph_time(torch, lambda: ops.lm_head_i8_codes_into(codes, q, wp, host["hs"], V, H,
                                                            logits, idx), 20)
    alg = V * H + V * 4 + H + V * 4
    return {"kernel": "lm_head_i8_kernel", "launches_per_token": 1, "mean_launch_us": t * 1e6,
            "alg_bytes_per_launch": alg, "achieved_gbs": alg / t / 1e9}


# ---------------------------------------------------------------- CPU leg

def cpu_baseline(torch, cfg, host, ctx, seconds):
    """The reference's own CPU engine (oracle/_ref/libtenzo_ref.so, compiled
    from the reference sources with its flags) on the same weights and cache,
    timed on a bounded sample of greedy decode steps at position ctx."""
    import oracle
    if not oracle.ref_available():
        return {"value": None, "unit": "tok/s", "cores": 0, "kind": "reference",
                "sample": "oracle/_ref not built on this host"}
    from tenzo_amd import synth
    R = oracle.ref()
    P = oracle._ptr
    L, Hkv = cfg.n_layers, cfg.n_kv_heads
    layers = []
    for tl1, scale, norms in host["layers"]:
        lw = synth.LayerWeights({p: tl1[p].cpu().numpy() for p in synth.PROJ}, scale,
                                norms["in_norm"], norms["attn_sub_norm"], norms["post_norm"],
                                norms["ffn_sub_norm"])
        layers.append(lw)
    max_seq = ctx + 8
    kc = np.zeros((L, Hkv, max_seq, 128), np.int8)
    vc = np.zeros_like(kc)
    ks = np.zeros((L, Hkv, max_seq), np.float32)
    vs = np.zeros_like(ks)
    kc[:, :, :ctx] = host["kc"].cpu().numpy()
    vc[:, :, :ctx] = host["vc"].cpu().numpy()
    ks[:, :, :ctx] = host["ks"].float().cpu().numpy()
    vs[:, :, :ctx] = host["vs"].float().cpu().numpy()
    sm = synth.SynthModel(synth.DecodeConfig(max_seq=max_seq), layers, host["final_norm"],
                          host["head"].cpu().numpy(), host["hs"].cpu().numpy(), kc, vc, ks, vs,
                          ctx)
    e = R.ref_engine_create(cfg.hidden, cfg.n_q_heads, cfg.n_kv_heads, L, cfg.ffn, cfg.vocab,
                            max_seq)
    keep = [oracle.ref_layer_struct(sm, l) for l in range(L)]
    for l, w in enumerate(keep):
        R.ref_engine_set_layer(e, l, ctypes.byref(w))
    R.ref_engine_set_head(e, P(sm.embed), P(sm.embed_scales), P(sm.final_norm), cfg.vocab,
                          cfg.hidden)
    times = []
    tok = 1
    t_end = time.perf_counter() + seconds
    while len(times) < 2 or (time.perf_counter() < t_end and len(times) < 50):
        R.ref_engine_set_kv(e, P(kc), P(vc), P(ks), P(vs), ctx)
        t0 = time.perf_counter()
        tok = R.ref_engine_step(e, tok, None)
        times.append(time.perf_counter() - t0)
    threads = R.ref_num_threads()
    R.ref_engine_destroy(e)
    med = float(np.median(times[1:] if len(times) > 2 else times))
    return {"value": 1.0 / med, "unit": "tok/s", "cores": int(threads), "kind": "reference",
            "sample": f"{len(times)} greedy decode steps at position {ctx} of the same model "
                      f"(median {med * 1e3:.1f} ms/token; reference TenzoEngine.cpp compiled "
                      f"with its own flags, OpenMP {threads} threads)"}


def mfma_roofline(torch, cfg, host, M):
    """The int8 MFMA contraction as the batched prefill runs it: the four
    projections of one layer at M rows (the whole pass), each replayed from a
    graph and timed with HIP events. Algorithmic work = 2*M*N*K integer ops;
    the dominant (largest) projection is reported against the 5.0 POP/s dense
    int8 peak."""
    from tenzo_amd import ops
    H, F, qd, kvd = cfg.hidden, cfg.ffn, cfg.q_dim, cfg.kv_dim
    tl1, _, _ = host["layers"][0]
    mats = {"qkv": (torch.cat([tl1["q"], tl1["k"], tl1["v"]]), qd + 2 * kvd, H),
            "o": (tl1["o"], H, H), "gate_up": (torch.cat([tl1["gate"], tl1["up"]]), 2 * F, H),
            "down": (tl1["down"], H, F)}
    out = {}
    reps = 20  # launches per captured graph, so replay overhead is amortised
    for name, (w, n, k) in mats.items():
        wp = ops.tl1_repack(w, n, k)
        codes, q, _ = ops.rmsnorm_quant31(torch.randn(M, k, device="cuda"), None)
        y = torch.empty((M, n), device="cuda")

        def launches():
            for _ in range(reps):
                ops.bitlinear_tl1_batch(codes, q, wp, 0.0159, n, k, y=y)

        t = graph_time(torch, launches, 5) / reps
        out[name] = {"N": n, "K": k, "us": round(t * 1e6, 2),
                     "tops": round(2.0 * M * n * k / t / 1e12, 1)}
    return out


def prefill_bench(torch, e, cfg, host, args):
    n = args.prefill
    if n > cfg.max_seq:
        raise SystemExit(f"--prefill {n} exceeds the context ({cfg.max_seq})")
    toks = np.random.default_rng(SEED).integers(0, cfg.vocab, n).astype(np.int32)
    e.rewind(0)
    e.prefill_batch(toks[:min(n, 64)])  # first use allocates the prefill buffers
    for _ in range(max(args.warmup, 1)):
        e.rewind(0)
        e.prefill_batch(toks)
    times = []
    for _ in range(args.steps):
        e.rewind(0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e.prefill_batch(toks)  # streaming attention; returns after the device finished
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    # the exact form (chunked attention, bit for bit the per-token kernels' results)
    e.rewind(0)
    e.prefill_batch(toks, exact=True)
    xt = []
    for _ in range(args.steps):
        e.rewind(0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e.prefill_batch(toks, exact=True)
        xt.append(time.perf_counter() - t0)
    dt_exact = float(np.median(xt))
    # the reference's way: one prefill_token per prompt token (persistent kernel)
    seq_n = min(n, 64)
    e.rewind(0)
    for t in toks[:4]:
        e.prefill(int(t))
    e.rewind(0)
    t0 = time.perf_counter()
    for t in toks[:seq_n]:
        e.prefill(int(t))
    seq_rate = seq_n / (time.perf_counter() - t0)
    rows = min(n, 512)
    roof = mfma_roofline(torch, cfg, host, rows)
    dom = max(roof.values(), key=lambda r: r["N"] * r["K"])
    # the headline is the exact form (the per-token path's results bit for bit); the
    # streaming form's attention sums in another order, so its KV codes can differ from the
    # per-token path's at rounding ties, and it is reported beside it
    out = {
        "metric": "prefill_tokens_per_s", "value": round(n / dt_exact, 1), "unit": "tok/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt_exact * 1e3, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"BitNet-b1.58-2B-shaped prompt prefill, {n} tokens from "
                               "position 0, batch 1 (tenzo_hip_engine_prefill, exact form)",
                   "prompt_tokens": n, "rows_per_pass": 512},
        "streaming_tok_s": round(n / dt, 1),
        "token_by_token_tok_s": round(seq_rate, 1),
        "speedup_vs_token_by_token": round(n / dt_exact / seq_rate, 1),
        "roofline": {"bound": "mfma", "kernel": "tl1_mfma_kernel (gate|up projection)",
                     "achieved": dom["tops"], "peak": 5000.0, "unit": "TOP/s",
                     "frac": round(dom["tops"] / 5000.0, 4), "traffic": None,
                     "rows": rows, "per_projection": roof},
    }
    print(json.dumps(out), flush=True)


TERN_ROW_BYTES = 32 + 32 + 4 + 4  # K row, V row, two fp32 scales per (kv head, token)
PAGED_ROW_BYTES = 128 + 128 + 4 + 4


def tern_bench(torch, e, cfg, host, args):
    """Decode with a ternary or paged KV cache (the engine mode asked for,
    persistent by default) and the mode's attention op at one layer's shape."""
    from tenzo_amd import ops
    ctx, mode = args.ctx, args.kv_mode
    tok = 1
    e.rewind(ctx)
    e.decode(tok, max(args.warmup, 1))
    e.rewind(ctx)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e.decode(tok, args.steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    # the attention op over layer 0's cache at position ctx (one kv append +
    # attention + chunk merge per call), replayed from a graph
    Hq, Hkv = cfg.n_q_heads, cfg.n_kv_heads
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED + 1)
    S = ctx + 1
    if mode != "paged_int8":
        kb = torch.zeros((1, Hkv, S, 32), dtype=torch.uint8, device="cuda")
        vb = torch.zeros_like(kb)
        ks = torch.zeros((1, Hkv, S), dtype=torch.float32, device="cuda")
        vs = torch.zeros_like(ks)
        kb[0, :, :ctx] = host["kc"][0]
        vb[0, :, :ctx] = host["vc"][0]
        ks[0, :, :ctx] = host["ks"][0]
        vs[0, :, :ctx] = host["vs"][0]
    q = torch.randn((1, Hq * 128), device="cuda", generator=gen)
    k = torch.randn((1, Hkv * 128), device="cuda", generator=gen)
    v = torch.randn((1, Hkv * 128), device="cuda", generator=gen)
    cs = ops.rope_table(cfg.theta, ctx, 1)[0].cuda()
    if mode == "paged_int8":
        # layer 0's cache in blocks 0, 1, ... (the engine's allocation order)
        nb = (S + 15) // 16

        def pool(x, width):
            full = torch.zeros((Hkv, nb * 16) + width, dtype=x.dtype, device="cuda")
            full[:, :ctx] = x[0]
            return full.reshape((Hkv, nb, 16) + width).transpose(0, 1).unsqueeze(1).contiguous()
        pk, pv = pool(host["kc"], (128,)), pool(host["vc"], (128,))
        pks, pvs = pool(host["ks"], ()), pool(host["vs"], ())
        bt = torch.arange(nb, dtype=torch.int32, device="cuda")
        kernel = "paged_scores + softmax + values + sum kernels"
        att_s = graph_time(torch, lambda: ops.attn_paged_int8_decode(q, k, v, pk, pv, pks, pvs, bt,
                                                                     0, cs, ctx), 200)
        att_bytes = Hkv * S * PAGED_ROW_BYTES + (2 * Hq + 2 * Hkv) * 128 * 4
    else:
        kernel = "attn_tern_chunk_kernel + attn_combine_kernel"
        att_s = graph_time(torch, lambda: ops.attn_tern_decode(mode, q, k, v, kb, vb, ks, vs, cs,
                                                               ctx), 200)
        att_bytes = Hkv * S * TERN_ROW_BYTES + (2 * Hq + 2 * Hkv) * 128 * 4
    gbs = att_bytes / att_s / 1e9
    cpu = None
    if not args.no_cpu and mode == "paged_int8":
        import oracle
        if oracle.ref_available():
            P = oracle._ptr
            hp = [t.cpu().numpy().copy() for t in (pk, pv, pks, pvs)]
            btn = bt.cpu().numpy().copy()
            qh, kh, vh = (t.cpu().numpy()[0] for t in (q, k, v))
            out = np.zeros(Hq * 128, np.float32)
            R = oracle.ref()
            n, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0) or n < 3:
                R.ref_attention_paged(Hq, Hkv, 1, 0, nb, ctx, P(qh.copy()), P(kh.copy()), P(vh),
                                      *(P(a) for a in hp), P(btn.copy()), (ctx + 15) // 16, P(out))
                n += 1
            cpu = {"value": round(n / (time.perf_counter() - t0), 2), "unit": "attention calls/s",
                   "cores": 1, "kind": "reference",
                   "sample": f"PagedKVCache::forward_attention_raw, one layer, Hq {Hq} Hkv {Hkv}, "
                             f"position {ctx}, {n} calls (single-threaded in the reference)"}
    elif not args.no_cpu:
        import oracle
        if oracle.ref_available():
            P = oracle._ptr
            m = 1 if mode == "tl1_fused" else 2
            hk = [t.cpu().numpy()[0].copy() for t in (kb, vb, ks, vs)]
            qh, kh, vh = (t.cpu().numpy()[0] for t in (q, k, v))
            out = np.zeros(Hq * 128, np.float32)
            R = oracle.ref()
            n, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0) or n < 3:
                R.ref_attention_tern(m, Hq, Hkv, S, ctx, P(qh.copy()), P(kh.copy()), P(vh),
                                     *(P(a) for a in hk), P(out))
                n += 1
            cpu = {"value": round(n / (time.perf_counter() - t0), 2), "unit": "attention calls/s",
                   "cores": R.ref_num_threads(), "kind": "reference",
                   "sample": f"FusedKVCache::forward_attention_raw ({mode}), one layer, "
                             f"Hq {Hq} Hkv {Hkv}, position {ctx}, {n} calls"}
    out = {
        "metric": f"decode tok/s BitNet-2B-shape bs=1 ctx {ctx}, {mode} KV",
        "value": round(args.steps / dt, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": ("int8 KV, fp32 scales" if mode == "paged_int8" else
                  "ternary KV (int32 dot, fp32 softmax)"), "data": "synthetic",
        "config": {"workload": f"BitNet-b1.58-2B-shaped greedy decode step, batch 1, context "
                               f"{ctx}, {mode} KV cache ({e.mode} engine mode)",
                   "engine_mode": e.mode},
        "roofline": {"bound": "hbm", "kernel": kernel,
                     "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "alg_bytes_per_launch": int(att_bytes),
                     "mean_launch_us": round(att_s * 1e6, 2)},
        "gpu_attention_calls_per_s": round(1.0 / att_s, 1),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


# ------------------------------------------------------------------- main

# --------------------------------------------------------- stage trace

STAGE_NAMES = ("QKV", "ATT", "O", "GU", "DOWN")


def stage_trace(e, cfg, ctx, runs=8):
    """Per-stage timing of the persistent kernel from its barrier trace
    (tenzo_hip_engine_trace: every workgroup stamps the 100 MHz wall clock
    when it reaches and when it leaves each grid barrier). For each stage:
    "work" = last arrival at its barrier - first departure from the previous
    one, "barrier" = first departure - last arrival, medians over `runs`
    steps at position ctx (the first two are dropped), averaged over layers
    1..L-1; with the stage's algorithmic bytes and GB/s."""
    e.trace(True)
    tok = 1
    traces = []
    for _ in range(runs):
        e.rewind(ctx)
        tok = e.step(tok)
        traces.append(e.get_trace().astype(np.int64))
    e.trace(False)
    t = np.array(traces[2:])  # [R][stages][nwg][2] ticks of 10 ns
    S = t.shape[1]
    work = np.zeros(S)
    bar = np.zeros(S)
    for s_ in range(S):
        arr, lv = t[:, s_, :, 0], t[:, s_, :, 1]
        if s_:
            work[s_] = np.median((arr.max(axis=1) - t[:, s_ - 1, :, 1].min(axis=1)) * 0.01)
        bar[s_] = np.median((lv.min(axis=1) - arr.max(axis=1)) * 0.01)
    H, F, qd, kvd = cfg.hidden, cfg.ffn, cfg.q_dim, cfg.kv_dim
    sb = {"QKV": (qd + 2 * kvd) * H // 4, "ATT": cfg.n_kv_heads * (ctx + 1) * (2 * 128 + 4),
          "O": H * qd // 4, "GU": 2 * F * H // 4, "DOWN": H * F // 4}
    L = cfg.n_layers
    out = {}
    for k, name in enumerate(STAGE_NAMES):
        idx = [5 * l + k for l in range(1, L)]
        w, b = float(np.mean(work[idx])), float(np.mean(bar[idx]))
        out[name] = {"work_us": round(w, 2), "barrier_us": round(b, 2), "bytes": sb[name],
                     "gbs_work_and_barrier": round(sb[name] / ((w + b) * 1e-6) / 1e9, 1)}
    out["HEAD"] = {"work_us": round(float(work[S - 1]), 2),
                   "bytes": cfg.vocab * H + cfg.vocab * 4,
                   "gbs": round((cfg.vocab * H + cfg.vocab * 4) / (work[S - 1] * 1e-6) / 1e9, 1)}
    layer = sum(out[n]["work_us"] + out[n]["barrier_us"] for n in STAGE_NAMES)
    out["layer_us"] = round(layer, 2)
    out["step_us"] = round(float(np.median((t[:, S - 1, :, 0].max(axis=1) -
                                            t[:, 0, :, 1].min(axis=1)) * 0.01)), 1)
    out["barriers_per_step"] = 5 * L
    return out


# ------------------------------------------------------------ configs leg
#
# BASELINE.json's other configs, each timed as a kernel on its own: configs 1
# (one TL1 GEMV 6912x2560), 3 (Q4_0 11008x4096 with fp16 and Q8_0 activations,
# and the reference's Q8_0-weight GEMV at the same shape), 4 (GPTQ / AWQ
# K 4096 x N 14336, group 128, batch 1 and 8) and 5 (INT8-KV decode attention,
# 20 q / 5 kv heads, batch 1 and 16, context 1k / 8k / 32k). The weights (or
# caches) are rotated over enough distinct copies that a pass reads >= 1 GiB,
# so the reads come from HBM rather than the 256 MB last-level cache; every
# call of a pass is captured into one HIP graph and the graph replayed between
# two HIP events. Algorithmic bytes per call: the packed weights (scales,
# zeros) or the cache rows and scales read, plus activations and outputs.
# The compiled reference's function for each (oracle/_ref) is timed beside it
# in a child process on the host cores.

GIB = 1 << 30


def _copies(nbytes, floor=GIB):
    return max(2, -(-floor // nbytes))


def _per_call(torch, calls, reps=3):
    return graph_time(torch, lambda: [c() for c in calls], reps) / len(calls)


def _entry(alg, t, copies):
    gbs = alg / t / 1e9
    return {"alg_bytes": int(alg), "mean_us": round(t * 1e6, 2), "achieved_gbs": round(gbs, 1),
            "frac": round(gbs / PEAK_HBM_GBS, 4), "copies": int(copies)}


def _gguf_dev(torch, gen, copies, N, K, bpb):
    """copies x N rows of K/32 GGUF blocks of bpb bytes: random codes, fp16
    scales |N(0, 0.01)|."""
    nbk = K // 32
    w = torch.randint(0, 256, (copies, N, nbk, bpb), dtype=torch.uint8, device="cuda",
                      generator=gen)
    d = (torch.randn((copies, N, nbk), device="cuda", generator=gen).abs() * 0.01).half()
    w[..., :2] = d.view(torch.uint8).view(copies, N, nbk, 2)
    return w


def tl1_methods(torch):
    """The masked-v_dot4 TL1 GEMV against the reference's table method (LDS
    tables per activation pair, v_perm lookups) on the same weights: config
    1's 6912 x 2560 (latency-bound: a wave sees about one 64-column chunk)
    and 65536 x 8192 (134 MB: each wave loops over 32 chunks)."""
    from tenzo_amd import ops
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED + 9)
    out = {}
    for N, K in ((6912, 2560), (65536, 8192)):
        nb = ops.tl1_packed_bytes(N, K)
        c = _copies(nb)
        W = tl1_random_dev(torch, c * nb, gen).view(c, nb)
        codes, q, _ = ops.rmsnorm_quant31(torch.randn(K, device="cuda", generator=gen))
        y = torch.empty(N, device="cuda")
        alg = N * K // 4 + K + N * 4
        for name, fn in (("v_dot4", lambda i: ops.bitlinear_tl1_into(codes, q, W[i], 0.0159, N, K, y)),
                         ("table", lambda i: ops.bitlinear_tl1_lut(codes, q, W[i], 0.0159, N, K, y=y))):
            t = _per_call(torch, [lambda i=i: fn(i) for i in range(c)])
            out[f"tl1_{N}x{K}_{name}"] = _entry(alg, t, c)
        del W
    return out


def configs_bench(torch):
    from tenzo_amd import _lib, ops
    L = _lib.load()
    P, S = ops._ptr, ops._stream
    gen = torch.Generator(device="cuda")
    gen.manual_seed(SEED + 7)
    out = {}
    # config 1: one TL1 GEMV, 6912 x 2560, on fp32 activations: the per-token
    # absmax quantization and the GEMV (build_lut + compute_from_lut, the unit
    # the CPU leg times), one launch (tl1_gemv_f32_kernel); fp32 in, fp32 out
    N, K = 6912, 2560
    nb = ops.tl1_packed_bytes(N, K)
    c = _copies(nb)
    W = tl1_random_dev(torch, c * nb, gen).view(c, nb)
    xa = torch.randn(K, device="cuda", generator=gen)
    y = torch.empty(N, device="cuda")
    P_ = ops._ptr
    t = _per_call(torch, [lambda i=i: L.tenzo_hip_bitlinear_tl1_f32(P_(xa), P_(W[i]), 0.0159, 1, N,
                                                                     K, P_(y), S())
                          for i in range(c)])
    out["c1_tl1_6912x2560"] = _entry(N * K // 4 + K * 4 + N * 4, t, c)
    # the GEMV alone on codes quantized once (int8 codes in)
    codes, q, _ = ops.rmsnorm_quant31(xa)
    t = _per_call(torch, [lambda i=i: ops.bitlinear_tl1_into(codes, q, W[i], 0.0159, N, K, y)
                          for i in range(c)])
    out["c1_tl1_6912x2560_codes_in"] = _entry(N * K // 4 + K + N * 4, t, c)
    # the same GEMV by the reference's table method (LDS tables per activation
    # pair, v_perm lookups): the measurement behind the masked-v_dot4 choice
    t = _per_call(torch, [lambda i=i: ops.bitlinear_tl1_lut(codes, q, W[i], 0.0159, N, K, y=y)
                          for i in range(c)])
    out["c1_tl1_6912x2560_table_method"] = _entry(N * K // 4 + K + N * 4, t, c)
    del W
    # config 3: Q4_0 (fp16 and Q8_0 activations) and Q8_0 weights, 11008 x 4096
    N, K = 11008, 4096
    nbk = K // 32
    y = torch.empty(N, device="cuda")
    a16 = torch.randn(K, device="cuda", generator=gen).half()
    c = _copies(N * nbk * 18)
    W = _gguf_dev(torch, gen, c, N, K, 18)
    t = _per_call(torch, [lambda i=i: L.tenzo_hip_gemv_q4_0(P(a16), 1, P(W[i]), P(y), K, N, 1,
                                                            S()) for i in range(c)])
    out["c3_q4_0_fp16act"] = _entry(N * nbk * 18 + K * 2 + N * 4, t, c)
    qa = _gguf_dev(torch, gen, 1, 1, K, 34)[0, 0]
    t = _per_call(torch, [lambda i=i: L.tenzo_hip_gemv_q4_0_q8_0(P(qa), P(W[i]), P(y), K, N, 1,
                                                                 S()) for i in range(c)])
    out["c3_q4_0_q8_0act"] = _entry(N * nbk * 18 + nbk * 34 + N * 4, t, c)
    del W
    c = _copies(N * nbk * 34)
    W = _gguf_dev(torch, gen, c, N, K, 34)
    t = _per_call(torch, [lambda i=i: L.tenzo_hip_gemv_q8_0(P(a16), 1, P(W[i]), P(y), K, N, 1,
                                                            S()) for i in range(c)])
    out["c3_q8_0_weights"] = _entry(N * nbk * 34 + K * 2 + N * 4, t, c)
    del W
    # config 4: GPTQ / AWQ, K 4096 x N 14336, group 128, fp16 scales
    K, N, G = 4096, 14336, 128
    wbytes = K // 8 * N * 4 + K // G * N * 2 + K // G // 8 * N * 4
    c = _copies(wbytes)
    qw = torch.randint(-2**31, 2**31 - 1, (c, K // 8, N), dtype=torch.int32, device="cuda",
                       generator=gen)
    sc = (torch.randn((c, K // G, N), device="cuda", generator=gen).abs() * 0.01).half()
    qz = torch.randint(-2**31, 2**31 - 1, (c, K // G // 8, N), dtype=torch.int32, device="cuda",
                       generator=gen)
    for kind in ("gptq", "awq"):
        fn = getattr(L, f"tenzo_hip_gemv_{kind}")
        for B in (1, 8):
            a = torch.randn((B, K), device="cuda", generator=gen).half()
            yb = torch.empty((B, N), device="cuda")
            t = _per_call(torch, [lambda i=i: fn(P(a), 1, P(qw[i]), P(sc[i]), 1, P(qz[i]), P(yb),
                                                 K, N, G, B, S()) for i in range(c)])
            out[f"c4_{kind}_b{B}"] = _entry(wbytes + B * K * 2 + B * N * 4, t, c)
    del qw, sc, qz
    # config 5: INT8-KV decode attention, 20 / 5 heads of 128
    Hq, Hkv = 20, 5
    cs = ops.rope_table(500000.0, 0, 1)[0].cuda()
    for B in (1, 16):
        for ctx in (1024, 8192, 32768):
            per = B * Hkv * ctx * (2 * 128 + 2 * 2)  # K and V codes + fp16 scales read
            c = _copies(per)
            kc = torch.randint(-127, 128, (c, B, Hkv, ctx, 128), dtype=torch.int8,
                               device="cuda", generator=gen)
            vc = torch.randint(-127, 128, (c, B, Hkv, ctx, 128), dtype=torch.int8,
                               device="cuda", generator=gen)
            ks = (torch.rand((c, B, Hkv, ctx), device="cuda", generator=gen) * 0.03 + 0.01).half()
            vs = (torch.rand((c, B, Hkv, ctx), device="cuda", generator=gen) * 0.03 + 0.01).half()
            qv = torch.randn((B, Hq * 128), device="cuda", generator=gen).half().float()
            kv = torch.randn((B, Hkv * 128), device="cuda", generator=gen)
            o = torch.empty((B, Hq * 128), device="cuda")
            pos = ctx - 1
            t = _per_call(torch, [lambda i=i: L.tenzo_hip_attn_int8_decode(
                P(qv), P(kv), P(kv), P(kc[i]), P(vc[i]), P(ks[i]), P(vs[i]), P(cs), B, Hq, Hkv,
                ctx, pos, P(o), None, None, S()) for i in range(c)])
            out[f"c5_attn_b{B}_ctx{ctx // 1024}k"] = _entry(per + B * (Hq + 2 * Hkv) * 512, t, c)
            del kc, vc, ks, vs
    torch.cuda.empty_cache()
    return out


def cpu_configs(seconds=1.0):
    """The compiled reference's functions for the same configs on the host (run
    in a child process: no GPU). Each is timed for about `seconds` (at least
    two calls after one warm-up) over copies of the weights totalling >= 256 MB
    where one copy would fit in the host's caches."""
    import oracle
    from tenzo_amd import formats
    if not oracle.ref_available():
        return {}
    R = oracle.ref()
    Pp = oracle._ptr
    rng = np.random.default_rng(SEED + 7)
    res = {}

    def clock(name, calls, alg):
        calls[0]()
        n, t0 = 0, time.perf_counter()
        while n < 2 or (time.perf_counter() - t0 < seconds and n < 10000):
            calls[n % len(calls)]()
            n += 1
        dt = (time.perf_counter() - t0) / n
        res[name] = {"us": round(dt * 1e6, 1), "gbs": round(alg / dt / 1e9, 2)}

    N, K = 6912, 2560
    c = _copies(N * K // 2, 256 << 20)
    W = rng.integers(-128, 128, size=(c, N * K // 2), dtype=np.int8)
    x = rng.standard_normal(K).astype(np.float32)
    y = np.empty(N, np.float32)
    clock("c1_tl1_6912x2560", [lambda i=i: R.ref_tl1_gemv(Pp(x), Pp(W[i]), K, N, 0.0159, Pp(y))
                               for i in range(c)], N * K // 4 + K * 4 + N * 4)
    del W
    N, K = 11008, 4096
    nbk = K // 32
    a = rng.standard_normal(K).astype(np.float16).astype(np.float32)
    y = np.empty(N, np.float32)
    for name, bpb, fn in (("c3_q4_0_fp16act", 18, R.ref_q4_0), ("c3_q8_0_weights", 34, R.ref_q8_0)):
        w = rng.integers(0, 256, size=(N * nbk, bpb), dtype=np.uint8)
        w[:, :2] = (np.abs(rng.normal(0, 0.01, N * nbk)).astype(np.float16)
                    .view(np.uint8).reshape(-1, 2))
        clock(name, [lambda w=w: fn(Pp(a), Pp(w), Pp(y), K, N)], N * nbk * bpb + K * 4 + N * 4)
    K, N, G = 4096, 14336, 128
    qw = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint32)
    sc = np.abs(rng.normal(0, 0.01, size=(K // G, N))).astype(np.float16).astype(np.float32)
    qz = rng.integers(0, 2**32, size=(K // G // 8 + 1, N), dtype=np.uint32)
    y = np.empty(N, np.float32)
    wbytes = K // 8 * N * 4 + K // G * N * 4 + K // G // 8 * N * 4
    for kind in ("gptq", "awq"):
        fn = getattr(R, f"ref_{kind}")
        for B in (1, 8):
            A = rng.standard_normal((B, K)).astype(np.float16).astype(np.float32)
            clock(f"c4_{kind}_b{B}",
                  [lambda: [fn(Pp(A[b]), Pp(qw), Pp(sc), Pp(qz), Pp(y), K, N, G)
                            for b in range(B)]], B * (wbytes + K * 4 + N * 4))
    Hq, Hkv = 20, 5
    for B in (1, 16):
        for ctx in (1024, 8192, 32768):
            ms = ctx + 1
            kc = rng.integers(-127, 128, size=(B, Hkv, ms, 128), dtype=np.int8)
            ks = rng.uniform(0.01, 0.04, size=(B, Hkv, ms)).astype(np.float32)
            q = rng.standard_normal((B, Hq * 128)).astype(np.float32)
            k = rng.standard_normal((B, Hkv * 128)).astype(np.float32)
            reps = max(2, min(20, int(2e8 // (B * Hkv * ctx * 260))))
            dt = R.ref_attention_int8_time(B, Hq, Hkv, ms, ctx - 1, Pp(kc), Pp(kc), Pp(ks), Pp(ks),
                                           Pp(q), Pp(k), Pp(k), reps)
            alg = B * Hkv * ctx * (2 * 128 + 2 * 4)
            res[f"c5_attn_b{B}_ctx{ctx // 1024}k"] = {"us": round(dt * 1e6, 1),
                                                      "gbs": round(alg / dt / 1e9, 2)}
            del kc
    return res


def host_cpu():
    """CPU model, sockets and physical cores of the host (lscpu), the OpenMP
    threads and placement the reference legs run with."""
    info = {}
    try:
        import subprocess
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        kv = dict(l.split(":", 1) for l in txt.splitlines() if ":" in l)
        kv = {k.strip(): v.strip() for k, v in kv.items()}
        info = {"model": kv.get("Model name"), "sockets": kv.get("Socket(s)"),
                "cores_per_socket": kv.get("Core(s) per socket"),
                "threads_per_core": kv.get("Thread(s) per core"), "cpus": kv.get("CPU(s)")}
    except (OSError, ValueError):
        pass
    info["cpus_usable"] = len(os.sched_getaffinity(0))
    info["omp"] = {k: os.environ.get(k) for k in ("OMP_NUM_THREADS", "OMP_PLACES",
                                                    "OMP_PROC_BIND")}
    return info


def run_cpu_configs(seconds):
    """cpu_configs in a child process (OpenMP placed on cores, spread), its
    JSON line parsed."""
    import subprocess
    env = dict(os.environ, OMP_PLACES="cores", OMP_PROC_BIND="spread")
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-configs-child",
                        "--cpu-seconds", str(seconds)], capture_output=True, text=True,
                       env=env, timeout=900)
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    if r.returncode != 0 or not lines:
        return {"error": f"child exited {r.returncode}: {r.stderr[-300:]}"}
    return json.loads(lines[-1])


def merge_configs(gpu, cpu):
    for name, e in gpu.items():
        ref = cpu.get(name) if isinstance(cpu, dict) else None
        e["cpu_ref_us"] = ref["us"] if ref else None
        e["cpu_ref_gbs"] = ref["gbs"] if ref else None
    return gpu


def main():
    args = parse()
    if args.cpu_configs_child:  # the child of run_cpu_configs: host only, no GPU
        out = {"host": host_cpu()}
        out.update(cpu_configs(min(args.cpu_seconds, 2.0)))
        print(json.dumps(out), flush=True)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not implemented)"}))
        sys.exit(2)
    import torch
    from tenzo_amd import synth
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU (the decode path has no CPU fallback)")
    cfg = synth.BITNET_2B
    if args.configs_only:
        print(json.dumps({"configs": configs_bench(torch)}), flush=True)
        return
    if args.tl1_methods:
        print(json.dumps({"tl1_methods": tl1_methods(torch)}), flush=True)
        return
    ctx = 0 if args.prefill else args.ctx
    tern = args.kv_mode != "int8_fused"
    if tern and args.prefill:
        raise SystemExit("--prefill runs the int8_fused cache")
    e, host = build_model(torch, cfg, ctx, args.kv_mode)
    if tern:
        e.set_mode(args.mode)  # the persistent kernel runs every KV mode
        tern_bench(torch, e, cfg, host, args)
        e.close()
        return
    if args.prefill:
        prefill_bench(torch, e, cfg, host, args)
        e.close()
        return
    e.set_mode(args.mode)
    mode = e.mode
    if args.stage_trace:
        print(json.dumps({"stage_trace": stage_trace(e, cfg, ctx),
                          "config": {"workload": "BitNet-2B decode step", "context": ctx}}),
              flush=True)
        e.close()
        return
    if args.pmc_probe:
        src = torch.empty(PROBE_COPY_BYTES // 4, dtype=torch.int32, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # the calibration kernel: PROBE_COPY_BYTES read and written
        torch.cuda.synchronize()
        e.rewind(ctx)
        e.decode(1, args.steps)
        torch.cuda.synchronize()
        e.close()
        print(f"pmc probe: 1 copy of {PROBE_COPY_BYTES} bytes, {args.steps} decode steps at "
              f"context {ctx}", flush=True)
        return

    # warm up (also captures graphs / loads code), then the timed decode:
    # `steps` greedy tokens chained on the device from position ctx
    tok = 1
    if args.warmup:
        e.rewind(ctx)
        e.decode(tok, args.warmup)
    e.rewind(ctx)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks, ev_ms = e.decode(tok, args.steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt / args.steps * 1e3
    tok_s = args.steps / dt
    # the reference API's loop: one tenzo_generate_step (token back to the
    # host) per token, at position ctx
    api_steps = max(5, args.steps // 5)
    e.rewind(ctx)
    t0 = time.perf_counter()
    for _ in range(api_steps):
        e.rewind(ctx)
        tok = e.step(tok)
    api_tok_s = api_steps / (time.perf_counter() - t0)
    # the timed path's tokens against the per-stage kernels (graph mode) on the
    # same engine and weights: the same greedy tokens from the same state
    # (attention sums in another order, so a logit tie could split them; a
    # difference is reported, not hidden)
    token_check = None
    if mode == "persistent":
        nchk = 4
        e.rewind(ctx)
        ptoks, _ = e.decode(1, nchk)
        e.set_mode("graph")
        e.rewind(ctx)
        gtoks, _ = e.decode(1, nchk)
        e.set_mode(mode)
        token_check = {"steps": nchk, "against": "graph", "tokens_equal":
                       [int(t) for t in ptoks] == [int(t) for t in gtoks]}
        # the first step from the same state: the two paths' logits (relative to the
        # largest |logit|); later steps start from states that differ (each path
        # appends the KV rows its own attention order gives, and an ulp at a code's
        # rounding tie is not damped by this random-weight model)
        lg0 = {}
        for m in (mode, "graph"):
            e.set_mode(m)
            e.rewind(ctx)
            e.step(1)
            lg0[m] = e.logits()
        e.set_mode(mode)
        token_check["step0_logits_rel"] = float(np.abs(lg0[mode] - lg0["graph"]).max() /
                                                np.abs(lg0["graph"]).max())
        if not token_check["tokens_equal"]:
            print(f"bench: persistent tokens {list(ptoks)} differ from the graph path's "
                  f"{list(gtoks)}", file=sys.stderr, flush=True)
            # where they part: both paths rerun the same inputs up to that step, and
            # the two candidate tokens' logits are compared in each (a near tie of
            # the two largest logits, relative to the largest |logit|, is what a
            # different attention summation order can split)
            k = next(i for i in range(nchk) if int(ptoks[i]) != int(gtoks[i]))
            pa, ga = int(ptoks[k]), int(gtoks[k])
            gaps = {}
            for m in (mode, "graph"):
                e.set_mode(m)
                e.rewind(ctx)
                t = 1
                for i in range(k + 1):
                    t = e.step(t if i == 0 else int(ptoks[i - 1]))
                lg = e.logits()
                gaps[m] = float(lg[pa] - lg[ga]) / float(np.abs(lg).max())
            e.set_mode(mode)
            token_check.update({"first_diff_step": k, "tokens": [pa, ga],
                                "rel_gap_persistent": gaps[mode], "rel_gap_graph": gaps["graph"]})

    # algorithmic HBM bytes of a step at the mean context of the timed run
    step_bytes = cfg.step_bytes(ctx + 1 + args.steps // 2)["total"]
    step_gbs = step_bytes / (dt / args.steps) / 1e9

    # the dominant kernel: the decode step itself (one launch per token in the
    # persistent mode); its mean duration from HIP events on the engine stream
    kern_s = ev_ms / 1e3 / args.steps
    dom_name = "decode_step_kernel" if mode == "persistent" else "decode step (stage kernels)"
    roofline = {"bound": "hbm", "kernel": dom_name,
                "achieved": round(step_bytes / kern_s / 1e9, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(step_bytes / kern_s / 1e9 / PEAK_HBM_GBS, 4),
                "traffic": measured_traffic() if mode == "persistent" else None,
                "alg_bytes_per_launch": int(step_bytes),
                "mean_launch_us": round(kern_s * 1e6, 2)}
    # the metric's GEMV + attention share: TL1 weights and KV cache bytes over
    # the step's kernel time less the LM-head stage (from the stage trace)
    st = stage_trace(e, cfg, ctx) if mode == "persistent" else None
    sb = cfg.step_bytes(ctx + 1 + args.steps // 2)
    ga_bytes = sb["tl1"] + sb["kv"]
    gemv_attn = None
    if st is not None:
        ga_s = kern_s - st["HEAD"]["work_us"] * 1e-6
        gemv_attn = {"bytes": int(ga_bytes), "time_us": round(ga_s * 1e6, 1),
                     "gbs": round(ga_bytes / ga_s / 1e9, 1),
                     "frac": round(ga_bytes / ga_s / 1e9 / PEAK_HBM_GBS, 4)}
    rl_tl1 = tl1_roofline(torch, cfg, host)
    rl_head = head_roofline(torch, cfg, host)
    cpu = None if args.no_cpu else cpu_baseline(torch, cfg, host, ctx, args.cpu_seconds)
    if cpu is not None:
        cpu["host"] = host_cpu()
        cpu["gbs"] = round(step_bytes * cpu["value"] / 1e9, 2) if cpu.get("value") else None
    configs = None
    if not args.no_configs:
        e.close()
        e = None
        torch.cuda.empty_cache()
        gpu_cfg = configs_bench(torch)
        host_cfg = {} if args.no_cpu else run_cpu_configs(args.cpu_seconds)
        configs = merge_configs(gpu_cfg, host_cfg)
        if isinstance(host_cfg, dict) and "host" in host_cfg:
            configs["cpu_host"] = host_cfg["host"]
        elif isinstance(host_cfg, dict) and "error" in host_cfg:
            configs["cpu_error"] = host_cfg["error"]

    out = {
        "metric": "decode tok/s BitNet-2B-shape bs=1 ctx 4k; GEMV+attn HBM GB/s % of peak",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8/ternary (int32 acc, fp32 out)",
        "data": "synthetic (random-init BitNet-2B-shaped weights, N(0,1) KV prefill)",
        "config": {"workload": "BitNet-b1.58-2B-shaped greedy decode step, batch 1, "
                               f"context {ctx}, INT8 KV fp16 scales, int8 LM head",
                   "layers": cfg.n_layers, "hidden": cfg.hidden, "ffn": cfg.ffn,
                   "heads": [cfg.n_q_heads, cfg.n_kv_heads, 128], "vocab": cfg.vocab,
                   "rope_theta": cfg.theta, "engine_mode": mode},
        "step_hbm_bytes": step_bytes, "step_gbs": round(step_gbs, 1),
        "step_frac_of_peak": round(step_gbs / PEAK_HBM_GBS, 4),
        "roofline": roofline,
        "gemv_attn": gemv_attn,
        "stages": st,
        "api_generate_step_tok_s": round(api_tok_s, 2),
        "token_check": token_check,
        # what "bit-exact" is measured against: RMSNorm (and so every activation
        # code) reproduces the reference build's 1/sqrt, the RSQRTSS estimate
        # of the x86 host it was compiled on plus one Newton step
        "parity_pin": {"rms_norm": "reference build host's RSQRTSS estimate (Intel x86, AVX2/FMA "
                                   "build, -ffast-math), table tenzo_amd/csrc/rsqrt_est_table.inc "
                                   "+ one Newton step; 8-chain FMA sum of squares",
                       "chained_decode_test": "tests/test_gpu_bitnet_full.py::"
                                              "test_full_shape_chained_decode"},
        "stage_kernels": {"tl1_gemv": {k: (round(v, 2) if isinstance(v, float) else v)
                                       for k, v in rl_tl1.items()},
                          "lm_head_i8": {k: (round(v, 2) if isinstance(v, float) else v)
                                         for k, v in rl_head.items()}},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    if e is not None:
        e.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
