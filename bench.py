"""State-op decode benchmark on one MI355X: tiered v4 vs fresh at the
Nemotron-Nano-9B-v2 mixer shape (27 Mamba2 layers, H=128, P=80, N=128, G=8).

A step is one decode token through the state op of all layers, inputs resident
in HBM, synthetic seeded data. Per layer-token the tiered path launches prep and
stream (windows up to 16 tokens, 32 for a single bf16 copy, are flushed inside the stream kernel) or prep,
stream and flush (longer windows); the untiered path prep and stream. Prints one
JSON line (the driver contract); progress goes to stderr.

    python bench.py [--steps 64] [--warmup 8] [--B 256] [--c 4] [--k 32] [--cold fp32]
"""
import argparse
import dataclasses
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

L_DEF, H, P, N, G = 27, 128, 80, 128, 8
PEAK_HBM_GBS = 8000.0


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# algorithmic byte model (bytes per request per layer-token)
def bytes_io():
    # x bf16 + B, C bf16 + dt bf16 in, y fp32 out
    return H * P * 2 + 2 * G * N * 2 + H * 2 + H * P * 4


def bytes_fresh_token():
    return 2 * H * P * N * 4 + bytes_io()


def bytes_v4_token(k, c, cold, master="fp32", skip=0.0, exact=False):
    """skip: fraction of heads whose cold term a gated readout drops; such a head reads
    no cold column on the c - 1 tokens of a window that do not flush. exact: the rank-c
    correction's reads of the buffered x and dt (a token finds (c - 1) / 2 of them on
    average) and its window dots per group (written by prep, read by the stream kernel,
    (c + 1) / 2 each)."""
    nc = N - k
    esz = {"fp32": 4, "bf16": 2, "fp8": 1}[cold]
    hot = 2 * H * P * k * 4
    scale = H * P * 4 if cold == "fp8" else 0  # e4m3 row scales
    keep = (c - 1) / c * (1.0 - skip)  # tokens that read the read copy (no flush, cold term kept)
    if cold == "fp32" or (cold == "bf16" and master == "bf16"):
        # a single copy: read by every token (at the flush, the stale readout and the replay's
        # start in one), rewritten at the flush
        read = H * P * nc * esz * (keep + 1 / c)
        flush = H * P * nc * esz
    else:
        # beside a master: the read copy (+ row scale) is read by the tokens that do not flush;
        # the flush token reads the master and the row scale (its stale readout requantizes the
        # master's values) and writes master, read copy and scale
        msz = 4 if master == "fp32" else 2
        read = (H * P * nc * esz + scale) * keep + scale / c
        flush = H * P * nc * (2 * msz + esz) + scale
    ring_entry = H * P * 2 + H * 4 + G * nc * 4  # x bf16, dt, B' cold
    ring = (c - 1) / c * 2 * ring_entry  # written by c-1 of c tokens, read once at the flush
    corr = (H * P * 2 * (c - 1) / 2 + H * 4 * (c - 1) / 2 + 2 * G * 4 * (c + 1) / 2) if exact else 0.0
    return hot + read + flush / c + ring + corr + bytes_io()


def bytes_rotation():
    return G * N * N * 4


# ---------------------------------------------------------------------------
def make_layers(L, dev, seed):
    """Per layer: dt_bias = log(expm1(U(1e-3, 1e-1))), A = -exp(U(0, ln 16)), D ~ N(0,1) per head;
    R = Q of QR(N(0,1)) with the sign fix, per group."""
    from nested_ssm_amd import LayerParams

    gen = torch.Generator().manual_seed(seed)
    out = []
    f = dict(device=dev, dtype=torch.float32)
    for _ in range(L):
        u = 1e-3 + (1e-1 - 1e-3) * torch.rand(H, generator=gen, dtype=torch.float64)
        dt_bias = torch.log(torch.expm1(u))
        A = -torch.exp(torch.rand(H, generator=gen, dtype=torch.float64) * 2.772588722239781)
        D = torch.randn(H, generator=gen, dtype=torch.float64)
        Q, Rr = torch.linalg.qr(torch.randn(G, N, N, generator=gen, dtype=torch.float64))
        R = Q * torch.sign(torch.diagonal(Rr, dim1=-2, dim2=-1))[..., None, :]
        out.append(LayerParams(H, P, N, G, dt_bias.to(**f), A.to(**f), D.to(**f), R.to(**f).contiguous()))
    return out


def make_inputs(L, B, dev, seed, pool=2):
    g = torch.Generator(device=dev).manual_seed(seed)
    sets = []
    for _ in range(pool):
        per = []
        for _ in range(L):
            x = torch.randn(B, H, P, device=dev, generator=g).to(torch.bfloat16)
            Bm = (torch.randn(B, G, N, device=dev, generator=g) / N ** 0.5).to(torch.bfloat16)
            Cm = (torch.randn(B, G, N, device=dev, generator=g) / N ** 0.5).to(torch.bfloat16)
            dt = torch.randn(B, H, device=dev, generator=g).to(torch.bfloat16)
            per.append((x, Bm, Cm, dt))
        sets.append(per)
    return sets


def rand_state(B, dev, g):
    return torch.randn(B, H, P, N, device=dev, generator=g).mul_(0.1)


def timed(step_fn, steps, warmup, launches_per_step):
    """Warmup, then time exactly `steps` steps with events on the launch stream."""
    for i in range(warmup):
        step_fn(i)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for i in range(steps):
        step_fn(warmup + i)
    e1.record(st)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    return ms / steps, ms / (steps * launches_per_step)


def graphed(step_fn, n_inputs):
    """One HIP graph per input set, each capturing a whole step (all layers), after a
    first call on the capture stream has sized its workspace; returns a step function
    that replays them in turn. The state ops allocate nothing, issue no memset and keep
    their phase on the device, so the replays do what the eager steps do."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step_fn(0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graphs = []
    for i in range(n_inputs):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            step_fn(i)
        graphs.append(gr)
    torch.cuda.synchronize()
    return lambda i: graphs[i % n_inputs].replay()


def per_launch_ms(launch_fn, n):
    """Average duration of n launches, each bracketed by its own event pair."""
    st = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i, (a, b) in enumerate(evs):
        a.record(st)
        launch_fn(i)
        b.record(st)
    torch.cuda.synchronize()
    return sum(a.elapsed_time(b) for a, b in evs) / n


def bench_fresh(args, layers, inputs, dev):
    """The untiered update in the model's own basis, as the reference's fresh baselines run
    (scale/bench_v4_decode.py:85-91, :236-254): no rotation of B and C (prep's identity path)."""
    from nested_ssm_amd import fresh_step

    layers = [dataclasses.replace(lp, R=None) for lp in layers]
    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    states = [rand_state(args.B, dev, g) for _ in range(args.layers)]
    ys = [torch.empty(args.B, H, P, device=dev) for _ in range(args.layers)]

    def step(i):
        inp = inputs[i % len(inputs)]
        for l in range(args.layers):
            fresh_step(layers[l], states[l], *inp[l], y=ys[l])

    run = graphed(step, len(inputs)) if args.graph else step
    ms_step, ms_launch = timed(run, args.steps, args.warmup, args.layers)

    def one(i):
        l = i % args.layers
        fresh_step(layers[l], states[l], *inputs[0][l], y=ys[l])

    ms_ev = per_launch_ms(one, min(4 * args.layers, 108))
    del states
    torch.cuda.empty_cache()
    return ms_step, ms_launch, ms_ev


def bench_v4(args, layers, inputs, dev):
    from nested_ssm_amd import V4Tier
    from nested_ssm_amd.ops import x_ring_for

    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    tiers, ys = [], []
    for l in range(args.layers):
        t = V4Tier(args.B, H, P, G, k_hot=args.k, c=args.c, cold=args.cold, device=dev, master=args.master,
                   x_ring=x_ring_for(args.c, args.exact))
        S0 = rand_state(args.B, dev, g)
        phase = (torch.randint(0, args.c, (args.B,), device=dev, generator=g, dtype=torch.int32)
                 if args.ragged else None)
        t.join(layers[l], S0, phase=phase)
        del S0
        tiers.append(t)
        ys.append(torch.empty(args.B, H, P, device=dev))
    torch.cuda.synchronize()

    counts = torch.zeros(args.layers, 2, dtype=torch.int64, device=dev) if args.qgate > 0 else None
    rd = dict(exact=args.exact, hot_only=args.coldoff, qgate=args.qgate)

    def step(i):
        inp = inputs[i % len(inputs)]
        for l in range(args.layers):
            tiers[l].step(layers[l], *inp[l], y=ys[l], counts=None if counts is None else counts[l], **rd)

    # warmup is rounded to whole flush windows so the timed steps start phase-aligned
    # (with --graph the capture's sizing call advances the phase by one token)
    warm = ((args.warmup + args.c - 1) // args.c) * args.c
    run = step
    if args.graph:
        run = graphed(step, len(inputs))
        warm = max(warm, args.c) - 1
    ms_step, ms_launch = timed(run, args.steps, warm, args.layers)

    # per-launch events over whole flush windows (c tokens of layer 0 .. L-1)
    seq = []
    for tok in range(args.c):
        for l in range(args.layers):
            seq.append((tok, l))

    def one(i):
        tok, l = seq[i % len(seq)]
        tiers[l].step(layers[l], *inputs[tok % len(inputs)][l], y=ys[l],
                      counts=None if counts is None else counts[l], **rd)

    ms_ev = per_launch_ms(one, len(seq) * max(1, 108 // len(seq)))
    tier_gb = sum(t.nbytes() for t in tiers) / 1e9
    # fraction of heads whose cold term the readout dropped
    if args.coldoff:
        args.skip = 1.0
    elif counts is not None:
        n, kept = counts.sum(0).tolist()
        args.skip = 1.0 - kept / n if n else 0.0
    del tiers
    torch.cuda.empty_cache()
    return ms_step, ms_launch, ms_ev, tier_gb


DEPLOY_POINTS = [
    # the v4-c4 storage points beyond the fp32 headline (scale/v4_fused_decode.py:149: the
    # bf16 snapshot master; the reference bench's bf16 arm; the e4m3 deployment point)
    ("v4 k32 c4 single bf16 copy, B=256", dict(B=256, cold="bf16", master="bf16")),
    ("v4 k32 c4 e4m3 cold + bf16 master, B=256", dict(B=256, cold="fp8", master="bf16")),
    ("v4 k32 c4 e4m3 cold + bf16 master, B=448", dict(B=448, cold="fp8", master="bf16")),
    # the rank-c exact correction readout (corr=1) at the longest window
    ("v4 k32 c64 fp32 exact readout, B=256", dict(B=256, c=64, exact=True)),
    # the ragged continuous batch: 384 requests at random phases (each token flushes about
    # B/c of them), fp32 cold, every (c, k_hot) pair of the sweep
    ("ragged B=384 k32 c8 fp32", dict(B=384, k=32, c=8, ragged=True)),
    ("ragged B=384 k32 c16 fp32", dict(B=384, k=32, c=16, ragged=True)),
    ("ragged B=384 k32 c64 fp32", dict(B=384, k=32, c=64, ragged=True)),
    ("ragged B=384 k64 c8 fp32", dict(B=384, k=64, c=8, ragged=True)),
    ("ragged B=384 k64 c16 fp32", dict(B=384, k=64, c=16, ragged=True)),
    ("ragged B=384 k64 c64 fp32", dict(B=384, k=64, c=64, ragged=True)),
]


def readout_name(args) -> str:
    return ("exact" if args.exact else "hot-only" if args.coldoff
            else f"query-gated tau={args.qgate:g}" if args.qgate > 0 else "stale")


def traffic_key(args, head="v4") -> str:
    """The workload's key in the profiles' `traffic[...]` lines."""
    if head != "v4":
        return f"fresh B={args.B}"
    readout = readout_name(args)
    return (f"v4 B={args.B} k={args.k} c={args.c} {args.cold}" + (" bf16-master" if args.master == "bf16" else "")
            + ("" if readout == "stale" else f" {readout}") + (" ragged" if args.ragged else ""))


def bench_deploy(args, layers, inputs, dev, fresh_ms_256):
    """The deployment points of DEPLOY_POINTS, each against fresh at its own batch size.
    Same layers, seeds and timing as the headline; fresh is measured once per batch size."""
    import copy

    out = {}
    fresh_ms = {256: fresh_ms_256}
    by_b = {}
    for name, kw in DEPLOY_POINTS:
        by_b.setdefault(kw["B"], []).append((name, kw))
    for B, pts in by_b.items():
        inp = inputs if B == args.B else make_inputs(args.layers, B, dev, args.seed + 7)
        if B not in fresh_ms:
            a = copy.copy(args)
            a.B = B
            log(f"deploy: fresh B={B} ...")
            fresh_ms[B] = bench_fresh(a, layers, inp, dev)[0]
        for name, kw in pts:
            a = copy.copy(args)
            a.__dict__.update(kw)
            if a.cold == "fp32":
                a.master = "fp32"
            a.skip = 0.0
            if a.steps % a.c:
                a.steps += a.c - a.steps % a.c
            log(f"deploy: {name} ...")
            v_step, _, v_ev, _ = bench_v4(a, layers, inp, dev)
            vb = a.B * bytes_v4_token(a.k, a.c, a.cold, a.master, exact=a.exact) + bytes_rotation()
            f_ms = fresh_ms[B]
            tr, tr_src = measured_traffic(traffic_key(a))
            out[name] = {"value": round(a.B / v_step * 1e3, 1), "unit": "state-op tokens/s",
                         "ms_per_step": round(v_step, 4), "fresh_ms_per_step": round(f_ms, 4),
                         "speedup_vs_fresh": round(f_ms / v_step, 3),
                         "byte_bound_speedup": round(bytes_fresh_token() / bytes_v4_token(a.k, a.c, a.cold, a.master,
                                                                                          exact=a.exact), 3),
                         "achieved_gbs": round(vb / (v_ev * 1e-3) / 1e9, 1),
                         "frac": round(vb / (v_ev * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                         "algorithmic_bytes_per_launch": int(vb), "avg_launch_us_events": round(v_ev * 1e3, 2),
                         "traffic": tr, "traffic_source": tr_src, "steps": a.steps}
            log(f"deploy: {name}: {v_step:.3f} ms/step, {out[name]['speedup_vs_fresh']}x fresh")
        del inp
        torch.cuda.empty_cache()
    return out


def bench_prologue(args, dev):
    """The mixer's conv prologue at the 9B shape (conv_dim 12288 = x 10240 + B, C 2 x 1024,
    width 4, bf16): nssm_conv_update (one launch: state shift, conv, SiLU, x/B/C split)
    vs transformers' causal_conv1d_update + split + bf16 casts (the adapter's path when
    a padding mask is given); and the epilogue gated norm. Microseconds per layer-token and
    GB/s of algorithmic bytes: for the HIP launches the device time (HIP graph replays of 27
    launches, as one decode step issues them) and the eager time (one Python call per launch,
    host-bound at this size); the torch paths eagerly, as the reference runs them."""
    from transformers.models.nemotron_h import modeling_nemotron_h as M

    from nested_ssm_amd import conv_update

    I, gn, W = H * P, G * N, 4
    dim = I + 2 * gn
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(args.seed + 3)
    proj = torch.randn(args.B, I + dim + H, device=dev, generator=g).to(bf)
    hbc = proj[:, I:I + dim]
    st = torch.randn(args.B, dim, W, device=dev, generator=g).to(bf)
    w = (torch.randn(dim, W, device=dev, generator=g) * 0.5).to(bf)
    bias = torch.randn(dim, device=dev, generator=g).to(bf)

    def ours(_):
        conv_update(hbc, st, w, bias, I, gn)

    def stock(_):
        o = M.causal_conv1d_update(hbc[..., None], st, w, bias, activation="silu")[..., 0]
        x, B, C = torch.split(o, [I, gn, gn], dim=-1)
        x.to(bf).contiguous(), B.to(bf).contiguous(), C.to(bf).contiguous()

    # the epilogue norm: y fp32 [B, I], gate a bf16 slice of the in_proj output, group 1280
    from nested_ssm_amd import gated_rmsnorm

    y = torch.randn(args.B, I, device=dev, generator=g)
    gate = proj[:, :I]
    norm = M.Zamba2RMSNormGated(I, group_size=I // G, eps=1e-5).to(dev, bf)
    norm_out = torch.empty(args.B, I, device=dev, dtype=bf)

    def ours_norm(_):
        gated_rmsnorm(y, gate, norm.weight, I // G, 1e-5, out=norm_out)

    def stock_norm(_):
        norm(y.to(bf)[:, None], gate[:, None])

    n = 200
    res = {}
    for name, fn in (("nssm_conv_update", ours), ("nssm_gated_rmsnorm", ours_norm)):
        reps = 27
        replay = graphed(lambda _: [fn(i) for i in range(reps)], 1)
        ms, _ = timed(replay, n // 4, 5, 1)
        res[name + "_us"] = round(ms * 1e3 / reps, 2)
        ms, _ = timed(fn, n, 20, 1)
        res[name + "_eager_us"] = round(ms * 1e3, 2)
    for name, fn in (("torch_causal_conv1d_update", stock), ("torch_Zamba2RMSNormGated", stock_norm)):
        ms, _ = timed(fn, n, 20, 1)
        res[name + "_us"] = round(ms * 1e3, 2)
    nbytes = args.B * (dim * 2 + 2 * dim * W * 2 + dim * 2) + dim * W * 2 + dim * 2
    res["algorithmic_bytes"] = nbytes
    res["nssm_conv_update_gbs"] = round(nbytes / (res["nssm_conv_update_us"] * 1e-6) / 1e9, 1)
    nb_norm = args.B * I * (4 + 2 + 2) + I * 2
    res["norm_algorithmic_bytes"] = nb_norm
    res["nssm_gated_rmsnorm_gbs"] = round(nb_norm / (res["nssm_gated_rmsnorm_us"] * 1e-6) / 1e9, 1)
    res["shape"] = (f"B={args.B}, conv_dim={dim} (x {I}, B/C {gn} each), width {W}; norm over {I} channels "
                    f"in groups of {I // G}; bf16")
    return res


def stream_probe(dev, achieved_gbs, gib=2, reps=10):
    """The device's practical HBM rate in this run, beside the state op's: nssm_stream_probe's
    plain streaming read of `gib` GiB and copy of `gib` / 2 GiB (read + write counted), each the
    mean of `reps` launches timed with HIP events on the stream they run on. The 8 TB/s peak
    stays the roofline's denominator; this says how much of the gap any streaming kernel keeps."""
    from nested_ssm_amd._lib import check, lib

    L = lib()
    n = gib << 30
    src = torch.zeros(n // 4, device=dev)
    dst = torch.empty_like(src)
    s = torch.cuda.current_stream()
    out = {"kernel": "nssm_stream_probe (non-temporal 16-byte loads, 4096 workgroups)", "read_bytes": n}
    for mode, key, nb in ((0, "read_gbs", n), (1, "copy_gbs", n // 2)):
        for _ in range(3):
            check(L.nssm_stream_probe(src.data_ptr(), dst.data_ptr(), nb, mode, s.cuda_stream), "nssm_stream_probe")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(reps):
            L.nssm_stream_probe(src.data_ptr(), dst.data_ptr(), nb, mode, s.cuda_stream)
        e1.record(s)
        e1.synchronize()
        sec = e0.elapsed_time(e1) / reps * 1e-3
        out[key] = round(nb * (2 if mode else 1) / sec / 1e9, 1)
    out["copy_bytes_each_way"] = n // 2
    out["state_op_achieved_over_read"] = round(achieved_gbs / out["read_gbs"], 4)
    del src, dst
    torch.cuda.empty_cache()
    return out


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), as lscpu reports it."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(args, budget_s):
    """The oracle's reference step (full fp32 state updated every token, stale
    cold readout, scale/v4_native_decode.py semantics) on the host, one layer at
    B requests; tokens/s for the whole L-layer model = B / (L * t_layer)."""
    import oracle

    threads = torch.get_num_threads()
    gen = torch.Generator().manual_seed(args.seed)
    prm = oracle.make_layer_params(H, P, N, G, gen)
    B = args.B
    ref = oracle.NativeV4(B, H, P, N, args.k, args.c, cold=args.cold, exact=args.exact, master=args.master)
    ref.join(torch.arange(B), oracle.make_state(B, H, P, N, gen))
    x, Bm, Cm, dt = oracle.make_step_inputs(B, H, P, N, G, gen)
    rd = dict(hot_only=args.coldoff, qgate=args.qgate)
    ref.step(x, Bm, Cm, dt, prm, **rd)  # warm
    t0 = time.perf_counter()
    n = 0
    while True:
        ref.step(x, Bm, Cm, dt, prm, **rd)
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= 16:
            break
    t_layer = (time.perf_counter() - t0) / n
    return {
        "value": round(B / (args.layers * t_layer), 2),
        "unit": "state-op tokens/s",
        "cores": threads,
        "cpu": cpu_model(),
        "kind": "port",
        "sample": f"oracle NativeV4 step ({args.cold} cold, k={args.k}, c={args.c}"
                  f"{', exact readout' if args.exact else ''}{', hot-only readout' if args.coldoff else ''}"
                  f"{f', query gate {args.qgate:g}' if args.qgate > 0 else ''}), 1 layer x B={B} x {n} tokens "
                  f"on the host, {t_layer * 1e3:.0f} ms/layer-token, scaled to {args.layers} layers",
    }


TRAFFIC_COPY_BYTES = 256 << 20  # the calibration copy of a traffic pass
# per-dispatch counter rows of the launches of one layer-token (join and materialize are
# outside the timed steps and left out)
TRAFFIC_KERNELS = {"v4": ("prep_kernel<", "unit_kernel", "flush_kernel<"), "fresh": ("prep_kernel<", "fresh_kernel(")}


def workload_argv(args):
    """bench.py flags that rebuild this workload (for a child pass)."""
    av = ["--B", str(args.B), "--k", str(args.k), "--c", str(args.c), "--cold", args.cold, "--master", args.master,
          "--seed", str(args.seed), "--qgate", repr(args.qgate)]
    return av + [f for f, on in (("--exact", args.exact), ("--coldoff", args.coldoff), ("--ragged", args.ragged))
                 if on]


def traffic_pass(args, head, dev):
    """The child side of live_traffic: 2 layers of the workload over whole flush windows
    (at least 8 tokens, then bench_v4's per-launch pass of one more window), then one
    nssm_stream_probe copy of TRAFFIC_COPY_BYTES for the counters' scale."""
    from nested_ssm_amd._lib import check, lib

    args.layers, args.warmup, args.graph = 2, 0, False
    args.steps = ((8 + args.c - 1) // args.c) * args.c
    layers = make_layers(args.layers, dev, args.seed)
    inputs = make_inputs(args.layers, args.B, dev, args.seed + 7)
    (bench_v4 if head == "v4" else bench_fresh)(args, layers, inputs, dev)
    src = torch.zeros(TRAFFIC_COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    check(lib().nssm_stream_probe(src.data_ptr(), dst.data_ptr(), TRAFFIC_COPY_BYTES, 1,
                                  torch.cuda.current_stream().cuda_stream), "nssm_stream_probe")
    torch.cuda.synchronize()


def live_traffic(args, head):
    """HBM bytes per layer-token of this workload, measured in this run: two child passes of
    `bench.py --traffic-pass` under `rocprofv3 --pmc FETCH_SIZE`, then `--pmc WRITE_SIZE`
    (one counter block per pass), each counter scaled by what it reads for the pass's copy
    of known size. Returns (bytes, None) or (None, the reason it could not be measured)."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3") or ("/opt/rocm/bin/rocprofv3" if os.path.exists("/opt/rocm/bin/rocprofv3")
                                         else None)
    if prof is None:
        return None, "rocprofv3 not found"
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    total = 0.0
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        d = tempfile.mkdtemp(prefix="nssm_pmc_")
        cmd = ["timeout", "-s", "KILL", "150", prof, "--pmc", ctr, "-f", "csv", "-d", d, "-o", "pmc", "--",
               sys.executable, os.path.join(ROOT, "bench.py"), "--traffic-pass", "--only", head] + workload_argv(args)
        try:
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=180, env=env)
            rows = []
            for root, _, files in os.walk(d):
                for f in files:
                    if f.endswith("counter_collection.csv"):
                        rows += [x for x in csv.DictReader(open(os.path.join(root, f))) if x["Counter_Name"] == ctr]
        except (OSError, subprocess.SubprocessError) as e:
            return None, f"{ctr} pass: {e}"
        finally:
            shutil.rmtree(d, ignore_errors=True)
        if r.returncode != 0 or not rows:
            return None, f"{ctr} pass exited {r.returncode} with {len(rows)} counter rows"
        per = {}
        for x in rows:
            per.setdefault(x["Kernel_Name"], []).append(float(x["Counter_Value"]))
        copy = [v for k, vs in per.items() if "stream_probe_kernel<true>" in k for v in vs]
        if not copy or copy[0] <= 0:
            return None, f"{ctr} pass: no calibration copy"
        scale = TRAFFIC_COPY_BYTES / copy[0]  # bytes per counter unit
        found = [k for k in per if any(s in k for s in TRAFFIC_KERNELS[head])]
        if not any("prep_kernel<" in k for k in found) or len(found) < 2:
            return None, f"{ctr} pass: kernels of the workload missing"
        total += sum(sum(per[k]) / len(per[k]) * scale for k in found)
    return int(round(total)), None


def measured_traffic(key):
    """HBM bytes per layer-token measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    (calibrated against a plain copy) in an earlier profiled run of this workload and
    recorded in profiles/*.md as `traffic[<key>]: <bytes>`: (bytes, that file), or
    (None, None) when no profile covers it. Not measured in this run."""
    import glob
    import re

    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        for m in re.finditer(r"traffic\[(.*?)\]:\s*(\d+)", open(path).read()):
            if m.group(1) == key:
                return int(m.group(2)), os.path.relpath(path, ROOT)
    return None, None


def kernel_label(head, args):
    """The launches of one layer-token (the unit the roofline is measured on)."""
    if head == "fresh":
        return "prep_kernel<false> + fresh_kernel (one layer-token, two launches)"
    if args.c <= (32 if args.cold == "bf16" and args.master == "bf16" else 16):
        return (f"prep_kernel<true> + unit_kernel<{args.k}, {args.cold}, fused flush> "
                f"(one layer-token, two launches)")
    return (f"prep_kernel<true> + unit_kernel<{args.k}, {args.cold}> + flush_kernel<{args.k}, {args.cold}> "
            f"(one layer-token, three launches)")


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--B", type=int, default=256)
    ap.add_argument("--layers", type=int, default=L_DEF)
    ap.add_argument("--k", type=int, default=32)
    ap.add_argument("--c", type=int, default=4)
    ap.add_argument("--cold", default="fp32", choices=["fp32", "bf16", "fp8"])
    ap.add_argument("--master", default="fp32", choices=["fp32", "bf16"],
                    help="precision of the cold master for bf16 / fp8 cold (bf16: the reference fused "
                         "path's bf16 master; bf16 cold is then a single copy)")
    ap.add_argument("--exact", action="store_true", help="v4 with the rank-c exact correction readout (corr=1)")
    ap.add_argument("--coldoff", action="store_true", help="v4 with the hot-only readout (coldoff=1)")
    ap.add_argument("--qgate", type=float, default=0.0,
                    help="v4 with the query-gated stale readout at this threshold (qgate=tau)")
    ap.add_argument("--graph", action="store_true", help="time HIP graph replays of whole steps (all layers)")
    ap.add_argument("--ragged", action="store_true",
                    help="v4 requests join with random phases (each token flushes about B/c of them)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the host baseline")
    ap.add_argument("--no-deploy", action="store_true",
                    help="skip the bf16 / e4m3 storage points measured beside the default headline")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of host work for the baseline")
    ap.add_argument("--only", choices=["v4", "fresh", "prologue"], default=None,
                    help="profile one path only (prologue: the conv prologue and epilogue norm)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (5 times), for scaling HBM counters")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the rocprofv3 counter passes that measure the headline's HBM traffic")
    ap.add_argument("--traffic-pass", action="store_true",
                    help="(internal) the workload of one counter pass: 2 layers, whole windows, and a copy")
    args = ap.parse_args(argv)
    if args.cold == "fp32":
        args.master = "fp32"  # fp32 cold is its own master
    if args.exact and (args.coldoff or args.qgate > 0):
        ap.error("--exact cannot be combined with --coldoff or --qgate")
    args.skip = 0.0
    return args


def main():
    args = parse_args()

    if args.copy_calibration_mib:
        n = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.randn(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_dispatch_each_way": n * 4, "dispatches": 5}), flush=True)
        return

    if args.traffic_pass:
        traffic_pass(args, args.only or "v4", "cuda")
        return

    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): the tiered state op has no "
              f"cross-GPU exchange (requests shard across GPUs with no collective)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    if args.steps % args.c:
        args.steps += args.c - args.steps % args.c
        log(f"steps rounded up to {args.steps} (a multiple of c, so flushes are counted evenly)")

    dev = "cuda"
    if args.only == "prologue":
        print(json.dumps({"prologue_epilogue": bench_prologue(args, dev)}), flush=True)
        return
    log(f"device {torch.cuda.get_device_name(0)}; B={args.B} L={args.layers} k={args.k} c={args.c} cold={args.cold}")
    layers = make_layers(args.layers, dev, args.seed)
    inputs = make_inputs(args.layers, args.B, dev, args.seed + 7)
    torch.cuda.synchronize()

    res = {}
    if args.only != "v4":
        log("fresh ...")
        f_step, f_launch, f_ev = bench_fresh(args, layers, inputs, dev)
        res["fresh"] = (f_step, f_launch, f_ev)
        fb = args.B * bytes_fresh_token()
        log(f"fresh: {f_step:.3f} ms/step, {args.B / f_step * 1e3:,.0f} tok/s, launch {f_ev * 1e3:.1f} us "
            f"-> {fb / (f_ev * 1e-3) / 1e9:,.0f} GB/s")
    if args.only != "fresh":
        log("v4 ...")
        v_step, v_launch, v_ev, tier_gb = bench_v4(args, layers, inputs, dev)
        res["v4"] = (v_step, v_launch, v_ev)
        vb = args.B * bytes_v4_token(args.k, args.c, args.cold, args.master, args.skip, args.exact) + bytes_rotation()
        log(f"v4: {v_step:.3f} ms/step, {args.B / v_step * 1e3:,.0f} tok/s, launch {v_ev * 1e3:.1f} us "
            f"-> {vb / (v_ev * 1e-3) / 1e9:,.0f} GB/s (tiers {tier_gb:.1f} GB)")

    deploy = None
    headline_default = (args.B == 256 and args.c == 4 and args.k == 32 and args.cold == "fp32" and not args.exact
                        and not args.coldoff and args.qgate <= 0 and not args.ragged and not args.graph)
    if args.only is None and headline_default and not args.no_deploy:
        deploy = bench_deploy(args, layers, inputs, dev, res["fresh"][0])

    prologue = None
    if args.only is None:
        log("conv prologue ...")
        prologue = bench_prologue(args, dev)
        log(f"prologue: nssm_conv_update {prologue['nssm_conv_update_us']} us "
            f"({prologue['nssm_conv_update_gbs']} GB/s), torch {prologue['torch_causal_conv1d_update_us']} us; "
            f"epilogue norm: nssm_gated_rmsnorm {prologue['nssm_gated_rmsnorm_us']} us "
            f"({prologue['nssm_gated_rmsnorm_gbs']} GB/s), torch {prologue['torch_Zamba2RMSNormGated_us']} us")

    head = "v4" if "v4" in res else "fresh"
    ms_step, ms_launch, ms_ev = res[head]
    per_launch_bytes = (args.B * bytes_v4_token(args.k, args.c, args.cold, args.master, args.skip, args.exact)
                        + bytes_rotation() if head == "v4" else args.B * bytes_fresh_token())
    achieved = per_launch_bytes / (ms_ev * 1e-3) / 1e9
    readout = readout_name(args)
    traffic, traffic_src = measured_traffic(traffic_key(args, head))
    traffic_src = (f"{traffic_src}: rocprofv3 FETCH_SIZE + WRITE_SIZE of an earlier profiled run of this workload, "
                   f"scaled against a plain copy" if traffic_src else None)
    live_err = None
    under_profiler = any(k.startswith("ROCPROFILER") for k in os.environ)
    if args.only is None and not args.no_traffic and not under_profiler:
        log("traffic passes (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE) ...")
        live, live_err = live_traffic(args, head)
        if live is not None:
            traffic, traffic_src = live, (
                "measured in this run: rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE, over 2 layers of this "
                "workload (whole windows), each scaled by its reading for a copy of 256 MiB in the same pass")
            log(f"traffic: {traffic:,} B per layer-token ({traffic / per_launch_bytes:.3f} of the algorithmic)")
        else:
            log(f"traffic passes failed ({live_err}); the profiled figure is reported")
    out = {
        "metric": "state-op tokens/s at 9B shape B=256 (v4-c4 vs fresh); achieved HBM GB/s vs peak",
        "value": round(args.B / ms_step * 1e3, 1),
        "unit": "state-op tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded; bf16 x/B/C/dt, fp32 state ~N(0,0.1^2), random orthogonal R per layer-group)",
        "config": {
            "workload": (f"{head} state op, Nemotron-Nano-9B-v2 mixer shape, {args.layers} layers, B={args.B}"
                         + (f", k_hot={args.k}, c={args.c}, {args.cold} cold"
                            + (", bf16 master" if args.master == "bf16" and args.cold != "fp32" else "") + ", "
                            f"{'random phases' if args.ragged else 'phase-aligned'}" if head == "v4" else "")
                         + (f", {readout} readout" if head == "v4" and readout != "stale" else "")
                         + (", HIP graph replay" if args.graph else "")),
            "layers": args.layers, "B": args.B, "H": H, "P": P, "N": N, "G": G,
            "k_hot": args.k, "c": args.c, "cold": args.cold, "readout": readout,
            "master": args.master if args.cold != "fp32" else "fp32",
        },
        **({"cold_skip_frac": round(args.skip, 4)} if head == "v4" and readout not in ("stale", "exact") else {}),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            **({"traffic_over_algorithmic": round(traffic / per_launch_bytes, 4)} if traffic else {}),
            **({"traffic_live_error": live_err} if live_err else {}),
            "kernel": kernel_label(head, args),
            "algorithmic_bytes_per_launch": int(per_launch_bytes),
            "avg_launch_us_events": round(ms_ev * 1e3, 2),
            "avg_launch_us_region": round(ms_launch * 1e3, 2),
        },
    }
    if "fresh" in res and "v4" in res:
        out["fresh_tok_s"] = round(args.B / res["fresh"][0] * 1e3, 1)
        out["fresh_ms_per_step"] = round(res["fresh"][0], 4)
        fb = args.B * bytes_fresh_token()
        out["fresh_achieved_gbs"] = round(fb / (res["fresh"][2] * 1e-3) / 1e9, 1)
        out["speedup_v4_vs_fresh"] = round(res["fresh"][0] / res["v4"][0], 3)
    if deploy is not None:
        out["deployment_points"] = deploy
    if prologue is not None:
        out["prologue_epilogue"] = prologue
    if args.only is None:
        log("stream probe ...")
        out["stream_probe"] = stream_probe(dev, achieved)
        log(f"stream probe: read {out['stream_probe']['read_gbs']:,.0f} GB/s, copy "
            f"{out['stream_probe']['copy_gbs']:,.0f} GB/s (read + write)")
    if not args.no_cpu:
        log("cpu baseline ...")
        out["cpu_baseline"] = cpu_baseline(args, args.cpu_budget)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
