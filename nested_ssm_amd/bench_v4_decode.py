"""Drop-in for scale/bench_v4_decode.py: decode state-op speed of v4 tiered
execution vs fresh at the Nemotron-9B mixer dims (L=27, H=128, P=80, N=128),
on the MI355X kernels.

Same CLI (`--Bs --pb --cs --smoke`, scale/bench_v4_decode.py:303-334), same
`run_point(B, pb, c, device, iters=20, warmup=5) -> dict` keys
(:285-300), same `timed` (:63-73) and `fp8_cold_readout(qc, S8, scale, out)`
(:55-60), same output file bench_v4_decode.json. The arms run the Mamba2
recurrence of the decode step (rotation, dt softplus, per-head decay, D skip)
with random synthetic values, 27 layers per step:

  fresh / fresh_ssu   untiered state op (nssm_fresh_step)
  v4                  tiered, fp32 cold (one exact copy)
  v4bf16 / v4ssu      tiered, one bf16 cold copy (the reference's SnapH / SnapM bf16
                      snapshot masters, scale/bench_v4_decode.py:160-175, 258-276)
  v4fp8               tiered, e4m3 cold read copy (per-row scale) + fp32 master
                      (the reference's fp32 acc_cold, :196-221)
  hotonly             hot tier only, cold columns dropped
  eager3              the untiered recurrence in plain torch ops (unfused engine)
  v4async             not run (the reference measured the side-stream variant
                      as no gain); reported NaN

Unlike the reference's arms (constant 0.98 flush decay, scale/bench_v4_decode.py:123-124)
every arm here computes the exact step.
"""
import argparse
import json
import math

import torch

from .ops import LayerParams, V4Tier, fp8_cold_readout, fresh_step  # noqa: F401

L, H, P, N = 27, 128, 80, 128  # Nemotron-9B mamba2 mixer dims
G = 8


def timed(fn, iters, warmup, sync_buf=None):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(True), torch.cuda.Event(True)
    t0.record()
    for _ in range(iters):
        fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / iters


def _layer_params(device, seed=0):
    gen = torch.Generator().manual_seed(seed)
    f = dict(device=device, dtype=torch.float32)
    out = []
    for _ in range(L):
        u = 1e-3 + (1e-1 - 1e-3) * torch.rand(H, generator=gen, dtype=torch.float64)
        A = -torch.exp(torch.rand(H, generator=gen, dtype=torch.float64) * math.log(16.0))
        Q, Rr = torch.linalg.qr(torch.randn(G, N, N, generator=gen, dtype=torch.float64))
        R = Q * torch.sign(torch.diagonal(Rr, dim1=-2, dim2=-1))[..., None, :]
        out.append(LayerParams(H, P, N, G, torch.log(torch.expm1(u)).to(**f), A.to(**f),
                               torch.randn(H, generator=gen, dtype=torch.float64).to(**f), R.to(**f).contiguous()))
    return out


def run_point(B, pb, c, device, iters=20, warmup=5):
    dt = torch.bfloat16
    g = torch.Generator(device=device).manual_seed(0)
    x = torch.randn(B, H, P, device=device, generator=g).to(dt)
    Bm = (torch.randn(B, G, N, device=device, generator=g) / N ** 0.5).to(dt)
    Cm = (torch.randn(B, G, N, device=device, generator=g) / N ** 0.5).to(dt)
    draw = torch.randn(B, H, device=device, generator=g).to(dt)
    prms = _layer_params(device)
    y = torch.empty(B, H, P, device=device)
    res = {}

    # ---- fresh ----
    S = [torch.randn(B, H, P, N, device=device, generator=g).mul_(0.1) for _ in range(L)]

    def fresh():
        for l in range(L):
            fresh_step(prms[l], S[l], x, Bm, Cm, draw, y=y)
    res["fresh_ms"] = timed(fresh, iters, warmup)
    res["fresh_ssu_ms"] = res["fresh_ms"]

    def tiered(cold, k, master="fp32"):
        tiers = []
        for l in range(L):
            t = V4Tier(B, H, P, G, k_hot=k, c=c, cold=cold, device=device, master=master)
            t.join(prms[l], S[l])
            tiers.append(t)

        def run():
            for l in range(L):
                tiers[l].step(prms[l], x, Bm, Cm, draw, y=y)
        it_c = max(iters, 4 * c)  # flush amortization
        ms = timed(run, it_c, ((warmup + c - 1) // c) * c)
        del tiers
        torch.cuda.empty_cache()
        return ms

    res["hotonly_ms"] = tiered("off", pb) if pb < N else res["fresh_ms"]
    if pb < N:
        res["v4_ms"] = tiered("fp32", pb)
        res["v4bf16_ms"] = tiered("bf16", pb, master="bf16")
        res["v4fp8_ms"] = tiered("fp8", pb)
    else:
        res["v4_ms"] = res["v4bf16_ms"] = res["v4fp8_ms"] = res["fresh_ms"]
    res["v4ssu_ms"] = res["v4bf16_ms"]
    res["speedup_ssu"] = res["fresh_ssu_ms"] / res["v4ssu_ms"]
    res["v4async_ms"] = float("nan")

    # ---- eager: the same recurrence in unfused torch ops ----
    def eager3():
        for l in range(L):
            p = prms[l]
            Bp = torch.einsum("bgn,gmn->bgm", Bm.float(), p.R).repeat_interleave(H // G, dim=1)
            Cp = torch.einsum("bgn,gmn->bgm", Cm.float(), p.R).repeat_interleave(H // G, dim=1)
            d = torch.nn.functional.softplus(draw.float() + p.dt_bias)
            S[l] = S[l] * torch.exp(d * p.A)[..., None, None] + (d[..., None, None] * Bp[:, :, None, :]) * \
                x.float()[..., None]
            torch.einsum("bhpn,bhn->bhp", S[l], Cp)
    res["eager3_ms"] = timed(eager3, max(2, iters // 4), 1)
    del S
    torch.cuda.empty_cache()

    state_gb = L * B * H * N * P * 4 / 1e9
    res.update(B=B, pb=pb, c=c, state_gb=state_gb,
               fresh_toks=B / res["fresh_ms"] * 1e3,
               v4_toks=B / res["v4_ms"] * 1e3,
               v4async_toks=B / res["v4async_ms"] * 1e3,
               v4bf16_toks=B / res["v4bf16_ms"] * 1e3,
               hotonly_toks=B / res["hotonly_ms"] * 1e3,
               eager3_toks=B / res["eager3_ms"] * 1e3,
               speedup_vs_fresh=res["fresh_ms"] / res["v4_ms"],
               speedup_async=res["fresh_ms"] / res["v4async_ms"],
               speedup_bf16=res["fresh_ms"] / res["v4bf16_ms"],
               speedup_fp8=res["fresh_ms"] / res["v4fp8_ms"],
               v4fp8_toks=B / res["v4fp8_ms"] * 1e3,
               speedup_vs_eager3=res["eager3_ms"] / res["v4_ms"],
               fresh_bw_tbs=2 * state_gb / res["fresh_ms"])
    return res


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--Bs", type=int, nargs="+", default=[64, 256, 512, 1024])
    ap.add_argument("--pb", type=int, default=32)
    ap.add_argument("--cs", type=int, nargs="+", default=[4, 8, 16, 64])
    ap.add_argument("--smoke", action="store_true")
    ap.add_argument("--out", default="bench_v4_decode.json")
    args = ap.parse_args(argv)
    if args.smoke:
        args.Bs, args.cs = [16], [4]
    device = "cuda"
    out = {"dims": dict(L=L, H=H, P=P, N=N), "cfg": vars(args), "points": []}
    for B in args.Bs:
        for c in args.cs:
            try:
                r = run_point(B, args.pb, c, device)
            except torch.cuda.OutOfMemoryError:
                torch.cuda.empty_cache()
                print(f"B={B} c={c}: OOM, skip", flush=True)
                continue
            out["points"].append(r)
            print(f"B={B:>5} pb={args.pb} c={c:>3} | state {r['state_gb']:6.1f}GB | "
                  f"fresh {r['fresh_ms']:7.2f}ms ({r['fresh_toks']:>9,.0f} tok/s, "
                  f"BW~{r['fresh_bw_tbs']:.2f}TB/s) | v4 {r['v4_ms']:7.2f}ms ({r['v4_toks']:>9,.0f} tok/s) | "
                  f"v4-BF16COLD {r['v4bf16_ms']:7.2f}ms ({r['v4bf16_toks']:>9,.0f} tok/s) | "
                  f"v4-FP8COLD {r['v4fp8_ms']:7.2f}ms ({r['v4fp8_toks']:>9,.0f} tok/s) | "
                  f"hot-only {r['hotonly_ms']:6.2f}ms | eager3 {r['eager3_ms']:7.2f}ms | "
                  f"speedup: fp32 {r['speedup_vs_fresh']:.2f}x BF16COLD {r['speedup_bf16']:.2f}x "
                  f"FP8COLD {r['speedup_fp8']:.2f}x", flush=True)
    with open(args.out, "w") as fh:
        json.dump(out, fh, indent=1)
    print(f"saved {args.out}", flush=True)
    return out


if __name__ == "__main__":
    main()
