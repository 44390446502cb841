"""GPU: the decode step captured in a HIP graph (torch.cuda.graph) and replayed.

The step enqueues kernels only (no allocation after the first call on a stream,
no memset, no host synchronisation; the phase lives on the device), so a whole
multi-layer token can be captured once and replayed. Each test keeps an eager twin
of every tier, replays the graph several times with eager work and host
synchronisations between the replays, and checks every replay's y and the tier
state against the eager twin bit for bit (the kernels are deterministic)."""
import pytest
import torch

from helpers import dev_params
from nested_ssm_amd import V4Tier, fresh_step

import oracle

pytestmark = pytest.mark.gpu

H, P, N, G = 16, 80, 128, 2


def _layers(n, seed):
    gen = torch.Generator().manual_seed(seed)
    return [dev_params(oracle.make_layer_params(H, P, N, G, gen)) for _ in range(n)]


def _inputs(b, n, g):
    return [(torch.randn(b, H, P, device="cuda", generator=g).to(torch.bfloat16),
             (torch.randn(b, G, N, device="cuda", generator=g) / N ** 0.5).to(torch.bfloat16),
             (torch.randn(b, G, N, device="cuda", generator=g) / N ** 0.5).to(torch.bfloat16),
             torch.randn(b, H, device="cuda", generator=g).to(torch.bfloat16)) for _ in range(n)]


@pytest.mark.parametrize("c,cold,exact,master", [(4, "fp32", False, "fp32"), (4, "fp8", True, "fp32"),
                                                 (40, "fp32", False, "fp32"), (40, "bf16", True, "fp32"),
                                                 (4, "fp8", False, "bf16"), (40, "bf16", False, "bf16")])
def test_v4_step_graph_replays_match_eager(c, cold, exact, master):
    b, nl, k = 6, 3, 32
    layers = _layers(nl, seed=c)
    g = torch.Generator(device="cuda").manual_seed(1)
    S0 = [torch.randn(b, H, P, N, device="cuda", generator=g).mul_(0.1) for _ in range(nl)]
    phase = torch.randint(0, c, (b,), device="cuda", generator=g, dtype=torch.int32)
    tg = [V4Tier(b, H, P, G, k_hot=k, c=c, cold=cold, master=master) for _ in range(nl)]
    te = [V4Tier(b, H, P, G, k_hot=k, c=c, cold=cold, master=master) for _ in range(nl)]
    for l in range(nl):
        tg[l].join(layers[l], S0[l], phase=phase)
        te[l].join(layers[l], S0[l], phase=phase)
    static = _inputs(b, nl, g)
    ys = [torch.empty(b, H, P, device="cuda") for _ in range(nl)]

    def token(tiers, inp, out):
        for l in range(nl):
            tiers[l].step(layers[l], *inp[l], y=out[l], exact=exact)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # first call on the capture stream sizes its workspace
        token([V4Tier(b, H, P, G, k_hot=k, c=c, cold=cold, master=master) for _ in range(nl)], static,
              [torch.empty_like(y) for y in ys])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        token(tg, static, ys)
    torch.cuda.synchronize()
    for step in range(2 * c + 3):
        fresh = _inputs(b, nl, g)
        for dst, src in zip(static, fresh):
            for d, s_ in zip(dst, src):
                d.copy_(s_)
        graph.replay()
        ye = [torch.empty_like(y) for y in ys]
        token(te, fresh, ye)  # eager work between the replays
        torch.cuda.synchronize()
        for l in range(nl):
            assert torch.equal(ys[l], ye[l]), f"y layer {l} replay {step}"
            assert torch.equal(tg[l].hot, te[l].hot), f"hot layer {l} replay {step}"
            assert torch.equal(tg[l].t, te[l].t)
    for l in range(nl):
        assert torch.equal(tg[l].materialize(layers[l]), te[l].materialize(layers[l]))


def test_fresh_step_graph_replays_match_eager():
    b, nl = 5, 3
    layers = _layers(nl, seed=9)
    g = torch.Generator(device="cuda").manual_seed(2)
    Sg = [torch.randn(b, H, P, N, device="cuda", generator=g).mul_(0.1) for _ in range(nl)]
    Se = [s.clone() for s in Sg]
    static = _inputs(b, nl, g)
    ys = [torch.empty(b, H, P, device="cuda") for _ in range(nl)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for l in range(nl):
            fresh_step(layers[l], Sg[l].clone(), *static[l], y=torch.empty_like(ys[l]))
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for l in range(nl):
            fresh_step(layers[l], Sg[l], *static[l], y=ys[l])
    torch.cuda.synchronize()
    for step in range(6):
        inp = _inputs(b, nl, g)
        for dst, src in zip(static, inp):
            for d, s_ in zip(dst, src):
                d.copy_(s_)
        graph.replay()
        for l in range(nl):
            ye = fresh_step(layers[l], Se[l], *inp[l])
            torch.cuda.synchronize()
            assert torch.equal(ys[l], ye), f"y layer {l} replay {step}"
            assert torch.equal(Sg[l], Se[l])


@pytest.mark.parametrize("c,cold,master", [(4, "fp32", "fp32"), (64, "fp32", "fp32"), (64, "fp8", "bf16")])
def test_noalloc_step_first_called_inside_a_capture(c, cold, master):
    """nssm_v4_step_noalloc serves code under graph capture: its per-device set-up (the
    scratch array's device address, looked up with hipGetSymbolAddress, and at c = 64 the
    flush kernel's LDS limit) runs on its first call, which here happens inside the capture
    (no earlier no-allocation call in this process: this file is collected before the
    no-allocation tests). The replays, with eager work and host synchronisations between
    them, give y and tiers bit-identical to eager nssm_v4_step twins; a window the stream
    kernel replays (c = 4) and one the flush kernel replays (c = 64)."""
    b, nl, k = 6, 2, 32
    layers = _layers(nl, seed=30 + c)
    g = torch.Generator(device="cuda").manual_seed(3)
    S0 = [torch.randn(b, H, P, N, device="cuda", generator=g).mul_(0.1) for _ in range(nl)]
    phase = torch.randint(0, c, (b,), device="cuda", generator=g, dtype=torch.int32)
    tg = [V4Tier(b, H, P, G, k_hot=k, c=c, cold=cold, master=master) for _ in range(nl)]
    te = [V4Tier(b, H, P, G, k_hot=k, c=c, cold=cold, master=master) for _ in range(nl)]
    for l in range(nl):
        tg[l].join(layers[l], S0[l], phase=phase)
        te[l].join(layers[l], S0[l], phase=phase)
    static = _inputs(b, nl, g)
    ys = [torch.empty(b, H, P, device="cuda") for _ in range(nl)]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for l in range(nl):
            tg[l].step(layers[l], *static[l], y=ys[l], noalloc=True)
    torch.cuda.synchronize()
    for step in range(c + 3 if c <= 16 else 5):
        fresh = _inputs(b, nl, g)
        for dst, src in zip(static, fresh):
            for d, s_ in zip(dst, src):
                d.copy_(s_)
        graph.replay()
        ye = [te[l].step(layers[l], *fresh[l]) for l in range(nl)]  # eager work between the replays
        torch.cuda.synchronize()
        for l in range(nl):
            assert torch.equal(ys[l], ye[l]), f"y layer {l} replay {step}"
            for f in ("hot", "cold_t", "master", "scale", "t", "nv", "glog"):
                a_, e_ = getattr(tg[l], f), getattr(te[l], f)
                if a_ is not None:
                    assert torch.equal(a_.view(torch.uint8), e_.view(torch.uint8)), f"{f} layer {l} replay {step}"
