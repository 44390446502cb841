"""GPU: nssm_v4_step_noalloc (the step whose workspace is the library's fixed per-GPU
scratch array) against nssm_v4_step with a caller workspace, both through the C ABI, on
twin tiers: two calls in a row, the second with fewer requests (in other slots), for a
window the stream kernel replays and one the flush kernel replays. The kernels are the
same, so y and every tier buffer must agree bit for bit after each call."""
import ctypes

import pytest
import torch

import oracle
from helpers import dev_params
from nested_ssm_amd import V4Tier, _lib
from nested_ssm_amd.ops import _inputs, _stream, step_workspace

pytestmark = pytest.mark.gpu

H, P, N, G = 128, 80, 128, 8


def _same(a: torch.Tensor, b: torch.Tensor, what: str):
    assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), what


@pytest.mark.parametrize("cold,master,c", [("fp32", "fp32", 4), ("fp8", "bf16", 64), ("bf16", "fp32", 40)])
def test_noalloc_step_equals_the_workspace_step(cold, master, c):
    L = _lib.lib()
    gen = torch.Generator().manual_seed(500 + c)
    prm = oracle.make_layer_params(H, P, N, G, gen)
    dprm = dev_params(prm)
    slots = 96
    S0 = oracle.make_state(slots, H, P, N, gen).cuda()
    phase = torch.randint(0, c, (slots,), generator=gen, dtype=torch.int32).cuda()
    tiers = [V4Tier(slots, H, P, G, k_hot=32, c=c, cold=cold, master=master) for _ in range(2)]
    tiers[0].join(dprm, S0, phase=phase)
    for f in _lib.TIER_FIELDS:  # the twin is a bitwise copy, unwritten ring rows included
        if tiers[0]._field(f) is not None:
            tiers[1]._field(f).copy_(tiers[0]._field(f))
    pc = dprm.c_struct()
    tc = [t.c_struct() for t in tiers]
    # first call: every slot; second call: 7 requests in scattered slots
    calls = [(slots, None), (7, torch.tensor([90, 3, 41, 17, 66, 0, 58], dtype=torch.int32).cuda())]
    for n, (b, sl) in enumerate(calls):
        x, B, C, dt = (v.cuda() for v in oracle.make_step_inputs(b, H, P, N, G, gen))
        ic = _inputs(dprm, x, B, C, dt, sl)
        y_ws = torch.full((b, H, P), float("nan"), device="cuda")
        y_na = torch.full((b, H, P), float("nan"), device="cuda")
        ws = step_workspace(b, H, G, c)
        rc = L.nssm_v4_step(ctypes.byref(pc), ctypes.byref(tc[0]), ctypes.byref(ic), y_ws.data_ptr(),
                            ws.data_ptr(), ws.numel(), _stream())
        assert rc == 0, L.nssm_strerror(rc)
        rc = L.nssm_v4_step_noalloc(ctypes.byref(pc), ctypes.byref(tc[1]), ctypes.byref(ic), y_na.data_ptr(),
                                    _stream())
        assert rc == 0, L.nssm_strerror(rc)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(y_na).all()), f"call {n}: y not written"
        _same(y_na, y_ws, f"call {n} ({b} requests): y")
        for f in _lib.TIER_FIELDS:
            a, w = tiers[1]._field(f), tiers[0]._field(f)
            if a is not None:
                _same(a, w, f"call {n} ({b} requests): tier {f}")
