"""Shared helpers for the parity tests: seeded inputs built on the CPU (so the
oracle and the GPU see identical bits) and copied to the device."""
import torch

import oracle
from nested_ssm_amd import LayerParams


def dev_params(prm: oracle.LayerParams, device="cuda") -> LayerParams:
    f = dict(device=device, dtype=torch.float32)
    R = None if prm.R is None else prm.R.to(**f).contiguous()
    return LayerParams(prm.H, prm.P, prm.N, prm.G, prm.dt_bias.to(**f), prm.A.to(**f), prm.D.to(**f), R,
                       prm.dt_min)


def to_dev(*ts, device="cuda"):
    return [None if t is None else t.to(device).contiguous() for t in ts]


def max_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30))


def assert_close32(got: torch.Tensor, ref: torch.Tensor, what: str, rtol=1e-5, atol=1e-5):
    """The fp32 parity bar: |got - ref| <= atol + rtol |ref| elementwise (computed on
    the device of `ref`, or the CPU when the two differ)."""
    if got.device != ref.device:
        got, ref = got.detach().cpu(), ref.detach().cpu()
    got = got.detach().float()
    ref = ref.detach().float()
    err = (got - ref).abs()
    bound = atol + rtol * ref.abs()
    bad = err > bound
    if bool(bad.any()):
        i = int(torch.argmax((err - bound).flatten()))
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.numel()} elements outside rtol={rtol} "
                             f"atol={atol}; worst at flat index {i}: got {got.flatten()[i].item():.8g} "
                             f"ref {ref.flatten()[i].item():.8g} (max abs err {err.max().item():.3g})")


def assert_close_flips(got: torch.Tensor, ref: torch.Tensor, what: str, rel=1e-4, frac_max=1e-2, rtol=1e-5,
                       atol=1e-5):
    """The bar for values rounded to bf16 from fp32 results that two paths build in
    different summation orders (one fp32 ulp apart, they can round to neighbouring
    bf16 values, 2^-8 relative, in isolated elements): norm-wise relative error
    <= rel and at most frac_max of the elements beyond the fp32 bar."""
    got, ref = got.detach().cpu().float(), ref.detach().cpu().float()
    r = max_rel(got, ref)
    assert r <= rel, f"{what}: norm-wise rel err {r:.3g} > {rel:g}"
    frac = float(((got - ref).abs() > atol + rtol * ref.abs()).float().mean())
    assert frac <= frac_max, f"{what}: {frac:.3%} of elements beyond the fp32 bar"
    return r
