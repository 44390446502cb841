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


class Fresh64:
    """The exact (fp64) fresh trajectory of a state on the GPU, in plain torch: the state the
    tiers represent, for checks at full size. S <- exp(a) S + (dt x) (x) B', y = S C' + D x with
    B' = R B, C' = R C per group, dt = softplus(dt_raw + dt_bias) (threshold 20, as torch and the
    kernels), a = dt A; every operand is the kernels' input (bf16 or fp32) converted exactly to
    fp64."""

    def __init__(self, prm: LayerParams, S: torch.Tensor):
        self.H, self.G = prm.H, prm.G
        self.R = None if prm.R is None else prm.R.double()
        self.dt_bias, self.A, self.D = prm.dt_bias.double(), prm.A.double(), prm.D.double()
        self.S = S.double()

    def _rot(self, v: torch.Tensor) -> torch.Tensor:
        v = v.double()
        if self.R is not None:
            v = torch.einsum("bgn,gmn->bgm", v, self.R)
        return v.repeat_interleave(self.H // self.G, dim=1)

    def step(self, x, B, C, dt_raw, slots=None):
        """Advance the rows `slots` (all when None); returns (a [b,H], C' [b,H,N], D x [b,H,P])."""
        d = torch.nn.functional.softplus(dt_raw.double() + self.dt_bias[None, :])
        a = d * self.A[None, :]
        Bp, Cp = self._rot(B), self._rot(C)
        u = (d[..., None] * x.double())[..., None]  # [b,H,P,1]
        if slots is None:
            self.S.mul_(torch.exp(a)[..., None, None]).addcmul_(u, Bp[:, :, None, :])
        else:
            sl = slots.long()
            self.S[sl] = self.S[sl] * torch.exp(a)[..., None, None] + u * Bp[:, :, None, :]
        return a, Cp, x.double() * self.D[None, :, None]

    def readout(self, Cp, cols=None, rows=None):
        """S[rows][..., cols] . C'[..., cols] (fp64)."""
        S = self.S if rows is None else self.S[rows.long()]
        if cols is not None:
            S, Cp = S[..., cols], Cp[..., cols]
        return torch.einsum("bhpn,bhn->bhp", S, Cp)
