"""Drop-in for the teacher-forced evaluation forward of scale/nemo9b_eval.py on the
MI355X kernels.

Same module surface: the `CFG` dict (keys mode, c, pb, lag, cold_bf16, warm, state_bf16,
state_fp8, cold_fp8; scale/nemo9b_eval.py:12-17) and `naive_mixer_forward(self,
input_states, cache_params=None, cache_position=None, attention_mask=None, **kw)`, bound to
a NemotronHMamba2Mixer as the reference's driver does (`m.forward =
naive_mixer_forward.__get__(m)`, scale/nemo9b_eval.py:185-186) to score whole sequences with
the per-token loop of scale/nemo9b_eval.py:41-85. A forward runs in_proj, the causal conv1d
and the activation in torch (as the reference), then one state-op launch pair per token:
mode "fresh" (or "v4" with pb >= d_state) the untiered step; mode "v4" the teacher-forced
readout of a tier with pb hot columns that starts each sequence from a zero state
(nssm_v4_step_teacher; the exact readout for the first `warm` tokens); mode "c1" (every
column stale, :79-80) the same readout of a tier with no hot column (k_hot = 0); with
lag = 1 (:44,59,70, readers one snapshot behind) either mode's lagged form
(nssm_v4_step_teacher_lagged); then the gated norm and out_proj.

The rotation R is read from the mixer (an ActRotMask-wrapped act, `_v4R` or `v4R`) and
applied in fp32 inside the kernels; the wrapper's own activation is used, not its rotation.
A width below d_state (set_width, scale/nemotron_retrofit.py:114-116, as the driver's
"hot-alone" needle arm sets it, scale/nemo9b_eval.py:198) zeroes the rotated B and C at and
above `width` (ActRotMask._mask): the kernels get the rotation with those rows zeroed,
diag(mask) R (the identity's when there is no R), which is the same product.

cold_fp8 stores the tier's e4m3 format, the per-row scale amax / 448 + 1e-12 of
scale/vllm_v4_patch.py:106-111, where this loop scales per column (amax over the head
dimension, :62-64); the readout stays within the 2e-2 fp8 bar of that column emulation.
Deviations, each raising NotImplementedError: state_bf16, state_fp8, a width given per
request (a tensor), lag other than 0 or 1, and warm > 0 over a bf16 or e4m3 snapshot, in
mode "c1" or with lag = 1.
"""
import torch

from . import hf
from .ops import N_STATE, V4Tier, fresh_step

CFG = {"mode": "fresh", "c": 16, "pb": 32, "lag": 0, "cold_bf16": 0, "warm": 0,
       "state_bf16": 0, "state_fp8": 0, "cold_fp8": 0}


def _dt_min(m) -> float:
    lim = getattr(m, "time_step_limit", None)
    return float(lim[0]) if lim is not None else float(getattr(m, "time_step_min", 0.0))


def _wrapped(m) -> bool:
    act = m.act
    return hasattr(act, "R") and hasattr(act, "act")


def _activation(m):
    """The mixer's activation without a rotation wrapper's rotation (the kernels rotate)."""
    return m.act.act if _wrapped(m) else m.act


def _width(m) -> int:
    """The rotation wrapper's width (set_width), d_state without a wrapper."""
    N = m.ssm_state_size
    w = getattr(m.act, "width", N) if _wrapped(m) else N
    if torch.is_tensor(w):
        raise NotImplementedError("a width per request (a tensor, ActRotMask._mask) is not served by the kernels")
    return min(int(w), N)


def _params(m):
    """The kernels' layer parameters: the mixer's, with the width mask folded into R."""
    prm = hf.layer_params(m, _dt_min(m))
    w = _width(m)
    if w < m.ssm_state_size:
        G, N = m.n_groups, m.ssm_state_size
        R = prm.R if prm.R is not None else torch.eye(N, device=prm.A.device).repeat(G, 1, 1)
        R = R.clone()
        R[:, w:, :] = 0.0  # rows m >= width: B'_m = C'_m = 0 (ActRotMask._mask)
        prm.R = R.contiguous()
    return prm


def _check_cfg(cfg):
    for key in ("state_bf16", "state_fp8"):
        if cfg.get(key, 0):
            raise NotImplementedError(f"CFG[{key!r}] = {cfg[key]} is not served by the MI355X kernels")
    if int(cfg.get("lag", 0)) not in (0, 1):
        raise NotImplementedError(f"CFG['lag'] = {cfg['lag']}: lags 0 and 1 are served by the kernels")
    if cfg["mode"] not in ("fresh", "v4", "c1"):
        raise NotImplementedError(f"mode {cfg['mode']!r}: 'fresh', 'v4' and 'c1' are served by the kernels")


def teacher_forced_inputs(m, input_states):
    """in_proj, causal conv1d + activation and the split (scale/nemo9b_eval.py:21-37):
    gate [B,T,I], and the state op's bf16 inputs x [B,T,H,P], B, C [B,T,G,N], dt [B,T,H]."""
    B_, T, _ = input_states.shape
    H, P, N, G = m.num_heads, m.head_dim, m.ssm_state_size, m.n_groups
    proj = m.in_proj(input_states)
    d_mlp = (proj.shape[-1] - 2 * m.intermediate_size - 2 * G * N - H) // 2
    _, _, gate, hBC, dt = proj.split([d_mlp, d_mlp, m.intermediate_size, m.intermediate_size + 2 * G * N, H],
                                     dim=-1)
    hBC = _activation(m)(m.conv1d(hBC.transpose(1, 2))[..., :T].transpose(1, 2))
    x, B, C = torch.split(hBC, [m.intermediate_size, G * N, G * N], dim=-1)
    bf = torch.bfloat16
    return (gate, x.reshape(B_, T, H, P).to(bf), B.reshape(B_, T, G, N).to(bf), C.reshape(B_, T, G, N).to(bf),
            dt.to(bf))


def _tier(m, b, pb, c, cold, device, lag=False):
    """The mixer's evaluation tier, kept between forwards of the same batch and split."""
    key = (b, pb, c, cold, lag)
    t = getattr(m, "_tf_tier", None)
    if t is None or t[0] != key:
        t = (key, V4Tier(b, m.num_heads, m.head_dim, m.n_groups, k_hot=pb, c=c, cold=cold, device=device,
                         lag=lag))
        m._tf_tier = t
    return t[1]


def state_op(m, x, B, C, dt, cfg=None):
    """The per-token loop of scale/nemo9b_eval.py:41-84 over bf16 inputs [B,T,...] on the GPU;
    returns y [B,T,H,P] fp32 (D x included)."""
    cfg = CFG if cfg is None else cfg
    _check_cfg(cfg)
    B_, T = x.shape[:2]
    N = m.ssm_state_size
    if N != N_STATE:
        raise ValueError(f"the MI355X kernels need d_state = {N_STATE} (mixer has {N})")
    prm = _params(m)
    dev = x.device
    ys = torch.empty(B_, T, m.num_heads, m.head_dim, device=dev, dtype=torch.float32)
    mode, pb, c, warm = cfg["mode"], int(cfg["pb"]), int(cfg["c"]), int(cfg.get("warm", 0))
    zeros = torch.zeros(B_, m.num_heads, m.head_dim, N, device=dev, dtype=torch.float32)
    y_t = torch.empty(B_, m.num_heads, m.head_dim, device=dev, dtype=torch.float32)
    if mode == "fresh" or (mode == "v4" and pb >= N):
        for t in range(T):  # the state starts from zeros and evolves in place
            fresh_step(prm, zeros, x[:, t].contiguous(), B[:, t].contiguous(), C[:, t].contiguous(),
                       dt[:, t].contiguous(), y=y_t)
            ys[:, t].copy_(y_t)
        return ys
    cold = "fp8" if cfg.get("cold_fp8") else "bf16" if cfg.get("cold_bf16") else "fp32"
    if warm > 0 and cold != "fp32":
        raise NotImplementedError("warm tokens read the exact state; over a bf16 / e4m3 snapshot the kernels' "
                                  "exact readout reads the rounded snapshot instead")
    k = 0 if mode == "c1" else pb  # c1: every column read from the snapshot
    lag = bool(int(cfg.get("lag", 0)))
    if warm > 0 and k == 0:
        raise NotImplementedError("warm tokens in mode 'c1': a tier without hot columns has no exact readout")
    if warm > 0 and lag:
        raise NotImplementedError("warm tokens with lag = 1: the exact readout does not keep the lagged snapshot")
    tier = _tier(m, B_, k, c, cold, dev, lag)
    # the sequence starts from zeros at position 0, a flush position: phase c - 1
    tier.join(prm, zeros, phase=torch.full((B_,), c - 1, dtype=torch.int32, device=dev))
    for t in range(T):
        tier.step(prm, x[:, t].contiguous(), B[:, t].contiguous(), C[:, t].contiguous(), dt[:, t].contiguous(),
                  y=y_t, exact=t < warm, teacher=t >= warm)
        ys[:, t].copy_(y_t)
    return ys


def naive_mixer_forward(self, input_states, cache_params=None, cache_position=None, attention_mask=None, **kw):
    """scale/nemo9b_eval.py:19-89 on the GPU kernels: a whole sequence through the mixer with
    the per-token readout CFG selects (no cache, as the reference's evaluation runs)."""
    B_, T, _ = input_states.shape
    gate, x, B, C, dt = teacher_forced_inputs(self, input_states)
    y = state_op(self, x, B, C, dt)
    y = y.reshape(B_, T, -1).to(input_states.dtype)
    y = self.norm(y, gate)
    return self.out_proj(y)
