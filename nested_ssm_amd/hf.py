"""Transformers NemotronH integration of the MI355X decode-step kernels.

Shared engine of the two drop-in modules v4_native_decode and v4_fused_decode.
A patched NemotronHMamba2Mixer runs prefill through the stock transformers
forward, then captures the state into a V4Tier (join); every single-token
decode call then runs

    prologue  in_proj (torch GEMM); causal conv1d update + SiLU + x/B/C split
              (nssm_conv_update; transformers' own functions under a padding mask)
    state op  nssm_v4_step / _exact / _gated, or nssm_fresh_step (pb >= N)
    epilogue  gated RMSNorm (nssm_gated_rmsnorm), out_proj (torch GEMM)

all HIP launches in libnssm_hip.so.

Rotation: the installed transformers (5.15) mixer never calls `self.act`, so a
rotation wrapper on `act` (ActRotMask, scale/nemotron_retrofit.py:15-56) would
not rotate B and C in prefill. Because the per-head decay is a scalar, the
model is invariant under an orthogonal rotation of the state basis
(S' = S R^T, y' = y): prefill runs unrotated and the captured state is rotated
once, S' = S R^T, before the tiers are filled; decode then rotates B and C
inside the kernels. Before any multi-token call that continues a decoded
sequence, the exact current state is rebuilt from the tiers (materialize) and
rotated back, so the stock forward sees the state it expects.
"""
import torch
from torch import nn

from . import ops
from .ops import N_STATE, LayerParams, V4Tier

MIXER = "NemotronHMamba2Mixer"


def _modeling():
    from transformers.models.nemotron_h import modeling_nemotron_h as M

    return M


# ---------------------------------------------------------------------------
class ActRotMask(nn.Module):
    """Container for the per-group rotation R of a mixer, identity-initialised
    (scale/nemotron_retrofit.py:15-56): `m.act = ActRotMask(m.act, inter,
    ngroups, dstate)` then `m.act.R.data.copy_(R_i)`. forward() keeps the
    reference's training-path semantics (activation, then rotation and width
    mask of the B and C slices); the decode kernels read `R` directly."""

    def __init__(self, act, inter, ngroups, dstate):
        super().__init__()
        self.act = act
        self.inter, self.ng, self.ds = inter, ngroups, dstate
        self.conv_dim = inter + 2 * ngroups * dstate
        self.R = nn.Parameter(torch.eye(dstate).repeat(ngroups, 1, 1))
        self.width = dstate

    def _rot(self, x):  # (B, T, G*N) -> (B, T, G, N) rotated, einsum('btgn,gmn->btgm')
        b, t, _ = x.shape
        return torch.einsum("btgn,gmn->btgm", x.view(b, t, self.ng, self.ds), self.R.to(x.dtype))

    def _mask(self, x):  # (B, T, G, N): the coordinates at and above width zeroed (per request for a tensor)
        b, t = x.shape[:2]
        w = self.width
        if torch.is_tensor(w):
            keep = torch.arange(self.ds, device=x.device)[None, :] < w.to(x.device)[:, None]  # [B, N]
            x = x * keep.to(x.dtype)[:, None, None, :]
        elif w < self.ds:
            x = torch.cat([x[..., :w], torch.zeros_like(x[..., w:])], -1)
        return x.reshape(b, t, self.ng * self.ds)

    def rotmask(self, x):
        return self._mask(self._rot(x))

    def forward(self, x):
        x = self.act(x)
        if x.dim() == 3 and x.shape[-1] == self.conv_dim:
            h, B, C = torch.split(x, [self.inter, self.ng * self.ds, self.ng * self.ds], dim=-1)
            x = torch.cat([h, self._mask(self._rot(B)), self._mask(self._rot(C))], dim=-1)
        return x


def get_wrappers(model):
    """Every ActRotMask of a model (scale/nemotron_retrofit.py:111-112)."""
    return [m for m in model.modules() if isinstance(m, ActRotMask)]


def set_width(model, w):
    """Set the width mask of every wrapper (scale/nemotron_retrofit.py:114-116): rotated B and C
    coordinates at and above w are zeroed (the evaluation forward folds a scalar w into R)."""
    for m in get_wrappers(model):
        m.width = w


def mixer_rotation(m):
    """R [G, N, N] attached to a mixer by any of the reference's conventions:
    ActRotMask (m.act.R), the fused install (m._v4R) or the vLLM port (m.v4R)."""
    for R in (getattr(m.act, "R", None), getattr(m, "_v4R", None), getattr(m, "v4R", None)):
        if R is not None:
            return R.detach()
    return None


def layer_params(m, dt_min: float) -> LayerParams:
    dev = m.A_log.device
    return LayerParams.from_mixer_values(m.dt_bias, m.A_log, m.D, mixer_rotation(m), P=m.head_dim,
                                         G=m.n_groups, dt_min=dt_min, device=dev)


def rotate_state(S: torch.Tensor, R: torch.Tensor, inverse: bool = False) -> torch.Tensor:
    """S R^T per head (the head's group rotation); inverse: S R. fp32."""
    H, G = S.shape[1], R.shape[0]
    Rh = R.float().repeat_interleave(H // G, dim=0)  # [H, N, N]
    if inverse:
        return torch.einsum("bhpm,hmn->bhpn", S.float(), Rh.contiguous())
    return torch.einsum("bhpn,hmn->bhpm", S.float(), Rh.contiguous())


_QGATE_KEYS = ("qgate_n", "qgate_kept")


class V4State(dict):
    """Per-mixer decode state (`m._v4state`). Keys: "tier" (V4Tier or None for
    the untiered path), "params" (LayerParams), "pb", "c". Item "t" reads and
    writes the decode phase kept on the device (callers reset it between
    prompts, scale/probe_selfspec_policy.py:127-128). Writing it re-captures the
    tier at the new phase: the exact current state is rebuilt (materialize) and
    joined again with t = value, so the snapshot, the buffered window and glog
    restart together (the reference keeps its older snapshot and lets the window
    grow past c tokens, which a tier holding at most c buffered tokens cannot
    represent). Items "qgate_n" and "qgate_kept" (present once a query-gated token
    has run, as in scale/v4_native_decode.py:153-154) read the gated and kept head
    counts kept on the device (scale/run_recall_native.py:116-118 reads them with
    .get)."""

    def __getitem__(self, key):
        if key == "t":
            tier = dict.get(self, "tier")
            return int(tier.t[0, 0].item()) if tier is not None else dict.get(self, "t_fresh", 0)
        if key in _QGATE_KEYS:
            qc = dict.get(self, "qcounts")
            if qc is None:
                raise KeyError(key)
            return int(qc[_QGATE_KEYS.index(key)].item())
        return dict.__getitem__(self, key)

    def get(self, key, default=None):
        try:
            return self[key]
        except KeyError:
            return default

    def __contains__(self, key):
        if key in _QGATE_KEYS:
            return dict.get(self, "qcounts") is not None
        return key == "t" or dict.__contains__(self, key)

    def __setitem__(self, key, value):
        if key == "t":
            t = int(value)
            if t < 0:
                raise ValueError(f"_v4state['t'] must be >= 0 (got {t})")
            tier = dict.get(self, "tier")
            if tier is None:
                dict.__setitem__(self, "t_fresh", t)
            elif tier.cold == "off":  # no cold tier: the phase only counts tokens
                tier.t.fill_(t)
            else:
                prm = dict.__getitem__(self, "params")
                phase = torch.full((tier.slots,), t, dtype=torch.int32, device=tier.hot.device)
                tier.join(prm, tier.materialize(prm), phase=phase)
            return
        dict.__setitem__(self, key, value)


# ---------------------------------------------------------------------------
def decode_inputs(m, hidden_states, cache_params, attention_mask):
    """One decode token through in_proj and the causal conv1d update + SiLU (one
    nssm_conv_update launch; transformers' own functions when a padding mask is
    given): gate [b,1,I] and x [b,H,P], B, C [b,G,N], dt [b,H] in bf16, as the
    kernels take them."""
    M = _modeling()
    b = hidden_states.shape[0]
    H, P, G, N = m.num_heads, m.head_dim, m.n_groups, m.ssm_state_size
    hidden_states = M.apply_mask_to_padding_states(hidden_states, attention_mask)
    proj = m.in_proj(hidden_states)
    gate, hbc, dt = proj.split([m.intermediate_size, m.conv_dim, H], dim=-1)
    conv_state = cache_params.layers[m.layer_idx].conv_states[0]
    bf = torch.bfloat16
    w = m.conv1d.weight.squeeze(1)
    if (attention_mask is None and m.activation in ("silu", "swish") and hbc.dtype in (torch.float32, bf)
            and conv_state.dtype == hbc.dtype and w.dtype == hbc.dtype and conv_state.is_contiguous()):
        # conv update + SiLU + split in one HIP launch (scale/v4_fused_decode.py:42-44)
        x, B, C = ops.conv_update(hbc[:, 0], conv_state, w.contiguous(), m.conv1d.bias, m.intermediate_size,
                                  G * N)
    else:
        hbc = M.causal_conv1d_update(hbc.transpose(1, 2), conv_state, w, m.conv1d.bias,
                                     activation=m.activation).transpose(1, 2)
        hbc = M.apply_mask_to_padding_states(hbc, attention_mask)
        x, B, C = torch.split(hbc, [m.intermediate_size, G * N, G * N], dim=-1)
    return (gate, x.reshape(b, H, P).to(bf).contiguous(), B.reshape(b, G, N).to(bf).contiguous(),
            C.reshape(b, G, N).to(bf).contiguous(), dt.reshape(b, H).to(bf).contiguous())


def decode_epilogue(m, y, gate, dtype):
    """y [b,H,P] fp32 (D x included) -> gated RMSNorm (one nssm_gated_rmsnorm launch for
    the mixer's Zamba2RMSNormGated) -> out_proj."""
    b = y.shape[0]
    norm = m.norm
    g = gate[:, 0]
    if (type(norm).__name__ == "Zamba2RMSNormGated" and g.dtype == dtype and norm.weight.dtype == dtype
            and dtype in (torch.float32, torch.bfloat16) and g.stride(-1) == 1):
        out = ops.gated_rmsnorm(y.reshape(b, -1), g, norm.weight, norm.group_size, norm.variance_epsilon)
        return m.out_proj(out.reshape(b, 1, -1))
    out = norm(y.to(dtype).reshape(b, 1, -1), gate)
    return m.out_proj(out.to(dtype))


def decode_step(m, hidden_states, cache_params, attention_mask):
    """The tiered (or untiered, pb >= N) decode step of one mixer."""
    st = m._v4state
    gate, x, B, C, dt = decode_inputs(m, hidden_states, cache_params, attention_mask)
    prm = st["params"]
    tier = dict.get(st, "tier")
    check_readout_cfg(m.v4cfg, st["pb"], m.ssm_state_size)
    if tier is None:
        S = cache_params.layers[m.layer_idx].recurrent_states[0]
        y = ops.fresh_step(prm, S, x, B, C, dt)
    else:
        # the readout keys are read per token (callers switch them at run time), in the
        # reference's order: corr (rank-c exact correction, scale/v4_native_decode.py:81-117),
        # else coldoff (hot-only draft readout, :118-127), else the stale readout,
        # query-gated when qgate > 0 (:147-156)
        cfg = m.v4cfg
        exact = bool(cfg.get("corr"))
        hot_only = not exact and bool(cfg.get("coldoff"))
        tau = 0.0 if exact or hot_only else float(cfg.get("qgate") or 0.0)
        if not hot_only and int(cfg["c"]) != tier.c:
            if int(cfg["c"]) > ops.MAX_WINDOW:
                raise NotImplementedError(f"window c={cfg['c']} exceeds the kernels' {ops.MAX_WINDOW}: it is "
                                          "supported with the hot-only readout (coldoff=1) only")
            raise NotImplementedError(f"v4cfg['c'] changed from {tier.c} to {cfg['c']} after capture; the "
                                      "tier's flush window is fixed when the prefill state is captured")
        counts = None
        if tau > 0:
            counts = dict.get(st, "qcounts")
            if counts is None:
                counts = torch.zeros(2, dtype=torch.int64, device=x.device)
                dict.__setitem__(st, "qcounts", counts)
        y = tier.step(prm, x, B, C, dt, exact=exact, hot_only=hot_only, qgate=tau, counts=counts)
    return decode_epilogue(m, y, gate, hidden_states.dtype)


def check_readout_cfg(cfg, pb: int, N: int):
    """Readout keys the kernels do not serve: a hot/cold split changed after capture
    (the tier's split is fixed when it is captured) and the top-k cold column gather
    (ktop < N - pb, scale/v4_native_decode.py:129-143: a data-dependent gather of cold
    columns, not a tier readout)."""
    if min(int(cfg["pb"]), N) != min(pb, N):
        raise NotImplementedError(f"v4cfg['pb'] changed from {pb} to {cfg['pb']} after capture; the tier's "
                                  "hot/cold split is fixed at capture")
    ktop = int(cfg.get("ktop") or 0)
    if pb < N and 0 < ktop < N - pb and not cfg.get("corr") and not cfg.get("coldoff"):
        raise NotImplementedError("v4cfg['ktop'] (top-k cold column gather) is not implemented by the "
                                  "MI355X kernels")


def _cold_kind(cfg) -> str:
    if "cold" in cfg:
        return cfg["cold"]
    return "bf16" if cfg.get("cold_bf16") else "fp32"


def capture(m, cache_params, dt_min: float):
    """End of prefill: tiers from the cache's fp32 state (rotated into R's basis)."""
    cfg = m.v4cfg
    pb, c = int(cfg["pb"]), int(cfg["c"])
    check_readout_cfg(cfg, pb, m.ssm_state_size)
    if c > ops.MAX_WINDOW and pb < m.ssm_state_size:
        # the hot-only readout never reads the cold tier, which evolves exactly at any
        # window: it runs on the largest window the kernels take
        if not cfg.get("coldoff"):
            raise NotImplementedError(f"window c={c} exceeds the kernels' {ops.MAX_WINDOW} (supported with "
                                      "coldoff=1 only)")
        c = ops.MAX_WINDOW
    layer = cache_params.layers[m.layer_idx]
    S = layer.recurrent_states[0]
    prm = layer_params(m, dt_min)
    Srot = rotate_state(S, prm.R) if prm.R is not None else S.float()
    b = S.shape[0]
    if pb >= m.ssm_state_size:
        if prm.R is not None:
            layer.recurrent_states[0].copy_(Srot)
        m._v4state = V4State(tier=None, params=prm, pb=pb, c=c, rotated=prm.R is not None)
        return
    kind = _cold_kind(cfg)
    master = cfg.get("master", "fp32") if kind in ("bf16", "fp8") else "fp32"
    # the x ring's layout follows the readout configured at capture (either layout serves
    # every readout if corr changes later)
    tier = V4Tier(b, m.num_heads, m.head_dim, m.n_groups, k_hot=pb, c=c, cold=kind, device=S.device,
                  master=master, x_ring=ops.x_ring_for(c, bool(cfg.get("corr"))))
    tier.join(prm, Srot.contiguous())
    m._v4state = V4State(tier=tier, params=prm, pb=pb, c=c, rotated=prm.R is not None)


def restore_cache(m, cache_params):
    """Exact current state back into the cache, in the unrotated basis, before a
    stock multi-token forward continues a decoded sequence."""
    st = m._v4state
    layer = cache_params.layers[m.layer_idx]
    prm = st["params"]
    tier = dict.get(st, "tier")
    if tier is not None and tier.cold == "off":
        raise NotImplementedError("cold='off' drops the cold columns: a multi-token call cannot continue "
                                  "from a hot-only decoded sequence")
    S = tier.materialize(prm) if tier is not None else layer.recurrent_states[0].float()
    if prm.R is not None:
        S = rotate_state(S, prm.R, inverse=True)
    layer.recurrent_states[0].copy_(S)
    m._v4state = None


def dispatch(m, hidden_states, cache_params, attention_mask, kw, orig_forward, dt_min, decode_fn):
    """Body of a patched mixer forward: single-token decode through `decode_fn`
    (the tiered step) once a tier exists; anything else through the stock
    forward, after which the tier is (re)captured."""
    seq_len = hidden_states.shape[1]
    has_prev = cache_params is not None and cache_params.has_previous_state(m.layer_idx)
    if has_prev and m._v4state is not None:
        if seq_len == 1 and not cache_params.layers[m.layer_idx].record_past:
            return decode_fn(m, hidden_states, cache_params, attention_mask)
        restore_cache(m, cache_params)
    out = orig_forward(m, hidden_states, cache_params=cache_params, attention_mask=attention_mask, **kw)
    if cache_params is not None:
        capture(m, cache_params, dt_min)
    return out


def mixers(model):
    return [m for m in model.modules() if type(m).__name__ == MIXER]


def check_mixer_shape(m):
    if m.ssm_state_size != N_STATE:
        raise ValueError(f"the MI355X kernels need d_state = {N_STATE} (mixer has {m.ssm_state_size})")
    if m.head_dim % 16:
        raise ValueError(f"the MI355X kernels need head_dim % 16 == 0 (mixer has {m.head_dim})")
