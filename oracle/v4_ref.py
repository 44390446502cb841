"""CPU restatement of the reference decode step (test infrastructure only).

Every function cites the reference file:line it follows (omin-Kwon/nested_ssm).
Tensors are torch CPU tensors; `dtype` selects fp32 (the parity convention)
or fp64 (for pinning the fp32 path against exact-ish arithmetic).
"""
from dataclasses import dataclass
import math
from typing import Optional

import torch
import torch.nn.functional as F

E4M3_MAX = 448.0


# ---------------------------------------------------------------------------
# parameters and synthetic inputs
@dataclass
class LayerParams:
    H: int
    P: int
    N: int
    G: int
    dt_bias: torch.Tensor  # [H]
    A: torch.Tensor        # [H] = -exp(A_log)
    D: torch.Tensor        # [H]
    R: Optional[torch.Tensor]  # [G, N, N] or None (identity)
    dt_min: float = 0.0

    def to(self, dtype):
        return LayerParams(self.H, self.P, self.N, self.G, self.dt_bias.to(dtype), self.A.to(dtype),
                           self.D.to(dtype), None if self.R is None else self.R.to(dtype), self.dt_min)


def make_rotation(G: int, N: int, gen: torch.Generator) -> torch.Tensor:
    """Q of QR(N(0,1)) with the sign fix Q * sign(diag(R_qr)), as the reference
    retracts R to orthogonal (scale/nemotron_retrofit.py:359-363)."""
    W = torch.randn(G, N, N, generator=gen, dtype=torch.float64)
    Q, Rr = torch.linalg.qr(W)
    sgn = torch.sign(torch.diagonal(Rr, dim1=-2, dim2=-1))
    return (Q * sgn[..., None, :]).to(torch.float32).contiguous()


def make_layer_params(H: int, P: int, N: int, G: int, gen: torch.Generator, rotation: bool = True,
                      dt_min: float = 0.0) -> LayerParams:
    """Per-head dt_bias = log(expm1(U(1e-3, 1e-1))), A = -exp(U(0, ln 16)), D ~ N(0,1);
    per-group R (the synthetic distributions of the benchmark configurations)."""
    u = 1e-3 + (1e-1 - 1e-3) * torch.rand(H, generator=gen, dtype=torch.float64)
    dt_bias = torch.log(torch.expm1(u)).to(torch.float32)
    A = -torch.exp(torch.rand(H, generator=gen, dtype=torch.float64) * math.log(16.0)).to(torch.float32)
    D = torch.randn(H, generator=gen, dtype=torch.float32)
    R = make_rotation(G, N, gen) if rotation else None
    return LayerParams(H, P, N, G, dt_bias, A, D, R, dt_min)


def make_state(slots: int, H: int, P: int, N: int, gen: torch.Generator, std: float = 0.1) -> torch.Tensor:
    """fp32 state ~ N(0, std^2) (std read as 0.1)."""
    return torch.randn(slots, H, P, N, generator=gen, dtype=torch.float32) * std


def make_step_inputs(b: int, H: int, P: int, N: int, G: int, gen: torch.Generator):
    """One decode token: x ~ N(0,1), B, C ~ N(0,1)/sqrt(N), dt_raw ~ N(0,1), all bf16."""
    x = torch.randn(b, H, P, generator=gen).to(torch.bfloat16)
    B = (torch.randn(b, G, N, generator=gen) / math.sqrt(N)).to(torch.bfloat16)
    C = (torch.randn(b, G, N, generator=gen) / math.sqrt(N)).to(torch.bfloat16)
    dt = torch.randn(b, H, generator=gen).to(torch.bfloat16)
    return x, B, C, dt


# ---------------------------------------------------------------------------
# building blocks
def rotate(X: torch.Tensor, R: Optional[torch.Tensor]) -> torch.Tensor:
    """B' = R_g B per group: einsum('bgn,gmn->bgm') — scale/v4_fused_decode.py:47-48,
    scale/nemotron_retrofit.py:24-27, scale/vllm_v4_patch.py:41-45."""
    if R is None:
        return X
    return torch.einsum("bgn,gmn->bgm", X, R.to(X.dtype))


def softplus_dt(dt_raw: torch.Tensor, dt_bias: torch.Tensor, dt_min: float = 0.0) -> torch.Tensor:
    """dt = softplus(dt_raw + dt_bias) [b,H], optional clamp(dt, dt_min) —
    scale/v4_native_decode.py:54-55 (clamp only on that path)."""
    dt = F.softplus(dt_raw + dt_bias[None, :])
    if dt_min > 0:
        dt = torch.clamp(dt, min=dt_min)
    return dt


def _heads(v: torch.Tensor, H: int) -> torch.Tensor:
    """Group -> head broadcast: head h reads group h // (H/G) — scale/v4_native_decode.py:59-61."""
    G = v.shape[1]
    return v.repeat_interleave(H // G, dim=1)


def mask_width(X: torch.Tensor, width: Optional[int]) -> torch.Tensor:
    """ActRotMask._mask with a scalar width (set_width): the rotated coordinates at and
    above `width` zeroed, the others kept (scale/nemotron_retrofit.py:29-37, :114-116)."""
    if width is None or width >= X.shape[-1]:
        return X
    return torch.cat([X[..., :width], torch.zeros_like(X[..., width:])], -1)


def _prep(x, B, C, dt_raw, prm: LayerParams, dtype, width: Optional[int] = None):
    xf = x.to(dtype)
    Bp = _heads(mask_width(rotate(B.to(dtype), prm.R), width), prm.H)
    Cp = _heads(mask_width(rotate(C.to(dtype), prm.R), width), prm.H)
    dt = softplus_dt(dt_raw.to(dtype), prm.dt_bias, prm.dt_min)
    a = dt * prm.A[None, :]
    return xf, Bp, Cp, dt, a


def quant_fp8(s: torch.Tensor):
    """Per-row e4m3fn quantization, scale = amax_over_last_dim / 448 + 1e-12 —
    scale/vllm_v4_patch.py:106-111 (_quant_store). Returns (codes, scale[...,1])."""
    sc = s.abs().amax(dim=-1, keepdim=True) / E4M3_MAX + 1e-12
    return (s / sc).to(torch.float8_e4m3fn), sc


def read_fp8(q: torch.Tensor, sc: torch.Tensor) -> torch.Tensor:
    """Dequantized snapshot q.float() * scale — scale/vllm_v4_patch.py:116-120 (_read_snap)."""
    return q.float() * sc


def fp8_readout(q: torch.Tensor, S8: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """y[r,p] = sum_n q[r,n] scale[r,n] fp8(S8[r,n,p]) — the _fp8_matvec docstring,
    scale/bench_v4_decode.py:33-52."""
    return torch.einsum("rn,rnp->rp", q.float() * scale.float(), S8.float())


# ---------------------------------------------------------------------------
# conv prologue
def conv_update(hbc: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor, bias, intermediate: int,
                gn: int, mask=None):
    """One decode token's causal depthwise conv1d update + SiLU and the x / B / C
    split (scale/v4_fused_decode.py:42-44 via causal-conv1d 1.6.2.post1
    causal_conv1d_update, restated by transformers' modeling_nemotron_h):
      state <- [state[..., 1:], hbc];  u = silu(bias + sum_w state[..., w] weight[:, w])
    computed in the model dtype (bf16: the conv and the SiLU outputs rounded to bf16),
    times mask[b] if given; returns bf16 x [b, I], B [b, gn], C [b, gn]; conv_state is
    updated in place."""
    dt = hbc.dtype
    new = torch.cat([conv_state[..., 1:], hbc[..., None]], dim=-1)
    conv_state.copy_(new)
    acc = (new.float() * weight.float()[None]).sum(-1)
    if bias is not None:
        acc = acc + bias.float()[None]
    u = acc.to(dt).float()
    u = (u / (1.0 + torch.exp(-u))).to(dt).float()
    if mask is not None:
        u = (u * mask.float()[:, None]).to(dt).float()
    u = u.to(torch.bfloat16)
    return u[:, :intermediate], u[:, intermediate:intermediate + gn], u[:, intermediate + gn:]


def gated_rmsnorm(y: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, group_size: int, eps: float):
    """The mixer's epilogue norm (transformers' Zamba2RMSNormGated, applied as
    self.norm(y.to(dtype), gate) at scale/v4_native_decode.py:170-171): y cast to the
    model dtype, times silu(gate) in fp32, RMS-normalised per group, cast back, times weight."""
    dt = gate.dtype
    v = y.to(dt).float() * torch.nn.functional.silu(gate.float())
    b, I = v.shape
    vg = v.view(b, I // group_size, group_size)
    vg = vg * torch.rsqrt(vg.pow(2).mean(-1, keepdim=True) + eps)
    return weight * vg.view(b, I).to(dt)


# ---------------------------------------------------------------------------
# fresh (untiered) step
def fresh_step(S: torch.Tensor, x, B, C, dt_raw, prm: LayerParams, dtype=torch.float32,
               width: Optional[int] = None) -> torch.Tensor:
    """S <- exp(dt A) S + (dt B') x;  y = S C' + D x  (S updated in place, y returned).
    scale/v4_native_decode.py:49-78 with pb >= N (the R applied by ActRotMask),
    the same recurrence as transformers' mamba2_selective_state_update. width: B' and C'
    masked to their first `width` coordinates (mask_width)."""
    xf, Bp, Cp, dt, a = _prep(x, B, C, dt_raw, prm, dtype, width)
    dA = torch.exp(a)[..., None, None]
    dB = dt[..., None, None] * Bp[:, :, None, :]
    S.copy_(S * dA + dB * xf[..., None])
    y = torch.einsum("bhpn,bhn->bhp", S, Cp)
    return y + xf * prm.D[None, :, None]


def hot_only_step(S_hot: torch.Tensor, x, B, C, dt_raw, prm: LayerParams, dtype=torch.float32) -> torch.Tensor:
    """Hot tier only, cold columns dropped (cold == "off"): the update and readout
    of the first k = S_hot.shape[-1] rotated columns, scale/v4_fused_decode.py:52-56
    and :140-142. S_hot updated in place; y = S_hot C'[:k] + D x."""
    k = S_hot.shape[-1]
    xf, Bp, Cp, dt, a = _prep(x, B, C, dt_raw, prm, dtype)
    S_hot.copy_(S_hot * torch.exp(a)[..., None, None] + (dt[..., None, None] * Bp[:, :, None, :k]) * xf[..., None])
    return torch.einsum("bhpn,bhn->bhp", S_hot, Cp[..., :k]) + xf * prm.D[None, :, None]


# ---------------------------------------------------------------------------
class NativeV4:
    """v4 with the full state kept fresh and a stale cold snapshot — the
    reference semantics: scale/v4_native_decode.py:58-167 (decode) and
    :234-243 (snapshot at prefill end), with the per-slot phase of
    scale/vllm_v4_patch.py:123-179 so requests may join and leave.

    cold: "fp32" (snapshot clone), "bf16" (snap.to(bf16).float(),
    v4_native_decode.py:162-163), "fp8" (per-row scale, vllm_v4_patch.py:106-120).
    fp8_restore_each_step re-stores the dequantized old snapshot for slots that
    do not flush, as scale/vllm_v4_patch.py:173-175 does.

    master: the precision the cold state is kept in between flushes. "fp32": the
    exact state (the native and vLLM paths keep the full fp32 state). "bf16": the
    fused path's bf16 master, scale/v4_fused_decode.py:149,156-158 (bf16 cold: the
    snapshot is the master; fp8 cold: a bf16 shadow master beside the e4m3 copy)
    and the bf16 arm of scale/bench_v4_decode.py:160-175: the cold columns are
    rounded to bf16 (RNE) at the join and at every flush and evolve in fp32 in
    between; the read copy is taken from the rounded values. (The reference rounds
    the decay product and the window update separately, :79-84; one rounding of the
    fp32 result is this convention.)

    step(..., hot_only=True) is the draft readout of coldoff=1
    (scale/v4_native_decode.py:118-127): y from the hot columns only. step(..., qgate=tau)
    is the query-gated cold skip (scale/v4_native_decode.py:147-156): a head's cold term is
    dropped when sum_{n>=k} C'_n^2 / max(sum_n C'_n^2, 1e-9) < tau; qgate_n / qgate_kept
    count heads and kept heads. In both the tier's bookkeeping (t, glog, snapshot) runs as
    in the stale readout (the reference's coldoff branch skips it, :118-127).

    exact=True is the rank-c exact correction readout (corr=1,
    scale/v4_native_decode.py:81-117): the log-decay G_t includes this token, this
    token's (B'_cold, dt x, G_t) is buffered before the readout, and
      y_cold = exp(G_t) (snap . C'_cold) + sum_j exp(G_t - G_j) (C'_cold . B'_j) (dt_j x_j)
    over the buffer since the snapshot; the bookkeeping (t, glog, snapshot) is the
    stale path's.
    """

    def __init__(self, slots: int, H: int, P: int, N: int, k: int, c: int, cold: str = "fp32",
                 dtype=torch.float32, fp8_restore_each_step: bool = True, exact: bool = False,
                 master: str = "fp32"):
        assert 0 < k <= N and c >= 1 and cold in ("fp32", "bf16", "fp8")
        assert master in ("fp32", "bf16") and not (cold == "fp32" and master == "bf16")
        self.k, self.c, self.cold, self.dtype, self.master = k, c, cold, dtype, master
        self.fp8_restore = fp8_restore_each_step
        self.exact = exact
        self.buf = [[] for _ in range(slots)]  # exact readout: per slot (B'_cold [H,Nc], dt x [H,P], G [H])
        self.S = torch.zeros(slots, H, P, N, dtype=dtype)
        Nc = N - k
        self.snap = torch.zeros(slots, H, P, Nc, dtype=dtype)          # fp32 / bf16-rounded values
        self.q8 = torch.zeros(slots, H, P, Nc, dtype=torch.float8_e4m3fn)
        self.sc8 = torch.ones(slots, H, P, 1, dtype=torch.float32)
        self.glog = torch.zeros(slots, H, dtype=dtype)
        self.t = torch.zeros(slots, dtype=torch.int64)
        self.qgate_n = 0
        self.qgate_kept = 0

    def _store(self, slots, s_cold):
        if self.cold == "fp8":
            q, sc = quant_fp8(s_cold.float())
            self.q8[slots] = q
            self.sc8[slots] = sc
        elif self.cold == "bf16":
            self.snap[slots] = s_cold.to(torch.bfloat16).to(self.dtype)
        else:
            self.snap[slots] = s_cold.clone()

    def _read(self, slots):
        if self.cold == "fp8":
            return read_fp8(self.q8[slots], self.sc8[slots]).to(self.dtype)
        return self.snap[slots]

    def _round_master(self, S: torch.Tensor) -> torch.Tensor:
        """S with its cold columns rounded to the master precision."""
        if self.master == "fp32":
            return S
        k = self.k
        return torch.cat([S[..., :k], S[..., k:].to(torch.bfloat16).to(S.dtype)], dim=-1)

    def join(self, slots: torch.Tensor, S_new: torch.Tensor, phase: Optional[torch.Tensor] = None):
        """End of prefill for `slots`: S = S_new, snapshot of its cold columns, glog = 0,
        t = phase (0 by default) — scale/vllm_v4_patch.py:123-137."""
        slots = torch.as_tensor(slots, dtype=torch.long)
        self.S[slots] = self._round_master(S_new.to(self.dtype))
        self._store(slots, self.S[slots][..., self.k:])
        self.glog[slots] = 0
        self.t[slots] = 0 if phase is None else torch.as_tensor(phase, dtype=torch.int64)
        for s in slots.tolist():
            self.buf[s] = []

    def step(self, x, B, C, dt_raw, prm: LayerParams, slots: Optional[torch.Tensor] = None,
             hot_only: bool = False, qgate: float = 0.0) -> torch.Tensor:
        assert not (self.exact and (hot_only or qgate > 0)), "the exact readout takes precedence"
        b = x.shape[0]
        slots = torch.arange(b) if slots is None else torch.as_tensor(slots, dtype=torch.long)
        k, c = self.k, self.c
        prm = prm.to(self.dtype)
        xf, Bp, Cp, dt, a = _prep(x, B, C, dt_raw, prm, self.dtype)
        S = self.S[slots]
        S = S * torch.exp(a)[..., None, None] + (dt[..., None, None] * Bp[:, :, None, :]) * xf[..., None]
        self.S[slots] = S
        glog = self.glog[slots]
        if self.exact:
            g1 = glog + a  # G_t, inclusive of this token
            y_cold = torch.einsum("bhpn,bhn->bhp", self._read(slots), Cp[..., k:]) * torch.exp(g1)[..., None]
            for i, s in enumerate(slots.tolist()):
                self.buf[s].append((Bp[i, :, k:].clone(), dt[i][:, None] * xf[i], g1[i].clone()))
                Bs = torch.stack([e[0] for e in self.buf[s]])   # [j,H,Nc]
                Xs = torch.stack([e[1] for e in self.buf[s]])   # [j,H,P]
                Gs = torch.stack([e[2] for e in self.buf[s]])   # [j,H]
                sj = torch.einsum("jhn,hn->jh", Bs, Cp[i, :, k:])
                w = torch.exp(g1[i][None] - Gs) * sj
                y_cold[i] = y_cold[i] + torch.einsum("jh,jhp->hp", w, Xs)
        else:
            y_cold = torch.einsum("bhpn,bhn->bhp", self._read(slots), Cp[..., k:]) * torch.exp(glog)[..., None]
            if hot_only:
                y_cold = torch.zeros_like(y_cold)
            elif qgate > 0:
                e = Cp * Cp
                rho = e[..., k:].sum(-1) / e.sum(-1).clamp(min=1e-9)  # [b,H]
                keep = rho >= qgate
                self.qgate_n += keep.numel()
                self.qgate_kept += int(keep.sum())
                y_cold = y_cold * keep[..., None].to(y_cold.dtype)
        y = torch.einsum("bhpn,bhn->bhp", S[..., :k], Cp[..., :k]) + y_cold
        t = self.t[slots] + 1
        self.t[slots] = t
        flush = (t % c == 0)
        if self.master != "fp32" and bool(flush.any()):
            S = torch.where(flush[:, None, None, None], self._round_master(S), S)
            self.S[slots] = S
        if self.cold == "fp8" and self.fp8_restore:
            old = self._read(slots)
            self._store(slots, torch.where(flush[:, None, None, None], S[..., k:], old))
        elif bool(flush.any()):
            fs = slots[flush]
            self._store(fs, S[flush][..., k:])
        if self.exact:
            for i, s in enumerate(slots.tolist()):
                if bool(flush[i]):
                    self.buf[s] = []
        self.glog[slots] = torch.where(flush[:, None], torch.zeros_like(glog), glog + a)
        return y + xf * prm.D[None, :, None]


# ---------------------------------------------------------------------------
class TieredV4:
    """v4 with tier-split storage and a chunked flush — scale/v4_fused_decode.py:28-95
    (hot slice updated every token, stale cold readout with exp(glog), ring of
    (dt x, B'_cold, dt A), flush = exp(sum a) snap + sum_j exp(sum_{i>j} a_i)
    (dt_j x_j) (x) B'_j, :76-85), generalised to per-slot phases. The hot/cold
    split does not hold the full state: the exact cold state exists only right
    after a flush. materialize() rebuilds it from the pending ring entries."""

    def __init__(self, slots: int, H: int, P: int, N: int, G: int, k: int, c: int, dtype=torch.float32,
                 master: str = "fp32"):
        assert 0 < k < N and c >= 1 and master in ("fp32", "bf16")
        self.H, self.P, self.N, self.G, self.k, self.c, self.dtype = H, P, N, G, k, c, dtype
        # "bf16": the cold tier is a bf16 master, rounded at join and at every flush
        self.master = master
        self.hot = torch.zeros(slots, H, P, k, dtype=dtype)
        self.cold = torch.zeros(slots, H, P, N - k, dtype=dtype)
        self.glog = torch.zeros(slots, H, dtype=dtype)
        self.t = torch.zeros(slots, dtype=torch.int64)
        self.ring = [[] for _ in range(slots)]  # per slot: list of (dt [H], x [H,P], B'cold [H,Nc])

    def join(self, slots, S_new, phase=None):
        slots = torch.as_tensor(slots, dtype=torch.long)
        S_new = S_new.to(self.dtype)
        self.hot[slots] = S_new[..., :self.k]
        self.cold[slots] = self._round(S_new[..., self.k:])
        self.glog[slots] = 0
        self.t[slots] = 0 if phase is None else torch.as_tensor(phase, dtype=torch.int64)
        for s in slots.tolist():
            self.ring[s] = []

    def _round(self, cold):
        return cold if self.master == "fp32" else cold.to(torch.bfloat16).to(self.dtype)

    def _replay(self, cold0, entries, A):
        """exp(sum a) cold0 + sum_j exp(sum_{i>j} a_i) dt_j x_j (x) B'_j."""
        if not entries:
            return cold0
        dts = torch.stack([e[0] for e in entries])           # [m,H]
        a = dts * A[None, :]
        suf = torch.flip(torch.cumsum(torch.flip(a, [0]), 0), [0]) - a
        w = torch.exp(suf) * dts                             # [m,H]
        X = torch.stack([e[1] for e in entries])              # [m,H,P]
        Bc = torch.stack([e[2] for e in entries])             # [m,H,Nc]
        upd = torch.einsum("mh,mhp,mhn->hpn", w, X, Bc)
        return cold0 * torch.exp(a.sum(0))[:, None, None] + upd

    def step(self, x, B, C, dt_raw, prm: LayerParams, slots=None):
        b = x.shape[0]
        slots = torch.arange(b) if slots is None else torch.as_tensor(slots, dtype=torch.long)
        k, c = self.k, self.c
        prm = prm.to(self.dtype)
        xf, Bp, Cp, dt, a = _prep(x, B, C, dt_raw, prm, self.dtype)
        hot = self.hot[slots] * torch.exp(a)[..., None, None] + \
            (dt[..., None, None] * Bp[:, :, None, :k]) * xf[..., None]
        self.hot[slots] = hot
        y = torch.einsum("bhpn,bhn->bhp", hot, Cp[..., :k]) + \
            torch.einsum("bhpn,bhn->bhp", self.cold[slots], Cp[..., k:]) * torch.exp(self.glog[slots])[..., None]
        t = self.t[slots] + 1
        self.t[slots] = t
        for i, s in enumerate(slots.tolist()):
            entry = (dt[i], xf[i], Bp[i, :, k:])
            if int(t[i]) % c == 0:
                self.cold[s] = self._round(self._replay(self.cold[s], self.ring[s] + [entry], prm.A))
                self.ring[s] = []
                self.glog[s] = 0
            else:
                self.ring[s].append(entry)
                self.glog[s] = self.glog[s] + a[i]
        return y + xf * prm.D[None, :, None]

    def materialize(self, slots, prm: LayerParams) -> torch.Tensor:
        slots = torch.as_tensor(slots, dtype=torch.long)
        prm = prm.to(self.dtype)
        out = []
        for s in slots.tolist():
            cold = self._replay(self.cold[s], self.ring[s], prm.A)
            out.append(torch.cat([self.hot[s], cold], dim=-1))
        return torch.stack(out)


# ---------------------------------------------------------------------------
class TeacherForcedV4:
    """The teacher-forced v4 readout of the reference's per-token evaluation forward,
    scale/nemo9b_eval.py:41-85 (naive_mixer_forward, mode "v4"), per slot:

      S_t = exp(a_t) S_{t-1} + (dt_t x_t) (x) B'_t                        (:53-54)
      Gtot_t = Gtot_{t-1} + a_t                                           (:60)
      if t % c == 0: SnapL, gSnapL = Snap, gSnap                          (:59)
                     Snap = q(S_t), gSnap = Gtot_t   (after the update)   (:61-71)
      (Rd, gRd) = (SnapL, gSnapL) if lag else (Snap, gSnap)               (:70)
      y_t = S_t[:k] C'_t[:k] + exp(Gtot_t - gRd) (Rd[k:] C'_t[k:]) + D x_t   (:72-84)
      (y_t = S_t C'_t + D x_t while t < warm, :75-78)

    lag = 1 is the loop's asynchronous-flush model: readers see the snapshot one flush
    behind (the one before the last).

    t counts the sequence's tokens from 0 (join sets it, with the state and its snapshot).
    q: "fp32" the clone, "bf16" S.to(bf16).float() (:66-67), "fp8" e4m3 with either the
    reference's per-column scale (fp8_scale="column": amax over P, clamp(1e-6) / 448,
    :62-64) or the tier's per-row one (fp8_scale="row": amax over the cold columns / 448 +
    1e-12, scale/vllm_v4_patch.py:106-111).

    k = 0 is the loop's mode "c1" (:79-80): every column read from the snapshot,
    y_t = exp(Gtot_t - gSnap) (Snap C'_t) + D x_t. master="bf16" keeps the cold columns as
    a bf16 master (the fused path's, scale/v4_fused_decode.py:149,156-158), as NativeV4
    does: they are rounded to bf16 (RNE) at the join and at every snapshot, evolve in fp32
    in between, and the snapshot is taken from the rounded values."""

    def __init__(self, slots: int, H: int, P: int, N: int, k: int, c: int, cold: str = "fp32",
                 fp8_scale: str = "row", warm: int = 0, dtype=torch.float32, master: str = "fp32", lag: int = 0):
        assert 0 <= k <= N and c >= 1 and cold in ("fp32", "bf16", "fp8") and fp8_scale in ("row", "column")
        assert master in ("fp32", "bf16") and not (cold == "fp32" and master == "bf16") and lag in (0, 1)
        self.k, self.c, self.cold, self.fp8_scale, self.warm, self.dtype = k, c, cold, fp8_scale, warm, dtype
        self.master, self.lag = master, lag
        self.S = torch.zeros(slots, H, P, N, dtype=dtype)
        self.snap = torch.zeros(slots, H, P, N - k, dtype=dtype)
        self.snapl = torch.zeros(slots, H, P, N - k, dtype=dtype)
        self.gtot = torch.zeros(slots, H, dtype=dtype)
        self.gsnap = torch.zeros(slots, H, dtype=dtype)
        self.gsnapl = torch.zeros(slots, H, dtype=dtype)
        self.t = torch.zeros(slots, dtype=torch.int64)

    def _q(self, S: torch.Tensor) -> torch.Tensor:
        """The snapshot of full states S: its cold columns in the snapshot precision."""
        k = self.k
        if self.cold == "bf16":
            return S[..., k:].to(torch.bfloat16).to(self.dtype)
        if self.cold == "fp8":
            if self.fp8_scale == "column":
                sc = S.abs().amax(-2, keepdim=True).clamp(min=1e-6) / E4M3_MAX
                return ((S / sc).to(torch.float8_e4m3fn).to(self.dtype) * sc)[..., k:]
            q, sc = quant_fp8(S[..., k:].float())
            return read_fp8(q, sc).to(self.dtype)
        return S[..., k:].clone()

    def _round_master(self, S: torch.Tensor) -> torch.Tensor:
        """S with its cold columns rounded to the master precision."""
        if self.master == "fp32":
            return S
        k = self.k
        return torch.cat([S[..., :k], S[..., k:].to(torch.bfloat16).to(S.dtype)], dim=-1)

    def join(self, slots, S_new: torch.Tensor, t0: Optional[torch.Tensor] = None):
        """A sequence at position t0 (default 0) with state S_new: the snapshot, and the lagged
        one, is S_new."""
        slots = torch.as_tensor(slots, dtype=torch.long)
        self.S[slots] = self._round_master(S_new.to(self.dtype))
        self.snap[slots] = self._q(self.S[slots])
        self.snapl[slots] = self.snap[slots]
        self.gtot[slots] = 0
        self.gsnap[slots] = 0
        self.gsnapl[slots] = 0
        self.t[slots] = 0 if t0 is None else torch.as_tensor(t0, dtype=torch.int64)

    def step(self, x, B, C, dt_raw, prm: LayerParams, slots: Optional[torch.Tensor] = None,
             width: Optional[int] = None) -> torch.Tensor:
        """One token; width: B' and C' masked to their first `width` coordinates (the
        rotation wrapper's set_width, mask_width)."""
        b = x.shape[0]
        slots = torch.arange(b) if slots is None else torch.as_tensor(slots, dtype=torch.long)
        k, c = self.k, self.c
        prm = prm.to(self.dtype)
        xf, Bp, Cp, dt, a = _prep(x, B, C, dt_raw, prm, self.dtype, width)
        S = self.S[slots] * torch.exp(a)[..., None, None] + (dt[..., None, None] * Bp[:, :, None, :]) * xf[..., None]
        self.S[slots] = S
        gtot = self.gtot[slots] + a
        self.gtot[slots] = gtot
        t = self.t[slots]
        snapt = t % c == 0
        if bool(snapt.any()):
            ss = slots[snapt]
            if self.master != "fp32":
                S = torch.where(snapt[:, None, None, None], self._round_master(S), S)
                self.S[slots] = S
            self.snapl[ss] = self.snap[ss]
            self.gsnapl[ss] = self.gsnap[ss]
            self.snap[ss] = self._q(S[snapt])
            self.gsnap[ss] = gtot[snapt]
        rd, grd = (self.snapl, self.gsnapl) if self.lag else (self.snap, self.gsnap)
        glog = gtot - grd[slots]
        y_v4 = torch.einsum("bhpn,bhn->bhp", S[..., :k], Cp[..., :k]) + \
            torch.einsum("bhpn,bhn->bhp", rd[slots], Cp[..., k:]) * torch.exp(glog)[..., None]
        y_fresh = torch.einsum("bhpn,bhn->bhp", S, Cp)
        y = torch.where((t < self.warm)[:, None, None], y_fresh, y_v4)
        self.t[slots] = t + 1
        return y + xf * prm.D[None, :, None]
