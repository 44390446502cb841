"""Host-side API over the C ABI: torch tensors in, HIP kernels on the current stream.

PyTorch is only the allocator and stream provider here; every state update
runs in libnssm_hip.so. Nothing in this module has a CPU path: inputs must be
CUDA (HIP) tensors and the library must be built.
"""
import ctypes
import os
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import COLD_KINDS, NssmError, TIER_FIELDS, check, lib

N_STATE = 128
MAX_WINDOW = 64  # largest flush window c the kernels take


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


_WORKSPACES = {}


def step_workspace(b: int, H: int, G: int, c: int, device=None) -> torch.Tensor:
    """Workspace for one step call on the current stream of `device` (cached per
    device and stream, grown on demand; calls on one stream run in order)."""
    need = lib().nssm_step_workspace_bytes(b, H, G, N_STATE, c)
    if need < 0:
        check(int(need), "nssm_step_workspace_bytes")
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(max(int(need), 256), device=dev, dtype=torch.uint8)
        _WORKSPACES[key] = ws
    return ws


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# Duplicate slot ids in one call make the kernels' per-slot read-modify-writes race (the
# tier rows, t / nv / glog and the ring of that slot), silently corrupting its state.
# Two checks: on the device (nssm_check_slots, one small launch before each call with
# slot_ids; no sync, graph-safe; V4Tier.slot_errors() reads what it found), on unless
# set_checks(device_slots=False) or NSSM_DEVICE_SLOT_CHECK=0; and on the host (raises at
# once, but needs a host sync and so skips graph capture), off unless
# set_checks(slot_ids=True) or NSSM_CHECK_SLOTS=1.
_CHECK_SLOTS = os.environ.get("NSSM_CHECK_SLOTS", "0") not in ("", "0")
_DEVICE_SLOT_CHECK = os.environ.get("NSSM_DEVICE_SLOT_CHECK", "1") not in ("", "0")


def set_checks(slot_ids: bool = False, device_slots: bool = True) -> None:
    """Turn the host-side check that a call's slot_ids are unique on or off (it
    synchronises the host with the device on every step, join and materialize), and the
    device-side one (nssm_check_slots before each call with slot_ids)."""
    global _CHECK_SLOTS, _DEVICE_SLOT_CHECK
    _CHECK_SLOTS = bool(slot_ids)
    _DEVICE_SLOT_CHECK = bool(device_slots)


def _check_unique(slot_ids: Optional[torch.Tensor], what: str) -> None:
    if not _CHECK_SLOTS or slot_ids is None:
        return
    if slot_ids.is_cuda and torch.cuda.is_current_stream_capturing():
        return
    if torch.unique(slot_ids).numel() != slot_ids.numel():
        raise ValueError(f"{what}: slot_ids must be unique (duplicates race on the same tier rows)")


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, shape: tuple):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU (got {t.device}); there is no CPU path")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype} (got {t.dtype})")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)} (got {tuple(t.shape)})")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


@dataclass
class LayerParams:
    """Per-layer constants on the GPU: dt_bias, A = -exp(A_log), D [H] fp32, R [G,N,N] fp32."""
    H: int
    P: int
    N: int
    G: int
    dt_bias: torch.Tensor
    A: torch.Tensor
    D: torch.Tensor
    R: Optional[torch.Tensor] = None
    dt_min: float = 0.0

    @classmethod
    def from_mixer_values(cls, dt_bias, A_log, D, R=None, P=80, G=8, dt_min=0.0, device="cuda"):
        """Build from the mixer's parameters (A_log as stored by NemotronH)."""
        f = dict(device=device, dtype=torch.float32)
        H = dt_bias.numel()
        A = -torch.exp(A_log.detach().float()).to(**f)
        Rt = None if R is None else R.detach().to(**f).contiguous()
        N = N_STATE if Rt is None else Rt.shape[-1]
        return cls(H, P, N, G, dt_bias.detach().to(**f).contiguous(), A.contiguous(),
                   D.detach().to(**f).contiguous(), Rt, dt_min)

    def validate(self):
        if self.N != N_STATE:
            raise ValueError(f"d_state must be {N_STATE} (got {self.N})")
        for nm in ("dt_bias", "A", "D"):
            _need(getattr(self, nm), nm, torch.float32, (self.H,))
        if self.R is not None:
            _need(self.R, "R", torch.float32, (self.G, self.N, self.N))

    def c_struct(self) -> _lib.LayerParams:
        self.validate()
        return _lib.LayerParams(self.H, self.P, self.N, self.G, _ptr(self.dt_bias), _ptr(self.A),
                                _ptr(self.D), _ptr(self.R), float(self.dt_min))


def _inputs(prm: LayerParams, x, B, C, dt, slot_ids) -> _lib.StepInputs:
    b = x.shape[0]
    _need(x, "x", torch.bfloat16, (b, prm.H, prm.P))
    _need(B, "B", torch.bfloat16, (b, prm.G, prm.N))
    _need(C, "C", torch.bfloat16, (b, prm.G, prm.N))
    _need(dt, "dt", torch.bfloat16, (b, prm.H))
    if slot_ids is not None:
        _need(slot_ids, "slot_ids", torch.int32, (b,))
    return _lib.StepInputs(b, _ptr(x), _ptr(B), _ptr(C), _ptr(dt), _ptr(slot_ids))


def fresh_step(prm: LayerParams, state: torch.Tensor, x, B, C, dt, y: Optional[torch.Tensor] = None,
               slot_ids: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Untiered step over state [slots,H,P,N] fp32 (in place); returns y [b,H,P] fp32."""
    slots = state.shape[0]
    _need(state, "state", torch.float32, (slots, prm.H, prm.P, prm.N))
    b = x.shape[0]
    if y is None:
        y = torch.empty(b, prm.H, prm.P, device=x.device, dtype=torch.float32)
    _need(y, "y", torch.float32, (b, prm.H, prm.P))
    pc, ic = prm.c_struct(), _inputs(prm, x, B, C, dt, slot_ids)
    _check_unique(slot_ids, "fresh_step")
    ws = step_workspace(b, prm.H, prm.G, 0, x.device)
    check(lib().nssm_fresh_step(ctypes.byref(pc), state.data_ptr(), slots, ctypes.byref(ic), y.data_ptr(),
                                ws.data_ptr(), ws.numel(), _stream()), "nssm_fresh_step")
    return y


def x_ring_for(c: int, exact: bool) -> str:
    """The x ring layout for a tier read mostly with the given readout: "unit" for the exact
    readout over windows longer than 16 tokens (its per-token window reads, c - 1 tokens per
    head, then outweigh the appends: 9B shape, c = 64, 9.02 -> 8.84 ms per step), "row"
    otherwise (exact c = 16: 8.03-8.07 -> 8.14-8.16 ms with "unit"; the stale readouts read the
    ring only at a flush)."""
    return "unit" if exact and c > 16 else "row"


class V4Tier:
    """Tiered state of one layer for `slots` sequence slots (hot fp32 [slots,H,P,K],
    cold fp32/bf16/fp8 [slots,H,P,NC] (+ master and per-row scale), ring of the last
    c tokens, per-(slot, head) t / nv / glog). Layout as in include/nssm.h.

    master: the precision the cold state is kept in between flushes. "fp32" (the
    default): an exact fp32 master beside a bf16 / e4m3 read copy (the native and
    vLLM paths keep the full fp32 state, scale/v4_native_decode.py:65-67). "bf16":
    the fused path's bf16 master (scale/v4_fused_decode.py:149,156-158): bf16 cold
    is then one bf16 copy, rewritten with the RNE of each flush; fp8 cold keeps a
    bf16 master beside the e4m3 copy. fp32 cold is its own fp32 master.

    k_hot = 0 (every column cold, the evaluation forward's mode "c1") serves the
    teacher-forced readout only (step(..., teacher=True)).

    lag=True keeps the lagged snapshot of the evaluation forward's lag = 1
    (scale/nemo9b_eval.py:44,59,70): a second read copy (cold2, scale2) and the log-decay
    between the two snapshots per (slot, head) (wlag); such a tier is read with the lagged
    teacher-forced readout (step(..., teacher=True)) only.

    x_ring: the layout of the ring's x (NSSM_XRING_*): "row" ([slots, H, c, P], the default:
    the cheapest per-token append) or "unit" ([slots, H, P / 8, c, 8]: the exact readout's
    window reads are one run per unit). Both serve every readout; only their speed differs."""

    def __init__(self, slots: int, H: int, P: int, G: int, k_hot: int = 32, c: int = 4, cold: str = "fp32",
                 device="cuda", N: int = N_STATE, master: str = "fp32", lag: bool = False, x_ring: str = "row"):
        if x_ring not in _lib.XRING_LAYOUTS:
            raise ValueError(f"x_ring must be one of {sorted(_lib.XRING_LAYOUTS)} (got {x_ring!r})")
        if x_ring == "unit" and P % 8:
            raise ValueError(f"x_ring='unit' needs P a multiple of 8 (got {P})")
        self.x_layout = _lib.XRING_LAYOUTS[x_ring]
        if cold not in COLD_KINDS:
            raise ValueError(f"cold must be one of {sorted(COLD_KINDS)} (got {cold!r})")
        if cold != "off" and (cold, master) not in _lib.STORAGE_KINDS:
            raise ValueError(f"cold={cold!r} cannot be kept with master={master!r} "
                             f"(supported: {sorted(_lib.STORAGE_KINDS)})")
        self.slots, self.H, self.P, self.G, self.N, self.k, self.c, self.cold = slots, H, P, G, N, k_hot, c, cold
        self.master_dtype = master if cold != "off" else None
        self.kind = COLD_KINDS["off"] if cold == "off" else _lib.STORAGE_KINDS[(cold, master)]
        sizes = (ctypes.c_int64 * 10)()
        check(lib().nssm_tier_sizes(slots, H, P, N, G, k_hot, c, self.kind, sizes), "nssm_tier_sizes")
        NC = N - k_hot
        dev = torch.device(device)
        e = lambda shape, dt: torch.empty(shape, device=dev, dtype=dt)  # noqa: E731
        self.hot = e((slots, H, P, k_hot), torch.float32)
        tiered = cold != "off"  # "off": hot tier only, the cold columns are dropped
        cold_dt = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp8": torch.uint8, "off": None}[cold]
        self.cold_t = e((slots, H, P, NC), cold_dt) if tiered else None
        self.scale = e((slots, H, P), torch.float32) if cold == "fp8" else None
        master_dt = {_lib.COLD_BF16: torch.float32, _lib.COLD_FP8: torch.float32,
                     _lib.COLD_FP8_BF16M: torch.bfloat16}.get(self.kind)
        self.master = e((slots, H, P, NC), master_dt) if master_dt is not None else None
        xshape = (slots, H, c, P) if self.x_layout == _lib.XRING_ROW else (slots, H, P // 8, c, 8)
        self.ring_x = e(xshape, torch.bfloat16) if tiered else None
        self.ring_dt = e((slots, H, c), torch.float32) if tiered else None
        self.ring_b = e((slots, G, c, NC), torch.float32) if tiered else None
        self.t = torch.zeros((slots, H), device=dev, dtype=torch.int32)
        self.nv = torch.zeros((slots, H), device=dev, dtype=torch.int32)
        self.glog = torch.zeros((slots, H), device=dev, dtype=torch.float32)
        if lag and not tiered:
            raise ValueError("the lagged readout needs a cold tier")
        self.lag = lag
        self.cold2 = torch.empty_like(self.cold_t) if lag else None
        self.scale2 = torch.empty_like(self.scale) if lag and self.scale is not None else None
        self.wlag = torch.zeros((slots, H), device=dev, dtype=torch.float32) if lag else None
        # the device-side slot id check's owner words and (call counter, error bits)
        self.slot_owner = torch.zeros(slots, device=dev, dtype=torch.int64)
        self.slot_state = torch.zeros(2, device=dev, dtype=torch.int32)
        got = [self._field(f) for f in TIER_FIELDS]
        for f, tns, want in zip(TIER_FIELDS, got, sizes):
            have = 0 if tns is None else tns.numel() * tns.element_size()
            if have != want:
                raise NssmError(f"tier buffer {f}: {have} bytes allocated, library expects {want}")

    def _field(self, f):
        return self.cold_t if f == "cold" else getattr(self, f)

    def _rows(self, t: Optional[torch.Tensor], blocked: bool) -> Optional[torch.Tensor]:
        """[slots, H, P, NC] in row order. The bf16 read copies and the bf16 master are
        stored unit-blocked (8 rows of a unit segment-major: [NC // 32][8][32] per unit, then
        [8][16] for a trailing 16-column segment when NC % 32 == 16), which this unpacks (a
        copy); other arrays are returned as they are."""
        if t is None or not blocked:
            return t
        S, H, P, NC = t.shape
        n32 = NC // 32 * 32
        blocks = t.reshape(S * H * P // 8, 8 * NC)
        rows = blocks[:, :8 * n32].reshape(-1, NC // 32, 8, 32).transpose(1, 2).reshape(-1, 8, n32)
        if n32 < NC:
            rows = torch.cat([rows, blocks[:, 8 * n32:].reshape(-1, 8, NC - n32)], dim=-1)
        return rows.reshape(S, H, P, NC)

    def cold_rows(self) -> Optional[torch.Tensor]:
        """The cold copy [slots, H, P, NC] in row order."""
        return self._rows(self.cold_t, self.kind in (_lib.COLD_BF16_SINGLE, _lib.COLD_BF16))

    def master_rows(self) -> Optional[torch.Tensor]:
        """The cold master [slots, H, P, NC] in row order (None without a separate master)."""
        return self._rows(self.master, self.kind == _lib.COLD_FP8_BF16M)

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self._field(f) for f in TIER_FIELDS) if t is not None)

    def c_struct(self) -> _lib.Tier:
        return _lib.Tier(self.slots, self.k, self.c, self.kind, *[_ptr(self._field(f)) for f in TIER_FIELDS],
                         self.x_layout)

    def lag_struct(self) -> _lib.Lag:
        return _lib.Lag(_ptr(self.cold2), _ptr(self.scale2), _ptr(self.wlag))

    def check_slots(self, slot_ids: torch.Tensor) -> None:
        """Enqueue nssm_check_slots for one call's slot_ids (int32 [b] on the GPU): no sync;
        what it finds accumulates until slot_errors()."""
        _need(slot_ids, "slot_ids", torch.int32, (slot_ids.shape[0],))
        check(lib().nssm_check_slots(slot_ids.data_ptr(), slot_ids.shape[0], self.slots, self.slot_owner.data_ptr(),
                                     self.slot_state.data_ptr(), _stream()), "nssm_check_slots")

    def _device_check(self, slot_ids: Optional[torch.Tensor]) -> None:
        if _DEVICE_SLOT_CHECK and slot_ids is not None:
            self.check_slots(slot_ids)

    def slot_errors(self) -> int:
        """The device-side slot check's findings since the last call (synchronises): bit 0,
        two requests of one call named the same slot; bit 1, an id outside [0, slots). Clears them."""
        bits = int(self.slot_state[1].item())
        self.slot_state[1:].zero_()
        return bits

    def join(self, prm: LayerParams, state: torch.Tensor, slot_ids: Optional[torch.Tensor] = None,
             phase: Optional[torch.Tensor] = None):
        """Capture full states [b,H,P,N] fp32 into slots (end of prefill)."""
        b = state.shape[0]
        _need(state, "state", torch.float32, (b, self.H, self.P, self.N))
        if slot_ids is not None:
            _need(slot_ids, "slot_ids", torch.int32, (b,))
        if phase is not None:
            _need(phase, "phase", torch.int32, (b,))
        _check_unique(slot_ids, "V4Tier.join")
        self._device_check(slot_ids)
        pc, tc = prm.c_struct(), self.c_struct()
        check(lib().nssm_v4_join(ctypes.byref(pc), ctypes.byref(tc), state.data_ptr(), b, _ptr(slot_ids),
                                 _ptr(phase), _stream()), "nssm_v4_join")
        if self.lag:  # both snapshots are the joined state (a slot's rows are contiguous in every layout)
            sl = (torch.arange(b, device=state.device) if slot_ids is None else slot_ids).long()
            self.cold2.index_copy_(0, sl, self.cold_t.index_select(0, sl))
            if self.scale2 is not None:
                self.scale2.index_copy_(0, sl, self.scale.index_select(0, sl))
            self.wlag.index_fill_(0, sl, 0.0)

    def step(self, prm: LayerParams, x, B, C, dt, y: Optional[torch.Tensor] = None,
             slot_ids: Optional[torch.Tensor] = None, exact: bool = False, hot_only: bool = False,
             qgate: float = 0.0, counts: Optional[torch.Tensor] = None, noalloc: bool = False,
             teacher: bool = False) -> torch.Tensor:
        """One decode token for b requests (slot_ids: their slots, default 0..b-1).
        exact=True reads the cold tier with the rank-c exact correction (corr=1,
        scale/v4_native_decode.py:81-117) instead of the stale readout. hot_only=True is
        the hot-only draft readout (coldoff=1, scale/v4_native_decode.py:118-127);
        qgate=tau > 0 drops the cold term of the heads whose query puts less than tau of
        its energy on the cold columns (scale/v4_native_decode.py:147-156), and adds the
        gated and kept head counts to counts (int64 [2] on the GPU) when given. The tier
        evolves the same way in every case. teacher=True is the teacher-forced readout of
        scale/nemo9b_eval.py:41-85 (nssm_v4_step_teacher: a flush token reads the state it
        flushes to, the others the snapshot with the decay inclusive of this token; join a
        sequence's start at phase c - 1 to flush at positions t % c == 0 as that loop does);
        on a lagged tier its lag = 1 form (nssm_v4_step_teacher_lagged: the snapshot before
        the last).
        noalloc=True runs the stale readout through
        nssm_v4_step_noalloc, whose workspace is the library's fixed per-GPU scratch array
        (with y given, the call allocates nothing; calls overlapping on one GPU race)."""
        b = x.shape[0]
        gated = hot_only or qgate > 0
        if exact and gated:
            raise ValueError("exact readout cannot be combined with hot_only or qgate")
        if noalloc and (exact or gated or teacher):
            raise ValueError("noalloc serves the stale readout only")
        if teacher and (exact or gated):
            raise ValueError("the teacher-forced readout cannot be combined with exact, hot_only or qgate")
        if self.k == 0 and not teacher:
            raise ValueError("a tier with k_hot = 0 (every column cold) serves the teacher-forced readout only")
        if self.lag and not teacher:
            raise ValueError("a lagged tier serves the (lagged) teacher-forced readout only")
        if y is None:
            y = torch.empty(b, prm.H, prm.P, device=x.device, dtype=torch.float32)
        _need(y, "y", torch.float32, (b, prm.H, prm.P))
        if counts is not None:
            _need(counts, "counts", torch.int64, (2,))
        pc, ic, tc = prm.c_struct(), _inputs(prm, x, B, C, dt, slot_ids), self.c_struct()
        _check_unique(slot_ids, "V4Tier.step")
        self._device_check(slot_ids)
        if noalloc:
            check(lib().nssm_v4_step_noalloc(ctypes.byref(pc), ctypes.byref(tc), ctypes.byref(ic), y.data_ptr(),
                                             _stream()), "nssm_v4_step_noalloc")
            return y
        ws = step_workspace(b, prm.H, prm.G, self.c, x.device)
        args = (ctypes.byref(pc), ctypes.byref(tc), ctypes.byref(ic), y.data_ptr(), ws.data_ptr(), ws.numel())
        if gated:
            check(lib().nssm_v4_step_gated(*args, int(hot_only), float(qgate), _ptr(counts), _stream()),
                  "nssm_v4_step_gated")
        elif self.lag:
            lc = self.lag_struct()
            check(lib().nssm_v4_step_teacher_lagged(args[0], args[1], ctypes.byref(lc), *args[2:], _stream()),
                  "nssm_v4_step_teacher_lagged")
        else:
            fn, name = ((lib().nssm_v4_step_exact, "nssm_v4_step_exact") if exact else
                        (lib().nssm_v4_step_teacher, "nssm_v4_step_teacher") if teacher else
                        (lib().nssm_v4_step, "nssm_v4_step"))
            check(fn(*args, _stream()), name)
        return y

    def materialize(self, prm: LayerParams, slot_ids: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Exact current full state [b,H,P,N] fp32 of the slots (the tier is unchanged)."""
        b = self.slots if slot_ids is None else slot_ids.shape[0]
        if out is None:
            out = torch.empty(b, self.H, self.P, self.N, device=self.hot.device, dtype=torch.float32)
        _need(out, "out", torch.float32, (b, self.H, self.P, self.N))
        if slot_ids is not None:
            _need(slot_ids, "slot_ids", torch.int32, (b,))
        _check_unique(slot_ids, "V4Tier.materialize")
        self._device_check(slot_ids)
        pc, tc = prm.c_struct(), self.c_struct()
        check(lib().nssm_v4_materialize(ctypes.byref(pc), ctypes.byref(tc), out.data_ptr(), b, _ptr(slot_ids),
                                        _stream()), "nssm_v4_materialize")
        return out


def fp8_cold_readout(qc: torch.Tensor, S8: torch.Tensor, scale: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """y[r,p] = sum_n qc[r,n] scale[r,n] fp8(S8[r,n,p]) (scale/bench_v4_decode.py:55-60)."""
    R_, Nc, Pd = S8.shape
    s8 = S8.view(torch.uint8) if S8.dtype == torch.float8_e4m3fn else S8
    _need(qc, "qc", torch.float32, (R_, Nc))
    _need(s8, "S8", torch.uint8, (R_, Nc, Pd))
    _need(scale, "scale", torch.float32, (R_, Nc))
    _need(out, "out", torch.float32, (R_, Pd))
    check(lib().nssm_fp8_readout(qc.data_ptr(), s8.data_ptr(), scale.data_ptr(), out.data_ptr(), R_, Nc, Pd,
                                 _stream()), "nssm_fp8_readout")
    return out


def rotate(X: torch.Tensor, R: torch.Tensor) -> torch.Tensor:
    """out[t,g,m] = sum_n R[g,m,n] X[t,g,n] for bf16 X [T,G,N]; fp32 out."""
    T, G, N = X.shape
    _need(X, "X", torch.bfloat16, (T, G, N))
    _need(R, "R", torch.float32, (G, N, N))
    out = torch.empty(T, G, N, device=X.device, dtype=torch.float32)
    check(lib().nssm_rotate(X.data_ptr(), R.data_ptr(), out.data_ptr(), T, G, N, _stream()), "nssm_rotate")
    return out


def conv_update(hbc: torch.Tensor, conv_state: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                intermediate: int, gn: int, mask: Optional[torch.Tensor] = None):
    """One decode token's causal conv1d update + SiLU and the x / B / C split, on the
    GPU in one launch: conv_state [b,dim,W] is updated in place; returns bf16
    x [b, intermediate], B [b, gn], C [b, gn]. hbc [b, dim] may be a row-strided slice
    (unit stride over channels); hbc, conv_state, weight [dim, W], bias [dim] share
    the model dtype (fp32 or bf16). Replaces causal_conv1d_update(..., "silu") and the
    split at scale/v4_fused_decode.py:42-44."""
    b, dim = hbc.shape
    W = conv_state.shape[-1]
    dt = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16}.get(hbc.dtype)
    if dt is None:
        raise NssmError(f"conv_update: model dtype {hbc.dtype} is not fp32 or bf16")
    if not hbc.is_cuda or hbc.stride(1) != 1:
        raise NssmError("conv_update: hbc must be a CUDA tensor with unit stride over channels")
    _need(conv_state, "conv_state", hbc.dtype, (b, dim, W))
    _need(weight, "weight", hbc.dtype, (dim, W))
    if bias is not None:
        _need(bias, "bias", hbc.dtype, (dim,))
    if mask is not None:
        _need(mask, "mask", torch.float32, (b,))
    bf = torch.bfloat16
    x = torch.empty(b, intermediate, device=hbc.device, dtype=bf)
    B = torch.empty(b, gn, device=hbc.device, dtype=bf)
    C = torch.empty(b, gn, device=hbc.device, dtype=bf)
    check(lib().nssm_conv_update(b, dim, W, dt, hbc.data_ptr(), hbc.stride(0), conv_state.data_ptr(),
                                 weight.data_ptr(), _ptr(bias), _ptr(mask), intermediate, gn, x.data_ptr(),
                                 B.data_ptr(), C.data_ptr(), _stream()), "nssm_conv_update")
    return x, B, C


def gated_rmsnorm(y: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, group_size: int, eps: float,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The mixer's epilogue norm on the GPU in one launch: y [b, I] fp32 (D x included)
    cast to the model dtype, times silu(gate), RMS-normalised per group of group_size
    channels, times weight (transformers' Zamba2RMSNormGated; self.norm(y, gate) at
    scale/v4_native_decode.py:170-171). gate [b, I] may be a row-strided slice; gate,
    weight [I] and the returned out [b, I] share the model dtype (fp32 or bf16)."""
    b, I = y.shape
    dt = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16}.get(gate.dtype)
    if dt is None:
        raise NssmError(f"gated_rmsnorm: model dtype {gate.dtype} is not fp32 or bf16")
    _need(y, "y", torch.float32, (b, I))
    _need(weight, "weight", gate.dtype, (I,))
    if not gate.is_cuda or gate.stride(1) != 1 or tuple(gate.shape) != (b, I):
        raise NssmError("gated_rmsnorm: gate must be a CUDA [b, I] tensor with unit stride over channels")
    if out is None:
        out = torch.empty(b, I, device=y.device, dtype=gate.dtype)
    _need(out, "out", gate.dtype, (b, I))
    check(lib().nssm_gated_rmsnorm(b, I, group_size, dt, y.data_ptr(), gate.data_ptr(), gate.stride(0),
                                   weight.data_ptr(), float(eps), out.data_ptr(), _stream()), "nssm_gated_rmsnorm")
    return out


def set_launch(units_per_wg: int = 0) -> None:
    """Override the stream kernel's units (waves of 8 headdim rows) per workgroup
    (0 = automatic; at most 4, and a step raises when it does not divide P / 8)."""
    check(lib().nssm_set_launch(units_per_wg), "nssm_set_launch")
