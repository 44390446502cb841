"""Drop-in for scale/v4_native_decode.py on the MI355X kernels.

Same module surface: `M` (the transformers NemotronH module; callers set
`M.is_fast_path_available`), `install(model, pb=32, c=16, cold_bf16=1,
corr=0, coldoff=0) -> int` (scale/v4_native_decode.py:247-256), the per-mixer
`v4cfg` dict and `_v4state`, and the module-level `_v4_decode(self,
input_states, cache_params, attention_mask)` that probes may wrap
(scale/v4_native_decode.py:28-172). Prefill runs the stock forward; the tier
is captured at its end (scale/v4_native_decode.py:223-244); decode tokens run
the tiered state op on the GPU. As in the reference's native decode, dt is
clamped at the mixer's time_step_min (scale/v4_native_decode.py:55), and the
cold snapshot is bf16 when cold_bf16=1 (an exact fp32 master is kept beside
it) or an exact fp32 copy otherwise.

The readout keys are read from v4cfg at every token, in the reference's order:
corr=1 the rank-c exact correction readout (scale/v4_native_decode.py:81-117), else
coldoff=1 the hot-only draft readout (:118-127), else the stale readout, query-gated when
v4cfg["qgate"] > 0 (:147-156; `_v4state.get("qgate_n")` / `get("qgate_kept")` count the
gated and kept heads since the prompt's capture). Under coldoff the tier evolves exactly
(the reference advances only t). A window beyond the kernels' 64 tokens (c=1<<30,
scale/probe_selfspec_alpha.py:59) runs on a 64-token window while coldoff=1 and raises on
a stale readout; ktop > 0 raises NotImplementedError. The installed transformers has no
`torch_forward`; the mixer's `forward` is patched instead.
"""
from transformers.models.nemotron_h import modeling_nemotron_h as M

from . import hf

_orig_forward = M.NemotronHMamba2Mixer.forward


def _dt_min(self) -> float:
    lim = getattr(self, "time_step_limit", None)
    return float(lim[0]) if lim is not None else float(getattr(self, "time_step_min", 0.0))


def _v4_decode(self, input_states, cache_params, attention_mask):
    """One decode token of a mixer through the tiered state op (pb < N) or the
    untiered one (pb >= N)."""
    return hf.decode_step(self, input_states, cache_params, attention_mask)


def _dispatch(self, input_states, cache_params=None, attention_mask=None, **kw):
    return hf.dispatch(self, input_states, cache_params, attention_mask, kw, _orig_forward, _dt_min(self),
                       lambda *a: _v4_decode(*a))


def install(model, pb=32, c=16, cold_bf16=1, corr=0, coldoff=0):
    n = 0
    for m in hf.mixers(model):
        hf.check_mixer_shape(m)
        m.v4cfg = dict(pb=pb, c=c, cold_bf16=cold_bf16, corr=corr, coldoff=coldoff)
        m._v4state = None
        m.forward = _dispatch.__get__(m)
        n += 1
    return n
