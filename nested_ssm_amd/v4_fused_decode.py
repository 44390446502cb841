"""Drop-in for scale/v4_fused_decode.py on the MI355X kernels.

Same module surface: `install(model, pb=32, c=16, cold="bf16") -> int`
(scale/v4_fused_decode.py:163-175) with cold in {"bf16", "fp32", "fp8", "off"}, the
rotation read from an ActRotMask-wrapped `m.act.R` into `m._v4R`, and the
module-level `_v4_fused_decode(self, hidden_states, cache_params,
attention_mask)` (scale/v4_fused_decode.py:28-95). Prefill runs the stock
forward and the tier is captured at its end (scale/v4_fused_decode.py:109-160).
No dt clamp, as the reference's fused kernel path. The cold tier is kept over the
reference's bf16 master by default (master="bf16": bf16 cold is one bf16 copy, fp8
cold an e4m3 copy beside a bf16 shadow master, scale/v4_fused_decode.py:149,156-158);
master="fp32" keeps an exact fp32 master instead. cold="off" keeps the hot tier only
(the cold columns are dropped).
"""
from transformers.models.nemotron_h import modeling_nemotron_h as M

from . import hf

_orig_forward = M.NemotronHMamba2Mixer.forward


def _v4_fused_decode(self, hidden_states, cache_params, attention_mask):
    return hf.decode_step(self, hidden_states, cache_params, attention_mask)


def _dispatch(self, hidden_states, cache_params=None, attention_mask=None, **kw):
    return hf.dispatch(self, hidden_states, cache_params, attention_mask, kw, _orig_forward, 0.0,
                       lambda *a: _v4_fused_decode(*a))


def install(model, pb=32, c=16, cold="bf16", master="bf16"):
    n = 0
    for m in hf.mixers(model):
        hf.check_mixer_shape(m)
        m.v4cfg = dict(pb=pb, c=c, cold=cold, master=master if cold in ("bf16", "fp8") else "fp32")
        m._v4state = None
        m._v4R = m.act.R.detach().float() if hasattr(m.act, "R") else None
        m.forward = _dispatch.__get__(m)
        n += 1
    return n
