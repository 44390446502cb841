"""nested_ssm_amd — MI355X (gfx950) Mamba2 decode-step state update with nested
hot/cold tiering ("v4"), behind the decode-step call signatures of
omin-Kwon/nested_ssm (scale/v4_native_decode.py, scale/v4_fused_decode.py,
scale/bench_v4_decode.py).

The kernels live in libnssm_hip.so (C ABI: include/nssm.h), built in-tree by
`python -m nested_ssm_amd.build`. There is no CPU fallback.
"""
from ._lib import COLD_KINDS, NssmError, lib  # noqa: F401
from .ops import (  # noqa: F401
    LayerParams, V4Tier, conv_update, fp8_cold_readout, fresh_step, gated_rmsnorm, rotate, set_checks, set_launch,
)

__version__ = "0.1.0"
