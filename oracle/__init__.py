"""CPU oracle for the Mamba2 v4 tiered decode step — TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU, the arithmetic of the
reference repository's decode step (omin-Kwon/nested_ssm, scale/*.py). It
serves only to check the product: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it, and never as the thing that is
measured or shipped. The
product path (nested_ssm_amd) never imports it and has no CPU fallback.

Precision convention (one fp32 convention for the whole path, as the
reference's variants disagree on bf16 intermediates):
  * bf16 inputs (x, B, C, dt) are upcast to fp32 first, as
    scale/nemo9b_eval.py:35-40 does; every later operation is fp32.
  * R is applied in fp32 without re-rounding to bf16 (scale/v4_fused_decode.py:47-48
    rounds to bf16; scale/v4_native_decode.py applies it in bf16) — deviation.
  * The flush contraction is fp32 (scale/v4_fused_decode.py:80-82 runs it in bf16) — deviation.
  * glog is per (slot, head) as in scale/v4_fused_decode.py:130 and
    scale/vllm_v4_patch.py:100 (scale/v4_native_decode.py:241 keeps the same
    value replicated over P).

Pinning status of each function (how it is checked, in tests/test_oracle.py):
  rotate            closed form vs fp64 matmul; orthogonality of make_rotation
  fresh_step        transformers' own mamba2_selective_state_update (fp32
                    inputs), an fp64 per-element loop, rotation invariance
  NativeV4          k = N reduces to fresh; c = 1 is one-step stale; state
                    after every flush equals the fresh state; fp64 brute force
  NativeV4 exact    (corr=1) y equals the fresh trajectory's y in fp64 with ragged
                    phases and join/leave (the stale readout and a buffer missing
                    this token's term fail it); with an e4m3 snapshot, fresh y plus
                    the closed-form quantisation term exp(G_t) (q sc - snap) . C'
  TieredV4          equals NativeV4 in fp64 (chunked replay == per-token
                    recurrence), including ragged phases and join/leave
  master="bf16"     (NativeV4, TieredV4) the fp64 fresh recurrence with the cold
                    columns rounded to bf16 at the join and after every flush
                    (rounding at every token, never, or quantizing the e4m3 copy
                    from the unrounded state each fails); TieredV4 == NativeV4
                    with ragged phases and join/leave
  NativeV4 gated    (hot_only, qgate) hot_only y = the hot part of the stale y with D x;
                    qgate on constructed queries C = R^T e_n (all energy on one column):
                    a cold column is kept, a hot one dropped at any tau, and the counters
                    count heads; the state is the ungated one's in every mode
  TeacherForcedV4   (scale/nemo9b_eval.py:41-85) the fp64 closed form from a fresh
                    trajectory with the snapshot taken at the last t = c floor(t / c) after
                    its update and the decay summed over (ts, t] (a snapshot before the
                    update or an exclusive decay fails it; the decode readout of NativeV4
                    is shown to differ); c = 1 and k = N give the fresh readout; k = 0
                    (mode "c1") the same closed form with no hot term; master="bf16" the
                    fp64 trajectory with the cold columns rounded to bf16 at the join and
                    at every snapshot (no rounding, or rounding every token, fails it);
                    lag=1 the same closed form one snapshot behind (the state after
                    token c (floor(t / c) - 1), the joined state before the first two
                    snapshots, decay from it to t; the unlagged snapshot fails it)
  mask_width        (set_width) the first `width` rotated coordinates of an explicit fp64
                    rotation kept, the rest zero; a fresh trajectory under it keeps the
                    masked state columns at zero and equals the trajectory of the
                    width-dimensional rotated model
  quant_fp8 / read  torch float8_e4m3fn cast; scale = amax/448 + 1e-12 per row
  fp8_readout       closed form of the reference docstring vs an fp64 loop
  hot_only_step     the hot columns of an fp64 fresh trajectory (they never read the cold ones)
  conv_update       transformers' own causal_conv1d_update (silu) in fp32 and bf16, and an
                    fp64 loop over the shifted window
  gated_rmsnorm     transformers' own Zamba2RMSNormGated module in fp32 and bf16, and an
                    fp64 per-group loop
"""
from .v4_ref import (  # noqa: F401
    LayerParams, NativeV4, TeacherForcedV4, TieredV4, conv_update, fp8_readout, fresh_step, gated_rmsnorm, hot_only_step,
    make_layer_params,
    make_rotation, make_state, make_step_inputs, mask_width, quant_fp8, read_fp8, rotate, softplus_dt,
)
