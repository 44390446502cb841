"""ctypes binding of libnssm_hip.so (the C ABI in include/nssm.h).

Loading fails loudly: there is no CPU fallback anywhere in this package.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnssm_hip.so")

COLD_FP32, COLD_BF16, COLD_FP8, COLD_NONE = 0, 1, 2, 3
COLD_BF16_SINGLE, COLD_FP8_BF16M = 4, 5  # bf16 masters (NSSM_COLD_BF16_SINGLE / NSSM_COLD_FP8_BF16M)
COLD_KINDS = {"fp32": COLD_FP32, "bf16": COLD_BF16, "fp8": COLD_FP8, "off": COLD_NONE}
# (cold read copy, master precision) -> storage kind
STORAGE_KINDS = {("fp32", "fp32"): COLD_FP32, ("bf16", "fp32"): COLD_BF16, ("fp8", "fp32"): COLD_FP8,
                 ("bf16", "bf16"): COLD_BF16_SINGLE, ("fp8", "bf16"): COLD_FP8_BF16M}
DT_F32, DT_BF16 = 0, 1  # model dtypes of nssm_conv_update (NSSM_DT_*)
XRING_ROW, XRING_UNIT = 0, 1  # x ring layouts (NSSM_XRING_*)
XRING_LAYOUTS = {"row": XRING_ROW, "unit": XRING_UNIT}

TIER_FIELDS = ("hot", "cold", "scale", "master", "ring_x", "ring_dt", "ring_b", "t", "nv", "glog")

c_i32 = ctypes.c_int32
c_vp = ctypes.c_void_p


class LayerParams(ctypes.Structure):
    _fields_ = [("H", c_i32), ("P", c_i32), ("N", c_i32), ("G", c_i32),
                ("dt_bias", c_vp), ("A", c_vp), ("D", c_vp), ("R", c_vp),
                ("dt_min", ctypes.c_float)]


class StepInputs(ctypes.Structure):
    _fields_ = [("b", c_i32), ("x", c_vp), ("B", c_vp), ("C", c_vp), ("dt", c_vp),
                ("slot_ids", c_vp)]


class Tier(ctypes.Structure):
    _fields_ = [("slots", c_i32), ("k_hot", c_i32), ("c", c_i32), ("cold_kind", c_i32)] + \
               [(f, c_vp) for f in TIER_FIELDS] + [("x_layout", c_i32)]


class Lag(ctypes.Structure):
    _fields_ = [("cold", c_vp), ("scale", c_vp), ("wlog", c_vp)]


_lib = None


class NssmError(RuntimeError):
    pass


def lib():
    """Load libnssm_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NssmError(f"{LIB_PATH} is missing: build it with `python -m nested_ssm_amd.build` "
                        "(there is no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    P_ = ctypes.POINTER
    L.nssm_abi_version.restype = ctypes.c_int
    L.nssm_strerror.restype = ctypes.c_char_p
    L.nssm_strerror.argtypes = [ctypes.c_int]
    L.nssm_tier_sizes.argtypes = [c_i32] * 8 + [P_(ctypes.c_int64)]
    c_i64 = ctypes.c_int64
    L.nssm_step_workspace_bytes.argtypes = [c_i32] * 5
    L.nssm_step_workspace_bytes.restype = c_i64
    L.nssm_fresh_step.argtypes = [P_(LayerParams), c_vp, c_i32, P_(StepInputs), c_vp, c_vp, c_i64, c_vp]
    L.nssm_v4_step.argtypes = [P_(LayerParams), P_(Tier), P_(StepInputs), c_vp, c_vp, c_i64, c_vp]
    L.nssm_v4_step_exact.argtypes = [P_(LayerParams), P_(Tier), P_(StepInputs), c_vp, c_vp, c_i64, c_vp]
    L.nssm_v4_step_noalloc.argtypes = [P_(LayerParams), P_(Tier), P_(StepInputs), c_vp, c_vp]
    L.nssm_v4_step_teacher.argtypes = [P_(LayerParams), P_(Tier), P_(StepInputs), c_vp, c_vp, c_i64, c_vp]
    L.nssm_v4_step_teacher_lagged.argtypes = [P_(LayerParams), P_(Tier), P_(Lag), P_(StepInputs), c_vp, c_vp, c_i64,
                                              c_vp]
    L.nssm_v4_step_gated.argtypes = [P_(LayerParams), P_(Tier), P_(StepInputs), c_vp, c_vp, c_i64, c_i32,
                                     ctypes.c_float, c_vp, c_vp]
    L.nssm_v4_join.argtypes = [P_(LayerParams), P_(Tier), c_vp, c_i32, c_vp, c_vp, c_vp]
    L.nssm_v4_materialize.argtypes = [P_(LayerParams), P_(Tier), c_vp, c_i32, c_vp, c_vp]
    L.nssm_fp8_readout.argtypes = [c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_vp]
    L.nssm_rotate.argtypes = [c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_vp]
    L.nssm_check_slots.argtypes = [c_vp, c_i32, c_i32, c_vp, c_vp, c_vp]
    L.nssm_gated_rmsnorm.argtypes = [c_i32, c_i32, c_i32, c_i32, c_vp, c_vp, c_i64, c_vp, ctypes.c_float, c_vp, c_vp]
    L.nssm_conv_update.argtypes = [c_i32, c_i32, c_i32, c_i32, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i32, c_i32,
                                   c_vp, c_vp, c_vp, c_vp]
    L.nssm_set_launch.argtypes = [c_i32]
    L.nssm_stream_probe.argtypes = [c_vp, c_vp, c_i64, c_i32, c_vp]
    L.nssm_host_f32_to_e4m3fn.argtypes = [c_vp, c_vp, ctypes.c_int64]
    L.nssm_host_e4m3fn_to_f32.argtypes = [c_vp, c_vp, ctypes.c_int64]
    L.nssm_host_f32_to_bf16.argtypes = [c_vp, c_vp, ctypes.c_int64]
    for fn in ("nssm_fresh_step", "nssm_v4_step", "nssm_v4_step_noalloc", "nssm_v4_step_exact", "nssm_v4_step_gated",
               "nssm_v4_step_teacher", "nssm_v4_step_teacher_lagged",
               "nssm_v4_join",
               "nssm_v4_materialize",
               "nssm_fp8_readout", "nssm_rotate", "nssm_conv_update", "nssm_gated_rmsnorm", "nssm_set_launch",
               "nssm_stream_probe", "nssm_tier_sizes", "nssm_check_slots"):
        getattr(L, fn).restype = ctypes.c_int
    for fn in ("nssm_host_f32_to_e4m3fn", "nssm_host_e4m3fn_to_f32", "nssm_host_f32_to_bf16"):
        getattr(L, fn).restype = None
    _lib = L
    return L


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().nssm_strerror(rc).decode()
        raise NssmError(f"{what} failed: {msg} (code {rc})")


# symbols include/nssm.h declares (checked by the CPU test-suite)
EXPORTED = ("nssm_tier_sizes", "nssm_step_workspace_bytes", "nssm_fresh_step", "nssm_v4_step", "nssm_v4_step_noalloc",
            "nssm_v4_step_exact", "nssm_v4_step_teacher", "nssm_v4_step_teacher_lagged",
            "nssm_v4_step_gated", "nssm_v4_join",
            "nssm_v4_materialize", "nssm_fp8_readout", "nssm_rotate", "nssm_conv_update", "nssm_gated_rmsnorm",
            "nssm_check_slots",
            "nssm_set_launch", "nssm_stream_probe",
            "nssm_host_f32_to_e4m3fn", "nssm_host_e4m3fn_to_f32", "nssm_host_f32_to_bf16",
            "nssm_strerror", "nssm_abi_version")
