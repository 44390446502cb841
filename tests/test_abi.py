"""CPU checks of the C ABI (no kernel launches): the library loads, exports
every entry point include/nssm.h declares, its scalar format conversions are
bit-identical to torch's casts, and argument validation returns error codes."""
import ctypes
import os
import re

import pytest
import torch

import nested_ssm_amd
from nested_ssm_amd import _lib
from nested_ssm_amd.ops import LayerParams, V4Tier, _need

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nssm.h")


def header_functions():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(nssm_[a-z0-9_]+)\s*\(", txt)))


def header_defines():
    return dict(re.findall(r"#define\s+(NSSM_[A-Z0-9_]+)\s+\(?(-?\d+)\)?", open(HEADER).read()))


def test_library_loads_and_exports_every_declared_function():
    L = _lib.lib()
    names = header_functions()
    assert len(names) >= 12
    for nm in names:
        assert hasattr(L, nm), f"{nm} declared in include/nssm.h but not exported"
    assert sorted(_lib.EXPORTED) == names


def test_abi_version_and_codes_match_header():
    d = header_defines()
    L = _lib.lib()
    assert L.nssm_abi_version() == int(d["NSSM_ABI_VERSION"])
    assert int(d["NSSM_COLD_FP32"]) == _lib.COLD_FP32
    assert int(d["NSSM_COLD_BF16"]) == _lib.COLD_BF16
    assert int(d["NSSM_COLD_FP8"]) == _lib.COLD_FP8
    assert int(d["NSSM_COLD_NONE"]) == _lib.COLD_NONE
    assert int(d["NSSM_COLD_BF16_SINGLE"]) == _lib.COLD_BF16_SINGLE
    assert int(d["NSSM_COLD_FP8_BF16M"]) == _lib.COLD_FP8_BF16M
    assert (int(d["NSSM_XRING_ROW"]), int(d["NSSM_XRING_UNIT"])) == (_lib.XRING_ROW, _lib.XRING_UNIT)
    assert (int(d["NSSM_DT_F32"]), int(d["NSSM_DT_BF16"])) == (_lib.DT_F32, _lib.DT_BF16)
    for code in ("NSSM_E_NULL", "NSSM_E_DIMS", "NSSM_E_ALIGN", "NSSM_E_KIND", "NSSM_E_LAUNCH", "NSSM_E_TUNING",
                 "NSSM_E_WORKSPACE", "NSSM_E_SCRATCH"):
        msg = L.nssm_strerror(int(d[code])).decode()
        assert msg and msg != "unknown nssm error"
    assert L.nssm_strerror(0).decode() == "ok"


def _host_f32_to_e4m3(x: torch.Tensor) -> torch.Tensor:
    x = x.contiguous().float()
    out = torch.empty(x.numel(), dtype=torch.uint8)
    _lib.lib().nssm_host_f32_to_e4m3fn(x.data_ptr(), out.data_ptr(), x.numel())
    return out.view(x.shape)


def test_e4m3fn_encode_matches_torch_on_a_dense_sweep():
    # every fp32 bit pattern with 11 low mantissa bits dropped over |x| in [2^-12, 512):
    # covers subnormals, every rounding tie class and the overflow edge
    lo = torch.tensor(2.0 ** -12).view(torch.int32).item()
    hi = torch.tensor(512.0).view(torch.int32).item()
    bits = torch.arange(lo, hi, 1 << 11, dtype=torch.int64).to(torch.int32)
    x = bits.view(torch.float32)
    x = torch.cat([x, -x, torch.tensor([0.0, -0.0, 448.0, 464.0, 463.9999, 480.0, 2.0 ** -9, 2.0 ** -10,
                                        1.5 * 2.0 ** -9, 2.0 ** -6, 0.9999 * 2.0 ** -6])])
    want = x.to(torch.float8_e4m3fn).view(torch.uint8)
    got = _host_f32_to_e4m3(x)
    bad = (got != want).nonzero()
    assert bad.numel() == 0, f"{bad.numel()} mismatches, first x={x[bad[0]].item()!r}"


def test_e4m3fn_encode_random_and_nan():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(200000, generator=g) * torch.logspace(-5, 2.6, 200000)
    assert torch.equal(_host_f32_to_e4m3(x), x.to(torch.float8_e4m3fn).view(torch.uint8))
    nan = _host_f32_to_e4m3(torch.tensor([float("nan")]))
    assert int(nan[0]) & 0x7F == 0x7F


def test_e4m3fn_decode_all_codes():
    codes = torch.arange(256, dtype=torch.uint8)
    out = torch.empty(256, dtype=torch.float32)
    _lib.lib().nssm_host_e4m3fn_to_f32(codes.data_ptr(), out.data_ptr(), 256)
    want = codes.view(torch.float8_e4m3fn).float()
    same = (out == want) | (torch.isnan(out) & torch.isnan(want))
    assert bool(same.all())
    assert torch.equal(torch.signbit(out[~torch.isnan(out)]), torch.signbit(want[~torch.isnan(want)]))


def test_bf16_rne_matches_torch():
    g = torch.Generator().manual_seed(1)
    x = torch.cat([torch.randn(100000, generator=g) * 1e3, torch.randn(100000, generator=g) * 1e-30,
                   torch.tensor([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.3895e38, -1e-45])])
    out = torch.empty(x.numel(), dtype=torch.int16)
    _lib.lib().nssm_host_f32_to_bf16(x.data_ptr(), out.data_ptr(), x.numel())
    assert torch.equal(out, x.to(torch.bfloat16).view(torch.int16))


def test_tier_sizes():
    L = _lib.lib()
    sz = (ctypes.c_int64 * 10)()
    assert L.nssm_tier_sizes(256, 128, 80, 128, 8, 32, 4, _lib.COLD_FP32, sz) == 0
    rows = 256 * 128 * 80
    assert sz[0] == rows * 32 * 4 and sz[1] == rows * 96 * 4 and sz[2] == 0 and sz[3] == 0
    assert sz[4] == 256 * 128 * 4 * 80 * 2 and sz[6] == 256 * 8 * 4 * 96 * 4
    assert L.nssm_tier_sizes(448, 128, 80, 128, 8, 32, 4, _lib.COLD_FP8, sz) == 0
    assert sz[1] == 448 * 128 * 80 * 96 and sz[2] == 448 * 128 * 80 * 4 and sz[3] == 448 * 128 * 80 * 96 * 4
    # bf16 masters: one bf16 copy (no master); e4m3 copy + row scale + bf16 master
    assert L.nssm_tier_sizes(256, 128, 80, 128, 8, 32, 4, _lib.COLD_BF16_SINGLE, sz) == 0
    assert sz[1] == rows * 96 * 2 and sz[2] == 0 and sz[3] == 0 and sz[6] == 256 * 8 * 4 * 96 * 4
    assert L.nssm_tier_sizes(448, 128, 80, 128, 8, 32, 4, _lib.COLD_FP8_BF16M, sz) == 0
    assert sz[1] == 448 * 128 * 80 * 96 and sz[2] == 448 * 128 * 80 * 4 and sz[3] == 448 * 128 * 80 * 96 * 2
    assert L.nssm_tier_sizes(4, 8, 80, 128, 1, 32, 4, 6, sz) == -4
    assert L.nssm_tier_sizes(4, 8, 80, 64, 1, 32, 4, 0, sz) == -2  # d_state must be 128
    assert L.nssm_tier_sizes(4, 8, 80, 128, 1, 32, 65, 0, sz) == -2  # c above 64
    assert L.nssm_tier_sizes(4, 8, 80, 128, 1, 32, 4, 7, sz) == -4
    assert L.nssm_tier_sizes(4, 8, 80, 128, 1, 32, 4, 3, sz) == 0  # hot only
    assert sz[0] == 4 * 8 * 80 * 32 * 4 and all(sz[i] == 0 for i in range(1, 7))


def test_entry_points_validate_before_launching():
    """Bad arguments return codes without touching a device (fake pointers never dereferenced)."""
    L = _lib.lib()
    fake = 4096
    prm = _lib.LayerParams(8, 80, 128, 1, fake, fake, fake, None, 0.0)
    inp = _lib.StepInputs(4, fake, fake, fake, fake, None)
    assert L.nssm_fresh_step(None, fake, 4, ctypes.byref(inp), fake, fake, 1 << 30, None) == -1
    bad = _lib.LayerParams(8, 80, 64, 1, fake, fake, fake, None, 0.0)
    assert L.nssm_fresh_step(ctypes.byref(bad), fake, 4, ctypes.byref(inp), fake, fake, 1 << 30, None) == -2
    bad = _lib.LayerParams(8, 72, 128, 1, fake, fake, fake, None, 0.0)  # P not a multiple of 16
    assert L.nssm_fresh_step(ctypes.byref(bad), fake, 4, ctypes.byref(inp), fake, fake, 1 << 30, None) == -2
    bad = _lib.LayerParams(8, 80, 128, 3, fake, fake, fake, None, 0.0)  # H % G
    assert L.nssm_fresh_step(ctypes.byref(bad), fake, 4, ctypes.byref(inp), fake, fake, 1 << 30, None) == -2
    assert L.nssm_fresh_step(ctypes.byref(prm), fake + 4, 4, ctypes.byref(inp), fake, fake, 1 << 30, None) == -3
    assert L.nssm_fresh_step(ctypes.byref(prm), fake, 2, ctypes.byref(inp), fake, fake, 1 << 30, None) == -2  # b > slots
    tier = _lib.Tier(4, 32, 4, 9, *([fake] * 10))
    assert L.nssm_v4_step(ctypes.byref(prm), ctypes.byref(tier), ctypes.byref(inp), fake, fake, 1 << 30, None) == -4
    tier = _lib.Tier(4, 48, 4, 0, *([fake] * 10))  # k_hot not 16, 32, 64 or 96
    assert L.nssm_v4_step(ctypes.byref(prm), ctypes.byref(tier), ctypes.byref(inp), fake, fake, 1 << 30, None) == -2
    tier = _lib.Tier(4, 32, 0, 0, *([fake] * 10))  # c = 0
    assert L.nssm_v4_step(ctypes.byref(prm), ctypes.byref(tier), ctypes.byref(inp), fake, fake, 1 << 30, None) == -2
    tier = _lib.Tier(4, 32, 4, 2, *([fake] * 2 + [None] + [fake] * 7))  # fp8 without a scale buffer
    assert L.nssm_v4_step(ctypes.byref(prm), ctypes.byref(tier), ctypes.byref(inp), fake, fake, 1 << 30, None) == -1
    tier = _lib.Tier(4, 32, 4, 0, *([fake] * 10), 2)  # x ring layout neither row nor unit
    assert L.nssm_v4_step(ctypes.byref(prm), ctypes.byref(tier), ctypes.byref(inp), fake, fake, 1 << 30, None) == -4
    # workspace: NULL, too small, misaligned
    need = L.nssm_step_workspace_bytes(4, 8, 1, 128, 0)
    assert need == 4 * (2 * 128 + 12 * 8) * 4
    # tiered: plus per-(request, group) flush flags [b][G] (padded to a multiple of 4),
    # window weights [b][H][c] and the exact readout's window dots [b][G][c]
    assert L.nssm_step_workspace_bytes(4, 8, 1, 128, 4) == need + 4 * 4 + (4 * 8 * 4 + 4 * 1 * 4) * 4
    assert L.nssm_step_workspace_bytes(3, 8, 2, 128, 4) == 4 * (3 * (2 * 2 * 128 + 12 * 8 + 8 * 4 + 2 * 4) + 8)
    assert L.nssm_step_workspace_bytes(4, 8, 3, 128, 4) == -2
    assert L.nssm_fresh_step(ctypes.byref(prm), fake, 4, ctypes.byref(inp), fake, None, need, None) == -7
    assert L.nssm_fresh_step(ctypes.byref(prm), fake, 4, ctypes.byref(inp), fake, fake, need - 4, None) == -7
    assert L.nssm_fresh_step(ctypes.byref(prm), fake, 4, ctypes.byref(inp), fake, fake + 8, need, None) == -3
    # conv prologue: dim = I + 2 GN, width <= 8, dtype fp32 / bf16
    assert L.nssm_conv_update(2, 10, 4, 0, fake, 10, fake, fake, None, None, 4, 2, fake, fake, fake, None) == -2
    assert L.nssm_conv_update(2, 8, 9, 0, fake, 8, fake, fake, None, None, 4, 2, fake, fake, fake, None) == -2
    assert L.nssm_conv_update(2, 8, 4, 5, fake, 8, fake, fake, None, None, 4, 2, fake, fake, fake, None) == -4
    assert L.nssm_conv_update(2, 8, 4, 0, None, 8, fake, fake, None, None, 4, 2, fake, fake, fake, None) == -1
    assert L.nssm_conv_update(0, 8, 4, 0, fake, 8, fake, fake, None, None, 4, 2, fake, fake, fake, None) == 0
    # epilogue norm: I a multiple of gs, gs <= 2048, dtype fp32 / bf16
    assert L.nssm_gated_rmsnorm(2, 100, 30, 0, fake, fake, 100, fake, ctypes.c_float(1e-5), fake, None) == -2
    assert L.nssm_gated_rmsnorm(2, 4096, 4096, 0, fake, fake, 4096, fake, ctypes.c_float(1e-5), fake, None) == -2
    assert L.nssm_gated_rmsnorm(2, 128, 64, 3, fake, fake, 128, fake, ctypes.c_float(1e-5), fake, None) == -4
    assert L.nssm_gated_rmsnorm(2, 128, 64, 0, None, fake, 128, fake, ctypes.c_float(1e-5), fake, None) == -1
    # the exact readout needs a cold tier; x must be 8-byte aligned
    tier = _lib.Tier(4, 32, 4, _lib.COLD_KINDS["off"], *([fake] * 10))
    assert L.nssm_v4_step_exact(ctypes.byref(prm), ctypes.byref(tier), ctypes.byref(inp), fake, fake, 1 << 30,
                                None) == -4
    odd = _lib.StepInputs(4, fake + 2, fake, fake, fake, None)
    assert L.nssm_v4_step_exact(ctypes.byref(prm), ctypes.byref(tier), ctypes.byref(odd), fake, fake, 1 << 30,
                                None) == -3
    # gated readout: the threshold must be a finite number, the counters 8-byte aligned
    t32 = _lib.Tier(4, 32, 4, _lib.COLD_FP32, *([fake] * 10))
    gargs = (ctypes.byref(prm), ctypes.byref(t32), ctypes.byref(inp), fake, fake, 1 << 30)
    assert L.nssm_v4_step_gated(*gargs, 0, float("nan"), None, None) == -2
    assert L.nssm_v4_step_gated(*gargs, 0, float("inf"), None, None) == -2
    assert L.nssm_v4_step_gated(*gargs, 0, 0.5, fake + 4, None) == -3
    assert L.nssm_v4_step_gated(*gargs[:1], None, *gargs[2:], 1, 0.0, None, None) == -1
    # the ring's x rows are read 16 bytes at a time: ring_x must be 16-byte aligned
    ptrs = [fake] * 10
    ptrs[4] = fake + 8
    t8 = _lib.Tier(4, 32, 4, _lib.COLD_FP32, *ptrs)
    assert L.nssm_v4_step(ctypes.byref(prm), ctypes.byref(t8), ctypes.byref(inp), fake, fake, 1 << 30, None) == -3
    assert L.nssm_set_launch(5) == -6
    assert L.nssm_set_launch(-1) == -6
    # 4 units per workgroup do not divide P / 8 = 10 rows blocks: refused before any launch
    assert L.nssm_set_launch(4) == 0
    t32 = _lib.Tier(4, 32, 4, _lib.COLD_FP32, *([fake] * 10))
    assert L.nssm_v4_step(ctypes.byref(prm), ctypes.byref(t32), ctypes.byref(inp), fake, fake, 1 << 30, None) == -6
    assert L.nssm_set_launch(0) == 0


def test_python_layer_rejects_cpu_tensors_and_wrong_dtypes():
    x = torch.zeros(2, 8, 80, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no CPU path"):
        _need(x, "x", torch.bfloat16, (2, 8, 80))
    prm = LayerParams(8, 80, 128, 1, torch.zeros(8), torch.zeros(8), torch.zeros(8))
    with pytest.raises(ValueError, match="no CPU path"):
        nested_ssm_amd.fresh_step(prm, torch.zeros(2, 8, 80, 128), x, x, x, x)
    with pytest.raises(ValueError):
        V4Tier(2, 8, 80, 1, cold="int4")
    with pytest.raises(ValueError, match="x_ring"):
        V4Tier(2, 8, 80, 1, x_ring="tiled")


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libnssm_hip.so"))
    with pytest.raises(_lib.NssmError, match="no CPU fallback"):
        _lib.lib()


@pytest.mark.parametrize("NC", [96, 64, 32, 112])
def test_blocked_16bit_layout_unpacks_to_row_order(NC):
    """The bf16 read copies and the bf16 master are stored unit-blocked: element (row, col)
    at (row // 8) * 8 NC + (col // 32) * 256 + (row % 8) * w + col % 32 with w = 32, or
    16 in a trailing 16-column segment (NC = 112, k_hot = 16; include/nssm.h).
    V4Tier.cold_rows / master_rows unpack that order (checked here on the CPU against the
    formula; the GPU join test checks the kernels through them)."""
    from nested_ssm_amd.ops import V4Tier

    S, H, P = 2, 3, 16
    rows = S * H * P
    flat = torch.empty(rows * NC, dtype=torch.int64)
    for r in range(rows):
        for cidx in range(NC):
            w = min(32, NC - cidx // 32 * 32)
            off = (r // 8) * 8 * NC + (cidx // 32) * 256 + (r % 8) * w + cidx % 32
            flat[off] = r * 1000 + cidx
    got = V4Tier._rows(None, flat.view(S, H, P, NC), True)
    want = (torch.arange(rows)[:, None] * 1000 + torch.arange(NC)[None, :]).view(S, H, P, NC)
    assert torch.equal(got, want)
    if NC == 32:  # one segment: the blocked order is the row order
        assert torch.equal(flat.view(S, H, P, NC), want)


def test_duplicate_slot_ids_are_refused_when_checked(monkeypatch):
    """With the slot check on (the test suite turns it on), a call whose slot ids repeat
    raises before any launch; unique ids and no ids pass; with the check off nothing is
    checked (the product path does not sync the host for it)."""
    from nested_ssm_amd import ops

    monkeypatch.setattr(ops, "_CHECK_SLOTS", True)
    with pytest.raises(ValueError, match="unique"):
        ops._check_unique(torch.tensor([3, 1, 3], dtype=torch.int32), "V4Tier.step")
    ops._check_unique(torch.tensor([3, 1, 2], dtype=torch.int32), "V4Tier.step")
    ops._check_unique(None, "V4Tier.step")
    ops.set_checks(slot_ids=False)
    assert ops._CHECK_SLOTS is False
    ops._check_unique(torch.tensor([3, 3], dtype=torch.int32), "V4Tier.step")


def test_lagged_readout_argument_errors():
    """nssm_v4_step_teacher_lagged checks its second snapshot before any device call: NULL
    struct or buffers, the e4m3 kinds' scale, alignment; the tier's own checks come first."""
    L = _lib.lib()
    fake = 4096
    prm = _lib.LayerParams(8, 80, 128, 1, fake, fake, fake, None, 0.0)
    inp = _lib.StepInputs(4, fake, fake, fake, fake, None)
    tier = _lib.Tier(4, 32, 4, _lib.COLD_FP32, *([fake] * 10))
    e8 = _lib.Tier(4, 32, 4, _lib.COLD_FP8_BF16M, *([fake] * 10))
    call = lambda t, lag: L.nssm_v4_step_teacher_lagged(  # noqa: E731
        ctypes.byref(prm), ctypes.byref(t), lag, ctypes.byref(inp), fake, fake, 1 << 30, None)
    assert call(tier, None) == -1
    assert call(tier, ctypes.byref(_lib.Lag(None, None, fake))) == -1
    assert call(tier, ctypes.byref(_lib.Lag(fake, None, None))) == -1
    assert call(e8, ctypes.byref(_lib.Lag(fake, None, fake))) == -1  # e4m3 without row scales
    assert call(tier, ctypes.byref(_lib.Lag(fake + 4, None, fake))) == -3
    off = _lib.Tier(4, 32, 4, _lib.COLD_NONE, *([fake] * 10))
    assert call(off, ctypes.byref(_lib.Lag(fake, None, fake))) == -4  # no cold tier to lag
    bad = _lib.Tier(4, 48, 4, _lib.COLD_FP32, *([fake] * 10))
    assert call(bad, ctypes.byref(_lib.Lag(fake, None, fake))) == -2


def test_check_slots_argument_errors():
    """nssm_check_slots refuses NULL buffers, sizes out of range and a misaligned owner array
    before any device call."""
    L = _lib.lib()
    fake = 4096
    assert L.nssm_check_slots(None, 4, 8, fake, fake, None) == -1
    assert L.nssm_check_slots(fake, 4, 8, None, fake, None) == -1
    assert L.nssm_check_slots(fake, 4, 8, fake, None, None) == -1
    assert L.nssm_check_slots(fake, -1, 8, fake, fake, None) == -2
    assert L.nssm_check_slots(fake, 4, 0, fake, fake, None) == -2
    assert L.nssm_check_slots(fake, 4, 8, fake + 4, fake, None) == -3
    assert L.nssm_check_slots(fake, 0, 8, fake, fake, None) == 0  # nothing to check


def test_noalloc_step_refuses_calls_beyond_its_scratch():
    """nssm_v4_step_noalloc checks its arguments as nssm_v4_step does and refuses, before
    any device call, a call whose workspace would exceed NSSM_SCRATCH_BYTES."""
    L = _lib.lib()
    fake = 4096
    prm = _lib.LayerParams(128, 80, 128, 8, fake, fake, fake, None, 0.0)
    tier = _lib.Tier(4096, 32, 4, _lib.COLD_FP32, *([fake] * 10))
    need = lambda b: L.nssm_step_workspace_bytes(b, 128, 8, 128, 4)  # noqa: E731
    limit = 32 << 20
    assert need(2028) <= limit < need(2029)
    big = _lib.StepInputs(2029, fake, fake, fake, fake, None)
    assert L.nssm_v4_step_noalloc(ctypes.byref(prm), ctypes.byref(tier), ctypes.byref(big), fake, None) == -8
    assert "scratch" in L.nssm_strerror(-8).decode()
    assert L.nssm_v4_step_noalloc(None, ctypes.byref(tier), ctypes.byref(big), fake, None) == -1
    bad = _lib.Tier(4096, 48, 4, _lib.COLD_FP32, *([fake] * 10))
    assert L.nssm_v4_step_noalloc(ctypes.byref(prm), ctypes.byref(bad), ctypes.byref(big), fake, None) == -2


def test_stream_probe_argument_errors():
    """nssm_stream_probe refuses NULL buffers, sizes that are not whole 16 KiB chunks, an
    unknown mode and misaligned buffers before any device call."""
    L = _lib.lib()
    fake, chunk = 4096, 16384
    assert L.nssm_stream_probe(None, fake, chunk, 0, None) == -1
    assert L.nssm_stream_probe(fake, None, chunk, 1, None) == -1
    assert L.nssm_stream_probe(fake, fake, 0, 0, None) == -2
    assert L.nssm_stream_probe(fake, fake, chunk + 16, 0, None) == -2
    assert L.nssm_stream_probe(fake, fake, chunk, 2, None) == -2
    assert L.nssm_stream_probe(fake + 4, fake, chunk, 0, None) == -3
    assert L.nssm_stream_probe(fake, fake + 8, chunk, 1, None) == -3


@pytest.mark.parametrize("argv", [
    [], ["--c", "64", "--exact"], ["--B", "384", "--k", "64", "--c", "16", "--ragged"],
    ["--cold", "fp8", "--master", "bf16", "--B", "448"], ["--qgate", "0.25", "--seed", "3"], ["--coldoff"]])
def test_bench_traffic_pass_rebuilds_the_workload(argv):
    """bench.py's counter passes run the workload again in a child process from the flags
    workload_argv forms: parsed back, they name the same workload (batch, tier shape,
    storage, readout, phases, seed)."""
    import sys

    sys.path.insert(0, ROOT)
    import bench

    a = bench.parse_args(argv)
    b = bench.parse_args(bench.workload_argv(a) + ["--traffic-pass", "--only", "v4"])
    keys = ("B", "k", "c", "cold", "master", "exact", "coldoff", "qgate", "ragged", "seed")
    assert {k: getattr(a, k) for k in keys} == {k: getattr(b, k) for k in keys}
    assert b.traffic_pass and bench.traffic_key(a) == bench.traffic_key(b)
