"""GPU: the conv prologue (nssm_conv_update) against the oracle's conv_update on the
same inputs: the conv state update bit for bit; x / B / C (bf16) equal up to a
one-ulp bf16 flip in at most 1% of the elements (the fp32 sum of the window runs
in another order than the oracle's)."""
import pytest
import torch

import oracle
from nested_ssm_amd import conv_update

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,b,I,gn,W,with_bias,with_mask,extra", [
    # width 4: four channels per thread where I, gn, the strides and the hbc slice are
    # 4-channel aligned; width 2: one
    (torch.float32, 4, 128, 32, 4, True, False, 24), (torch.bfloat16, 4, 128, 32, 4, True, True, 24),
    (torch.bfloat16, 64, 10240, 1024, 4, True, False, 24), (torch.bfloat16, 6, 256, 64, 4, False, True, 24),
    (torch.bfloat16, 5, 132, 12, 4, True, True, 24), (torch.float32, 3, 64, 16, 2, False, True, 24),
    # width 4 on the one-channel-per-thread kernel: the hbc slice starts one element past a
    # 4-channel boundary, or I and gn are not multiples of 4
    (torch.bfloat16, 4, 128, 32, 4, True, True, 1), (torch.float32, 3, 64, 16, 4, True, False, 1),
    (torch.bfloat16, 5, 130, 10, 4, True, False, 24), (torch.float32, 2, 130, 10, 4, False, True, 24)])
def test_conv_update_matches_oracle(dtype, b, I, gn, W, with_bias, with_mask, extra):
    gen = torch.Generator().manual_seed(b + I + W)
    dim = I + 2 * gn
    # hbc is a slice of a wider in_proj output (row stride dim + 2 extra, first channel at extra)
    proj = torch.randn(b, dim + 2 * extra, generator=gen).to(dtype)
    hbc = proj[:, extra:extra + dim]
    st = torch.randn(b, dim, W, generator=gen).to(dtype)
    w = (torch.randn(dim, W, generator=gen) * 0.5).to(dtype)
    bias = torch.randn(dim, generator=gen).to(dtype) if with_bias else None
    mask = (torch.arange(b) % 3 != 1).float() if with_mask else None
    st_ref = st.clone()
    xr, Br, Cr = oracle.conv_update(hbc.clone(), st_ref, w, bias, I, gn, mask=mask)
    proj_d = proj.cuda()
    st_d = st.cuda()
    x, B, C = conv_update(proj_d[:, extra:extra + dim], st_d, w.cuda(), None if bias is None else bias.cuda(), I, gn,
                          mask=None if mask is None else mask.cuda())
    assert torch.equal(st_d.cpu(), st_ref)
    got = torch.cat([x, B, C], dim=-1).cpu().float()
    want = torch.cat([xr, Br, Cr], dim=-1).float()
    assert torch.allclose(got, want, rtol=2 ** -7, atol=1e-6)
    assert float((got != want).float().mean()) <= 0.01


@pytest.mark.parametrize("dtype,b,I,gs,off", [
    # one workgroup per group (gs not a multiple of 256, or the gate rows not 4-channel aligned)
    (torch.float32, 4, 256, 64, 8), (torch.bfloat16, 4, 256, 64, 8),
    (torch.bfloat16, 6, 2560, 1280, 1), (torch.float32, 2, 1024, 512, 2),
    # one wave per group (the 9B shape: 8 groups of 1280; 1 and 3 blocks of 256 per lane)
    (torch.bfloat16, 32, 10240, 1280, 8), (torch.float32, 3, 2048, 2048, 8),
    (torch.float32, 2, 1024, 256, 4), (torch.bfloat16, 5, 1536, 768, 4)])
def test_gated_rmsnorm_matches_oracle(dtype, b, I, gs, off):
    """The epilogue norm (nssm_gated_rmsnorm) against the oracle (itself equal to
    transformers' Zamba2RMSNormGated): fp32 rtol 1e-5; bf16 up to one-ulp flips in at
    most 1% of the outputs (the group's sum of squares runs in another order)."""
    from nested_ssm_amd import gated_rmsnorm

    gen = torch.Generator().manual_seed(b + I + off)
    y = torch.randn(b, I, generator=gen)
    proj = torch.randn(b, I + 40, generator=gen).to(dtype)  # gate is a slice of the in_proj output
    gate = proj[:, off:off + I]
    w = torch.randn(I, generator=gen).to(dtype)
    want = oracle.gated_rmsnorm(y, gate, w, gs, 1e-5).float()
    got = gated_rmsnorm(y.cuda(), proj.cuda()[:, off:off + I], w.cuda(), gs, 1e-5).cpu().float()
    if dtype == torch.float32:
        assert torch.allclose(got, want, rtol=1e-5, atol=1e-6)
    else:
        assert torch.allclose(got, want, rtol=2 ** -7, atol=1e-6)
        assert float((got != want).float().mean()) <= 0.01
