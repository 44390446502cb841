"""GPU: nssm_stream_probe, the streaming read / copy bench.py times beside the state op.
The copy moves every byte (more chunks than workgroups, so the grid-stride loop wraps),
and the read visits every chunk: a +inf planted in the last chunk reaches the one store
the read makes."""
import pytest
import torch

from nested_ssm_amd._lib import check, lib

pytestmark = pytest.mark.gpu

CHUNK = 16384  # bytes per workgroup chunk


def test_stream_probe_copy_moves_every_byte():
    n = 4096 * CHUNK + 7 * CHUNK  # 4103 chunks over 4096 workgroups
    g = torch.Generator(device="cuda").manual_seed(5)
    src = torch.randn(n // 4, device="cuda", generator=g)
    dst = torch.full_like(src, float("nan"))
    s = torch.cuda.current_stream()
    check(lib().nssm_stream_probe(src.data_ptr(), dst.data_ptr(), n, 1, s.cuda_stream), "nssm_stream_probe")
    torch.cuda.synchronize()
    assert torch.equal(dst, src)


def test_stream_probe_read_reaches_the_last_chunk():
    n = 4096 * CHUNK + 3 * CHUNK
    src = torch.zeros(n // 4, device="cuda")
    out = torch.zeros(4, device="cuda")
    s = torch.cuda.current_stream()
    check(lib().nssm_stream_probe(src.data_ptr(), out.data_ptr(), n, 0, s.cuda_stream), "nssm_stream_probe")
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros(4, device="cuda"))  # a finite sum stores nothing
    src[-1] = float("inf")
    check(lib().nssm_stream_probe(src.data_ptr(), out.data_ptr(), n, 0, s.cuda_stream), "nssm_stream_probe")
    torch.cuda.synchronize()
    assert torch.isinf(out).any()
