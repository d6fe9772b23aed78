"""The kernels' f32 -> bf16 rounding equals torch's (c10::BFloat16, round to
nearest even) bit for bit: random bit patterns, exact ties, denormals, values at
the overflow edge and infinities.  NaN inputs are not compared (the payload of a
quieted NaN is not part of the contract)."""
import pytest
import torch

from tilefoundry_amd._lib import lib, ptr

pytestmark = pytest.mark.gpu


def test_round_bf16_matches_torch(gpu_device):
    g = torch.Generator().manual_seed(0)
    bits = torch.randint(-2**31, 2**31 - 1, (1 << 20,), generator=g, dtype=torch.int64)
    x = bits.to(torch.int32).view(torch.float32)
    ties = (torch.randint(0, 2**16, (4096,), generator=g, dtype=torch.int32) << 16) | 0x8000
    near = (torch.randint(0, 2**16, (4096,), generator=g, dtype=torch.int32) << 16) | 0x7fff
    den = torch.randint(1, 2**23, (4096,), generator=g, dtype=torch.int32)
    special = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), 3.3895e38, -3.3895e38,
                            3.4028235e38, 1e-45, -1e-45, 1.0, -1.0, 65504.0])
    x = torch.cat([x, ties.view(torch.float32), near.view(torch.float32),
                   den.view(torch.float32), special])
    x = x[~torch.isnan(x)]
    want = x.to(torch.bfloat16).view(torch.int16)
    xd = x.to(gpu_device)
    out = torch.empty(x.numel(), dtype=torch.int16, device=gpu_device)
    lib().tfd_round_bf16(ptr(xd), ptr(out), x.numel(),
                         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = out.cpu()
    bad = (got != want).nonzero().flatten()
    assert bad.numel() == 0, [(float(x[i]), int(got[i]), int(want[i])) for i in bad[:8]]
