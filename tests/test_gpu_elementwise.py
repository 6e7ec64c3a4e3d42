"""Gather, combine and SiLU-and-mul on the GPU vs the oracle."""
import numpy as np
import pytest
import torch

from oracle import moe
from tests._helpers import banner

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_gather_hidden_exact(dtype, device):
    from exq_amd.kernels.exq_dispatch import gather_hidden
    banner(f"gather {dtype}")
    rng = np.random.default_rng(0)
    T, k, H = 16, 8, 2048
    hidden = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(dtype)
    order = rng.permutation(T * k)
    out = torch.empty(T * k, H, dtype=dtype, device=device)
    gather_hidden(hidden.to(device), torch.from_numpy(order).to(device), out, k)
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    ref = moe.gather_hidden(hidden.view(bits).numpy(), order, k)
    assert np.array_equal(out.cpu().view(bits).numpy(), ref)


@pytest.mark.parametrize("dtype,wdtype", [(torch.bfloat16, torch.float32),
                                          (torch.float16, torch.float16),
                                          (torch.float32, torch.bfloat16)])
def test_combine(dtype, wdtype, device):
    from exq_amd.kernels.exq_dispatch import combine
    banner(f"combine {dtype} {wdtype}")
    rng = np.random.default_rng(1)
    T, k, H = 13, 6, 384
    down = torch.from_numpy(rng.standard_normal((T * k, H)).astype(np.float32)).to(dtype)
    w = torch.from_numpy(rng.random((T, k)).astype(np.float32)).to(wdtype)
    order = rng.permutation(T * k)
    res = torch.empty(T, H, dtype=dtype, device=device)
    combine(down.to(device), torch.from_numpy(order).to(device), w.to(device), res)
    ref = moe.combine(down.float().numpy(), order, w.float().numpy())
    # fp32 accumulation then one rounding to the output dtype
    tol = {torch.float32: 1e-6, torch.float16: 1e-3, torch.bfloat16: 8e-3}[dtype]
    assert np.allclose(res.float().cpu().numpy(), ref, rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_silu_and_mul(dtype, device):
    from exq_amd.kernels.exq_dispatch import silu_and_mul
    banner(f"silu_and_mul {dtype}")
    rng = np.random.default_rng(2)
    x = torch.from_numpy((rng.standard_normal((37, 2 * 768)) * 4).astype(np.float32)).to(dtype)
    out = torch.empty(37, 768, dtype=dtype, device=device)
    silu_and_mul(x.to(device), out)
    ref = moe.silu_and_mul(x.float().numpy().astype(np.float64))
    tol = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 8e-3}[dtype]
    assert np.allclose(out.float().cpu().numpy(), ref, rtol=tol, atol=tol * 1e-2)
