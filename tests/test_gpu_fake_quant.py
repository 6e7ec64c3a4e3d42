"""Fake quantisation on the GPU (quantize_tensor_int4 / quantize_tensor_int8,
exq/eval/quant_shim.py:84-125) against the oracle's restatement, bit for bit:
fp32 / fp16 / bf16 weights, a last dimension that is not a multiple of 128
(padded short group), zero rows (the reference's known answer,
test_eval.py:151-163), exact half-way ties, and in-place use."""
import numpy as np
import pytest
import torch

from oracle import quant
from tests._helpers import banner

pytestmark = pytest.mark.gpu


def _weights(shape, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    w[0, 1] = 0.0                      # a zero row
    # a group whose max is 7 and holds exact half-way points (scale 1.0)
    w[1, 2, :128] = 0.0
    w[1, 2, 0] = 7.0
    w[1, 2, 1:9] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 3.5, -6.5, 6.5], dtype=np.float32)
    return w


def _oracle(w32: np.ndarray, bits: int) -> np.ndarray:
    return quant.fake_quant_int4(w32) if bits == 4 else quant.fake_quant_int8(w32)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("K", [256, 300])
def test_fake_quant_bit_exact(bits, dtype, K, device):
    from exq_amd.kernels import quantize_tensor_int4, quantize_tensor_int8
    banner(f"fake quant int{bits} {dtype} K={K}")
    w = torch.from_numpy(_weights((2, 5, K), K + bits)).to(dtype)
    fn = quantize_tensor_int4 if bits == 4 else quantize_tensor_int8
    got = fn(w.to(device))
    assert got.dtype == dtype and got.shape == w.shape
    # the oracle computes in fp32 from the stored values; one rounding to the dtype
    ref32 = _oracle(w.float().numpy(), bits)
    ref = torch.from_numpy(ref32).to(dtype)
    assert torch.equal(got.cpu(), ref)
    # zero rows stay exactly zero; the tie group rounds half to even
    assert torch.count_nonzero(got[0, 1]) == 0
    if bits == 4:
        tie = got[1, 2, :9].float().cpu().numpy()
        assert np.array_equal(tie, np.array([7, 0, 2, 2, -0, -2, 4, -6, 6], dtype=np.float32))


def test_fake_quant_in_place_and_errors(device):
    from exq_amd import _lib
    from exq_amd.kernels import quantize_tensor_int4
    w = torch.from_numpy(_weights((2, 5, 256), 9)).to(torch.float16).to(device)
    want = quantize_tensor_int4(w)
    L = _lib.lib()
    _lib.check(L.exq_fake_quant(w.data_ptr(), _lib.dtype_code(w.dtype), 10, 256, 4, 128,
                                w.data_ptr(), _lib.stream_handle(w.device)), "in place")
    assert torch.equal(w, want)
    with pytest.raises(_lib.ExqError, match="bits must be 4 or 8"):
        _lib.check(L.exq_fake_quant(w.data_ptr(), _lib.dtype_code(w.dtype), 10, 256, 3, 128,
                                    w.data_ptr(), _lib.stream_handle(w.device)), "bits")
    with pytest.raises(_lib.ExqError):
        quantize_tensor_int4(torch.zeros(4, 8))  # host tensor: no host path


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_fake_quant_nan_inf_and_0dim(dtype, device):
    """torch's amax / clamp keep NaN (quant_shim.py:92-95, 114-117): a NaN or
    infinite weight turns its whole INT8 row or INT4 group into NaN, and the
    other rows and groups are untouched.  A 0-dim tensor is one INT8 element;
    INT4 indexes shape[-1] and raises."""
    from exq_amd.kernels import quantize_tensor_int4, quantize_tensor_int8
    banner(f"fake quant NaN / inf / 0-dim {dtype}")
    w = torch.from_numpy(_weights((2, 6, 256), 3)).to(dtype)
    w[0, 0, 5] = float("nan")     # row 0, group 0
    w[0, 2, 200] = float("inf")   # row 2, group 1
    w[0, 3, 7] = float("-inf")    # row 3, group 0
    for bits, fn in ((4, quantize_tensor_int4), (8, quantize_tensor_int8)):
        got = fn(w.to(device)).cpu()
        ref = torch.from_numpy(_oracle(w.float().numpy(), bits)).to(dtype)
        assert torch.equal(torch.isnan(got), torch.isnan(ref))
        fin = ~torch.isnan(ref)
        assert torch.equal(got[fin], ref[fin])
        if bits == 8:
            assert torch.isnan(got[0, [0, 2, 3]]).all() and not torch.isnan(got[0, [1, 4, 5]]).any()
        else:
            assert torch.isnan(got[0, 0, :128]).all() and not torch.isnan(got[0, 0, 128:]).any()
            assert torch.isnan(got[0, 2, 128:]).all() and not torch.isnan(got[0, 2, :128]).any()
    s = torch.tensor(0.3, dtype=dtype)
    got = quantize_tensor_int8(s.to(device)).cpu()
    assert got.shape == () and torch.equal(got, torch.from_numpy(
        np.asarray(quant.fake_quant_int8(s.float().numpy()))).to(dtype))
    with pytest.raises(IndexError):
        quantize_tensor_int4(s.to(device))
