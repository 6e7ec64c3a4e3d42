"""On-disk cache of packed INT4 banks (exq_amd.runtime.PackedWeightCache):
a miss packs and writes, a hit returns the same tensors, and any change of
the weights, the group size or a damaged file is a miss.  The CPU tests pack
with the oracle restatement; the GPU test with the library's pack kernel."""
import numpy as np
import pytest
import torch

from exq_amd.runtime.pack_cache import PackedWeightCache, fingerprint
from oracle import quant


def _oracle_packer(w13, w2, group_size):
    out = []
    for w in (w13, w2):
        p, s = quant.pack_experts_int4(w.float().numpy(), group_size)
        out += [torch.from_numpy(p), torch.from_numpy(s.view(np.int16))]
    return tuple(out)


def _weights(seed, E=3, I=64, H=256):
    rng = np.random.default_rng(seed)
    w13 = torch.from_numpy((rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float16))
    w2 = torch.from_numpy((rng.standard_normal((E, H, I)) * 0.02).astype(np.float16))
    return w13, w2


def test_cache_miss_then_hit(tmp_path):
    c = PackedWeightCache(tmp_path, packer=_oracle_packer)
    w13, w2 = _weights(1)
    a = c.get_or_pack("layer0", w13, w2)
    assert (c.hits, c.misses) == (0, 1) and c.path("layer0").exists()
    c2 = PackedWeightCache(tmp_path, packer=_oracle_packer)  # a later run
    b = c2.get_or_pack("layer0", w13, w2)
    assert (c2.hits, c2.misses) == (1, 0)
    for x, y in zip(a, b):
        assert x.dtype == y.dtype and torch.equal(x, y)


def test_cache_invalidation(tmp_path):
    c = PackedWeightCache(tmp_path, packer=_oracle_packer)
    w13, w2 = _weights(2)
    c.get_or_pack("L", w13, w2)
    w13b = w13.clone()
    w13b[1, 5, 7] += 0.01                      # one element of a sampled-out row
    assert fingerprint(w13b, w2) != fingerprint(w13, w2)
    c.get_or_pack("L", w13b, w2)
    assert c.misses == 2
    c.get_or_pack("L", w13b, w2, group_size=64)  # group size is part of the key
    assert c.misses == 3
    c.path("L").write_bytes(b"not a safetensors file")
    bank = c.get_or_pack("L", w13b, w2, group_size=64)
    assert c.misses == 4 and bank[0].shape == (3, 128, 128)
    assert c.get_or_pack("L", w13b, w2, group_size=64)[1].shape == (3, 128, 4)
    assert c.hits == 1


@pytest.mark.gpu
def test_cache_with_gpu_packer(tmp_path, device):
    from exq_amd.kernels import pack_experts_int4
    w13, w2 = (w.to(device) for w in _weights(3))
    c = PackedWeightCache(tmp_path)
    a = c.get_or_pack("layer7", w13, w2)
    ref = pack_experts_int4(w13, 128) + pack_experts_int4(w2, 128)
    for x, y in zip(a, ref):
        assert torch.equal(x, y)
    b = PackedWeightCache(tmp_path).get_or_pack("layer7", w13, w2)
    for x, y in zip(b, ref):
        assert x.device == y.device and torch.equal(x, y)
