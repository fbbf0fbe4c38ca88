"""GPU checks of the measurement kernels bench.py relies on: lemoq_copy_probe
copies exactly (it calibrates the profiler's byte counters) and
lemoq_read_probe reads every byte (its per-block fold equals a numpy fold of
the same buffer), so the bandwidth it reports covers the whole buffer."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_bytes,blocks", [(16, 1), (4096, 3), ((1 << 20) + 48, 64)])
def test_copy_probe_copies_exactly(n_bytes, blocks, dev):
    from lemoq import _hip

    g = torch.Generator().manual_seed(n_bytes)
    src = torch.randint(0, 256, (n_bytes + 64,), dtype=torch.uint8, generator=g).to(dev)
    dst = torch.zeros((n_bytes + 64,), dtype=torch.uint8, device=dev)
    _hip.call("lemoq_copy_probe", _hip.ptr(src), _hip.ptr(dst), n_bytes, blocks, _hip.stream_of(dev))
    torch.cuda.synchronize()
    assert torch.equal(dst[:n_bytes], src[:n_bytes]) and (dst[n_bytes:] == 0).all()


def test_copy_probe_rejects_overlap_and_misalignment(dev):
    from lemoq import _hip

    buf = torch.zeros((4096,), dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError):
        _hip.call("lemoq_copy_probe", _hip.ptr(buf), _hip.ptr(buf) + 1024, 2048, 4, _hip.stream_of(dev))
    with pytest.raises(ValueError):
        _hip.call("lemoq_copy_probe", _hip.ptr(buf) + 8, _hip.ptr(buf) + 2048, 1024, 4, _hip.stream_of(dev))


@pytest.mark.parametrize("n16,blocks", [(1, 1), (1000, 2), (70001, 16), (300, 4), (65536, 16)])
def test_read_probe_folds_every_element(n16, blocks, dev):
    from lemoq import _hip

    g = np.random.default_rng(n16)
    words = g.integers(0, 1 << 32, size=(n16, 4), dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32).copy()).to(dev)
    out = torch.zeros((blocks,), dtype=torch.int32, device=dev)
    _hip.call("lemoq_read_probe", _hip.ptr(src), n16 * 16, _hip.ptr(out), blocks, _hip.stream_of(dev))
    torch.cuda.synchronize()
    # contiguous shares of per16 elements (ceil(n16 / blocks) rounded up to 256);
    # a block folds the 32-bit word sums of its share with xor; blocks past the
    # last non-empty share are not launched (their entries stay 0)
    per16 = -(-n16 // blocks)
    per16 = -(-per16 // 256) * 256
    sums = words.astype(np.uint64).sum(axis=1).astype(np.uint32)
    want = np.zeros((blocks,), dtype=np.uint32)
    for b in range(blocks):
        s = sums[b * per16: (b + 1) * per16]
        want[b] = np.bitwise_xor.reduce(s) if s.size else 0
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want)
