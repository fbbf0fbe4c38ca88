"""GPU parity of the bit-exact quantisers: RTN w8 (weights) and KV-INT8 (cache).

Mirrors the reference's bit-exact gates (tests/test_kv_int8_gpu.py:63-111,
tests/test_kv_int8_read_gpu.py:116-162, tests/test_quant_oracle.py:107-163):
codes and scales must equal the oracle's bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import randn
from oracle import quant as oq

pytestmark = pytest.mark.gpu


def _rtn_case(w: torch.Tensor, group: int, dev):
    from lemoq.quant.rtn import quantize_rtn

    got = quantize_rtn(w.to(dev), bits=8, group_size=group)
    ref = oq.rtn_quantize_w8(w.numpy(), group)
    assert np.array_equal(got["codes_padded"].cpu().numpy(), ref["codes_padded"])
    assert np.array_equal(got["scale"].cpu().numpy(), ref["scale"])
    assert np.array_equal(got["scale_f16"].cpu().numpy().view(np.uint16), ref["scale_f16"].view(np.uint16))


@pytest.mark.parametrize("rows,cols,group", [(64, 2048, 128), (37, 500, 128), (16, 256, 32), (8, 1024, 64)])
def test_rtn_w8_bit_exact(rows, cols, group, dev):
    w = randn(rows, cols, seed=rows * cols, std=0.02)
    _rtn_case(w, group, dev)


def test_rtn_w8_edge_values(dev):
    w = randn(4, 256, seed=3, std=0.02)
    w[0, :128] = 0.0  # all-zero group -> scale 1.0, codes 0
    w[1, :128] = torch.linspace(-1.0, 1.0, 128)
    # exact half-way ties: absmax 127 -> scale 1.0; values k+0.5 round to even
    w[2, :128] = 0.5 + torch.arange(128, dtype=torch.float32) - 64.0
    w[2, 0] = 127.0
    w[3, 128:] = -3.0  # constant negative group: -127 everywhere
    _rtn_case(w, 128, dev)


def _kv_rows(h, d, seed):
    return randn(1, h, 1, d, seed=seed).to(torch.float16)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_kv_int8_write_bit_exact(seed, dev):
    from lemoq.kernels.kv_int8 import kv_int8_write

    k = _kv_rows(16, 128, seed)
    v = _kv_rows(16, 128, seed + 100) * 3
    if seed == 1:
        k[0, 3] = 0.0  # zero row -> scale 1.0, codes 0
    kc, ks, vc, vs = kv_int8_write(k.to(dev), v.to(dev))
    for got_c, got_s, x in ((kc, ks, k), (vc, vs, v)):
        rc, rs = oq.kv_quantize_rows(x.numpy())
        assert np.array_equal(got_c.cpu().numpy(), rc)
        assert np.array_equal(got_s.cpu().numpy().view(np.uint16), rs.view(np.uint16))


def test_kv_int8_half_way_ties_round_to_even(dev):
    from lemoq.kernels.kv_int8 import kv_int8_write

    # amax 127 -> s = 1.0, so x/s = x; fp16 can hold k + 0.5 exactly
    row = torch.tensor([127.0] + [(i % 40) - 20 + 0.5 for i in range(127)], dtype=torch.float16)
    k = row.reshape(1, 1, 1, 128).repeat(1, 2, 1, 1).contiguous()
    kc, ks, _, _ = kv_int8_write(k.to(dev), k.to(dev))
    rc, _ = oq.kv_quantize_rows(k.numpy())
    assert np.array_equal(kc.cpu().numpy(), rc)
    assert int(kc[0, 0, 0, 1]) == -20  # -19.5 -> -20 (even), not -19


def test_kv_int8_cache_write_scatter_and_untouched_slots(dev):
    from lemoq.kernels.kv_int8 import kv_int8_cache_write

    H, S, D = 16, 40, 128
    bufs = {
        "kc": torch.full((1, H, S, D), 7, dtype=torch.int8, device=dev),
        "ks": torch.full((1, H, S), 2.0, dtype=torch.float16, device=dev),
        "vc": torch.full((1, H, S, D), -7, dtype=torch.int8, device=dev),
        "vs": torch.full((1, H, S), 3.0, dtype=torch.float16, device=dev),
    }
    before = {k: v.clone() for k, v in bufs.items()}
    k = _kv_rows(H, D, 11).to(dev)
    v = _kv_rows(H, D, 12).to(dev)
    pos = torch.tensor([17], dtype=torch.int64, device=dev)
    kv_int8_cache_write(bufs, k, v, pos)
    rc, rs = oq.kv_quantize_rows(k.cpu().numpy())
    assert np.array_equal(bufs["kc"][0, :, 17].cpu().numpy(), rc[0, :, 0])
    assert np.array_equal(bufs["ks"][0, :, 17].cpu().numpy().view(np.uint16), rs[0, :, 0].view(np.uint16))
    for name in bufs:
        a, b = bufs[name].clone(), before[name]
        a[0, :, 17] = b[0, :, 17]
        assert torch.equal(a, b), name + ": a slot other than pos changed"


def test_kv_int8_bulk_quantize_matches_rows_and_tail(dev):
    from lemoq.kernels.kv_int8 import kv_int8_bulk_quantize

    x = randn(1, 4, 24, 128, seed=5).to(torch.float16)
    bufs = kv_int8_bulk_quantize(x.to(dev), (x * 2).to(dev), filled=17)
    rc, rs = oq.kv_quantize_rows(x[0, :, :17].numpy())
    assert np.array_equal(bufs["kc"][0, :, :17].cpu().numpy(), rc)
    assert np.array_equal(bufs["ks"][0, :, :17].cpu().numpy().view(np.uint16), rs.view(np.uint16))
    assert (bufs["kc"][0, :, 17:] == 0).all() and (bufs["ks"][0, :, 17:] == 1.0).all()


def test_kv_direct_write_bitwise(dev):
    from types import SimpleNamespace

    from lemoq.kernels.kv_direct import kv_direct_write

    H, S, D = 16, 12, 128
    layer = SimpleNamespace(
        keys=randn(1, H, S, D, seed=1).to(torch.float16).to(dev),
        values=randn(1, H, S, D, seed=2).to(torch.float16).to(dev),
    )
    keys0, values0 = layer.keys.clone(), layer.values.clone()
    k = randn(1, H, 1, D, seed=3).to(torch.float16).to(dev)
    v = randn(1, H, 1, D, seed=4).to(torch.float16).to(dev)
    kv_direct_write(layer, k, v, torch.tensor([5], dtype=torch.int64, device=dev))
    from oracle.ops import write_kv_slot

    write_kv_slot(keys0, values0, 5, k, v)
    assert torch.equal(layer.keys, keys0) and torch.equal(layer.values, values0)


def test_kv_direct_write_stream_sentinels_and_graph(dev):
    """The reference's tests/test_kv_direct_write.py:100-147 on the device: a
    stream of positions 0..7 over two layers against the slot contract, the
    sentinel tail and the neighbouring slots untouched, the buffers kept (same
    addresses), a position outside the cache writing nothing, and the write
    captured once in a graph and replayed with the position advanced on the
    device between replays."""
    from types import SimpleNamespace

    from lemoq.kernels.kv_direct import kv_direct_write
    from oracle.ops import write_kv_slot

    H, S, D, L = 16, 16, 128, 2
    sentinel = torch.tensor(-7.25, dtype=torch.float16)
    layers = [SimpleNamespace(keys=torch.full((1, H, S, D), float(sentinel), dtype=torch.float16, device=dev),
                              values=torch.full((1, H, S, D), float(sentinel), dtype=torch.float16, device=dev))
              for _ in range(L)]
    ref = [(l.keys.cpu(), l.values.cpu()) for l in layers]
    addrs = [(l.keys.data_ptr(), l.values.data_ptr()) for l in layers]
    pos = torch.zeros(1, dtype=torch.int64, device=dev)

    def kv(li, t):
        return (randn(1, H, 1, D, seed=100 * li + 2 * t).to(torch.float16),
                randn(1, H, 1, D, seed=100 * li + 2 * t + 1).to(torch.float16))

    for t in range(8):
        pos.fill_(t)
        for li, layer in enumerate(layers):
            k, v = kv(li, t)
            kv_direct_write(layer, k.to(dev), v.to(dev), pos)
            write_kv_slot(ref[li][0], ref[li][1], t, k, v)
        for li, layer in enumerate(layers):
            assert torch.equal(layer.keys.cpu(), ref[li][0]) and torch.equal(layer.values.cpu(), ref[li][1]), (li, t)
    for li, layer in enumerate(layers):
        assert (layer.keys.cpu()[:, :, 8:] == sentinel).all() and (layer.values.cpu()[:, :, 8:] == sentinel).all()
        assert (layer.keys.data_ptr(), layer.values.data_ptr()) == addrs[li]

    # a position outside [0, S) writes nothing
    before = layers[0].keys.clone(), layers[0].values.clone()
    k, v = kv(0, 99)
    for bad in (S, S + 5, -1):
        pos.fill_(bad)
        kv_direct_write(layers[0], k.to(dev), v.to(dev), pos)
    assert torch.equal(layers[0].keys, before[0]) and torch.equal(layers[0].values, before[1])

    # one captured write, replayed at positions 9..12 set on the device
    k, v = kv(1, 50)
    kd, vd = k.to(dev), v.to(dev)
    pos.fill_(9)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        kv_direct_write(layers[1], kd, vd, pos)  # warm-up outside the capture
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        kv_direct_write(layers[1], kd, vd, pos)
    for t in range(9, 13):
        pos.fill_(t)
        g.replay()
        torch.cuda.synchronize()
        write_kv_slot(ref[1][0], ref[1][1], t, k, v)
        assert torch.equal(layers[1].keys.cpu(), ref[1][0]) and torch.equal(layers[1].values.cpu(), ref[1][1]), t
    assert (layers[1].keys.cpu()[:, :, 13:] == sentinel).all() and (layers[1].keys.cpu()[:, :, 8] == sentinel).all()
