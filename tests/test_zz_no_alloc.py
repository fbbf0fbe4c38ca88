"""The allocation-free split-K GEMM (lemoq_gemm_f16_splitk_noalloc) against the
workspace form it mirrors (lemoq_gemm_f16_splitk), through the C-ABI.

It runs the same kernels with the split partials in the library's fixed device
array instead of a caller workspace, so its outputs must equal the workspace
form's bit for bit: on two calls in a row, the second one smaller (the array
keeps the first call's contents, which the second must overwrite wherever it
reads), and on the single-split path, which needs no partials.  A request
larger than the array is refused before anything is launched.
"""

from __future__ import annotations

import pytest
import torch

from helpers import randn

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 4 << 20
CAPACITY = -5


def _both(hip, dev, m, n, k, splits, seed):
    P, st = hip.ptr, hip.stream_of(dev)
    w = randn(n, k, seed=seed, std=0.05).to(torch.float16).to(dev)
    x = randn(m, k, seed=seed + 1).to(torch.float16).to(dev)
    ws = torch.full((splits, m, n), float("nan"), dtype=torch.float32, device=dev)
    y_ref = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    y = torch.full((m, n), float("nan"), dtype=torch.float16, device=dev)
    hip.call("lemoq_gemm_f16_splitk", P(x), m, k, k, P(w), n, P(y_ref), n, splits, P(ws), st)
    hip.call("lemoq_gemm_f16_splitk_noalloc", P(x), m, k, k, P(w), n, P(y), n, splits, st)
    torch.cuda.synchronize()
    return y_ref.cpu(), y.cpu()


def test_noalloc_splitk_equals_workspace_form_on_two_calls(dev):
    from lemoq import _hip

    cases = [(1024, 64, 2048, 8, 11), (37, 64, 2048, 4, 12)]  # the second call smaller
    for m, n, k, splits, seed in cases:
        print("case: noalloc split-K m=%d n=%d k=%d splits=%d" % (m, n, k, splits), flush=True)
        ref, got = _both(_hip, dev, m, n, k, splits, seed)
        assert not torch.isnan(got.float()).any()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (m, n, k, splits)


def test_noalloc_single_split_and_capacity(dev):
    from lemoq import _hip

    print("case: noalloc split-K single split; capacity refusal", flush=True)
    ref, got = _both(_hip, dev, 5, 64, 512, 1, 13)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    lib = _hip.load()
    # splits * M * N one past the array: refused before launching (no device buffer is touched)
    m, n, splits = SCRATCH_FLOATS // (64 * 8) + 1, 64, 8
    fake = 1 << 20
    assert int(lib.lemoq_gemm_f16_splitk_noalloc(fake, m, 2048, 2048, fake, n, fake, n, splits, None)) == CAPACITY
    assert int(lib.lemoq_gemm_f16_splitk_noalloc(fake, 4, 2048, 2048, fake, n, None, n, 2, None)) == -1
