"""The GPU tests' parity bars (tests/parity.py) discriminate at the BASELINE configs' key counts.

On the CPU, with the oracle's own output standing in for a kernel's: the result rounded to bf16 (what
a correct bf16 kernel returns) passes both bars, while the two faults a long-key regression would
show -- the last quarter of the keys dropped (a split-merge or tile-index bug past some key count),
and the output scaled by 1.5 (a wrong row sum) -- fail. In the flat N(0,1) cases every output is
small (max|ref| < 0.1), so these faults move outputs by about the absolute 2e-2 bar or less; the
scale-aware bar rejects them. Sharpened queries (q x 4) make outputs O(1), where both bars reject
both faults.

Shapes: C4 (d = 64, 45,000 cached keys, one (estimator, head) slice, 64 query rows) and C3 ISAB-1
(d = 16, 128 inducing queries over 45,000 valid rows, 8 heads).
"""
import numpy as np
import pytest
import torch

from oracle import attention as O
from parity import ABS, passes

BF = torch.bfloat16


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(BF).double().numpy()


def _c4(qscale):
    g = torch.Generator().manual_seed(31)
    q = (torch.randn(1, 1, 64, 64, generator=g) * qscale).to(BF)
    k = torch.randn(1, 1, 45000, 64, generator=g).to(BF)
    v = torch.randn(1, 1, 45000, 64, generator=g).to(BF)
    ref = O.splash_sdpa_ref(q, k, v, 45000)
    dropped = O.splash_sdpa_ref(q, k, v, 45000 * 3 // 4)
    return ref, dropped


def _c3_isab1(qscale):
    g = torch.Generator().manual_seed(32)
    q = (torch.randn(1, 128, 128, generator=g) * 0.25 * qscale).to(BF)
    kv = torch.randn(1, 45000, 256, generator=g).to(BF)
    ref = O.hxq_ref(q, kv, np.array([45000]), 8)
    dropped = O.hxq_ref(q, kv, np.array([45000 * 3 // 4]), 8)
    return ref, dropped


@pytest.mark.parametrize("case", [_c4, _c3_isab1], ids=["c4_icl_45k", "c3_isab1_45k"])
@pytest.mark.parametrize("qscale", [1.0, 4.0], ids=["flat", "sharp"])
def test_bars_reject_long_key_faults(case, qscale):
    ref, dropped = case(qscale)
    assert passes(_bf16(ref), ref, BF), "a correctly rounded bf16 result must pass"
    assert not passes(_bf16(dropped), ref, BF), "last quarter of the keys dropped must fail"
    assert not passes(_bf16(ref * 1.5), ref, BF), "output scaled by 1.5 must fail"
    if qscale == 1.0:
        # why the scale-aware bar is needed: the flat case's outputs are tiny, so the absolute bar alone
        # accepts most of the fault (every output moves by at most half of max|ref|)
        assert float(np.abs(ref).max()) < 0.1
        assert float(np.abs(ref * 1.5 - ref).max()) <= 2.5 * ABS[BF]
    else:
        assert float(np.abs(ref).max()) > 0.3


def test_bars_fp32_mode():
    # fp32-input validation mode: 1e-4 absolute and 1e-3 x max|ref|; an fp32-rounded result passes,
    # the dropped-keys fault fails
    g = torch.Generator().manual_seed(33)
    q = torch.randn(1, 1, 32, 64, generator=g)
    k = torch.randn(1, 1, 20000, 64, generator=g)
    v = torch.randn(1, 1, 20000, 64, generator=g)
    ref = O.splash_sdpa_ref(q, k, v)
    f32 = ref.astype(np.float32).astype(np.float64)
    assert passes(f32, ref, torch.float32)
    assert not passes(O.splash_sdpa_ref(q, k, v, 15000), ref, torch.float32)
    assert not passes(ref * 1.01, ref, torch.float32)
