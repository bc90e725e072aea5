"""GPU parity of the folded first-ISAB attention (hxf_attention, folded_mab1) against the CPU oracle.

Mirrors the reference's check (scripts/tests/test_pallas_attn.py:289-318, shapes at :367-369): the
folded path against the unfolded fp32 attention on the same projections, plus the kernel alone
(softmax(qf x^T) x, head dim 128) with shared and per-batch folded queries, ragged and empty valid
lengths. Bars (tests/parity.py): max abs error <= 1e-4 for fp32 inputs, <= 2e-2 for bf16, and <= 1e-3
(fp32) / 2e-2 (bf16) times max |ref|.
"""
import pytest
import torch

from oracle import attention as O
from parity import check

H = 8
E = 128

pytestmark = pytest.mark.gpu


def _attn():
    import tabicl_mi355_attn as pk
    return pk


@pytest.mark.parametrize("name,B,hq,Lk,valid,dtype,shared", [
    ("small_fp32_shared", 4, 1024, 4096, 3000, torch.float32, True),
    ("small_bf16_shared", 4, 1024, 4096, 3000, torch.bfloat16, True),
    ("odd_fp32_per_batch", 3, 64, 777, 500, torch.float32, False),
    ("odd_bf16_per_batch", 3, 200, 1000, 999, torch.bfloat16, False),
])
def test_hxf_kernel(dev, name, B, hq, Lk, valid, dtype, shared):
    pk = _attn()
    g = torch.Generator().manual_seed(40)
    qf = (torch.randn(1 if shared else B, hq, E, generator=g) * 0.05).to(dtype)
    x = torch.randn(B, Lk, E, generator=g).to(dtype)
    print(f"[hxf] {name}", flush=True)
    out = pk.hxf_attention(qf.to(dev) if not shared else qf[0].to(dev), x.to(dev), torch.tensor(valid).to(dev))
    assert out.shape == (B, hq, E)
    check(out, O.hxf_ref(qf, x, valid), dtype, "hxf_kernel")


def test_hxf_ragged_and_empty_valid(dev):
    pk = _attn()
    g = torch.Generator().manual_seed(41)
    B, hq, Lk = 4, 96, 700
    qf = (torch.randn(1, hq, E, generator=g) * 0.05).to(torch.bfloat16)
    x = torch.randn(B, Lk, E, generator=g).to(torch.bfloat16)
    valid = torch.tensor([700, 65, 0, 1], dtype=torch.int32)
    out = pk.hxf_attention(qf.to(dev), x.to(dev), valid.to(dev))
    assert torch.isfinite(out.float()).all()
    check(out, O.hxf_ref(qf, x, valid.numpy()), torch.bfloat16, "hxf_ragged_and_empty_valid")
    assert float(out[2].abs().max()) == 0.0


def _mab1_inputs(B, Lq, Lk, seed):
    g = torch.Generator().manual_seed(seed)
    ind = torch.randn(Lq, E, generator=g) * 0.5
    x = torch.randn(B, Lk, E, generator=g)
    W = torch.randn(3 * E, E, generator=g) * E ** -0.5
    b = torch.randn(3 * E, generator=g) * 0.1
    return ind, x, W, b


@pytest.mark.parametrize("name,B,Lq,Lk,valid,sub", [
    ("small", 4, 128, 4096, 3000, None),
    ("infer_tile54", 54, 128, 53248, 45000, (0, 53)),   # oracle on two batch elements
])
@pytest.mark.parametrize("qkind", ["expanded", "per_batch"])
def test_folded_mab1_vs_unfolded(dev, name, B, Lq, Lk, valid, sub, qkind):
    import tabicl_mi355_mha as mha
    pk = _attn()
    ind, x, W, b = _mab1_inputs(B, Lq, Lk, 42)
    q = ind.to(dev).expand(B, Lq, E)
    if qkind == "per_batch":
        q = q.contiguous()
    print(f"[folded_mab1] {name} {qkind}", flush=True)
    with torch.no_grad():
        o = mha.folded_mab1(q, x.to(dev), torch.tensor(valid).to(dev), H, W.to(dev), b.to(dev), None, None, pk=pk)
    assert o is not None and o.shape == (B, Lq, E)
    idx = list(range(B)) if sub is None else list(sub)
    ref = O.folded_mab1_ref(ind, x[idx], valid, H, W, b)
    check(o[idx], ref, torch.float32, "folded_mab1_vs_unfolded")
