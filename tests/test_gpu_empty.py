"""Zero-size calls through the public ops: an empty batch or no query rows launches nothing and returns an
empty output of the right shape and dtype (the C ABI returns before any launch for B = 0 or Lq = 0; a grid of
zero workgroups would be a launch error)."""
import pytest
import torch

pytestmark = pytest.mark.gpu

H, E = 8, 128


def _pk():
    import tabicl_mi355_attn as pk
    return pk


@pytest.mark.parametrize("B,Lq", [(0, 40), (3, 0)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_smallhead_empty(dev, B, Lq, dtype):
    pk = _pk()
    Lk = 100
    q = torch.randn(B, Lq, E, device=dev).to(dtype)
    k = torch.randn(B, Lk, E, device=dev).to(dtype)
    v = torch.randn(B, Lk, E, device=dev).to(dtype)
    kv = torch.randn(B, Lk, 2 * E, device=dev).to(dtype)
    print(f"[empty] B={B} Lq={Lq} {dtype}", flush=True)
    out = pk.hx_attention(q, k, v, H)
    assert out.shape == (B, Lq, E) and out.dtype == dtype
    out = pk.hxq_attention(q, kv, torch.tensor(50, dtype=torch.int32, device=dev), H)
    assert out.shape == (B, Lq, E) and out.dtype == dtype
    out = pk.pk_cross_attention(q, kv, H, None, None, 0.25)
    assert out.shape == (B, Lq, E) and out.dtype == dtype
    qkv = torch.randn(B, Lq, 3 * E, device=dev).to(dtype)
    out = pk.pk_self_attention(qkv, H, None, None, 0.25)
    assert out.shape == (B, Lq, E) and out.dtype == dtype
    torch.cuda.synchronize()


@pytest.mark.parametrize("N,Tq", [(0, 300), (2, 0)])
def test_icl_empty(dev, N, Tq):
    import tabicl_mi355_icl as icl
    Tkv = 500
    q = torch.randn(N, H, Tq, 64, device=dev).to(torch.bfloat16)
    k = torch.randn(N, H, Tkv, 64, device=dev).to(torch.bfloat16)
    v = torch.randn(N, H, Tkv, 64, device=dev).to(torch.bfloat16)
    print(f"[empty icl] N={N} Tq={Tq}", flush=True)
    out = icl.icl_sdpa(q, k, v, 300)
    assert out.shape == q.shape and out.dtype == q.dtype
    out = icl.icl_sdpa(q, k, v, torch.full((max(N, 1),), 200, dtype=torch.int32, device=dev)[:N] if N else None)
    assert out.shape == q.shape
    torch.cuda.synchronize()
