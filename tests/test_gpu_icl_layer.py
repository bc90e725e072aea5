"""GPU parity of the ICL cache's projection paths: IclKVCache.append_projected (train rows and the
packed in-projection straight into the [estimator, block, head, row, d] cache) and
IclKVCache.attention_layer (Q projection, attention over the cache, out-projection).

Layout: the cached rows equal the same torch GEMM's K|V output split into heads by hand (bit-exact).
Math: float64 restatements of the projections (x W^T + b with W_q, W_k, W_v the thirds of the packed
[3 width, width] in-projection, results/tpu_patch.diff:308-310) around oracle.attention.splash_sdpa_ref,
to <= 2e-2 abs for bf16 (the attention kernel's bar; the projections add bf16 rounding of q, k, v).
"""
import numpy as np
import pytest
import torch

from oracle import attention as O

pytestmark = pytest.mark.gpu

H, D = 8, 64
W = H * D


def _icl():
    import tabicl_mi355_icl as icl
    return icl


def _weights(g):
    w_in = (torch.randn(3 * W, W, generator=g) * W ** -0.5).to(torch.bfloat16)
    b_in = (torch.randn(3 * W, generator=g) * 0.1).to(torch.bfloat16)
    w_out = (torch.randn(W, W, generator=g) * W ** -0.5).to(torch.bfloat16)
    b_out = (torch.randn(W, generator=g) * 0.1).to(torch.bfloat16)
    return w_in, b_in, w_out, b_out


def _proj64(x, w, b):
    return x.double().numpy() @ w.double().numpy().T + b.double().numpy()


def test_append_projected_layout_and_math(dev):
    icl = _icl()
    g = torch.Generator().manual_seed(40)
    E, NB, cap, T, row0 = 2, 3, 512, 300, 40
    x = torch.randn(E, T, W, generator=g).to(torch.bfloat16)
    w_in, b_in, _, _ = _weights(g)
    cache = icl.IclKVCache(E, NB, H, cap, D, torch.bfloat16, dev)
    print("[append_projected] layout", flush=True)
    xd, wd, bd = x.to(dev), w_in.to(dev), b_in.to(dev)
    cache.append_projected(1, xd, wd, bd, row0=row0)
    kv = torch.nn.functional.linear(xd, wd[W:], bd[W:]).view(E, T, 2, H, D)
    got_k = cache.keys[:, 1, :, row0:row0 + T]
    got_v = cache.values[:, 1, :, row0:row0 + T]
    assert torch.equal(got_k, kv[:, :, 0].permute(0, 2, 1, 3))
    assert torch.equal(got_v, kv[:, :, 1].permute(0, 2, 1, 3))
    # the K and V thirds of the packed weight, head h = dims 64 h .. 64 h + 63
    k64 = _proj64(x, w_in[W:2 * W], b_in[W:2 * W]).reshape(E, T, H, D).transpose(0, 2, 1, 3)
    v64 = _proj64(x, w_in[2 * W:], b_in[2 * W:]).reshape(E, T, H, D).transpose(0, 2, 1, 3)
    assert np.abs(got_k.double().cpu().numpy() - k64).max() <= 2e-2 * max(1.0, np.abs(k64).max())
    assert np.abs(got_v.double().cpu().numpy() - v64).max() <= 2e-2 * max(1.0, np.abs(v64).max())


def test_append_projected_rejects_bad_shapes(dev):
    icl = _icl()
    cache = icl.IclKVCache(1, 1, H, 64, D, torch.bfloat16, dev)
    x = torch.zeros(1, 8, W, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        cache.append_projected(0, x, torch.zeros(2 * W, W, dtype=torch.bfloat16, device=dev))
    with pytest.raises(ValueError):
        cache.append_projected(0, x[:, :, :100], torch.zeros(3 * W, W, dtype=torch.bfloat16, device=dev))


@pytest.mark.parametrize("valid", [250, None])
def test_attention_layer(dev, valid):
    icl = _icl()
    g = torch.Generator().manual_seed(41)
    E, NB, cap, T, Tq = 2, 2, 320, 300, 100
    xtr = torch.randn(E, T, W, generator=g).to(torch.bfloat16)
    xq = torch.randn(E, Tq, W, generator=g).to(torch.bfloat16)
    w_in, b_in, w_out, b_out = _weights(g)
    cache = icl.IclKVCache(E, NB, H, cap, D, torch.bfloat16, dev)
    cache.append_projected(0, xtr.to(dev), w_in.to(dev), b_in.to(dev))
    print(f"[attention_layer] valid={valid}", flush=True)
    vl = T if valid is None else valid
    out = cache.attention_layer(0, xq.to(dev), w_in.to(dev), b_in.to(dev), w_out.to(dev), b_out.to(dev),
                                valid_kv_len=vl, q_transform=lambda q: q * 1.25)
    assert out.shape == (E, Tq, W) and out.dtype == torch.bfloat16
    # float64 restatement; q, k, v rounded to bf16 as the layer hands them to the kernel
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16).double().numpy()  # noqa: E731
    q = bf(_proj64(xq, w_in[:W], b_in[:W]).reshape(E, Tq, H, D).transpose(0, 2, 1, 3) * 1.25)
    k = bf(_proj64(xtr, w_in[W:2 * W], b_in[W:2 * W]).reshape(E, T, H, D).transpose(0, 2, 1, 3))
    v = bf(_proj64(xtr, w_in[2 * W:], b_in[2 * W:]).reshape(E, T, H, D).transpose(0, 2, 1, 3))
    o = O.splash_sdpa_ref(q, k, v, np.array([vl]))
    o = bf(o.transpose(0, 2, 1, 3).reshape(E, Tq, W))
    ref = o @ w_out.double().numpy().T + b_out.double().numpy()
    err = float(np.abs(out.double().cpu().numpy() - ref).max())
    print(f"  max abs err {err:.3e} (ref max {np.abs(ref).max():.3e})", flush=True)
    assert err <= 2e-2 * max(1.0, float(np.abs(ref).max()))
