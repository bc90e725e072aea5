"""CPU tests of the dispatch module tabicl_mi355_mha (mirror of the reference's tabicl_tpu_mha.py):
layout algebra, impl choice, mask normalisation, merged RoPE, and install() on an upstream stand-in
(torch layouts only; the HIP routes are covered by tests/test_gpu_mha.py)."""
import numpy as np
import pytest
import torch

import upstream_stub as U
from oracle import attention as O

H, E = 8, 128


@pytest.fixture()
def mha(monkeypatch):
    import tabicl_mi355_mha as m
    monkeypatch.setattr(m, "_ANY_DEVICE", True)
    return m


@pytest.mark.parametrize("impl", ["std", "hxq", "hxk", "thl"])
@pytest.mark.parametrize("Lq,Lk", [(4, 104), (128, 300), (300, 128), (104, 104)])
def test_small_head_layouts_match_oracle(mha, impl, Lq, Lk):
    g = torch.Generator().manual_seed(Lq * 7 + Lk)
    q = torch.randn(3, Lq, E, generator=g) * 0.25
    k = torch.randn(3, Lk, E, generator=g)
    v = torch.randn(3, Lk, E, generator=g)
    bias = torch.zeros(3, Lk)
    bias[:, Lk - 5:] = float(torch.finfo(torch.float32).min)
    mask = bias.view(3, 1, 1, Lk)
    out = mha.small_head_attention(q, k, v, H, mask, impl)
    ref = O.attention_f64(q.numpy(), k.numpy(), v.numpy(), H, bias.double().numpy())
    np.testing.assert_allclose(out.double().numpy(), ref, atol=2e-5)


def test_pick_impl_rules(mha):
    assert mha.pick_impl("pk", 4, 104) == "std"
    assert mha.pick_impl("pk", 104, 104) == "pk"
    assert mha.pick_impl("hx", 128, 1024) == "hxq"
    assert mha.pick_impl("hx", 1024, 128) == "hxk"
    assert mha.pick_impl("", 128, 1024) == "hxq"
    assert mha.pick_impl("", 1024, 128) == "hxk"
    assert mha.pick_impl("", 104, 104) == "thl"
    assert mha.pick_impl("col1=pk,col2=pk,row=pk,cls=pk", 4, 104) == "pk"
    assert mha.pick_impl("row=std", 104, 104) == "std"
    with pytest.raises(ValueError):
        mha.small_head_attention(torch.zeros(1, 2, E), torch.zeros(1, 2, E), torch.zeros(1, 2, E), H, None, "nope")


def test_combined_mask_matches_oracle(mha):
    cases = [
        (torch.randn(3, 5), None),
        (None, torch.randn(2, 5)),
        (torch.randn(1, 1, 1, 5), torch.randn(2, 5)),
        (torch.zeros(3, 5, dtype=torch.bool), None),
        (torch.randn(4, 5), None),
        (None, torch.randn(1, 5)),
    ]
    for am, kp in cases:
        got = mha._combined_mask(am, kp, (2,), 8, 3, 5, torch.float32)
        want = O.combined_mask_ref(None if am is None else am.numpy(), None if kp is None else kp.numpy(),
                                   (2,), 8, 3, 5)
        if want is False or want is None:
            assert got is want
        else:
            np.testing.assert_allclose(got.numpy(), np.broadcast_to(want, got.shape), atol=0)


@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_merged_matches_oracle_and_head_split(mha, interleaved):
    rope = U.RopeStub(dim=16, theta=100000.0, interleaved=interleaved)
    x = torch.randn(2, 104, E, generator=torch.Generator().manual_seed(1))
    got = mha.rope_merged(rope, x, H)
    tabs = O.rope_tables_ref(rope.freqs.double().numpy(), 104, E, H, interleaved)
    np.testing.assert_allclose(got.double().numpy(), O.rope_merged_ref(x.numpy(), *tabs[:2], H, *tabs[2:]), atol=1e-5)
    split = rope.rotate_queries_or_keys(x.view(2, 104, H, 16).transpose(1, 2)).transpose(1, 2).reshape(2, 104, E)
    np.testing.assert_allclose(got.numpy(), split.numpy(), atol=1e-5)


@pytest.mark.parametrize("mode", ["std", "hxq", "hxk", "thl", "hx", "col1=hxq,col2=hxk,row=thl,cls=std"])
def test_install_layouts_match_upstream(mha, mode):
    g = torch.Generator().manual_seed(3)
    w, b, wo, bo = U.weights(E, 3)
    ref_mod, mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode=mode, proj="split")
    rope = U.RopeStub()
    x = torch.randn(2, 104, E, generator=g)
    kpm = torch.zeros(2, 104)
    kpm[:, 100:] = float(torch.finfo(torch.float32).min)
    ind = torch.randn(2, 16, E, generator=g)
    cases = [
        dict(query=x, key=x, value=x, rope=rope, key_padding_mask=kpm),  # row self attention with RoPE + mask
        dict(query=ind, key=x, value=x),  # column ISAB-1 (Lq < Lk)
        dict(query=x, key=ind, value=ind),  # column ISAB-2 (Lq > Lk)
        dict(query=x[:, :4], key=x, value=x, rope=rope),  # CLS queries
        dict(query=ind, key=x, value=x, ssmax_layer=U.SSMaxStub(H)),
    ]
    for kw in cases:
        q, k, v = kw.pop("query"), kw.pop("key"), kw.pop("value")
        want = U.call(ref_mod.multi_head_attention_forward, q, k, v, H, w, b, wo, bo, **kw)
        got = U.call(mod.multi_head_attention_forward, q, k, v, H, w, b, wo, bo, **kw)
        np.testing.assert_allclose(got.numpy(), want.numpy(), atol=2e-5)


def test_install_falls_back_for_cached_kv_and_wide_heads(mha):
    mod = U.make_module()
    calls = []
    orig = mod.multi_head_attention_forward

    def spy(*a, **k):
        calls.append(1)
        return orig(*a, **k)

    mod.multi_head_attention_forward = spy
    mha.install(mod, None, mode="std")
    w, b, wo, bo = U.weights(512, 5)
    x = torch.randn(1, 8, 512)
    U.call(mod.multi_head_attention_forward, x, x, x, 8, w, b, wo, bo)  # head dim 64 > 32: upstream
    assert calls == [1]
    assert mha.install(mod, None, mode="std") is True  # idempotent
    assert mha.install(U.make_module(), None, mode="off") is False
