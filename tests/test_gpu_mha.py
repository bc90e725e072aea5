"""GPU tests of the dispatch wrapper's HIP routes (PACKED -> pk_self / pk_cross, HXQ -> hxq, cached
ICL -> icl_sdpa) against the upstream stand-in running plain torch math on the same GPU.
Bar: max abs error <= 1e-4 with fp32 activations, <= 3e-2 with bf16 (projections rounded in bf16
on both sides, attention inputs differ by one bf16 rounding)."""
import pytest
import torch

import upstream_stub as U

pytestmark = pytest.mark.gpu
H, E = 8, 128


@pytest.fixture()
def mha(monkeypatch):
    import tabicl_mi355_mha as m
    monkeypatch.setattr(m, "_PACKED", True)
    monkeypatch.setattr(m, "_HXQ", True)
    return m


def _routes(monkeypatch, m):
    import tabicl_mi355_attn as pk
    import tabicl_mi355_icl as icl
    seen = []
    for mod, name in ((pk, "pk_self_attention"), (pk, "pk_cross_attention"), (pk, "hxq_attention"),
                      (pk, "hx_attention"), (icl, "icl_sdpa")):
        fn = getattr(mod, name)

        def wrap(*a, _fn=fn, _name=name, **k):
            seen.append(_name)
            return _fn(*a, **k)

        monkeypatch.setattr(mod, name, wrap)
    return seen


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 3e-2)])
def test_packed_and_hxq_routes(dev, mha, monkeypatch, dtype, tol):
    seen = _routes(monkeypatch, mha)
    g = torch.Generator().manual_seed(11)
    w, b, wo, bo = U.weights(E, 11, dev, dtype)
    ref_mod, mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="col1=pk,col2=pk,row=pk,cls=pk", proj="views")
    rope = U.RopeStub()
    x = torch.randn(4, 104, E, generator=g).to(dev, dtype)
    kpm = torch.zeros(4, 104)
    kpm[:, 101:] = float(torch.finfo(torch.float32).min)
    kpm = kpm.to(dev, dtype)
    ind = torch.randn(4, 128, E, generator=g).to(dev, dtype)
    rows = torch.randn(4, 2000, E, generator=g).to(dev, dtype)
    cases = [
        ("pk_self_attention", dict(query=x, key=x, value=x, rope=rope, key_padding_mask=kpm)),
        ("pk_cross_attention", dict(query=x[:, :4], key=x, value=x, rope=rope, key_padding_mask=kpm)),
        ("pk_cross_attention", dict(query=rows, key=ind, value=ind)),
        ("hxq_attention", dict(query=ind, key=rows, value=rows, ssmax_layer=U.SSMaxStub(H),
                               valid_kv_len=torch.tensor(1500, device=dev), src_len_override=torch.tensor(1500))),
    ]
    with torch.no_grad():
        for route, kw in cases:
            q, k, v = kw.pop("query"), kw.pop("key"), kw.pop("value")
            seen.clear()
            want = U.call(ref_mod.multi_head_attention_forward, q, k, v, H, w, b, wo, bo, **kw)
            got = U.call(mod.multi_head_attention_forward, q, k, v, H, w, b, wo, bo, **kw)
            assert route in seen, (route, seen)
            err = float((got.float() - want.float()).abs().max())
            assert err <= tol, (route, err)


def test_cached_icl_route(dev, mha, monkeypatch):
    seen = _routes(monkeypatch, mha)
    g = torch.Generator().manual_seed(12)
    Ew, nh, T, Tq = 512, 8, 20000, 300
    w, b, wo, bo = U.weights(Ew, 12, dev, torch.float32)
    ref_mod, mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="pk")
    kc = torch.randn(2, nh, T, 64, generator=g).to(dev, torch.bfloat16)
    vc = torch.randn(2, nh, T, 64, generator=g).to(dev, torch.bfloat16)
    q = torch.randn(2, Tq, Ew, generator=g).to(dev, torch.bfloat16)
    valid = torch.tensor(18000, device=dev)
    with torch.no_grad():
        kw = dict(cached_kv=U.KVEntry(kc, vc), valid_kv_len=valid, src_len_override=valid,
                  ssmax_layer=U.SSMaxStub(nh))
        want = U.call(ref_mod.multi_head_attention_forward, q, None, None, nh, w.bfloat16(), b.bfloat16(),
                      wo.bfloat16(), bo.bfloat16(), **kw)
        got = U.call(mod.multi_head_attention_forward, q, None, None, nh, w.bfloat16(), b.bfloat16(),
                     wo.bfloat16(), bo.bfloat16(), **kw)
    assert "icl_sdpa" in seen
    err = float((got.float() - want.float()).abs().max())
    assert err <= 3e-2, err
