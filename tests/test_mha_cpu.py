"""CPU tests of the dispatch module tabicl_mi355_mha: mode rules, mask normalisation (against an
element-by-element evaluation of upstream's broadcast rules), the torch small-head implementation,
the ICL hook's mask extraction, and the whole routing of install() driven through a restatement of
upstream's MultiheadAttentionBlock (tests/upstream_stub.block_attention) with torch "fake kernels"
in place of the HIP ops (the reference's own mock-backend pattern, scripts/tests/test_fold_cpu.py:25-70).
The HIP kernels themselves are covered by the -m gpu tests."""
import itertools
import types

import numpy as np
import pytest
import torch

import upstream_stub as U
from oracle import attention as O

H, E = 8, 128


@pytest.fixture()
def mha():
    import tabicl_mi355_mha as m
    return m


# ---------------------------------------------------------------------------------------------
# mode rules
# ---------------------------------------------------------------------------------------------
def test_pick_impl_rules(mha):
    assert mha.pick_impl("pk", 4, 104) == "std"  # CLS-sized query sets stay on torch in mode pk
    assert mha.pick_impl("pk", 17, 104) == "pk"
    assert mha.pick_impl("pk", 104, 104) == "pk"
    assert mha.pick_impl("hx", 128, 1024) == "hxq"
    assert mha.pick_impl("hx", 1024, 128) == "hxk"
    assert mha.pick_impl("hx", 104, 104) == "hxq"
    assert mha.pick_impl("", 128, 1024) == "hxq"
    assert mha.pick_impl("auto", 1024, 128) == "hxk"
    assert mha.pick_impl("", 104, 104) == "thl"
    assert mha.pick_impl("", 16, 104) == "hxq"  # cls rule
    assert mha.pick_impl("col1=pk,col2=pk,row=pk,cls=pk", 4, 104) == "pk"
    assert mha.pick_impl("row=std", 104, 104) == "std"
    assert mha.pick_impl("row=std", 128, 1024) == "hxq"  # unlisted roles keep their defaults
    for single in ("std", "hxq", "hxk", "thl"):
        assert mha.pick_impl(single, 3, 900) == single


# ---------------------------------------------------------------------------------------------
# masks: every supported form against an element-by-element evaluation of upstream's rules
# ---------------------------------------------------------------------------------------------
def _brute_mask(am, kp, batch_shape, nh, Lq, Lk):
    """Expected additive mask entry at every (*batch, head, i, j) under upstream's documented forms
    (results/tpu_patch.diff:327-366): a 2-D attn_mask is [Lq, Lk] for every batch element and head; a
    (1, 1, 1, Lk) attn_mask with a batch rank other than 1 is one key row; an attn_mask of full rank
    broadcasts dim by dim; a key_padding_mask is one key row per batch element (dims of size 1
    broadcast) or a single (1, Lk) row."""
    nb = len(batch_shape)
    full = (*batch_shape, nh, Lq, Lk)
    out = np.zeros(full, np.float64)
    for idx in itertools.product(*[range(n) for n in full]):
        i, j = idx[-2], idx[-1]
        val = 0.0
        if am is not None:
            if am.ndim == 2:
                val += am[i, j]
            elif am.ndim == 4 and nb != 1:
                val += am[0, 0, 0, j]
            else:
                val += am[tuple(0 if am.shape[d] == 1 else idx[d] for d in range(am.ndim))]
        if kp is not None:
            if kp.shape == (1, Lk) and (kp.ndim != nb + 1):
                val += kp[0, j]
            else:
                val += kp[tuple(0 if kp.shape[d] == 1 else idx[d] for d in range(nb)) + (j,)]
        out[idx] = val
    return out


_MASK_CASES = [
    # (name, attn_mask shape, key_padding_mask shape, batch_shape)
    ("2d", (3, 5), None, (2,)),
    ("2d_batch0", (3, 5), None, ()),
    ("4d_key_row_nb2", (1, 1, 1, 5), None, (2, 3)),
    ("4d_key_row_nb0", (1, 1, 1, 5), None, ()),
    ("full_rank_exact", (2, 8, 3, 5), None, (2,)),
    ("full_rank_broadcast", (2, 1, 3, 1), None, (2,)),
    ("full_rank_nb2", (1, 3, 8, 1, 5), None, (2, 3)),
    ("kpm_rows", None, (2, 5), (2,)),
    ("kpm_shared_row_nb1", None, (1, 5), (2,)),
    ("kpm_shared_row_nb2", None, (1, 5), (2, 3)),
    ("kpm_rank_nb2", None, (2, 1, 5), (2, 3)),
    ("both", (1, 1, 1, 5), (2, 5), (2,)),
    ("both_full", (2, 8, 3, 5), (1, 5), (2,)),
]


@pytest.mark.parametrize("name,am_shape,kp_shape,batch", _MASK_CASES, ids=[c[0] for c in _MASK_CASES])
def test_combined_mask_matches_upstream_rules(mha, name, am_shape, kp_shape, batch):
    g = torch.Generator().manual_seed(len(name))
    am = None if am_shape is None else torch.randn(am_shape, generator=g)
    kp = None if kp_shape is None else torch.randn(kp_shape, generator=g)
    want = _brute_mask(None if am is None else am.double().numpy(), None if kp is None else kp.double().numpy(),
                       batch, 8, 3, 5)
    got = mha._combined_mask(am, kp, batch, 8, 3, 5, torch.float32)
    np.testing.assert_allclose(torch.broadcast_to(got, want.shape).double().numpy(), want, atol=1e-6)
    ref = O.combined_mask_ref(None if am is None else am.numpy(), None if kp is None else kp.numpy(), batch, 8, 3, 5)
    np.testing.assert_allclose(np.broadcast_to(ref, want.shape), want, atol=1e-6)


@pytest.mark.parametrize("am,kp,batch", [
    (torch.zeros(3, 5, dtype=torch.bool), None, (2,)),  # boolean masks go to upstream
    (None, torch.zeros(2, 5, dtype=torch.bool), (2,)),
    (torch.zeros(4, 5), None, (2,)),  # 2-D of the wrong shape
    (torch.zeros(3, 8, 3, 5), None, (2,)),  # batch dim 3 vs 2
    (torch.zeros(1, 5, 1), None, (2,)),  # rank 3 with batch rank 1
    (None, torch.zeros(3, 5), (2,)),  # key padding rows for 3 batch elements, batch 2
    (None, torch.zeros(2, 4), (2,)),  # wrong key count
])
def test_combined_mask_refusals(mha, am, kp, batch):
    assert mha._combined_mask(am, kp, batch, 8, 3, 5, torch.float32) is False
    assert O.combined_mask_ref(None if am is None else am.numpy(), None if kp is None else kp.numpy(),
                               batch, 8, 3, 5) is False


def test_combined_mask_sums_in_query_dtype(mha):
    # upstream casts the summed mask to the query dtype (diff:370-371): finfo(float32).min is -inf in bf16
    kp = torch.zeros(2, 5)
    kp[:, 3:] = torch.finfo(torch.float32).min
    got = mha._combined_mask(None, kp, (2,), 8, 3, 5, torch.bfloat16)
    assert got.dtype == torch.float32 and torch.isinf(got[..., 3:]).all() and (got[..., :3] == 0).all()
    assert mha._combined_mask(None, None, (2,), 8, 3, 5, torch.float32) is None


def test_key_only_and_hook_bias(mha):
    m = torch.randn(2, 1, 1, 7)
    assert mha._key_only(m, 7).shape == (2, 7)
    assert mha._key_only(torch.randn(2, 8, 1, 7), 7) is False
    assert mha._key_only(torch.randn(2, 1, 3, 7), 7) is False
    q = torch.zeros(2, 3, 8, 10, 64)  # lead (2, 3)
    assert mha._hook_bias(None, q, 7) is None
    assert tuple(mha._hook_bias(torch.zeros(1, 1, 1, 1, 7), q, 7).shape) == (1, 7)
    b = mha._hook_bias(torch.arange(3.0).view(1, 3, 1, 1, 1).expand(1, 3, 1, 1, 7).contiguous(), q, 7)
    assert tuple(b.shape) == (6, 7) and torch.equal(b[:, 0], torch.tensor([0., 1, 2, 0, 1, 2]))
    assert mha._hook_bias(torch.zeros(2, 3, 8, 1, 7), q, 7) is False  # per head
    assert mha._hook_bias(torch.zeros(2, 3, 1, 10, 7), q, 7) is False  # per query
    assert mha._hook_bias(torch.zeros(1, 1, 1, 7, dtype=torch.bool), q, 7) is False
    assert mha._hook_bias(torch.zeros(4, 1, 1, 7), q, 7) is False  # 4 rows for a (2, 3) batch


@pytest.mark.parametrize("impl", ["std", "hxq", "hxk", "thl", "pk"])
@pytest.mark.parametrize("Lq,Lk", [(4, 104), (128, 300), (300, 128)])
def test_small_head_attention_matches_oracle(mha, impl, Lq, Lk):
    # on CPU tensors "pk" falls back to the torch form (the HIP kernel needs GPU tensors)
    g = torch.Generator().manual_seed(Lq * 7 + Lk)
    q = torch.randn(3, Lq, E, generator=g) * 0.25
    k = torch.randn(3, Lk, E, generator=g)
    v = torch.randn(3, Lk, E, generator=g)
    bias = torch.zeros(3, Lk)
    bias[:, Lk - 5:] = float(torch.finfo(torch.float32).min)
    out = mha.small_head_attention(q, k, v, H, bias.view(3, 1, 1, Lk), impl)
    np.testing.assert_allclose(out.double().numpy(), O.attention_f64(q.numpy(), k.numpy(), v.numpy(), H,
                                                                     bias.double().numpy()), atol=2e-5)
    with pytest.raises(ValueError):
        mha.small_head_attention(q, k, v, H, None, "nope")


def test_in_projection_forms_agree(mha):
    g = torch.Generator().manual_seed(2)
    w, b, _, _ = U.weights(E, 2)
    x, y = torch.randn(2, 7, E, generator=g), torch.randn(2, 9, E, generator=g)
    for query, key, value in ((x, x, x), (x, y, y), (x, y, torch.randn(2, 9, E, generator=g))):
        want = torch.nn.functional._in_projection_packed(query, key, value, w, b)
        for proj in ("packed", "split", "views"):
            for a, c in zip(mha.in_projection(query, key, value, w, b, proj), want):
                torch.testing.assert_close(a, c, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------------------------------------
# routing, end to end through the upstream block, with fake kernels
# ---------------------------------------------------------------------------------------------
def _t(a, like):
    return torch.from_numpy(np.ascontiguousarray(a)).to(like.dtype)


def _fake_pk():
    """The tabicl_mi355_attn surface the router calls, in float64 numpy (the oracle)."""
    def _bias_rows(kb, B, Lk):
        return None if kb is None else np.broadcast_to(O._f64(kb).reshape(-1, Lk), (B, Lk))

    def hx_attention(q, k, v, h, key_bias=None):
        lead, Lq, Lk = q.shape[:-2], q.shape[-2], k.shape[-2]
        q3, k3, v3 = q.reshape(-1, Lq, E), k.reshape(-1, Lk, E), v.reshape(-1, Lk, E)
        out = O.attention_f64(O._f64(q3), O._f64(k3), O._f64(v3), h, _bias_rows(key_bias, q3.shape[0], Lk))
        return _t(out, q).reshape(*lead, Lq, E)

    def hxq_attention(q, kv, valid_len, h, key_bias=None):
        Lq, Lk = q.shape[-2], kv.shape[-2]
        kv3 = kv.reshape(-1, Lk, 2 * E)
        q3 = q.reshape(-1, Lq, E).expand(kv3.shape[0], Lq, E)
        valid = None if valid_len is None else O._f64(torch.as_tensor(valid_len)).astype(np.int64)
        out = O.attention_f64(O._f64(q3), O._f64(kv3[..., :E]), O._f64(kv3[..., E:]), h,
                              _bias_rows(key_bias, kv3.shape[0], Lk), valid=valid)
        return _t(out, q).reshape(*kv.shape[:-2], Lq, E)

    def pk_self_attention(qkv, h, key_bias, rope, scale):
        L = qkv.shape[-2]
        x = qkv.reshape(-1, L, 3 * E)
        tabs = None if rope is None else O.rope_tables_ref(rope.freqs.double().numpy(), L, E, h, rope.interleaved)
        out = O.pk_self_ref(x, h, _bias_rows(key_bias, x.shape[0], L), tabs, scale)
        return _t(out, qkv).reshape(*qkv.shape[:-2], L, E)

    def pk_cross_attention(q, kv, h, key_bias, rope, scale):
        Lq, Lk = q.shape[-2], kv.shape[-2]
        kv3 = kv.reshape(-1, Lk, 2 * E)
        q3 = q.reshape(-1, Lq, E)
        tq = tk = None
        if rope is not None:
            tq = O.rope_tables_ref(rope.freqs.double().numpy(), Lq, E, h, rope.interleaved)
            tk = O.rope_tables_ref(rope.freqs.double().numpy(), Lk, E, h, rope.interleaved)
        out = O.pk_cross_ref(q3, kv3, h, _bias_rows(key_bias, kv3.shape[0], Lk), tq, tk, scale)
        return _t(out, q).reshape(*kv.shape[:-2], Lq, E)

    def hxf_attention(qf, x, valid_len, key_bias=None):
        Lk = x.shape[-2]
        x3 = x.reshape(-1, Lk, E)
        q3 = qf.reshape(-1, qf.shape[-2], E)
        q3 = q3.expand(x3.shape[0], *q3.shape[1:])
        valid = None if valid_len is None else O._f64(torch.as_tensor(valid_len)).astype(np.int64)
        out = O.attention_f64(O._f64(q3), O._f64(x3), O._f64(x3), 1, _bias_rows(key_bias, x3.shape[0], Lk),
                              valid=valid)
        return _t(out, x).reshape(*x.shape[:-2], q3.shape[1], E)

    yes = lambda *a, **k: True  # noqa: E731
    return types.SimpleNamespace(supported=yes, hxq_supported=yes, packed_supported=yes, hxf_supported=yes,
                                 hx_attention=hx_attention, hxq_attention=hxq_attention,
                                 pk_self_attention=pk_self_attention, pk_cross_attention=pk_cross_attention,
                                 hxf_attention=hxf_attention)


def _fake_icl():
    def icl_sdpa(q, k, v, valid_kv_len=None, key_bias=None):
        lead, D = q.shape[:-3], q.shape[-1]
        q4, k4, v4 = (t.reshape(-1, *t.shape[-3:]) for t in (q, k, v))
        valid = None if valid_kv_len is None else O._f64(torch.as_tensor(valid_kv_len)).astype(np.int64)
        out = O.splash_sdpa_ref(q4, k4, v4, valid, None if key_bias is None else O._f64(key_bias))
        return _t(out, q).reshape(*lead, *q4.shape[1:])

    return types.SimpleNamespace(icl_supported=lambda Tq, Tkv, D, dtype: D == 64, icl_sdpa=icl_sdpa)


@pytest.fixture()
def routed(mha, monkeypatch):
    """install() on an upstream stand-in with every route enabled and fake kernels on CPU tensors;
    yields (module, upstream reference module, list of fake kernels called)."""
    for name, val in (("few_queries", True), ("packed", True), ("folded", False)):
        monkeypatch.setattr(mha.KNOBS, name, val)
    mod, ref_mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="col1=pk,col2=pk,row=pk,cls=pk")
    monkeypatch.setattr(mha, "_DEVICE", "cpu")
    seen = []
    pk, icl = _fake_pk(), _fake_icl()
    for ns in (pk, icl):
        for name, fn in list(vars(ns).items()):
            if name.endswith("attention") or name == "icl_sdpa":
                def spy(*a, _fn=fn, _name=name, **k):
                    seen.append(_name)
                    return _fn(*a, **k)
                setattr(ns, name, spy)
    monkeypatch.setattr(mha, "_PK", pk)
    monkeypatch.setattr(mha, "_ICL", icl)
    yield mod, ref_mod, seen


def _block(mod, q, w, b, wo, bo, nh=H, **kw):
    with torch.no_grad():
        return U.block_attention(mod, q, nh, w, b, wo, bo, **kw)


def test_isab1_train_mask_from_tensor_train_size_takes_few_query_route(routed):
    mod, ref_mod, seen = routed
    g = torch.Generator().manual_seed(5)
    w, b, wo, bo = U.weights(E, 5)
    ind = torch.randn(3, 16, E, generator=g)
    rows = torch.randn(3, 300, E, generator=g)
    ts = torch.tensor(200)
    kw = dict(k=rows, v=rows, src_len_override=ts, valid_kv_len=ts, ssmax_layer=U.SSMaxStub(H))
    got = _block(mod, ind, w, b, wo, bo, **kw)
    want = _block(ref_mod, ind, w, b, wo, bo, **kw)
    assert seen == ["hxq_attention"]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_isab1_folded_route_takes_the_train_mask(routed, mha, monkeypatch):
    mod, ref_mod, seen = routed
    monkeypatch.setattr(mha.KNOBS, "folded", True)  # install() copies the knobs: a new install sees it
    monkeypatch.setattr(mha.KNOBS, "folded_force", True)  # the folded kernel itself, not projection + hxq
    g = torch.Generator().manual_seed(6)
    w, b, wo, bo = U.weights(E, 6)
    ind = torch.randn(16, E, generator=g).expand(3, 16, E)
    rows = torch.randn(3, 300, E, generator=g)
    ts = torch.tensor(123)
    mod2 = U.make_module()
    assert mha.install(mod2, None, mode="pk")
    kw = dict(k=rows, v=rows, src_len_override=ts, valid_kv_len=ts)
    got = _block(mod2, ind, w, b, wo, bo, **kw)
    want = _block(ref_mod, ind, w, b, wo, bo, **kw)
    assert seen == ["hxf_attention"]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_isab1_folded_route_key_mask_and_ssmax_without_override(routed, mha, monkeypatch):
    # a key-padding mask and SSMax with neither src_len_override nor valid_kv_len: SSMax takes the key
    # count, as upstream's sdpa does (k.size(-2), results/tpu_patch.diff:251-254)
    mod, ref_mod, seen = routed
    monkeypatch.setattr(mha.KNOBS, "folded", True)
    monkeypatch.setattr(mha.KNOBS, "folded_force", True)
    g = torch.Generator().manual_seed(9)
    w, b, wo, bo = U.weights(E, 9)
    ind = torch.randn(16, E, generator=g).expand(2, 16, E)
    rows = torch.randn(2, 300, E, generator=g)
    kpm = torch.zeros(2, 300)
    kpm[:, 270:] = torch.finfo(torch.float32).min
    mod2 = U.make_module()
    assert mha.install(mod2, None, mode="pk")
    kw = dict(k=rows, v=rows, key_padding_mask=kpm, ssmax_layer=U.SSMaxStub(H))
    got = _block(mod2, ind, w, b, wo, bo, **kw)
    want = _block(ref_mod, ind, w, b, wo, bo, **kw)
    assert seen == ["hxf_attention"]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_isab1_folded_knob_runs_projection_and_hxq_where_it_applies(routed, mha, monkeypatch):
    # TABICL_TPU_MHA_HXF=1 alone (not forced): the call goes to projection + hxq, faster on this GPU, with
    # the HXQ knob off too; the result is the same attention
    mod, ref_mod, seen = routed
    monkeypatch.setattr(mha.KNOBS, "folded", True)
    monkeypatch.setattr(mha.KNOBS, "few_queries", False)
    g = torch.Generator().manual_seed(10)
    w, b, wo, bo = U.weights(E, 10)
    ind = torch.randn(16, E, generator=g).expand(2, 16, E)
    rows = torch.randn(2, 300, E, generator=g)
    ts = torch.tensor(250)
    mod2 = U.make_module()
    assert mha.install(mod2, None, mode="pk")
    kw = dict(k=rows, v=rows, src_len_override=ts, valid_kv_len=ts, ssmax_layer=U.SSMaxStub(H))
    got = _block(mod2, ind, w, b, wo, bo, **kw)
    want = _block(ref_mod, ind, w, b, wo, bo, **kw)
    assert seen == ["hxq_attention"]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_isab1_reference_device_semantics_tensor_length(routed):
    # the caller hands over a tensor valid_kv_len and no mask (what upstream does on the reference's device)
    mod, ref_mod, seen = routed
    g = torch.Generator().manual_seed(7)
    w, b, wo, bo = U.weights(E, 7)
    ind = torch.randn(2, 16, E, generator=g)
    rows = torch.randn(2, 300, E, generator=g)
    vl = torch.tensor(250)
    with torch.no_grad():
        got = U.call(mod.multi_head_attention_forward, ind, rows, rows, H, w, b, wo, bo, valid_kv_len=vl)
        want = U.call(ref_mod.multi_head_attention_forward, ind, rows[:, :250], rows[:, :250], H, w, b, wo, bo)
    assert seen == ["hxq_attention"]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_row_self_attention_with_feature_mask_takes_packed_route(routed):
    mod, ref_mod, seen = routed
    g = torch.Generator().manual_seed(8)
    w, b, wo, bo = U.weights(E, 8)
    x = torch.randn(2, 24, E, generator=g)
    kpm = torch.zeros(2, 24)
    kpm[:, 20:] = torch.finfo(torch.float32).min
    rope = U.RopeStub()
    got = _block(mod, x, w, b, wo, bo, key_padding_mask=kpm, rope=rope)
    want = _block(ref_mod, x, w, b, wo, bo, key_padding_mask=kpm, rope=rope)
    assert seen == ["pk_self_attention"]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_isab2_cross_attention_takes_packed_route(routed):
    mod, ref_mod, seen = routed
    g = torch.Generator().manual_seed(9)
    w, b, wo, bo = U.weights(E, 9)
    rows, hidden = torch.randn(2, 40, E, generator=g), torch.randn(2, 16, E, generator=g)
    got = _block(mod, rows, w, b, wo, bo, k=hidden, v=hidden)
    want = _block(ref_mod, rows, w, b, wo, bo, k=hidden, v=hidden)
    assert seen == ["pk_cross_attention"]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("T,train", [(20000, 18000), (5000, 4500)])
def test_cached_icl_with_tensor_train_size_reaches_the_icl_kernel(routed, T, train):
    # 20000 >= the Splash threshold, 5000 below it (the ragged batch's small tables): both go to the kernel
    mod, ref_mod, seen = routed
    g = torch.Generator().manual_seed(T)
    Ew, nh = 256, 4
    w, b, wo, bo = U.weights(Ew, 10)
    kc = torch.randn(2, nh, T, 64, generator=g)
    vc = torch.randn(2, nh, T, 64, generator=g)
    q = torch.randn(2, 6, Ew, generator=g)
    ts = torch.tensor(train)
    kw = dict(cached_kv=U.KVEntry(kc, vc), valid_kv_len=ts, src_len_override=ts, ssmax_layer=U.SSMaxStub(nh))
    got = _block(mod, q, w, b, wo, bo, nh=nh, **kw)
    want = _block(ref_mod, q, w, b, wo, bo, nh=nh, **kw)
    assert seen == ["icl_sdpa"]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_icl_hook_keeps_gradient_calls(routed):
    # the ICL op has a backward: calls under autograd reach the kernel; a key mask that itself needs a
    # gradient (the op gives a mask none) goes to upstream
    mod, ref_mod, seen = routed
    g = torch.Generator().manual_seed(13)
    q = torch.randn(2, 4, 6, 64, generator=g, requires_grad=True)
    k, v = torch.randn(2, 4, 50, 64, generator=g), torch.randn(2, 4, 50, 64, generator=g)
    kb = torch.zeros(2, 1, 1, 50)
    kb[1, ..., 40:] = torch.finfo(torch.float32).min
    with torch.enable_grad():
        mod.sdpa_with_flattened_batch(q, k, v, kb, valid_kv_len=torch.tensor(45))
        assert seen == ["icl_sdpa"]
        got = mod.sdpa_with_flattened_batch(q, k, v, kb.clone().requires_grad_())
        want = ref_mod.sdpa_with_flattened_batch(q, k, v, kb)
    assert seen == ["icl_sdpa"]
    torch.testing.assert_close(got, want)


@pytest.mark.parametrize("with_mask", [False, True])
def test_cached_column_attention_takes_pk_cross(routed, with_mask):
    # the column blocks' second attention at query time: test rows over the cached head-split K/V of
    # the 128 inducing points (scripts/tabicl_tpu_bucketed.py:788-792) -> pk_cross on packed K|V rows;
    # with a key-padding mask over the inducing keys it becomes the key bias
    mod, ref_mod, seen = routed
    g = torch.Generator().manual_seed(12)
    w, b, wo, bo = U.weights(E, 12)
    rows = torch.randn(2, 3, 40, E, generator=g)  # [est, column, test row, E]
    kc = torch.randn(2, 3, H, 128, E // H, generator=g)
    vc = torch.randn(2, 3, H, 128, E // H, generator=g)
    kw = dict(cached_kv=U.KVEntry(kc, vc))
    if with_mask:
        kpm = torch.zeros(2, 3, 128)
        kpm[:, :, 100:] = torch.finfo(torch.float32).min
        kw["key_padding_mask"] = kpm
    got = _block(mod, rows, w, b, wo, bo, **kw)
    want = _block(ref_mod, rows, w, b, wo, bo, **kw)
    assert seen == ["pk_cross_attention"]
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


def test_cached_column_attention_declines(routed, mha, monkeypatch):
    # RoPE (the cache holds keys rotated at fit time), K/V whose batch differs from the query's, and the
    # knob off all leave the call to upstream
    mod, ref_mod, seen = routed
    g = torch.Generator().manual_seed(13)
    w, b, wo, bo = U.weights(E, 13)
    rows = torch.randn(2, 40, E, generator=g)
    kc = torch.randn(2, H, 128, E // H, generator=g)
    vc = torch.randn(2, H, 128, E // H, generator=g)
    _block(mod, rows, w, b, wo, bo, cached_kv=U.KVEntry(kc, vc), rope=U.RopeStub())
    _block(mod, rows, w, b, wo, bo, cached_kv=U.KVEntry(kc[:1], vc[:1]))
    assert seen == []
    monkeypatch.setattr(mha.KNOBS, "cached", False)
    mod2 = U.make_module()
    assert mha.install(mod2, None, mode="col1=pk,col2=pk,row=pk,cls=pk")
    got = _block(mod2, rows, w, b, wo, bo, cached_kv=U.KVEntry(kc, vc))
    want = _block(ref_mod, rows, w, b, wo, bo, cached_kv=U.KVEntry(kc, vc))
    assert seen == []
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-6)


def test_fallbacks_to_upstream(routed):
    mod, ref_mod, seen = routed
    g = torch.Generator().manual_seed(11)
    w, b, wo, bo = U.weights(E, 11)
    x = torch.randn(2, 24, E, generator=g)
    # a boolean mask: upstream handles it
    bm = torch.ones(24, 24, dtype=torch.bool)
    with torch.no_grad():
        got = U.call(mod.multi_head_attention_forward, x, x, x, H, w, b, wo, bo, attn_mask=bm)
    assert seen == []
    # a mask that varies over queries: not a key mask, so the packed route declines and upstream runs
    am = torch.randn(24, 24, generator=g)
    with torch.no_grad():
        got = U.call(mod.multi_head_attention_forward, x, x, x, H, w, b, wo, bo, attn_mask=am)
        want = U.call(ref_mod.multi_head_attention_forward, x, x, x, H, w, b, wo, bo, attn_mask=am)
    assert seen == []
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-6)
    # K/V requested back: upstream
    with torch.no_grad():
        U.call(mod.multi_head_attention_forward, x, x, x, H, w, b, wo, bo, need_kv=True)
    assert seen == []


def test_install_binds_the_reference_splash_ops(mha):
    # the upstream module's _tpu_splash_sdpa_{seg,full}_op attributes (the reference's op objects,
    # results/tpu_patch.diff:95-115) become the HIP ICL ops under the reference's op names
    import tabicl_mi355_icl as icl
    mod = U.make_module()
    assert mha.install(mod, None, mode="pk")
    assert mod._tpu_splash_sdpa_seg_op is icl.splash_sdpa_seg_op
    assert mod._tpu_splash_sdpa_full_op is icl.splash_sdpa_full_op
    assert torch.ops.tabicl.tpu_splash_sdpa_seg is not None and torch.ops.tabicl.tpu_splash_sdpa_full is not None
    q = torch.zeros(2, 8, 1024, 64, device="meta", dtype=torch.bfloat16)
    k = torch.zeros(2, 8, 4096, 64, device="meta", dtype=torch.bfloat16)
    out = torch.ops.tabicl.tpu_splash_sdpa_seg(q, k, k, torch.zeros((), dtype=torch.int32, device="meta"), 1024, 4096)
    assert out.shape == q.shape and out.dtype == q.dtype


def test_install_is_idempotent_and_off(mha):
    mod = U.make_module()
    assert mha.install(mod, None, mode="pk") is True
    f = mod.multi_head_attention_forward
    assert mha.install(mod, None, mode="pk") is True and mod.multi_head_attention_forward is f
    assert mha.install(U.make_module(), None, mode="off") is False
    assert mha.install(U.make_module(), None, mode="") is False


def test_block_stub_builds_the_train_mask():
    # the restated block turns a tensor train size into an additive finfo.min key mask off the reference's
    # device (diff:1526-1542): check the attention it drives equals attention over the train rows only
    mod = U.make_module()
    g = torch.Generator().manual_seed(12)
    w, b, wo, bo = U.weights(E, 12)
    x = torch.randn(2, 50, E, generator=g)
    ts = torch.tensor(30)
    got = _block(mod, x, w, b, wo, bo, train_size=ts)
    want = U.call(mod.multi_head_attention_forward, x, x[:, :30], x[:, :30], H, w, b, wo, bo)
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)
