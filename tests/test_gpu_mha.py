"""GPU tests of the dispatch layer driven the way upstream tabicl drives it: through the attention call
of MultiheadAttentionBlock.forward (tests/upstream_stub.block_attention, a restatement of
results/tpu_patch.diff:1509-1565), which on this device turns a tensor train size into an additive
finfo.min key mask before multi_head_attention_forward runs (diff:1526-1542). A route spy asserts that
the HIP op of the route ran, and the output is compared with the same upstream stand-in, not installed,
running torch math on the same GPU from the same inputs (the projections are the same GEMMs on both
sides, so the difference is the kernel's).

Bar (written here): max abs error <= 2e-2 with bf16 activations, <= 1e-4 with fp32; training
gradients through the dispatch (mean-square loss: small gradients) to the same factors times the
reference gradient's largest entry. The long-key routes
(cached ICL over 45,000 / 5,000 keys, ISAB-1 over 50,000 rows) also take the scale-aware bar of
tests/parity.py on the attention's part of the block output (output minus the out-projection bias):
max abs error <= 2e-2 (bf16) / 1e-3 (fp32) times its max. The SSMax stand-in scales q by s_h log n
(5-11 at these key counts), so the attention is sharp there and that part is O(1) (~3.4).
The small_head_attention "pk" branch (mask -> key bias -> hx kernel) is compared with the fp64 oracle.
"""
import numpy as np
import pytest
import torch

import upstream_stub as U
from oracle import attention as O
from parity import check

pytestmark = pytest.mark.gpu
H, E = 8, 128
TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}


@pytest.fixture()
def mha(monkeypatch):
    import tabicl_mi355_mha as m
    for name in ("packed", "few_queries"):
        monkeypatch.setattr(m.KNOBS, name, True)
    monkeypatch.setattr(m.KNOBS, "folded", False)
    return m


def _spy(monkeypatch):
    import tabicl_mi355_attn as pk
    import tabicl_mi355_icl as icl
    seen = []
    for mod, name in ((pk, "pk_self_attention"), (pk, "pk_cross_attention"), (pk, "hxq_attention"),
                      (pk, "hx_attention"), (pk, "hxf_attention"), (icl, "icl_sdpa")):
        fn = getattr(mod, name)

        def wrap(*a, _fn=fn, _name=name, **k):
            seen.append(_name)
            return _fn(*a, **k)

        monkeypatch.setattr(mod, name, wrap)
    return seen


def _weights(Ew, seed, dev, dtype):
    return U.weights(Ew, seed, dev, dtype)


def _err(a, b):
    return float((a.float() - b.float()).abs().max())


def _run(mod, ref_mod, q, w, b, wo, bo, nh=H, **kw):
    with torch.no_grad():
        got = U.block_attention(mod, q, nh, w, b, wo, bo, **kw)
        want = U.block_attention(ref_mod, q, nh, w, b, wo, bo, **kw)
    torch.cuda.synchronize()
    return got, want


@pytest.mark.parametrize("T,train", [(45000, 45000 - 56), (5000, 4500)])
def test_block_cached_icl_tensor_train_size(dev, mha, monkeypatch, T, train):
    # C4 (45k cached train rows, >= the Splash threshold) and a C5 table (5k rows, below it): the block's
    # train mask reaches the ICL hook as a key mask; the kernel reads it as the valid length
    seen = _spy(monkeypatch)
    g = torch.Generator().manual_seed(T)
    Ew, nh = 512, 8
    w, b, wo, bo = _weights(Ew, 12, dev, torch.bfloat16)
    mod, ref_mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="col1=pk,col2=pk,row=pk,cls=pk")
    kc = torch.randn(2, nh, T, 64, generator=g).to(dev, torch.bfloat16)
    vc = torch.randn(2, nh, T, 64, generator=g).to(dev, torch.bfloat16)
    kc[..., train:, :] = float("nan")  # rows past the train size must not be read
    vc[..., train:, :] = float("nan")
    q = torch.randn(2, 300, Ew, generator=g).to(dev, torch.bfloat16)
    ts = torch.tensor(train, device=dev)
    print(f"[mha] cached icl T={T}", flush=True)
    with torch.no_grad():
        got = U.block_attention(mod, q, nh, w, b, wo, bo, cached_kv=U.KVEntry(kc, vc), valid_kv_len=ts,
                                src_len_override=ts, ssmax_layer=U.SSMaxStub(nh))
        kr, vr = kc[..., :train, :].contiguous(), vc[..., :train, :].contiguous()
        want = U.call(ref_mod.multi_head_attention_forward, q, None, None, nh, w, b, wo, bo,
                      cached_kv=U.KVEntry(kr, vr), src_len_override=ts, ssmax_layer=U.SSMaxStub(nh))
    assert seen == ["icl_sdpa"], seen
    assert torch.isfinite(got.float()).all()
    check(got.double() - bo.double(), want.double() - bo.double(), torch.bfloat16, f"cached icl T={T}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_block_isab1_50k_rows_few_query_route(dev, mha, monkeypatch, dtype):
    # C3's first ISAB attention at full length (50,000 rows, 45,000 train) through the block
    seen = _spy(monkeypatch)
    g = torch.Generator().manual_seed(50)
    w, b, wo, bo = _weights(E, 13, dev, dtype)
    mod, ref_mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="col1=pk,col2=pk,row=pk,cls=pk")
    ind = torch.randn(128, E, generator=g).to(dev, dtype).expand(3, 128, E)
    rows = torch.randn(3, 50000, E, generator=g).to(dev, dtype)
    ts = torch.tensor(45000, device=dev)
    print(f"[mha] isab1 50k {dtype}", flush=True)
    got, want = _run(mod, ref_mod, ind, w, b, wo, bo, k=rows, v=rows, src_len_override=ts, valid_kv_len=ts,
                     ssmax_layer=U.SSMaxStub(H))
    assert seen == ["hxq_attention"], seen
    check(got.double() - bo.double(), want.double() - bo.double(), dtype, f"isab1 50k {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_block_cached_column_attention(dev, mha, monkeypatch, dtype):
    # the column blocks' second attention at query time (scripts/tabicl_tpu_bucketed.py:788-792): test rows
    # of each (estimator, column) over that column's cached K/V of the 128 inducing points, head-split as
    # upstream's need_kv returns them; the route writes them as packed K|V rows and runs pk_cross
    seen = _spy(monkeypatch)
    g = torch.Generator().manual_seed(54)
    w, b, wo, bo = _weights(E, 16, dev, dtype)
    mod, ref_mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="col1=pk,col2=pk,row=pk,cls=pk")
    rows = torch.randn(2, 13, 5000, E, generator=g).to(dev, dtype)  # [est, column, test row, E]
    kc = torch.randn(2, 13, H, 128, E // H, generator=g).to(dev, dtype)
    vc = torch.randn(2, 13, H, 128, E // H, generator=g).to(dev, dtype)
    print(f"[mha] cached column attention {dtype}", flush=True)
    got, want = _run(mod, ref_mod, rows, w, b, wo, bo, cached_kv=U.KVEntry(kc, vc))
    assert seen == ["pk_cross_attention"], seen
    check(got.double() - bo.double(), want.double() - bo.double(), dtype, f"cached column {dtype}")


def test_block_isab1_folded_route(dev, mha, monkeypatch):
    monkeypatch.setattr(mha.KNOBS, "folded", True)
    monkeypatch.setattr(mha.KNOBS, "folded_force", True)  # the folded kernel, not projection + hxq
    seen = _spy(monkeypatch)
    g = torch.Generator().manual_seed(51)
    w, b, wo, bo = _weights(E, 14, dev, torch.float32)
    mod, ref_mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="pk")
    ind = torch.randn(128, E, generator=g).to(dev).expand(2, 128, E)
    rows = torch.randn(2, 20000, E, generator=g).to(dev)
    ts = torch.tensor(17000, device=dev)
    got, want = _run(mod, ref_mod, ind, w, b, wo, bo, k=rows, v=rows, src_len_override=ts, valid_kv_len=ts)
    assert seen == ["hxf_attention"], seen
    assert _err(got, want) <= 1e-4


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_block_row_and_column_routes(dev, mha, monkeypatch, dtype):
    seen = _spy(monkeypatch)
    g = torch.Generator().manual_seed(52)
    w, b, wo, bo = _weights(E, 15, dev, dtype)
    mod, ref_mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="col1=pk,col2=pk,row=pk,cls=pk")
    rope = U.RopeStub()
    x = torch.randn(4, 104, E, generator=g).to(dev, dtype)
    kpm = torch.zeros(4, 104)
    kpm[:, 101:] = float(torch.finfo(torch.float32).min)  # padded feature slots (diff:1253-1271)
    kpm = kpm.to(dev, dtype)
    hidden = torch.randn(4, 128, E, generator=g).to(dev, dtype)
    rows = torch.randn(4, 2000, E, generator=g).to(dev, dtype)
    cases = [
        ("pk_self_attention", x, dict(rope=rope, key_padding_mask=kpm)),  # row stage
        ("pk_cross_attention", x[:, :4], dict(k=x, v=x, rope=rope, key_padding_mask=kpm)),  # CLS tokens
        ("pk_cross_attention", rows, dict(k=hidden, v=hidden)),  # column ISAB-2
        ("hxq_attention", hidden, dict(k=rows, v=rows, ssmax_layer=U.SSMaxStub(H),  # column ISAB-1, small table
                                       valid_kv_len=torch.tensor(1500, device=dev),
                                       src_len_override=torch.tensor(1500, device=dev))),
    ]
    for route, q, kw in cases:
        seen.clear()
        print(f"[mha] {route} {dtype}", flush=True)
        got, want = _run(mod, ref_mod, q, w, b, wo, bo, **kw)
        assert seen == [route], (route, seen)
        assert _err(got, want) <= TOL[dtype], route


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_small_head_attention_pk_branch(dev, mha, monkeypatch, dtype):
    # small_head_attention(impl="pk") with a key-padding mask: the mask becomes a key bias and the hx
    # kernel runs (reference scripts/tabicl_tpu_mha.py:177-188); a per-query mask takes the torch form
    import tabicl_mi355_attn as pk
    monkeypatch.setattr(mha, "_PK", pk)
    seen = _spy(monkeypatch)
    g = torch.Generator().manual_seed(53)
    q = (torch.randn(3, 200, E, generator=g) * 0.25).to(dtype)
    k = torch.randn(3, 300, E, generator=g).to(dtype)
    v = torch.randn(3, 300, E, generator=g).to(dtype)
    bias = torch.zeros(3, 300)
    bias[0, 250:] = float(torch.finfo(torch.float32).min)
    bias[1, :] = torch.randn(300, generator=g)
    mask = bias.view(3, 1, 1, 300)
    out = mha.small_head_attention(q.to(dev), k.to(dev), v.to(dev), H, mask.to(dev), "pk")
    ref = O.attention_f64(q.double().numpy(), k.double().numpy(), v.double().numpy(), H, bias.double().numpy())
    assert float(np.abs(out.double().cpu().numpy() - ref).max()) <= TOL[dtype]
    assert seen == ["hx_attention"]
    qmask = torch.randn(3, 1, 200, 300, generator=g)
    out2 = mha.small_head_attention(q.to(dev), k.to(dev), v.to(dev), H, qmask.to(dev), "pk")
    ref2 = np.zeros((3, 200, E))
    for i in range(200):  # per-query mask: each query row with its own bias row
        ref2[:, i:i + 1] = O.attention_f64(q[:, i:i + 1].double().numpy(), k.double().numpy(), v.double().numpy(), H,
                                           qmask[:, 0, i].double().numpy())
    assert float(np.abs(out2.double().cpu().numpy() - ref2).max()) <= TOL[dtype]


@pytest.mark.parametrize("case,dtype", [("row_rope", torch.bfloat16), ("row_rope", torch.float32),
                                        ("isab2_cross", torch.bfloat16), ("icl_train_size", torch.bfloat16),
                                        ("icl_train_size", torch.float32)])
def test_block_training_gradients(dev, mha, monkeypatch, case, dtype):
    # training through the installed dispatch, as the reference's CPU equivalence test does per mode
    # (scripts/tests/test_mha_cpu.py:78-104): the loss out.float().square().mean(), then the gradients of
    # the block input and of every weight, against the same stand-in without the dispatch (torch math on
    # the same GPU). Routes: the row stage's self attention with RoPE and a key-padding mask (pk_self),
    # ISAB-2 cross attention (pk_cross), the ICL stage's self attention with a tensor train size (the
    # additive train mask through the ICL hook to the masked ICL kernel and its backward)
    seen = _spy(monkeypatch)
    g = torch.Generator().manual_seed(60)
    icl_case = case == "icl_train_size"
    Ew, nh = (512, 8) if icl_case else (E, H)
    params = list(_weights(Ew, 61, dev, dtype))
    mod, ref_mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="col1=pk,col2=pk,row=pk,cls=pk")
    if case == "row_rope":
        x = torch.randn(8, 104, Ew, generator=g).to(dev, dtype)
        kpm = torch.zeros(8, 104)
        kpm[:, 90:] = torch.finfo(torch.float32).min
        kw = dict(rope=U.RopeStub(), key_padding_mask=kpm.to(dev, dtype))
        route = "pk_self_attention"
    elif case == "isab2_cross":
        x = torch.randn(4, 300, Ew, generator=g).to(dev, dtype)
        hidden = torch.randn(4, 128, Ew, generator=g).to(dev, dtype)
        kw = dict(k=hidden, v=hidden)
        route = "pk_cross_attention"
    else:
        x = torch.randn(2, 700, Ew, generator=g).to(dev, dtype)
        ts = torch.tensor(600, device=dev)
        kw = dict(train_size=ts, ssmax_layer=U.SSMaxStub(nh))
        route = "icl_sdpa"
    print(f"[mha] training gradients {case} {dtype}", flush=True)

    def run(m):
        leaves = [t.detach().clone().requires_grad_() for t in [x] + params]
        out = U.block_attention(m, leaves[0], nh, *leaves[1:], **kw)
        loss = out.float().square().mean()
        return loss.detach(), torch.autograd.grad(loss, leaves)

    loss, grads = run(mod)
    assert route in seen, seen
    ref_loss, ref_grads = run(ref_mod)
    torch.cuda.synchronize()
    # relative bars (the mean-square loss makes every gradient small): 2e-2 (bf16) / 1e-4 (fp32) of the
    # reference gradient's largest entry; the loss to the same relative bar
    tol = TOL[dtype]
    assert abs(float(loss) - float(ref_loss)) <= tol * abs(float(ref_loss))
    for name, a, b in zip(("x", "in_proj_w", "in_proj_b", "out_proj_w", "out_proj_b"), grads, ref_grads):
        scale = float(b.float().abs().max())
        err = _err(a, b)
        print(f"  d{name}: max abs err {err:.3e} (ref max {scale:.3e}, {err / scale:.2e} of it)", flush=True)
        assert torch.isfinite(a.float()).all() and scale > 0
        assert err <= tol * scale, (name, err, scale)
