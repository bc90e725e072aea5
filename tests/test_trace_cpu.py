"""Tracing the ops without a GPU: every registered op has a fake (meta) implementation and an autograd
formula, so forward and backward run on meta tensors (shapes and dtypes only), and torch.compile traces
them, and the installed dispatch wrapper around them, as one graph (fullgraph=True, backend aot_eager:
no code generation). The reference checks the same property of its wrapper with a Dynamo fullgraph
aot_eager trace (scripts/tests/test_mha_cpu.py:106-124). Nothing here launches a kernel.
"""
import pytest
import torch

import upstream_stub as U

META = dict(device="meta", dtype=torch.bfloat16)


class _Rope:
    """RotaryEmbedding stand-in (get_seq_pos / interleaved / freqs)."""
    interleaved = False
    freqs = 100000.0 ** (-torch.arange(0, 16, 2, dtype=torch.float32) / 16)

    def get_seq_pos(self, n, device=None, dtype=torch.float32):
        return torch.arange(n, device=device, dtype=dtype)


def _leaves(*shapes):
    return [torch.zeros(*s, **META, requires_grad=True) for s in shapes]


def _grads(out, leaves):
    gs = torch.autograd.grad(out.float().square().mean(), leaves)
    for g, t in zip(gs, leaves):
        assert g.shape == t.shape and g.dtype == t.dtype and g.device.type == "meta"
    return gs


def test_meta_forward_backward_every_op():
    import tabicl_mi355_attn as pk
    import tabicl_mi355_icl as icl
    B, L, E, H = 3, 104, 128, 8
    q, k, v = _leaves((B, L, E), (B, 300, E), (B, 300, E))
    out = pk.hx_attention(q, k, v, H)
    assert out.shape == q.shape and out.dtype == q.dtype
    _grads(out, [q, k, v])
    out = pk.hx_attention(q, k, v, H, torch.zeros(B, 300, device="meta"))
    _grads(out, [q, k, v])
    (qkv,) = _leaves((B, L, 3 * E))
    out = pk.pk_self_attention(qkv, H, None, _Rope(), 0.25)
    assert out.shape == (B, L, E)
    _grads(out, [qkv])
    qc, kv = _leaves((B, 40, E), (B, 128, 2 * E))
    out = pk.pk_cross_attention(qc, kv, H, None, _Rope(), 0.25)
    assert out.shape == (B, 40, E)
    _grads(out, [qc, kv])
    out = pk.hxq_attention(torch.zeros(B, 128, E, **META), torch.zeros(B, 5000, 2 * E, **META),
                           torch.tensor(4000, device="meta"), H)
    assert out.shape == (B, 128, E)
    # ICL: the training forward (statistics kept) without a mask, the plain op with one
    qi, ki, vi = _leaves((2, 8, 100, 64), (2, 8, 700, 64), (2, 8, 700, 64))
    out = icl.icl_sdpa(qi, ki, vi, 650)
    assert out.shape == qi.shape
    _grads(out, [qi, ki, vi])
    out = icl.icl_sdpa(qi, ki, vi, None, torch.zeros(2, 700, device="meta"))
    _grads(out, [qi, ki, vi])
    o, stat = icl.ICL_FWD_TRAIN(qi.detach(), ki.detach(), vi.detach(), None, 0.125)
    assert o.shape == qi.shape and stat.shape == (2, 8, 100, 2) and stat.dtype == torch.float32


def test_compile_fullgraph_ops():
    import tabicl_mi355_attn as pk
    import tabicl_mi355_icl as icl
    torch._dynamo.reset()
    qi, ki, vi = _leaves((2, 8, 100, 64), (2, 8, 700, 64), (2, 8, 700, 64))
    f = torch.compile(lambda q, k, v: icl.icl_sdpa(q, k, v, 650), backend="aot_eager", fullgraph=True)
    out = f(qi, ki, vi)
    assert out.shape == qi.shape
    _grads(out, [qi, ki, vi])
    (qkv,) = _leaves((3, 104, 384))
    rope = _Rope()
    g = torch.compile(lambda x: pk.pk_self_attention(x, 8, None, rope, 0.25), backend="aot_eager", fullgraph=True)
    out = g(qkv)
    assert out.shape == (3, 104, 128)
    _grads(out, [qkv])


@pytest.mark.parametrize("case", ["row_self", "cached_icl"])
def test_compile_fullgraph_installed_wrapper(case, monkeypatch):
    # the dispatch drop-in installed on an upstream stand-in, called as upstream's block calls it, traced
    # as one graph with the routes taken on meta tensors (the device gate pointed at "meta")
    import tabicl_mi355_mha as mha
    torch._dynamo.reset()
    for name, val in (("few_queries", True), ("packed", True), ("folded", False)):
        monkeypatch.setattr(mha.KNOBS, name, val)
    mod = U.make_module()
    assert mha.install(mod, None, mode="col1=pk,col2=pk,row=pk,cls=pk")
    monkeypatch.setattr(mha, "_DEVICE", "meta")
    if case == "row_self":
        E, nh = 128, 8
        w, b, wo, bo = (t.to(**META) for t in U.weights(E, 3))
        x = torch.zeros(4, 104, E, **META, requires_grad=True)

        def fn(x):
            return U.block_attention(mod, x, nh, w, b, wo, bo)
    else:
        E, nh = 256, 4
        w, b, wo, bo = (t.to(**META) for t in U.weights(E, 4))
        kc = torch.zeros(2, nh, 900, 64, **META)
        vc = torch.zeros(2, nh, 900, 64, **META)
        x = torch.zeros(2, 30, E, **META, requires_grad=True)
        train = torch.tensor(800, device="meta")

        def fn(x):
            return U.block_attention(mod, x, nh, w, b, wo, bo, cached_kv=U.KVEntry(kc, vc), valid_kv_len=train)
    out = torch.compile(fn, backend="aot_eager", fullgraph=True)(x)
    assert out.shape == x.shape
    _grads(out, [x])
