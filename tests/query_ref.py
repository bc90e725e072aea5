"""CPU restatement of the whole cached-KV query (test infrastructure): the reference's _make_query_fn
(scripts/tabicl_tpu_bucketed.py:768-834) restated from its call sites in float64 with the oracle's
attention, plus the random weights the query tests use. Used by tests/test_gpu_query.py (against the HIP
path) and tests/test_query_cpu.py (against the composition run on the CPU with oracle-backed kernels).

Feature grouping by explicit index loops, the in-linear with the skip rule, each layer's LayerNorm /
GEMMs / GELU in float64, `pk_cross_ref` for the column and CLS attention, `pk_self_ref` with the oracle's
RoPE tables for the row attention, and for the ICL stage the rounding points of the bf16 path (bf16 GEMM
inputs and outputs, fp32 LayerNorm and residual stream) around `splash_sdpa_ref`."""
import numpy as np
import torch
import torch.nn.functional as F

from oracle import attention as O

E, H, C, ICLW, ICLH = 128, 8, 4, 512, 8
NI = 128
SKIP = -100.0


class Rope:
    interleaved = False

    def __init__(self):
        self.freqs = torch.tensor(O.textbook_freqs(16, 100000.0), dtype=torch.float32)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)


def block_weights(width, ff, g, dtype):
    import tabicl_mi355_icl as icl

    def lin(o, i):
        return (torch.randn(o, i, generator=g) * i ** -0.5).to(dtype), (torch.randn(o, generator=g) * 0.1).to(dtype)

    in_w, in_b = lin(3 * width, width)
    out_w, out_b = lin(width, width)
    f1w, f1b = lin(ff, width)
    f2w, f2b = lin(width, ff)
    return icl.IclBlockWeights(1 + 0.1 * torch.randn(width, generator=g), 0.1 * torch.randn(width, generator=g),
                               in_w, in_b, out_w, out_b, 1 + 0.1 * torch.randn(width, generator=g),
                               0.1 * torch.randn(width, generator=g), f1w, f1b, f2w, f2b)


def map_tensors(w, fn):
    """The weights dataclass w with fn applied to every tensor (nested dataclasses and lists too)."""
    import dataclasses
    if isinstance(w, torch.Tensor):
        return fn(w)
    if isinstance(w, list):
        return [map_tensors(x, fn) for x in w]
    if dataclasses.is_dataclass(w):
        return dataclasses.replace(w, **{f.name: map_tensors(getattr(w, f.name), fn) for f in dataclasses.fields(w)})
    return w


def to_device(w, dev):
    return map_tensors(w, lambda t: t.to(dev))


def as_f64(w):
    return map_tensors(w, lambda t: t.detach().cpu().double())


def model(dtype, seed=90):
    import tabicl_mi355_query as Q
    g = torch.Generator().manual_seed(seed)
    col = Q.ColumnWeights((torch.randn(E, 3, generator=g) * 0.5).to(dtype), (0.1 * torch.randn(E, generator=g)).to(dtype),
                          [block_weights(E, 2 * E, g, dtype) for _ in range(3)])
    row = Q.RowWeights((0.5 * torch.randn(C, E, generator=g)).to(dtype), [block_weights(E, 2 * E, g, dtype) for _ in range(3)],
                       1 + 0.1 * torch.randn(E, generator=g), 0.1 * torch.randn(E, generator=g))
    iclb = [block_weights(ICLW, 2 * ICLW, g, torch.bfloat16) for _ in range(2)]

    def lin(o, i):
        return (torch.randn(o, i, generator=g) * i ** -0.5).to(torch.bfloat16), \
               (torch.randn(o, generator=g) * 0.1).to(torch.bfloat16)

    (w1, b1), (w2, b2) = lin(2 * ICLW, ICLW), lin(10, 2 * ICLW)
    dec = Q.DecoderWeights(1 + 0.1 * torch.randn(ICLW, generator=g), 0.1 * torch.randn(ICLW, generator=g), w1, b1, w2, b2)
    return Q.QueryWeights(col, row, iclb, dec), g


# ---- CPU restatement (float64) --------------------------------------------------------------------
def ln64(x, w, b, eps):
    return F.layer_norm(x, (x.shape[-1],), w, b, eps)


def ffn64(x, blk):
    h = ln64(x, blk.ln2_w, blk.ln2_b, blk.eps)
    return x + F.linear(F.gelu(F.linear(h, blk.ff1_w, blk.ff1_b)), blk.ff2_w, blk.ff2_b)


def grouping_loops(X, d):
    Bn, Tn, Hn = X.shape
    out = np.zeros((Bn, Tn, Hn, 3))
    for b in range(Bn):
        rf = int(d[b])
        for j in range(Hn):
            for i in range(3):
                out[b, :, j, i] = X[b, :, (j % rf + 2 ** i) % rf]
    return out


def column_ref(X, d, kvc, col):
    x = torch.from_numpy(grouping_loops(X.double().numpy(), d.numpy()))
    x = F.pad(x, (0, 0, C, 0), value=SKIP).transpose(1, 2)  # [B, HC, T, 3]
    src = F.linear(x, col.in_w, col.in_b)
    src = torch.where((x == SKIP).all(dim=-1, keepdim=True), torch.full_like(src, SKIP), src)
    for b, blk in enumerate(col.blocks):
        skip = (src == SKIP).all(dim=-1, keepdim=True).all(dim=-2, keepdim=True)
        q = F.linear(ln64(src, blk.ln1_w, blk.ln1_b, blk.eps), blk.in_w[:E], blk.in_b[:E])
        Bn, HC, Tn, _ = q.shape
        a = O.pk_cross_ref(q.reshape(Bn * HC, Tn, E), kvc[b].reshape(Bn * HC, NI, 2 * E), H, None, None, None, 0.25)
        out = src + F.linear(torch.from_numpy(a).reshape(Bn, HC, Tn, E), blk.out_w, blk.out_b)
        src = torch.where(skip, torch.full_like(out, SKIP), ffn64(out, blk))
    return src


def row_ref(src, d, row, rope):
    Bn, HC, Tn, _ = src.shape
    x = src.transpose(1, 2)
    x = torch.cat([row.cls_tokens.expand(Bn, Tn, C, E), x[:, :, C:]], dim=2)
    kb = torch.zeros(Bn, HC, dtype=torch.float64)
    for b in range(Bn):
        kb[b, int(d[b]) + C:] = float(torch.finfo(torch.float32).min)
    kb_rows = kb[:, None, :].expand(Bn, Tn, HC).reshape(Bn * Tn, HC)
    tabs = O.rope_tables_ref(rope.freqs.double().numpy(), HC, E, H, False)
    tq = O.rope_tables_ref(rope.freqs.double().numpy(), C, E, H, False)
    for blk in row.blocks[:-1]:
        qkv = F.linear(ln64(x, blk.ln1_w, blk.ln1_b, blk.eps), blk.in_w, blk.in_b)
        a = O.pk_self_ref(qkv.reshape(Bn * Tn, HC, 3 * E), H, kb_rows, tabs, 0.25)
        x = ffn64(x + F.linear(torch.from_numpy(a).reshape(Bn, Tn, HC, E), blk.out_w, blk.out_b), blk)
    blk = row.blocks[-1]
    hk = ln64(x, blk.ln1_w, blk.ln1_b, blk.eps)
    q = F.linear(hk[:, :, :C], blk.in_w[:E], blk.in_b[:E])
    kv = F.linear(hk, blk.in_w[E:], blk.in_b[E:])
    a = O.pk_cross_ref(q.reshape(Bn * Tn, C, E), kv.reshape(Bn * Tn, HC, 2 * E), H, kb_rows, tq, tabs, 0.25)
    cls = ffn64(x[:, :, :C] + F.linear(torch.from_numpy(a).reshape(Bn, Tn, C, E), blk.out_w, blk.out_b), blk)
    cls = ln64(cls, row.out_ln_w, row.out_ln_b, row.eps)
    return cls.flatten(-2)


def _bf(t):
    return t.to(torch.bfloat16).float()


def icl_ref(x, blocks, kc, vc, valid, dec):
    """ICL blocks + decoder with the bf16 path's rounding points (bf16 GEMM inputs and outputs, fp32
    LayerNorm and residual stream), attention from the fp64 oracle."""
    x = x.float()
    En, Tq = x.shape[0], x.shape[1]
    for b, w in enumerate(blocks):
        h = _bf(F.layer_norm(x, (ICLW,), w.ln1_w.float(), w.ln1_b.float(), w.eps))
        q = _bf(h @ w.in_w[:ICLW].float().T + w.in_b[:ICLW].float()).view(En, Tq, ICLH, 64).transpose(1, 2)
        att = O.splash_sdpa_ref(q, kc[:, b].float(), vc[:, b].float(), valid)
        att = _bf(torch.from_numpy(att).float()).transpose(1, 2).reshape(En, Tq, ICLW)
        x = x + _bf(att @ w.out_w.float().T + w.out_b.float())
        h = _bf(F.layer_norm(x, (ICLW,), w.ln2_w.float(), w.ln2_b.float(), w.eps))
        f = _bf(F.gelu(_bf(h @ w.ff1_w.float().T + w.ff1_b.float())))
        x = x + _bf(f @ w.ff2_w.float().T + w.ff2_b.float())
    h = _bf(F.layer_norm(x, (ICLW,), dec.ln_w.float(), dec.ln_b.float(), dec.eps))
    f = _bf(F.gelu(_bf(h @ dec.w1.float().T + dec.b1.float())))
    return _bf(f @ dec.w2.float().T + dec.b2.float())
