"""Test stand-in for the parts of upstream tabicl (2.2.0, as patched by the reference's
results/tpu_patch.diff) that the dispatch wrapper patches or is called from: a module-like namespace
with `multi_head_attention_forward` and `sdpa_with_flattened_batch`, the attention part of
`MultiheadAttentionBlock.forward` (`block_attention`), plus a RotaryEmbedding-like object.
Upstream is not vendored in the reference; this restates the behaviour the diff shows
(diff:196-281 sdpa routing and SSMax, diff:283-395 projections, RoPE, mask processing, cached K/V,
diff:1509-1542 the block's handling of a tensor train size / valid_kv_len) with plain torch math.
Test infrastructure only."""
from __future__ import annotations

import types
import torch
import torch.nn.functional as F
from torch import Tensor


class RopeStub:
    """RotaryEmbedding surface used by the reference (get_seq_pos, interleaved, freqs, forward,
    rotate_queries_or_keys on head-split [..., L, d]); textbook frequencies base^(-2i/dim)."""

    def __init__(self, dim: int = 16, theta: float = 100000.0, interleaved: bool = False):
        self.interleaved = interleaved
        self.freqs = theta ** (-torch.arange(0, dim, 2, dtype=torch.float32) / dim)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)

    def forward(self, seq, seq_len=None):
        f = seq.float().unsqueeze(-1) * self.freqs.to(seq.device)
        return f.repeat_interleave(2, dim=-1)

    def rotate_queries_or_keys(self, x: Tensor) -> Tensor:
        L, d = x.shape[-2], x.shape[-1]
        pos = torch.arange(L, device=x.device, dtype=torch.float32)
        f = pos[:, None] * self.freqs.to(x.device)[None, :]
        ang = f.repeat_interleave(2, dim=-1) if self.interleaved else torch.cat([f, f], dim=-1)
        rot = ang.shape[-1]
        xf = x.float()
        xr, xp = xf[..., :rot], xf[..., rot:]
        if self.interleaved:
            r = torch.stack([-xr[..., 1::2], xr[..., 0::2]], dim=-1).flatten(-2)
        else:
            r = torch.cat([-xr[..., rot // 2:], xr[..., :rot // 2]], dim=-1)
        out = torch.cat([xr * ang.cos() + r * ang.sin(), xp], dim=-1)
        return out.to(x.dtype)


class SSMaxStub(torch.nn.Module):
    """q * (s_h * log n) per head: stands in for the QASSMax layer (applied to q before attention)."""

    def __init__(self, nh: int):
        super().__init__()
        self.s = torch.linspace(0.5, 1.0, nh)

    def forward(self, q: Tensor, n) -> Tensor:
        n = torch.as_tensor(n, dtype=torch.float32, device=q.device)
        return q * (self.s.to(q.device)[:, None, None] * torch.log(n)).to(q.dtype)


def sdpa_with_flattened_batch(q, k, v, attn_mask=None, dropout_p=0.0, ssmax_layer=None, src_len_override=None,
                              valid_kv_len=None):
    lead = q.shape[:-3]
    q = q.reshape(-1, *q.shape[-3:])
    k = k.reshape(-1, *k.shape[-3:])
    v = v.reshape(-1, *v.shape[-3:])
    if attn_mask is not None and attn_mask.dim() >= 4:
        attn_mask = attn_mask.reshape(-1, *attn_mask.shape[-3:]) if attn_mask.shape[:-3].numel() > 1 else \
            attn_mask.reshape(1, *attn_mask.shape[-3:])
    if ssmax_layer is not None:
        q = ssmax_layer(q, src_len_override if src_len_override is not None else k.size(-2))
    s = (q.float() * q.shape[-1] ** -0.5) @ k.float().transpose(-2, -1)
    if attn_mask is not None:
        s = s + attn_mask.float()
    if valid_kv_len is not None:
        keep = torch.arange(k.shape[-2], device=q.device) < torch.as_tensor(valid_kv_len, device=q.device).reshape(-1, 1, 1, 1)
        s = s.masked_fill(~keep, float("-inf"))
    out = (torch.softmax(s, dim=-1) @ v.float()).to(q.dtype)
    return out.reshape(*lead, *out.shape[-3:])


def make_module():
    mod = types.SimpleNamespace()
    mod._tpu_splash_min_kv = lambda: 16384
    mod.sdpa_with_flattened_batch = sdpa_with_flattened_batch

    def multi_head_attention_forward(query, num_heads, in_proj_weight, in_proj_bias, dropout_p, out_proj_weight,
                                     out_proj_bias, key=None, value=None, cached_kv=None, training=True,
                                     key_padding_mask=None, attn_mask=None, rope=None, ssmax_layer=None, need_kv=False,
                                     src_len_override=None, valid_kv_len=None):
        key = query if key is None else key
        value = key if value is None else value
        *batch_shape, tgt_len, E = query.shape
        hd = E // num_heads
        if cached_kv is None:
            q, k, v = F._in_projection_packed(query, key, value, in_proj_weight, in_proj_bias)
            src_len = k.shape[-2]
            q = q.view(*batch_shape, tgt_len, num_heads, hd).transpose(-3, -2)
            k = k.view(*batch_shape, src_len, num_heads, hd).transpose(-3, -2)
            v = v.view(*batch_shape, src_len, num_heads, hd).transpose(-3, -2)
            if rope is not None:
                q = rope.rotate_queries_or_keys(q)
                k = rope.rotate_queries_or_keys(k)
        else:
            q = F.linear(query, in_proj_weight[:E], None if in_proj_bias is None else in_proj_bias[:E])
            q = q.view(*batch_shape, tgt_len, num_heads, hd).transpose(-3, -2)
            if rope is not None:
                q = rope.rotate_queries_or_keys(q)
            dt = torch.promote_types(q.dtype, cached_kv.key.dtype)
            q, k, v = q.to(dt), cached_kv.key.to(dt), cached_kv.value.to(dt)
            src_len = k.shape[-2]
        mask = None
        if attn_mask is not None:
            mask = attn_mask.view(*([1] * len(batch_shape)), 1, tgt_len, src_len) if attn_mask.dim() == 2 else attn_mask
        if key_padding_mask is not None:
            kpm = key_padding_mask.view(*key_padding_mask.shape[:-1], 1, 1, src_len)
            mask = kpm if mask is None else mask + kpm
        if mask is not None and mask.dtype != torch.bool and mask.dtype != q.dtype:
            mask = mask.to(dtype=q.dtype)  # diff:370-371 (a finfo(float32).min entry becomes -inf in bf16)
        out = mod.sdpa_with_flattened_batch(q, k, v, mask, dropout_p, ssmax_layer=ssmax_layer,
                                            src_len_override=src_len_override, valid_kv_len=valid_kv_len)
        out = out.transpose(-3, -2).contiguous().view(*batch_shape, tgt_len, E)
        out = F.linear(out, out_proj_weight, out_proj_bias)
        if need_kv:
            return out, k, v
        return out

    mod.multi_head_attention_forward = multi_head_attention_forward
    return mod


class KVEntry:
    def __init__(self, key: Tensor, value: Tensor):
        self.key, self.value = key, value


def weights(E: int, seed: int, device="cpu", dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(3 * E, E, generator=g) * E ** -0.5).to(device=device, dtype=dtype)
    b = (torch.randn(3 * E, generator=g) * 0.1).to(device=device, dtype=dtype)
    wo = (torch.randn(E, E, generator=g) * E ** -0.5).to(device=device, dtype=dtype)
    bo = (torch.randn(E, generator=g) * 0.1).to(device=device, dtype=dtype)
    return w, b, wo, bo


def call(fn, query, key, value, nh, w, b, wo, bo, **kw) -> Tensor:
    return fn(query, nh, w, b, 0.0, wo, bo, key=key, value=value, training=False, **kw)



def splash_min_kv() -> int:
    return 16384


def block_attention(mod, q, num_heads, w, b, wo, bo, k=None, v=None, cached_kv=None, train_size=None,  # noqa: ANN001
                    key_padding_mask=None, attn_mask=None, rope=None, ssmax_layer=None, src_len_override=None,
                    valid_kv_len=None):
    """The attention call of MultiheadAttentionBlock.forward as patched (diff:1509-1565), norms and the
    feed-forward part left out (the inputs count as already normalised):
      * a tensor train_size makes k = v = q and sets src_len_override / valid_kv_len to it (:1512-1517);
      * a tensor valid_kv_len is kept only on the reference's device ("tpu") with no grad, no other
        mask and at least splash_min_kv keys; everywhere else it becomes an additive mask, 0 for key
        positions below it and finfo(q.dtype).min from there on, of shape [1, .., 1, 1, src_len]
        (q.dim() - 2 leading ones), added to attn_mask, and valid_kv_len is cleared (:1526-1542).
    Then the module's multi_head_attention_forward is looked up and called, as layers.py does."""
    if train_size is None:
        k = q if k is None else k
        v = q if v is None else v
    elif isinstance(train_size, Tensor):
        k = v = q
        src_len_override = train_size if src_len_override is None else src_len_override
        valid_kv_len = train_size if valid_kv_len is None else valid_kv_len
    else:
        k = v = q[..., :train_size, :]
    src_seq_len = cached_kv.key.shape[-2] if cached_kv is not None else k.shape[-2]
    if isinstance(valid_kv_len, Tensor):
        keep = (q.device.type == "tpu" and not torch.is_grad_enabled() and attn_mask is None
                and key_padding_mask is None and src_seq_len >= splash_min_kv())
        if not keep:
            pos = torch.arange(src_seq_len, device=q.device)
            train_mask = torch.where(pos < valid_kv_len, torch.zeros((), dtype=q.dtype, device=q.device),
                                     torch.full((), torch.finfo(q.dtype).min, dtype=q.dtype, device=q.device))
            train_mask = train_mask.view(*([1] * (q.dim() - 2)), 1, 1, src_seq_len)
            attn_mask = train_mask if attn_mask is None else attn_mask + train_mask
            valid_kv_len = None
    if cached_kv is not None:
        return mod.multi_head_attention_forward(q, num_heads, w, b, 0.0, wo, bo, cached_kv=cached_kv, training=False,
                                                key_padding_mask=key_padding_mask, attn_mask=attn_mask, rope=rope,
                                                ssmax_layer=ssmax_layer, src_len_override=src_len_override,
                                                valid_kv_len=valid_kv_len)
    return mod.multi_head_attention_forward(q, num_heads, w, b, 0.0, wo, bo, key=k, value=v, training=False,
                                            key_padding_mask=key_padding_mask, attn_mask=attn_mask, rope=rope,
                                            ssmax_layer=ssmax_layer, src_len_override=src_len_override,
                                            valid_kv_len=valid_kv_len)
