"""Small-head multi-head attention dispatch for MI355X (TabICLv2 column / row stages: 8 heads x 16
dims; ICL stage: 8 heads x 64 dims over a cached K/V).

Drop-in for the reference's scripts/tabicl_tpu_mha.py: `install(attention_module, layers_module)`
patches upstream tabicl's `multi_head_attention_forward` (and `sdpa_with_flattened_batch` for the
cached-KV ICL attention) so that the attention itself runs in the HIP kernels of
libtabicl_attn.so (tabicl_mi355_attn / tabicl_mi355_icl), keeping the reference's routing order:

  HXF      inference first-ISAB attention with the K projection folded into the queries
           (folded_mab1 + hxf_attention; the K/V projection is never formed)   (reference :319-327)
  HXQ      inference first-ISAB attention (few queries over the train rows, keys >= valid ignored):
           q / packed K|V projections, SSMax on q, hxq_attention            (reference :328-342)
  fallback upstream for cached_kv / need_kv / dropout / valid_kv_len / head dim > MAX_HEAD_DIM /
           keys >= splash_min_kv / non-GPU tensors                            (reference :343-347)
  PACKED   packed projections + pk_self_attention / pk_cross_attention (RoPE, scale and key-only
           masks in the kernel)                                               (reference :350-371)
  layouts  small_head_attention(impl) with impl from pick_impl(mode, Lq, Lk)  (reference :372-385)
  ICL      sdpa_with_flattened_batch: cached-KV attention with d = 64 and no mask and no grad goes
           to icl_sdpa (the Splash hook's contract)                           (diff :261-265)

Knobs (same names as the reference where they select kernels):
  TABICL_TPU_MHA=hxq|hxk|thl|std|pk|hx|auto|<rules>, TABICL_TPU_MHA_MAX_HEAD_DIM (32),
  TABICL_TPU_MHA_PROJ=packed|split|views, TABICL_TPU_MHA_HXF=1, TABICL_TPU_MHA_HXQ=1, TABICL_TPU_MHA_PACKED=1,
  TABICL_TPU_MHA_ANY_DEVICE=1 (CPU equivalence tests: lets the wrapper's torch layouts run on CPU;
  the HIP kernels themselves never run on CPU tensors).
"""
from __future__ import annotations

import os
from typing import Optional

import torch
from torch import Tensor
from torch.nn import functional as F

_MODE = os.environ.get("TABICL_TPU_MHA", "").strip().lower()
_MAX_HEAD_DIM = int(os.environ.get("TABICL_TPU_MHA_MAX_HEAD_DIM", "32") or 32)
_ANY_DEVICE = os.environ.get("TABICL_TPU_MHA_ANY_DEVICE", "") == "1"
_PROJ = os.environ.get("TABICL_TPU_MHA_PROJ", "packed").strip().lower()
_HXQ = os.environ.get("TABICL_TPU_MHA_HXQ", "") == "1"
_HXF = os.environ.get("TABICL_TPU_MHA_HXF", "") == "1"
_PACKED = os.environ.get("TABICL_TPU_MHA_PACKED", "") == "1"
_ICL = os.environ.get("TABICL_MI355_ICL", "1") == "1"
_PK = None  # tabicl_mi355_attn, imported by install()
_ICL_MOD = None  # tabicl_mi355_icl, imported by install()
_DEVICE = "cuda"  # torch device type of the HIP kernels (ROCm builds report "cuda")


def in_projection(query: Tensor, key: Tensor, value: Tensor, w: Tensor, b: Optional[Tensor], proj: str):
    """q, k, v projections (reference scripts/tabicl_tpu_mha.py:95-111): "views" computes one matmul per
    distinct input and returns column views, "split" three matmuls on weight slices, otherwise
    torch's packed in-projection."""
    E = query.shape[-1]
    if proj == "views":
        if query is key and key is value:
            return F.linear(query, w, b).chunk(3, dim=-1)
        if key is value:
            w_q, w_kv = w.split([E, 2 * E])
            b_q, b_kv = (None, None) if b is None else b.split([E, 2 * E])
            k_p, v_p = F.linear(key, w_kv, b_kv).chunk(2, dim=-1)
            return F.linear(query, w_q, b_q), k_p, v_p
        proj = "split"
    if proj != "split":
        return F._in_projection_packed(query, key, value, w, b)
    w_q, w_k, w_v = w.split(E, dim=0)
    b_q, b_k, b_v = (None, None, None) if b is None else b.split(E)
    return F.linear(query, w_q, b_q), F.linear(key, w_k, b_k), F.linear(value, w_v, b_v)


def _head_mask(h: int, E: int, dtype: torch.dtype, device) -> Tensor:
    """[h, E] 0/1 selector of each head's d = E/h columns."""
    return torch.repeat_interleave(torch.eye(h, dtype=dtype, device=device), E // h, dim=1)


def _parse_rules(mode: str) -> dict:
    rules = {"col1": "hxq", "col2": "hxk", "row": "thl", "cls": "hxq"}
    for part in mode.split(","):
        if "=" in part:
            k, v = part.split("=", 1)
            rules[k.strip()] = v.strip()
    return rules


def pick_impl(mode: str, Lq: int, Lk: int) -> str:
    """Layout choice (reference :129-141): pk keeps CLS (Lq <= 16) on the torch path; hx picks
    query- or key-expansion by shape; rules map col1 (Lq < Lk), col2 (Lq > Lk), row (Lq == Lk),
    cls (Lq <= 16)."""
    if mode == "pk":
        return "std" if Lq <= 16 else "pk"
    if mode in ("hxq", "hxk", "thl", "std"):
        return mode
    if mode == "hx":
        return "hxq" if Lq <= Lk else "hxk"
    rules = _parse_rules(mode if "=" in mode else "")
    if Lq <= 16:
        return rules["cls"]
    if Lq == Lk:
        return rules["row"]
    return rules["col1"] if Lq < Lk else rules["col2"]


def small_head_attention(q: Tensor, k: Tensor, v: Tensor, h: int, mask: Optional[Tensor], impl: str) -> Tensor:
    """q [..., Lq, E] (already scaled), k / v [..., Lk, E]; additive mask broadcastable to
    [..., h|1, Lq|1, Lk] (reference :144-198). All impls compute per-head softmax(q_g k_g^T + mask) v_g
    with an fp32 softmax; "pk" runs the HIP kernel for key-only masks and otherwise uses "std"."""
    Lq, E = q.shape[-2], q.shape[-1]
    Lk = k.shape[-2]
    d = E // h
    if impl == "pk":
        if _PK is None or q.device.type != _DEVICE:
            return small_head_attention(q, k, v, h, mask, "std")
        kb = None
        if mask is not None:
            if mask.shape[-3] != 1 or mask.shape[-2] != 1:
                return small_head_attention(q, k, v, h, mask, "std")
            kb = mask.reshape(*mask.shape[:-3], Lk)
        if not _PK.supported(Lq, Lk, E, h, q.dtype):
            return small_head_attention(q, k, v, h, mask, "std")
        return _PK.hx_attention(q, k, v, h, kb)
    if impl == "hxq":  # query-head expansion: row block g of the expanded queries sees only head g
        M = _head_mask(h, E, q.dtype, q.device)
        q_exp = (q.unsqueeze(-3) * M[:, None, :]).reshape(*q.shape[:-2], h * Lq, E)
        s = (q_exp @ k.transpose(-2, -1)).float().reshape(*q.shape[:-2], h, Lq, Lk)
        if mask is not None:
            s = s + mask
        p = torch.softmax(s, dim=-1).to(v.dtype).reshape(*q.shape[:-2], h * Lq, Lk)
        o_full = (p @ v).reshape(*q.shape[:-2], h, Lq, E)
        return (o_full * M.to(o_full.dtype)[:, None, :]).sum(dim=-3)
    if impl == "hxk":  # key-head expansion: column block g of the scores belongs to head g
        M = _head_mask(h, E, k.dtype, k.device)
        k_exp = (k.unsqueeze(-3) * M[:, None, :]).reshape(*k.shape[:-2], h * Lk, E)
        v_exp = (v.unsqueeze(-3) * M.to(v.dtype)[:, None, :]).reshape(*v.shape[:-2], h * Lk, E)
        s = (q @ k_exp.transpose(-2, -1)).float().reshape(*q.shape[:-2], Lq, h, Lk)
        if mask is not None:
            s = s + mask.transpose(-3, -2)
        p = torch.softmax(s, dim=-1).to(v.dtype).reshape(*q.shape[:-2], Lq, h * Lk)
        return p @ v_exp
    if impl == "thl":  # transposed head layout: sequence on the last axis
        qt = q.transpose(-2, -1).reshape(*q.shape[:-2], h, d, Lq)
        kt = k.transpose(-2, -1).reshape(*k.shape[:-2], h, d, Lk)
        vt = v.transpose(-2, -1).reshape(*v.shape[:-2], h, d, Lk)
        s = (qt.transpose(-2, -1) @ kt).float()
        if mask is not None:
            s = s + mask
        p = torch.softmax(s, dim=-1).to(v.dtype)
        return (vt @ p.transpose(-2, -1)).reshape(*q.shape[:-2], E, Lq).transpose(-2, -1)
    if impl == "std":  # head split, matmul, fp32 softmax, matmul
        qh = q.reshape(*q.shape[:-1], h, d).transpose(-3, -2)
        kh = k.reshape(*k.shape[:-1], h, d).transpose(-3, -2)
        vh = v.reshape(*v.shape[:-1], h, d).transpose(-3, -2)
        s = (qh @ kh.transpose(-2, -1)).float()
        if mask is not None:
            s = s + mask
        p = torch.softmax(s, dim=-1).to(vh.dtype)
        return (p @ vh).transpose(-3, -2).reshape(*q.shape[:-1], E)
    raise ValueError(f"unknown small-head attention impl {impl!r}")


def rope_merged(rope, x: Tensor, h: int) -> Tensor:  # noqa: ANN001
    """RotaryEmbedding.rotate_queries_or_keys for merged-head x [..., L, E]: x*cos + R(x)*sin per
    head, R the signed rotate-half (pairs or halves), computed in fp32 and cast back
    (reference :201-248, "roll" form)."""
    L, E = x.shape[-2], x.shape[-1]
    import tabicl_mi355_attn as pk

    cos, sin, code, half, rot = pk.rope_tables(rope, L, E, h, x.device)
    if code == 0:
        return x
    d = E // h
    xf = x.float().reshape(*x.shape[:-1], h, d)
    rx = torch.zeros_like(xf)
    if code == 1:
        rx[..., 0:rot:2] = -xf[..., 1:rot:2]
        rx[..., 1:rot:2] = xf[..., 0:rot:2]
    else:
        rx[..., :half] = -xf[..., half:rot]
        rx[..., half:rot] = xf[..., :half]
    out = xf.reshape(x.shape) * cos + rx.reshape(x.shape) * sin
    return out.to(x.dtype)


def _combined_mask(attn_mask, key_padding_mask, batch_shape, nh: int, Lq: int, Lk: int, qdtype):  # noqa: ANN001
    """Upstream mask processing -> additive mask broadcastable to (*batch, nh, Lq, Lk); None if absent;
    False for bool masks and shapes that do not broadcast (caller falls back) (reference :251-290)."""
    nb = len(batch_shape)
    full = (*batch_shape, nh, Lq, Lk)
    m = None
    if attn_mask is not None:
        if attn_mask.dtype == torch.bool:
            return False
        if attn_mask.dim() == 2:
            if tuple(attn_mask.shape) != (Lq, Lk):
                return False
            m = attn_mask.view(*([1] * nb), 1, Lq, Lk)
        elif attn_mask.dim() == 4 and nb != 1 and tuple(attn_mask.shape[:3]) == (1, 1, 1) and attn_mask.shape[-1] == Lk:
            m = attn_mask.view(*([1] * nb), 1, 1, Lk)
        elif attn_mask.dim() == len(full):
            if any(g not in (1, e) for g, e in zip(attn_mask.shape, full)):
                return False
            m = attn_mask
        else:
            return False
    if key_padding_mask is not None:
        kp = key_padding_mask
        if kp.dtype == torch.bool:
            return False
        if not (tuple(kp.shape) == (1, Lk) or (kp.dim() == nb + 1 and kp.shape[-1] == Lk)):
            return False
        if any(g not in (1, e) for g, e in zip(kp.shape[:-1], batch_shape)):
            return False
        kpm = kp.view(*([1] * nb), 1, 1, Lk) if (kp.dim() == 2 and nb != 1) else kp.view(*kp.shape[:-1], 1, 1, Lk)
        m = kpm if m is None else m + kpm
    if m is not None:
        if m.dtype != qdtype:
            m = m.to(dtype=qdtype)
        m = m.float()
    return m


def folded_mab1(query: Tensor, key: Tensor, valid_kv_len: Tensor, num_heads: int, in_proj_weight: Tensor,
                in_proj_bias: Optional[Tensor], ssmax_layer=None, src_len_override=None, pk=None) -> Optional[Tensor]:  # noqa: ANN001
    """Folded first-ISAB attention (reference scripts/tabicl_tpu_mha.py:60-92): softmax(q_g K_g^T) V_g
    for every head, merged [..., Lq, E] before the output projection, with K = key W_k^T + b_k and
    V = key W_v^T + b_v never formed: U = softmax(Qf key^T) key with Qf_g = q_g W_k,g (q pre-scaled;
    q_g . b_k,g is constant per query row, so softmax drops it), then O_g = U_g W_v,g^T + b_v,g (rows
    of P sum to 1). None when the kernel does not apply."""
    pk = pk if pk is not None else _PK
    E = query.shape[-1]
    hd = E // num_heads
    qsrc = query
    while qsrc.dim() > 2 and qsrc.stride(0) == 0:  # inducing points expanded over the batch: fold once
        qsrc = qsrc[0]
    Lq = qsrc.shape[-2]
    nb_q = qsrc.shape[:-2].numel()
    nb_k = key.shape[:-2].numel()
    if pk is None or nb_q not in (1, nb_k) or not pk.hxf_supported(num_heads * Lq, key.shape[-2], E):
        return None
    w_q, w_k, w_v = in_proj_weight.split([E, E, E])
    b_q, _b_k, b_v = (None, None, None) if in_proj_bias is None else in_proj_bias.split([E, E, E])
    q = F.linear(qsrc, w_q, b_q)
    if ssmax_layer is not None:
        q = _ssmax(ssmax_layer, q, num_heads, src_len_override if src_len_override is not None else valid_kv_len)
    q = q * (hd ** -0.5)
    # Qf[.., g, i, :] = q[.., i, g, :] @ W_k,g  ([hd] x [hd, E]); batched over heads, right operand contiguous
    qh = q.unflatten(-1, (num_heads, hd)).transpose(-3, -2)
    qf = torch.matmul(qh, w_k.reshape(num_heads, hd, E).contiguous())
    u = pk.hxf_attention(qf.flatten(-3, -2), key, valid_kv_len)  # [*key_lead, h * Lq, E]
    # O[.., i, g, :] = U[.., g, i, :] @ W_v,g^T
    uh = u.unflatten(-2, (num_heads, Lq))
    o = torch.matmul(uh, w_v.reshape(num_heads, hd, E).transpose(-1, -2).contiguous().to(uh.dtype))
    o = o.transpose(-3, -2).flatten(-2, -1)
    return o + b_v if b_v is not None else o


def _ssmax(ssmax_layer, q: Tensor, num_heads: int, n) -> Tensor:  # noqa: ANN001
    hd = q.shape[-1] // num_heads
    qh = q.unflatten(-1, (num_heads, hd)).transpose(-3, -2)
    return ssmax_layer(qh.reshape(-1, *qh.shape[-3:]), n).view(qh.shape).transpose(-3, -2).flatten(-2, -1)


def install(att_module, layers_module=None, mode: Optional[str] = None, proj: Optional[str] = None) -> bool:  # noqa: ANN001
    """Patch `multi_head_attention_forward` in att_module (and layers_module, which imports it by
    name) and `sdpa_with_flattened_batch` for the ICL path (reference :293-393)."""
    mode = (_MODE if mode is None else mode).strip().lower()
    proj = (_PROJ if proj is None else proj).strip().lower()
    if not mode or mode in ("0", "off", "none"):
        return False
    if getattr(att_module, "_mi355_mha_installed", False):
        return True
    global _PK, _ICL_MOD
    import tabicl_mi355_attn as _pk_mod  # registers the tabicl_pk:: ops eagerly (never while tracing)
    import tabicl_mi355_icl as _icl_mod

    _PK, _ICL_MOD = _pk_mod, _icl_mod
    orig = att_module.multi_head_attention_forward
    splash_min_kv = getattr(att_module, "_tpu_splash_min_kv", lambda: int(os.environ.get("TABICL_TPU_SPLASH_MIN_KV", "16384")))

    def multi_head_attention_forward(query, num_heads, in_proj_weight, in_proj_bias, dropout_p,  # noqa: ANN001
                                     out_proj_weight, out_proj_bias, key=None, value=None, cached_kv=None,
                                     training=True, key_padding_mask=None, attn_mask=None, rope=None,
                                     ssmax_layer=None, need_kv=False, src_len_override=None, valid_kv_len=None):
        def _orig():
            return orig(query, num_heads, in_proj_weight, in_proj_bias, dropout_p, out_proj_weight, out_proj_bias,
                        key=key, value=value, cached_kv=cached_kv, training=training,
                        key_padding_mask=key_padding_mask, attn_mask=attn_mask, rope=rope, ssmax_layer=ssmax_layer,
                        need_kv=need_kv, src_len_override=src_len_override, valid_kv_len=valid_kv_len)

        E = query.shape[-1]
        hd = E // num_heads
        on_gpu = query.device.type == _DEVICE
        if (_HXF and isinstance(valid_kv_len, Tensor) and not torch.is_grad_enabled() and cached_kv is None
                and not need_kv and key is not None and key is value and rope is None and attn_mask is None
                and key_padding_mask is None and hd <= _MAX_HEAD_DIM and on_gpu
                and (not isinstance(src_len_override, Tensor) or src_len_override.numel() == 1)):
            o = folded_mab1(query, key, valid_kv_len, num_heads, in_proj_weight, in_proj_bias, ssmax_layer,
                            src_len_override)
            if o is not None:
                return F.linear(o, out_proj_weight, out_proj_bias)
        if (_HXQ and isinstance(valid_kv_len, Tensor) and not torch.is_grad_enabled() and cached_kv is None
                and not need_kv and key is not None and key is value and rope is None and attn_mask is None
                and key_padding_mask is None and hd <= _MAX_HEAD_DIM and on_gpu
                and _PK.hxq_supported(query.shape[-2], key.shape[-2], E, num_heads, query.dtype)):
            w_q, w_kv = in_proj_weight.split([E, 2 * E])
            b_q, b_kv = (None, None) if in_proj_bias is None else in_proj_bias.split([E, 2 * E])
            q = F.linear(query, w_q, b_q)
            kv = F.linear(key, w_kv, b_kv)  # [.., Lk, 2E]: K columns [0, E), V columns [E, 2E)
            if ssmax_layer is not None:
                q = _ssmax(ssmax_layer, q, num_heads, src_len_override if src_len_override is not None else valid_kv_len)
            out = _PK.hxq_attention(q * (hd ** -0.5), kv, valid_kv_len, num_heads)
            return F.linear(out, out_proj_weight, out_proj_bias)
        if ((not on_gpu and not _ANY_DEVICE) or cached_kv is not None or need_kv or key is None or value is None
                or hd > _MAX_HEAD_DIM or (training and dropout_p > 0.0) or valid_kv_len is not None
                or getattr(att_module, "_tpu_flash_attention_fn", None) is not None
                or key.shape[-2] >= splash_min_kv()):
            return _orig()
        *batch_shape, Lq, _ = query.shape
        Lk = key.shape[-2]
        if _PACKED and on_gpu and pick_impl(mode, Lq, Lk) == "pk" and key is value:
            self_attn = query is key
            if _PK.packed_supported(Lq, Lk, E, num_heads, self_attn, query.dtype):
                mask = _combined_mask(attn_mask, key_padding_mask, batch_shape, num_heads, Lq, Lk, query.dtype)
                kb = None
                if mask is not None and mask is not False:
                    kb = mask.reshape(*mask.shape[:-3], Lk) if mask.shape[-3] == 1 and mask.shape[-2] == 1 else False
                if mask is not False and kb is not False:
                    if self_attn:
                        qkv = F.linear(query, in_proj_weight, in_proj_bias)
                        out = _PK.pk_self_attention(qkv, num_heads, kb, rope, hd ** -0.5)
                    else:
                        w_q, w_kv = in_proj_weight.split([E, 2 * E])
                        b_q, b_kv = (None, None) if in_proj_bias is None else in_proj_bias.split([E, 2 * E])
                        qp = F.linear(query, w_q, b_q)
                        kv = F.linear(key, w_kv, b_kv)
                        if ssmax_layer is not None:
                            qp = _ssmax(ssmax_layer, qp, num_heads, src_len_override if src_len_override is not None else Lk)
                        out = _PK.pk_cross_attention(qp, kv, num_heads, kb, rope, hd ** -0.5)
                    return F.linear(out, out_proj_weight, out_proj_bias)
        q, k, v = in_projection(query, key, value, in_proj_weight, in_proj_bias, proj)
        mask = _combined_mask(attn_mask, key_padding_mask, batch_shape, num_heads, Lq, Lk, q.dtype)
        if mask is False:
            return _orig()
        if rope is not None:
            q = rope_merged(rope, q, num_heads)
            k = rope_merged(rope, k, num_heads)
        if ssmax_layer is not None:
            q = _ssmax(ssmax_layer, q, num_heads, src_len_override if src_len_override is not None else Lk)
        out = small_head_attention(q * (hd ** -0.5), k, v, num_heads, mask, pick_impl(mode, Lq, Lk))
        return F.linear(out, out_proj_weight, out_proj_bias)

    att_module.multi_head_attention_forward = multi_head_attention_forward
    if layers_module is not None:
        layers_module.multi_head_attention_forward = multi_head_attention_forward
    if _ICL and hasattr(att_module, "sdpa_with_flattened_batch"):
        att_module.sdpa_with_flattened_batch = _wrap_sdpa(att_module.sdpa_with_flattened_batch, splash_min_kv)
    att_module._mi355_mha_installed = True
    att_module._mi355_mha_mode = mode
    att_module._mi355_mha_proj = proj
    return True


def _wrap_sdpa(orig_sdpa, splash_min_kv):  # noqa: ANN001
    """sdpa_with_flattened_batch with the Splash branch of the reference patch (diff:261-265) on the
    HIP ICL kernel: GPU tensors, no dropout, no mask, no grad, long keys (>= splash_min_kv) or a
    valid length, head dim 64 -> SSMax on q (diff:251-254), then icl_sdpa(q, k, v, valid_kv_len)."""

    def sdpa_with_flattened_batch(q, k, v, attn_mask=None, dropout_p=0.0, ssmax_layer=None,  # noqa: ANN001
                                  src_len_override=None, valid_kv_len=None):
        if (q.device.type == _DEVICE and dropout_p == 0.0 and attn_mask is None and not torch.is_grad_enabled()
                and (k.shape[-2] >= splash_min_kv() or valid_kv_len is not None)
                and q.dtype in (torch.bfloat16, torch.float32) and q.dtype == k.dtype == v.dtype
                and _ICL_MOD.icl_supported(q.shape[-2], k.shape[-2], q.shape[-1], q.dtype)):
            lead = q.shape[:-3]
            q3 = q.reshape(-1, *q.shape[-3:])
            if ssmax_layer is not None:
                q3 = ssmax_layer(q3, src_len_override if src_len_override is not None else k.size(-2))
            out = _ICL_MOD.icl_sdpa(q3, k.reshape(-1, *k.shape[-3:]), v.reshape(-1, *v.shape[-3:]), valid_kv_len)
            return out.reshape(*lead, *out.shape[-3:])
        return orig_sdpa(q, k, v, attn_mask, dropout_p, ssmax_layer=ssmax_layer,
                         src_len_override=src_len_override, valid_kv_len=valid_kv_len)

    return sdpa_with_flattened_batch
