"""Attention dispatch of TabICLv2 on MI355X: the plugin boundary between upstream tabicl's attention
and the HIP kernels of libtabicl_attn.so.

`install(attention_module, layers_module)` is the drop-in for the reference's install
(scripts/tabicl_tpu_mha.py:293-393): it replaces upstream's `multi_head_attention_forward` (in both
modules: layers.py imports it by name) and, for the 8 x 64 ICL attention, the module's
`sdpa_with_flattened_batch` (whose Splash branch the reference hooks, results/tpu_patch.diff:261-281).

Routing contract kept from the reference (same knobs, same order, same fallbacks), with one route
ahead of it:
  0. small heads over cached K/V            TABICL_TPU_MHA_CACHED (default 1; no counterpart in the
     reference, whose route 3 sends these calls to upstream torch): the column blocks' second
     attention at query time (test rows over the cached inducing-point K/V)
  1. folded first-ISAB attention            TABICL_TPU_MHA_HXF=1      (reference :319-327)
  2. few queries over the train rows        TABICL_TPU_MHA_HXQ=1      (reference :328-342)
  3. upstream for: cached K/V (its attention reaches the ICL hook below), K/V requested back,
     dropout in training, head dim > TABICL_TPU_MHA_MAX_HEAD_DIM, a registered flash fn,
     keys >= the Splash threshold, tensors off the GPU                (reference :343-347)
  4. packed projections + fused kernels     TABICL_TPU_MHA_PACKED=1 and the mode picks "pk"
                                                                       (reference :350-371)
  5. the mode's small-head implementation   TABICL_TPU_MHA=<mode>     (reference :372-385)
The ICL hook sends every d = 64 attention without gradient, dropout or a non-key mask to the HIP
kernel (the reference: keys >= TABICL_TPU_SPLASH_MIN_KV without a mask, diff:263-265), and the
module's `_tpu_splash_sdpa_seg_op` / `_tpu_splash_sdpa_full_op` attributes (the reference's Splash
ops, diff:95-115) are bound to the same kernel under the reference's op names.

Where this differs from the reference, and why:
  * A key-validity length reaches routes 1, 2 and the ICL hook either as a tensor `valid_kv_len`
    (what upstream passes on the reference's device) or as the additive train mask upstream builds
    from it on every other device, this one included (diff:1526-1542: 0 below the train size,
    finfo.min after). Both routes and the hook take any key-only additive mask; the kernels read a
    mask of that prefix form as a valid length on the device and add any other mask term by term.
  * The reference's torch layouts hxq / hxk / thl keep a wide axis on TPU lanes; on this GPU they
    are the same math as upstream's own attention, so route 5 defers to upstream for every mode but
    "pk" (small_head_attention keeps the names and a single torch implementation for them).

Knobs (names of the reference): TABICL_TPU_MHA=hxq|hxk|thl|std|pk|hx|auto|<rules>,
TABICL_TPU_MHA_MAX_HEAD_DIM (32), TABICL_TPU_MHA_PROJ (accepted; every form computes the same
projections here), TABICL_TPU_MHA_HXF, _HXQ, _PACKED, _CACHED, TABICL_MI355_HXF_FORCE (route 1 runs the
folded kernel even where projection + hxq takes the call, which is faster here), TABICL_TPU_MHA_ANY_DEVICE (lets route 5's
torch math run on CPU tensors in tests; the HIP kernels never run on CPU tensors), TABICL_MI355_ICL
(default 1: install the ICL hook).
"""
from __future__ import annotations

import dataclasses
import math
import os
from dataclasses import dataclass
from typing import Optional

import torch
from torch import Tensor
from torch.nn import functional as F


def _env_flag(name: str, default: str = "") -> bool:
    return os.environ.get(name, default) == "1"


@dataclass
class Knobs:
    mode: str = os.environ.get("TABICL_TPU_MHA", "").strip().lower()
    max_head_dim: int = int(os.environ.get("TABICL_TPU_MHA_MAX_HEAD_DIM", "32") or 32)
    proj: str = os.environ.get("TABICL_TPU_MHA_PROJ", "packed").strip().lower()
    folded: bool = _env_flag("TABICL_TPU_MHA_HXF")
    few_queries: bool = _env_flag("TABICL_TPU_MHA_HXQ")
    packed: bool = _env_flag("TABICL_TPU_MHA_PACKED")
    cached: bool = _env_flag("TABICL_TPU_MHA_CACHED", "1")
    folded_force: bool = _env_flag("TABICL_MI355_HXF_FORCE")
    any_device: bool = _env_flag("TABICL_TPU_MHA_ANY_DEVICE")
    icl_hook: bool = _env_flag("TABICL_MI355_ICL", "1")


KNOBS = Knobs()
_DEVICE = "cuda"  # torch device type of the HIP kernels (ROCm builds report "cuda")
_PK = None  # tabicl_mi355_attn, bound by install() (imported eagerly, never while tracing)
_ICL = None  # tabicl_mi355_icl, bound by install()

_CLS_MAX_Q = 16  # query sets this short are the row stage's CLS tokens in the mode rules


# ---------------------------------------------------------------------------------------------
# mode rules (which calls the "pk" kernels serve)
# ---------------------------------------------------------------------------------------------
_DEFAULT_RULES = {"col1": "hxq", "col2": "hxk", "row": "thl", "cls": "hxq"}
_SINGLE_IMPLS = ("hxq", "hxk", "thl", "std")


def _rule_table(mode: str) -> dict:
    table = dict(_DEFAULT_RULES)
    for item in mode.split(","):
        name, sep, impl = item.partition("=")
        if sep:
            table[name.strip()] = impl.strip()
    return table


def pick_impl(mode: str, Lq: int, Lk: int) -> str:
    """Small-head implementation of a call with Lq queries and Lk keys under a TABICL_TPU_MHA mode
    (reference scripts/tabicl_tpu_mha.py:129-141): "pk" serves everything but CLS-sized query sets;
    a single impl name applies to all; "hx" picks by the longer side; otherwise per-role rules
    (cls: Lq <= 16, row: Lq == Lk, col1: Lq < Lk, col2: Lq > Lk)."""
    if mode == "pk":
        return "pk" if Lq > _CLS_MAX_Q else "std"
    if mode in _SINGLE_IMPLS:
        return mode
    if mode == "hx":
        return "hxk" if Lq > Lk else "hxq"
    table = _rule_table(mode) if "=" in mode else dict(_DEFAULT_RULES)
    role = "cls" if Lq <= _CLS_MAX_Q else "row" if Lq == Lk else "col1" if Lq < Lk else "col2"
    return table[role]


# ---------------------------------------------------------------------------------------------
# masks
# ---------------------------------------------------------------------------------------------
def _as_rank(m: Tensor, nb: int, Lq: int, Lk: int) -> Optional[Tensor]:
    """attn_mask as a view of rank nb + 3 broadcastable to (*batch, h, Lq, Lk) under upstream's rules
    (results/tpu_patch.diff:327-346), or None if upstream would reject it."""
    rank = nb + 3
    if m.dim() == 2:
        return m.view(*([1] * (rank - 2)), Lq, Lk) if tuple(m.shape) == (Lq, Lk) else None
    if m.dim() == 4 and nb != 1 and tuple(m.shape[:3]) == (1, 1, 1) and m.shape[-1] == Lk:
        return m.view(*([1] * (rank - 1)), Lk)
    if m.dim() == rank:
        return m
    return None


def _kpm_as_rank(kp: Tensor, batch_shape, nb: int, Lk: int) -> Optional[Tensor]:
    """key_padding_mask as a view of rank nb + 3 (diff:352-366), or None if upstream would reject it."""
    if kp.shape[-1] != Lk or not (tuple(kp.shape) == (1, Lk) or kp.dim() == nb + 1):
        return None
    lead = tuple(kp.shape[:-1])
    if kp.dim() == 2 and nb != 1:  # one shared row
        return kp.view(*([1] * nb), 1, 1, Lk)
    if any(g != 1 and g != b for g, b in zip(lead, batch_shape)):
        return None
    return kp.view(*lead, 1, 1, Lk)


def _combined_mask(attn_mask, key_padding_mask, batch_shape, nh: int, Lq: int, Lk: int, qdtype):  # noqa: ANN001
    """attn_mask and key_padding_mask as one additive fp32 mask broadcastable to (*batch, nh, Lq, Lk)
    (reference scripts/tabicl_tpu_mha.py:251-290, following upstream's mask processing,
    results/tpu_patch.diff:327-371). None when there is no mask; False when a mask is boolean or of a
    shape upstream rejects (the caller then defers to upstream, which handles or reports it). Like
    upstream the sum is taken in the query dtype."""
    nb = len(batch_shape)
    full = (*batch_shape, nh, Lq, Lk)
    terms = []
    if attn_mask is not None:
        if attn_mask.dtype == torch.bool:
            return False
        am = _as_rank(attn_mask, nb, Lq, Lk)
        if am is None or any(g != 1 and g != e for g, e in zip(am.shape, full)):
            return False
        terms.append(am)
    if key_padding_mask is not None:
        if key_padding_mask.dtype == torch.bool:
            return False
        kp = _kpm_as_rank(key_padding_mask, batch_shape, nb, Lk)
        if kp is None:
            return False
        terms.append(kp)
    if not terms:
        return None
    m = terms[0] if len(terms) == 1 else terms[0] + terms[1]
    return m.to(dtype=qdtype).float() if m.dtype != qdtype else m.float()


def _key_only(mask: Optional[Tensor], Lk: int) -> Optional[Tensor]:
    """A combined mask that varies over keys only, as [*lead, Lk] (lead dims 1 or the batch's); None
    for no mask; False if it varies over heads or queries."""
    if mask is None:
        return None
    if mask.shape[-3] != 1 or mask.shape[-2] != 1:
        return False
    return mask.reshape(*mask.shape[:-3], Lk)


# ---------------------------------------------------------------------------------------------
# the small-head implementations (route 5)
# ---------------------------------------------------------------------------------------------
def _heads(x: Tensor, h: int) -> Tensor:
    """[..., L, E] -> [..., h, L, E / h]."""
    return x.unflatten(-1, (h, x.shape[-1] // h)).transpose(-3, -2)


def _merge(x: Tensor) -> Tensor:
    """[..., h, L, d] -> [..., L, h d]."""
    return x.transpose(-3, -2).flatten(-2)


def small_head_attention(q: Tensor, k: Tensor, v: Tensor, h: int, mask: Optional[Tensor], impl: str) -> Tensor:
    """Per-head softmax(q_g k_g^T + mask) v_g for merged q [..., Lq, E] (already scaled), k / v
    [..., Lk, E] and an additive mask broadcastable to [..., h|1, Lq|1, Lk]; fp32 scores and softmax,
    probabilities in v's dtype (reference scripts/tabicl_tpu_mha.py:144-198). impl "pk" runs the HIP
    hx kernel when the mask varies over keys only (reference :177-188), otherwise and for
    "std" / "hxq" / "hxk" / "thl" (the reference's TPU layouts of the same math) one torch form."""
    if impl == "pk":
        if _PK is not None and q.device.type == _DEVICE:
            Lq, E, Lk = q.shape[-2], q.shape[-1], k.shape[-2]
            kb = _key_only(mask, Lk)
            if kb is not False and _PK.supported(Lq, Lk, E, h, q.dtype):
                return _PK.hx_attention(q, k, v, h, kb)
        impl = "std"
    if impl not in _SINGLE_IMPLS:
        raise ValueError(f"unknown small-head attention impl {impl!r}")
    s = torch.matmul(_heads(q, h), _heads(k, h).transpose(-2, -1).contiguous()).float()
    if mask is not None:
        s = s + mask
    p = torch.softmax(s, dim=-1).to(v.dtype)
    return _merge(torch.matmul(p, _heads(v, h).contiguous()))


def _rotate_merged(rope, x: Tensor, h: int) -> Tensor:  # noqa: ANN001
    """The module's own RoPE (rotate_queries_or_keys on head-split [..., h, L, d]) for merged x."""
    return _merge(rope.rotate_queries_or_keys(_heads(x, h)))


# ---------------------------------------------------------------------------------------------
# projections
# ---------------------------------------------------------------------------------------------
def _linear_rows(x: Tensor, w: Tensor, b: Optional[Tensor], rows: slice) -> Tensor:
    return F.linear(x, w[rows], None if b is None else b[rows])


def in_projection(query: Tensor, key: Tensor, value: Tensor, w: Tensor, b: Optional[Tensor],
                  proj: str = "packed"):
    """q, k, v projections with the in-projection weight [3E, E] (reference scripts/tabicl_tpu_mha.py:95-111):
    one GEMM per distinct input (self attention: one [.., 3E] product; shared key/value: [.., E] and
    [.., 2E]), column views of the results. `proj` is accepted for the reference's knob; every form
    gives the same projections."""
    E = query.shape[-1]
    if query is key and key is value:
        return F.linear(query, w, b).chunk(3, dim=-1)
    q = _linear_rows(query, w, b, slice(0, E))
    if key is value:
        kv = _linear_rows(key, w, b, slice(E, 3 * E))
        return (q, *kv.chunk(2, dim=-1))
    return q, _linear_rows(key, w, b, slice(E, 2 * E)), _linear_rows(value, w, b, slice(2 * E, 3 * E))


def _ssmax(ssmax_layer, q: Tensor, h: int, n) -> Tensor:  # noqa: ANN001
    """upstream's SSMax on merged q: the layer takes head-split [B', h, L, d] and the source length n
    (results/tpu_patch.diff:251-254)."""
    qh = _heads(q, h)
    lead = qh.shape[:-3]
    return _merge(ssmax_layer(qh.reshape(math.prod(lead), *qh.shape[-3:]), n).reshape(*lead, *qh.shape[-3:]))


# ---------------------------------------------------------------------------------------------
# folded first-ISAB attention (route 1)
# ---------------------------------------------------------------------------------------------
def _distinct_rows(x: Tensor) -> Tensor:
    """Strip leading dims along which x is an expanded view (stride 0): the inducing points are one
    set broadcast over the batch, so they are folded once."""
    while x.dim() > 2 and x.stride(0) == 0:
        x = x[0]
    return x


def folded_mab1(query: Tensor, key: Tensor, valid_kv_len: Optional[Tensor], num_heads: int, in_proj_weight: Tensor,
                in_proj_bias: Optional[Tensor], ssmax_layer=None, src_len_override=None, pk=None,  # noqa: ANN001
                key_bias: Optional[Tensor] = None) -> Optional[Tensor]:
    """Merged per-head softmax(q_g K_g^T) V_g (before the output projection) of the first ISAB
    attention, with K = key W_k^T + b_k and V = key W_v^T + b_v never formed (reference
    scripts/tabicl_tpu_mha.py:60-92). Per head g: q_g K_g^T = (q_g W_k,g) key^T + q_g . b_k,g, and the
    second term is the same for every key of a query row, so it leaves the softmax unchanged; the
    probabilities sum to 1, so P V_g = (P key) W_v,g^T + b_v,g. The kernel computes U = softmax(Qf key^T)
    key over the raw rows with Qf = [q_g W_k,g]_g (hq = h Lq folded queries of width E). Keys past
    valid_kv_len, or masked by the additive key_bias, are excluded. None when the kernel does not apply."""
    kern = _PK if pk is None else pk
    E = query.shape[-1]
    d = E // num_heads
    ind = _distinct_rows(query)
    Lq = ind.shape[-2]
    n_ind = ind.shape[:-2].numel()
    if kern is None or n_ind not in (1, key.shape[:-2].numel()) or not kern.hxf_supported(num_heads * Lq, key.shape[-2], E):
        return None
    w_q, w_k, w_v = in_proj_weight.chunk(3)
    b_q = None if in_proj_bias is None else in_proj_bias[:E]
    b_v = None if in_proj_bias is None else in_proj_bias[2 * E:]
    q = F.linear(ind, w_q, b_q)
    if ssmax_layer is not None:  # source length: the override, else the valid length, else every key
        n = src_len_override if src_len_override is not None else valid_kv_len
        q = _ssmax(ssmax_layer, q, num_heads, key.shape[-2] if n is None else n)
    q = q * d ** -0.5
    # Qf[.., g, i, :] = q[.., i, g d:(g + 1) d] @ W_k[g d:(g + 1) d, :]   (both operands contiguous)
    qf = torch.matmul(_heads(q, num_heads).contiguous(), w_k.reshape(num_heads, d, E).contiguous())
    u = kern.hxf_attention(qf.flatten(-3, -2), key, valid_kv_len, key_bias)  # [*key lead, h Lq, E]
    # O[.., i, g d:(g + 1) d] = U[.., g, i, :] @ W_v[g d:(g + 1) d, :]^T
    w_vt = w_v.reshape(num_heads, d, E).transpose(-1, -2).contiguous().to(u.dtype)
    o = _merge(torch.matmul(u.unflatten(-2, (num_heads, Lq)), w_vt))
    return o if b_v is None else o + b_v


# ---------------------------------------------------------------------------------------------
# one call of multi_head_attention_forward
# ---------------------------------------------------------------------------------------------
class _Call:
    """The arguments of one multi_head_attention_forward call plus what routing needs from them."""

    def __init__(self, query, num_heads, in_proj_weight, in_proj_bias, dropout_p, out_proj_weight,  # noqa: ANN001
                 out_proj_bias, key, value, cached_kv, training, key_padding_mask, attn_mask, rope,
                 ssmax_layer, need_kv, src_len_override, valid_kv_len):
        self.query, self.key, self.value = query, key, value
        self.h = num_heads
        self.w, self.b, self.wo, self.bo = in_proj_weight, in_proj_bias, out_proj_weight, out_proj_bias
        self.dropout_p, self.training = dropout_p, training
        self.cached_kv, self.need_kv = cached_kv, need_kv
        self.key_padding_mask, self.attn_mask = key_padding_mask, attn_mask
        self.rope, self.ssmax, self.src_len_override, self.valid_kv_len = rope, ssmax_layer, src_len_override, valid_kv_len
        self.E = query.shape[-1]
        self.d = self.E // num_heads
        self.batch_shape = tuple(query.shape[:-2])
        self.Lq = query.shape[-2]
        self.Lk = None if key is None else key.shape[-2]
        self.on_gpu = query.device.type == _DEVICE
        self._mask = ...

    def mask(self):
        """Combined additive mask (see _combined_mask), computed once."""
        if self._mask is ...:
            if self.Lk is None:
                self._mask = False
            else:
                self._mask = _combined_mask(self.attn_mask, self.key_padding_mask, self.batch_shape, self.h,
                                            self.Lq, self.Lk, self.query.dtype)
        return self._mask

    def key_constraint(self):
        """(valid length tensor or None, key-only mask [*lead, Lk] or None), or None when the call's keys
        are not constrained by a tensor length or a key-only additive mask (routes 1-2 need one)."""
        if self.attn_mask is None and self.key_padding_mask is None:
            return (self.valid_kv_len, None) if isinstance(self.valid_kv_len, Tensor) else None
        if self.valid_kv_len is not None and not isinstance(self.valid_kv_len, Tensor):
            return None
        m = self.mask()
        if m is None or m is False:
            return None
        kb = _key_only(m, self.Lk)
        return None if kb is False else (self.valid_kv_len, kb)

    def inducing_over_rows(self, max_head_dim: int) -> bool:
        """The shape of the inference first-ISAB attention: no grad, no cache, one key/value input, no
        RoPE, small heads, on the GPU."""
        return (not torch.is_grad_enabled() and self.cached_kv is None and not self.need_kv
                and self.key is not None and self.key is self.value and self.rope is None
                and self.d <= max_head_dim and self.on_gpu)

    def ssmax_n(self, default):  # noqa: ANN001
        return self.src_len_override if self.src_len_override is not None else default

    def out(self, merged: Tensor) -> Tensor:
        return F.linear(merged, self.wo, self.bo)


def _route_cached(c: _Call, knobs: Knobs) -> Optional[Tensor]:
    """Small heads over cached K/V: the column blocks' second attention at query time, test rows over
    the cached K/V of the 128 inducing points (scripts/tabicl_tpu_bucketed.py:788-792). Upstream's cached
    branch (results/tpu_patch.diff:305-318) projects q only, promotes q and the cache to one dtype and
    attends over the cache's head-split K/V [..., h, Lk, d]; the reference's TPU path leaves these calls
    to it (scripts/tabicl_tpu_mha.py:343-347), which on this GPU would be torch SDPA (the ICL hook takes
    the 64-wide heads only). Here the cache's K and V are written once per call into the packed
    [.., Lk, 2E] rows pk_cross reads (one copy of the Lk cached rows, 128 here) and pk_cross runs; SSMax
    takes n = src_len_override or the cached key count (diff:251-254). Declines RoPE (the cache holds
    keys rotated at fit time), a valid length, K/V requested back, gradients and dropout."""
    e = c.cached_kv
    if not (knobs.cached and e is not None and c.on_gpu and not c.need_kv and c.rope is None
            and c.valid_kv_len is None and c.d <= knobs.max_head_dim and not torch.is_grad_enabled()
            and not (c.training and c.dropout_p > 0.0)):
        return None
    k, v = e.key, e.value
    if (k.dim() < 3 or k.shape != v.shape or k.shape[-3] != c.h or k.shape[-1] != c.d
            or tuple(k.shape[:-3]) != c.batch_shape):
        return None
    Lk = k.shape[-2]
    if pick_impl(knobs.mode, c.Lq, Lk) != "pk":
        return None
    q = _linear_rows(c.query, c.w, c.b, slice(0, c.E))
    dt = torch.promote_types(q.dtype, k.dtype)
    if not _PK.packed_supported(c.Lq, Lk, c.E, c.h, False, dt):
        return None
    m = _combined_mask(c.attn_mask, c.key_padding_mask, c.batch_shape, c.h, c.Lq, Lk, dt)
    kb = None if m is None or m is False else _key_only(m, Lk)
    if m is False or kb is False:
        return None
    kv = torch.empty(*c.batch_shape, Lk, 2, c.h, c.d, dtype=dt, device=q.device)
    kv[..., 0, :, :] = k.transpose(-3, -2)
    kv[..., 1, :, :] = v.transpose(-3, -2)
    q = q.to(dt)
    if c.ssmax is not None:
        q = _ssmax(c.ssmax, q, c.h, c.ssmax_n(Lk))
    return c.out(_PK.pk_cross_attention(q, kv.flatten(-3), c.h, kb, None, c.d ** -0.5))


def _route_folded(c: _Call, knobs: Knobs) -> Optional[Tensor]:
    """Route 1. The folded kernel computes softmax(Qf x^T) x with h Lq folded queries of width E: 4x
    the attention FLOPs of projection + hxq (4 h Lq Lk E against 2 Lk E 2E + 4 Lq Lk E per batch
    element), to save the [.., Lk, 2E] projection that the reference avoids on its TPU for memory. On
    this GPU that trade loses at every shape measured (bf16 1.67 vs 0.94 ms, fp32 10.9 vs 4.3 ms at
    54 x 128 queries over 45k rows), so where the hxq kernel takes the call it runs as route 2 does,
    the same math to rounding; TABICL_MI355_HXF_FORCE=1 keeps the folded kernel."""
    if not (knobs.folded and c.inducing_over_rows(knobs.max_head_dim)):
        return None
    kc = c.key_constraint()
    if kc is None or (isinstance(c.src_len_override, Tensor) and c.src_len_override.numel() != 1):
        return None
    valid, kb = kc
    if valid is not None and valid.numel() != 1:
        return None
    if not knobs.folded_force and _PK.hxq_supported(c.Lq, c.Lk, c.E, c.h, c.query.dtype):
        return _route_few_queries(c, dataclasses.replace(knobs, few_queries=True))
    o = folded_mab1(c.query, c.key, valid, c.h, c.w, c.b, c.ssmax, c.src_len_override, key_bias=kb)
    return None if o is None else c.out(o)


def _route_few_queries(c: _Call, knobs: Knobs) -> Optional[Tensor]:
    if not (knobs.few_queries and c.inducing_over_rows(knobs.max_head_dim)):
        return None
    kc = c.key_constraint()
    if kc is None or not _PK.hxq_supported(c.Lq, c.Lk, c.E, c.h, c.query.dtype):
        return None
    valid, kb = kc
    q = _linear_rows(c.query, c.w, c.b, slice(0, c.E))
    kv = _linear_rows(c.key, c.w, c.b, slice(c.E, 3 * c.E))  # [.., Lk, 2E]: K columns [0, E), V [E, 2E)
    if c.ssmax is not None:
        q = _ssmax(c.ssmax, q, c.h, c.ssmax_n(valid if valid is not None else c.Lk))
    return c.out(_PK.hxq_attention(q * c.d ** -0.5, kv, valid, c.h, kb))


def _defers(c: _Call, knobs: Knobs, att_module, splash_min_kv) -> bool:  # noqa: ANN001
    return ((not c.on_gpu and not knobs.any_device) or c.cached_kv is not None or c.need_kv
            or c.key is None or c.value is None or c.d > knobs.max_head_dim
            or (c.training and c.dropout_p > 0.0) or c.valid_kv_len is not None
            or getattr(att_module, "_tpu_flash_attention_fn", None) is not None
            or c.Lk >= splash_min_kv())


def _route_packed(c: _Call, knobs: Knobs, mode: str) -> Optional[Tensor]:
    if not (knobs.packed and c.on_gpu and c.key is c.value and pick_impl(mode, c.Lq, c.Lk) == "pk"):
        return None
    self_attn = c.query is c.key
    if not _PK.packed_supported(c.Lq, c.Lk, c.E, c.h, self_attn, c.query.dtype):
        return None
    m = c.mask()
    kb = None if m is None or m is False else _key_only(m, c.Lk)
    if m is False or kb is False:
        return None
    if self_attn:
        qkv = F.linear(c.query, c.w, c.b)
        return c.out(_PK.pk_self_attention(qkv, c.h, kb, c.rope, c.d ** -0.5))
    q = _linear_rows(c.query, c.w, c.b, slice(0, c.E))
    kv = _linear_rows(c.key, c.w, c.b, slice(c.E, 3 * c.E))
    if c.ssmax is not None:
        q = _ssmax(c.ssmax, q, c.h, c.ssmax_n(c.Lk))
    return c.out(_PK.pk_cross_attention(q, kv, c.h, kb, c.rope, c.d ** -0.5))


def _route_hx(c: _Call, knobs: Knobs) -> Optional[Tensor]:
    """Mode "pk" without the packed route: projections, RoPE and SSMax in torch, the hx kernel."""
    m = c.mask()
    if m is False:
        return None
    q, k, v = in_projection(c.query, c.key, c.value, c.w, c.b, knobs.proj)
    if c.rope is not None:
        q, k = _rotate_merged(c.rope, q, c.h), _rotate_merged(c.rope, k, c.h)
    if c.ssmax is not None:
        q = _ssmax(c.ssmax, q, c.h, c.ssmax_n(c.Lk))
    return c.out(small_head_attention(q * c.d ** -0.5, k, v, c.h, m, "pk"))


def install(att_module, layers_module=None, mode: Optional[str] = None, proj: Optional[str] = None) -> bool:  # noqa: ANN001
    """Patch `multi_head_attention_forward` in att_module (and layers_module, which imports it by name)
    and install the ICL hook on att_module.sdpa_with_flattened_batch. Same signature, knobs and return
    value as the reference's install (scripts/tabicl_tpu_mha.py:293-393): False when the mode is off,
    True when installed (idempotent)."""
    knobs = Knobs(**{**KNOBS.__dict__})
    knobs.mode = (knobs.mode if mode is None else mode).strip().lower()
    knobs.proj = (knobs.proj if proj is None else proj).strip().lower()
    if knobs.mode in ("", "0", "off", "none"):
        return False
    if getattr(att_module, "_mi355_mha_installed", False):
        return True
    global _PK, _ICL
    import tabicl_mi355_attn as pk_mod  # registers the tabicl_pk:: ops now, never while tracing
    import tabicl_mi355_icl as icl_mod  # registers tabicl::icl_cached_attn

    _PK = pk_mod if _PK is None else _PK
    _ICL = icl_mod if _ICL is None else _ICL
    upstream = att_module.multi_head_attention_forward
    splash_min_kv = getattr(att_module, "_tpu_splash_min_kv",
                            lambda: int(os.environ.get("TABICL_TPU_SPLASH_MIN_KV", "16384")))

    def multi_head_attention_forward(query, num_heads, in_proj_weight, in_proj_bias, dropout_p,  # noqa: ANN001
                                     out_proj_weight, out_proj_bias, key=None, value=None, cached_kv=None,
                                     training=True, key_padding_mask=None, attn_mask=None, rope=None,
                                     ssmax_layer=None, need_kv=False, src_len_override=None, valid_kv_len=None):
        c = _Call(query, num_heads, in_proj_weight, in_proj_bias, dropout_p, out_proj_weight, out_proj_bias, key,
                  value, cached_kv, training, key_padding_mask, attn_mask, rope, ssmax_layer, need_kv,
                  src_len_override, valid_kv_len)
        out = _route_cached(c, knobs)
        if out is None:
            out = _route_folded(c, knobs)
        if out is None:
            out = _route_few_queries(c, knobs)
        if out is None and not _defers(c, knobs, att_module, splash_min_kv):
            out = _route_packed(c, knobs, knobs.mode)
            if out is None and c.on_gpu and pick_impl(knobs.mode, c.Lq, c.Lk) == "pk":
                out = _route_hx(c, knobs)
        if out is not None:
            return out
        return upstream(query, num_heads, in_proj_weight, in_proj_bias, dropout_p, out_proj_weight, out_proj_bias,
                        key=key, value=value, cached_kv=cached_kv, training=training,
                        key_padding_mask=key_padding_mask, attn_mask=attn_mask, rope=rope, ssmax_layer=ssmax_layer,
                        need_kv=need_kv, src_len_override=src_len_override, valid_kv_len=valid_kv_len)

    att_module.multi_head_attention_forward = multi_head_attention_forward
    if layers_module is not None:
        layers_module.multi_head_attention_forward = multi_head_attention_forward
    if knobs.icl_hook and hasattr(att_module, "sdpa_with_flattened_batch"):
        att_module.sdpa_with_flattened_batch = icl_hook(att_module.sdpa_with_flattened_batch)
    if knobs.icl_hook:  # the reference's Splash op attributes (diff:95-115), for code that calls them directly
        for form in ("seg", "full"):
            op = getattr(_ICL, f"splash_sdpa_{form}_op", None)
            if op is not None:
                setattr(att_module, f"_tpu_splash_sdpa_{form}_op", op)
    att_module._mi355_mha_installed = True
    att_module._mi355_mha_mode = knobs.mode
    att_module._mi355_mha_proj = knobs.proj
    return True


# ---------------------------------------------------------------------------------------------
# the ICL hook on sdpa_with_flattened_batch
# ---------------------------------------------------------------------------------------------
def _hook_bias(attn_mask: Optional[Tensor], q: Tensor, Tkv: int):
    """The hook's key mask: None (no mask), [1 | N, Tkv] fp32 for a mask that varies over keys only
    (N = the flattened batch of q [..., H, Tq, D]), False for anything else (boolean, or varying over
    heads or queries)."""
    if attn_mask is None:
        return None
    if attn_mask.dtype == torch.bool or attn_mask.shape[-1] != Tkv:
        return False
    m = attn_mask
    for _ in range(2):  # the query dim, then the head dim: both must be broadcast (size 1)
        if m.dim() >= 2:
            if m.shape[-2] != 1:
                return False
            m = m.squeeze(-2)
    lead = tuple(q.shape[:-3])
    extra = m.dim() - 1 - len(lead)
    if extra > 0:
        if any(s_ != 1 for s_ in m.shape[:extra]):
            return False
        m = m.reshape(*m.shape[extra:])
    if any(g != 1 and g != e for g, e in zip(m.shape[:-1][::-1], lead[::-1])):
        return False
    if m.shape[:-1].numel() == 1:
        return m.reshape(1, Tkv).float()
    return m.expand(*lead, Tkv).reshape(-1, Tkv).float()


def icl_hook(upstream_sdpa):  # noqa: ANN001
    """sdpa_with_flattened_batch with its attention on the HIP ICL kernel (the reference's Splash
    branch, results/tpu_patch.diff:261-281, on this GPU): q, k, v [..., H, T, D] on the GPU, same
    dtype (bf16 or fp32), D the kernel's head dim, no dropout, and either no mask or one that varies
    over keys only (and needs no gradient itself). SSMax is applied to q with n = src_len_override or the
    key count first (diff:251-254); valid_kv_len masks the key tail. Calls with a gradient take the
    library's backward kernels through the op's autograd formula, where the reference's take autograd
    through its tiled online softmax (diff:158-193, 263-270). Anything else goes to upstream."""

    global _ICL
    if _ICL is None:
        import tabicl_mi355_icl as icl_mod  # registers tabicl::icl_cached_attn now, never while tracing

        _ICL = icl_mod

    def sdpa_with_flattened_batch(q, k, v, attn_mask=None, dropout_p=0.0, ssmax_layer=None,  # noqa: ANN001
                                  src_len_override=None, valid_kv_len=None):
        Tkv = k.shape[-2]
        kb = _hook_bias(attn_mask, q, Tkv)
        if (kb is not False and q.device.type == _DEVICE and dropout_p == 0.0
                and not (torch.is_grad_enabled() and attn_mask is not None and attn_mask.requires_grad)
                and q.dtype in (torch.bfloat16, torch.float32) and q.dtype == k.dtype == v.dtype
                and _ICL.icl_supported(q.shape[-2], Tkv, q.shape[-1], q.dtype)):
            lead = q.shape[:-3]
            q3 = q.reshape(math.prod(lead), *q.shape[-3:])
            if ssmax_layer is not None:
                q3 = ssmax_layer(q3, src_len_override if src_len_override is not None else Tkv)
            out = _ICL.icl_sdpa(q3, k.reshape(q3.shape[0], *k.shape[-3:]), v.reshape(q3.shape[0], *v.shape[-3:]),
                                valid_kv_len, kb)
            return out.reshape(*lead, *out.shape[-3:])
        return upstream_sdpa(q, k, v, attn_mask, dropout_p, ssmax_layer=ssmax_layer,
                             src_len_override=src_len_override, valid_kv_len=valid_kv_len)

    return sdpa_with_flattened_batch
