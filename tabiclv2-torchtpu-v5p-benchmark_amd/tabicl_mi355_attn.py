"""Fused small-head attention (8 heads x 16 dims) on MI355X, as torch custom ops over HIP kernels.

Drop-in for the reference's scripts/tabicl_tpu_pallas_attn.py: same public functions, argument
meaning and op names (tabicl_pk::hx_fwd, hxq_fwd, pk_self_fwd, pk_cross_fwd), with the math done by
hand-written gfx950 kernels in libtabicl_attn.so (C ABI: include/tabicl_attn.h).

  hx_attention(q, k, v, h, key_bias=None)            q pre-scaled; merged [.., L, E] in and out
  hxq_attention(q, kv, valid_len, h, key_bias=None)  few queries, packed [.., Lk, 2E] K|V, keys >= valid ignored
  pk_self_attention(qkv, h, key_bias, rope, scale)   packed [.., L, 3E], in-kernel RoPE + scale
  pk_cross_attention(q, kv, h, key_bias, rope, scale)

Semantics per head g: softmax(q_g k_g^T + bias) v_g with fp32 scores and softmax, probabilities cast
to the value dtype before the PV product, output in the query dtype. Differences from the reference,
all extensions: any key length (keys stream through LDS; the reference stops at 1024), any query
length, a per-batch valid length for hxq, an additive key mask for hxq (the form upstream gives a
tensor train size off the reference's device), and a defined output (0) for a row with no valid key.
The ops take the reference's `lkp`, `bq` and `prec` arguments for schema compatibility and ignore
them: the kernels pick their own tiles, and fp32 inputs are always multiplied in full fp32.
The HIP library is the only compute path: the ops raise when it is missing (no CPU fallback).
"""
from __future__ import annotations

import math
import weakref
from typing import Optional

import torch
import torch.nn.functional as F
from torch import Tensor

import tabicl_mi355_native as _nat

_NEG = -1e30


# ---------------------------------------------------------------------------------------------
# host-side helpers with the reference's names and meaning
# ---------------------------------------------------------------------------------------------
def _pick_bq(Lq: int, lkp: int) -> int:
    """Query block of the reference kernel (scripts/tabicl_tpu_pallas_attn.py:36-44): Lq itself when it
    fits the cap min(512, 65536 // lkp) (at least 8), else the largest multiple of 8 within the cap that
    divides Lq, else 0. Kept for the op schema; the HIP kernels pick their own query tiling."""
    cap = max(8, min(512, 65536 // lkp))
    if Lq <= cap:
        return Lq
    fits = [b for b in range(8, cap + 1, 8) if Lq % b == 0]
    return fits[-1] if fits else 0


def _pick_bk(Lk: int) -> int:
    """Key block of the reference hxq kernel (scripts/tabicl_tpu_pallas_attn.py:312-316): the first of
    512, 1024, 256, 128 (that order) dividing Lk, else 0."""
    return next((b for b in (512, 1024, 256, 128) if Lk % b == 0), 0)


_PREC_CODES = {"highest": 2, "high": 1}


def _fp32_prec_code() -> int:
    """fp32 matmul precision code (reference scripts/tabicl_tpu_pallas_attn.py:755-759): highest 2,
    high 1, anything else 0. The HIP fp32 kernels always multiply in full fp32 (fp32 MFMA)."""
    return _PREC_CODES.get(torch.get_float32_matmul_precision(), 0)


def _bias3(key_bias: Optional[Tensor], lead, Lk: int, device) -> Tensor:
    """An additive key bias as fp32 [1, 1, Lk] (one row shared by every batch element) or [B, 1, Lk]
    (B = prod(lead)), the two forms of the reference (scripts/tabicl_tpu_pallas_attn.py:701-712);
    None gives a zero row."""
    if key_bias is None:
        return torch.zeros(1, 1, Lk, device=device, dtype=torch.float32)
    kb = key_bias.float()
    missing = len(lead) + 1 - kb.dim()
    if missing > 0:
        kb = kb.reshape((1,) * missing + tuple(kb.shape))
    if math.prod(kb.shape[:-1]) == 1:
        return _nat.aligned16(kb.reshape(1, 1, Lk))
    return _nat.aligned16(kb.expand(*lead, Lk).reshape(math.prod(lead), 1, Lk))


def rope_tables(rope_mod, L: int, E: int, h: int, device) -> tuple:  # noqa: ANN001
    """(cos, sin) fp32 [L, E]: one head's d = E / h columns repeated for every head, with cos = 1 and
    sin = 0 past the rotary dims; then the rope code (0 none, 1 pairs, 2 halves), half and rot
    (reference scripts/tabicl_tpu_pallas_attn.py:681-698). rope_mod follows the upstream RotaryEmbedding
    surface: get_seq_pos, interleaved, freqs and, for the interleaved form, forward (which returns the
    pairwise-repeated angles)."""
    d = E // h
    if rope_mod is None:
        return (torch.ones(L, E, device=device), torch.zeros(L, E, device=device), 0, 0, 0)
    pos = rope_mod.get_seq_pos(L, device=device, dtype=torch.float32)
    if rope_mod.interleaved:
        ang = rope_mod.forward(pos, seq_len=L).float()  # f0 f0 f1 f1 ...
    else:
        ang = torch.outer(pos.float(), rope_mod.freqs.float().to(device)).repeat(1, 2)  # f0 f1 ... f0 f1 ...
    rot = ang.shape[-1]
    cos = F.pad(ang.cos(), (0, d - rot), value=1.0)
    sin = F.pad(ang.sin(), (0, d - rot), value=0.0)
    return (cos.repeat(1, h).contiguous(), sin.repeat(1, h).contiguous(), 1 if rope_mod.interleaved else 2,
            rot // 2, rot)


def _dt_ok(dt: torch.dtype) -> bool:
    return dt in (torch.bfloat16, torch.float32)


def supported(Lq: int, Lk: int, E: int, h: int, dtype: torch.dtype = torch.bfloat16) -> bool:
    """hx kernel shape predicate (reference scripts/tabicl_tpu_pallas_attn.py:762-764). The HIP
    kernel needs E == 128, h == 8; it has no key-length cap (keys stream through LDS)."""
    return _dt_ok(dtype) and _nat.supported(_nat.OP_HX, Lq, Lk, E, h, dtype)


def hxq_supported(Lq: int, Lk: int, E: int, h: int, dtype: torch.dtype = torch.bfloat16) -> bool:
    """hxq predicate (reference scripts/tabicl_tpu_pallas_attn.py:319-320): the reference needs
    Lq % 8 == 0, Lq <= 256 and a key block dividing Lk; the HIP kernel takes any Lq and Lk."""
    return _dt_ok(dtype) and _nat.supported(_nat.OP_HXQ, Lq, Lk, E, h, dtype)


def packed_supported(Lq: int, Lk: int, E: int, h: int, self_attn: bool,
                     dtype: torch.dtype = torch.bfloat16) -> bool:
    """pk_self / pk_cross predicate (reference scripts/tabicl_tpu_pallas_attn.py:715-719)."""
    op = _nat.OP_PK_SELF if self_attn else _nat.OP_PK_CROSS
    if self_attn and Lq != Lk:
        return False
    return _dt_ok(dtype) and _nat.supported(op, Lq, Lk, E, h, dtype)


def hxf_supported(hq: int, Lk: int, E: int) -> bool:
    """Folded first-ISAB kernel (reference :425-426): E = 128 (the kernel's head dim), hq a multiple of
    8 and at most 2048 folded queries, any key length >= 1."""
    return E == 128 and hq % 8 == 0 and 0 < hq <= 2048 and Lk >= 1


# ---------------------------------------------------------------------------------------------
# torch custom ops (reference op names and schemas)
# ---------------------------------------------------------------------------------------------
def _contig(*ts: Tensor) -> None:
    for t in ts:
        if not t.is_contiguous():
            raise ValueError("tabicl_pk ops need contiguous inputs")


def _bias_ptr(bias: Tensor):
    """Device pointer of an op's key bias; an empty bias tensor (no rows) stands for no bias, which
    lets the kernels skip the additive term (a bias of zeros gives the same result, more slowly)."""
    return bias.data_ptr() if bias.numel() else None


def _bias_rows(bias: Tensor) -> int:
    return bias.shape[0] if bias.numel() else 0


def _flat(t: Tensor, *tail: int) -> Tensor:
    """t [..., *tail] as [n, *tail], n the product of its leading dims (reshape(-1, ...) is ambiguous
    for a tensor with no elements, e.g. zero query rows)."""
    return t.reshape(math.prod(t.shape[:t.dim() - len(tail)]), *tail)


def _bias_arg(key_bias: Optional[Tensor], lead, Lk: int, device) -> Tensor:
    """The op's bias argument for a wrapper's key_bias: _bias3's [1|B, 1, Lk] fp32, or an empty
    [0, 1, Lk] tensor for no bias."""
    if key_bias is None:
        return torch.empty(0, 1, Lk, device=device, dtype=torch.float32)
    return _bias3(key_bias, lead, Lk, device)


@torch.library.custom_op("tabicl_pk::hx_fwd", mutates_args=())
def _hx_fwd(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, h: int, lkp: int, bq: int, prec: int) -> Tensor:
    _nat.require_device(q, k, v, bias)
    _contig(q, k, v, bias)
    B, Lq, E = q.shape
    Lk = k.shape[1]
    out = torch.empty_like(q)
    _nat.call("tabicl_hx_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), _bias_ptr(bias), _bias_rows(bias),
              out.data_ptr(), B, Lq, Lk, E, h, _nat.dtype_code(q.dtype), _nat.stream_of(q))
    return out


@_hx_fwd.register_fake
def _(q, k, v, bias, h, lkp, bq, prec):  # noqa: ANN001
    return torch.empty_like(q)


@torch.library.custom_op("tabicl_pk::hxq_fwd", mutates_args=())
def _hxq_fwd(valid: Tensor, q: Tensor, kv: Tensor, h: int, bk: int, prec: int,
             key_bias: Optional[Tensor] = None) -> Tensor:
    """key_bias (extension, no counterpart in the reference's op): additive fp32 key mask [1|B, Lk];
    prefix masks (0 then <= -1e30, what upstream builds from a tensor train size) run as a valid
    length on the streaming kernel, other masks on a kernel that adds them term by term."""
    _nat.require_device(valid, q, kv, key_bias)
    _contig(valid, q, kv)
    B, Lq, E = q.shape
    Lk = kv.shape[1]
    if valid.dtype != torch.int32:
        raise ValueError("valid must be int32")
    out = torch.empty_like(q)
    code = _nat.dtype_code(q.dtype)
    ws = _hxq_workspace(B, Lq, Lk, E, h, code, q.device)
    wsp, wsn = (None, 0) if ws is None else (ws.data_ptr(), ws.numel())
    if key_bias is None:
        _nat.call("tabicl_hxq_fwd", valid.data_ptr(), valid.numel(), q.data_ptr(), kv.data_ptr(), out.data_ptr(),
                  B, Lq, Lk, E, h, code, wsp, wsn, _nat.stream_of(q))
        return out
    if key_bias.dtype != torch.float32 or key_bias.dim() != 2 or key_bias.shape[1] != Lk \
            or key_bias.shape[0] not in (1, B) or not key_bias.is_contiguous():
        raise ValueError(f"key_bias must be a contiguous float32 [1 or {B}, {Lk}] tensor, got "
                         f"{key_bias.dtype} {tuple(key_bias.shape)}")
    _nat.call("tabicl_hxq_fwd_masked", valid.data_ptr(), valid.numel(), key_bias.data_ptr(), key_bias.shape[0],
              q.data_ptr(), kv.data_ptr(), out.data_ptr(), B, Lq, Lk, E, h, code, wsp, wsn, _nat.stream_of(q))
    return out


_HXQ_WS_BYTES: dict = {}


def _hxq_workspace(B: int, Lq: int, Lk: int, E: int, h: int, code: int, device) -> Optional[Tensor]:
    """Scratch for the key-split path of the streaming kernel (size from the library, per shape and
    device), from torch's caching allocator on the launch stream; None when the call does not split."""
    key = (B, Lq, Lk, E, h, code, device.index)
    nbytes = _HXQ_WS_BYTES.get(key)
    if nbytes is None:
        nbytes = int(_nat.load().tabicl_hxq_workspace_bytes(B, Lq, Lk, E, h, code))
        _HXQ_WS_BYTES[key] = nbytes
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes > 0 else None


@_hxq_fwd.register_fake
def _(valid, q, kv, h, bk, prec, key_bias=None):  # noqa: ANN001
    return torch.empty_like(q)


def _check_tables(op: str, rope: int, L: int, E: int, h: int, cos: Tensor, sin: Tensor) -> None:
    """A RoPE form reads float32 cos / sin tables of L rows: E columns, or one head's E / h columns
    with the shared-table flag. Anything else would make the kernels read the wrong positions (or past
    the tables), so it is refused before launch."""
    if not rope:
        return
    cols = E // h if rope & ROPE_SHARED_TABLES else E
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != torch.float32 or tuple(t.shape) != (L, cols):
            raise ValueError(f"{op}: {name} table must be float32 [{L}, {cols}] for rope code {rope}, "
                             f"got {t.dtype} {tuple(t.shape)}")


@torch.library.custom_op("tabicl_pk::pk_self_fwd", mutates_args=())
def _pk_self_fwd(qkv: Tensor, bias: Tensor, cos: Tensor, sin: Tensor, h: int, lkp: int, rope: int, half: int,
                 rot: int, prec: int, scale: float) -> Tensor:
    B, L, E3 = qkv.shape
    E = E3 // 3
    _check_tables("pk_self_fwd", rope, L, E, h, cos, sin)
    _nat.require_device(qkv, bias, cos, sin)
    _contig(qkv, bias, cos, sin)
    out = torch.empty(B, L, E, device=qkv.device, dtype=qkv.dtype)
    _nat.call("tabicl_pk_self_fwd", qkv.data_ptr(), _bias_ptr(bias), _bias_rows(bias), cos.data_ptr(), sin.data_ptr(),
              out.data_ptr(), B, L, E, h, rope, half, rot, float(scale), _nat.dtype_code(qkv.dtype),
              _nat.stream_of(qkv))
    return out


@_pk_self_fwd.register_fake
def _(qkv, bias, cos, sin, h, lkp, rope, half, rot, prec, scale):  # noqa: ANN001
    B, L, E3 = qkv.shape
    return qkv.new_empty(B, L, E3 // 3)


@torch.library.custom_op("tabicl_pk::pk_cross_fwd", mutates_args=())
def _pk_cross_fwd(q: Tensor, kv: Tensor, bias: Tensor, cq: Tensor, sq: Tensor, ck: Tensor, sk: Tensor, h: int,
                  lkp: int, bq: int, rope: int, half: int, rot: int, prec: int, scale: float) -> Tensor:
    Bq, Lq, E = q.shape
    B, Lk, _ = kv.shape
    _check_tables("pk_cross_fwd", rope, Lq, E, h, cq, sq)
    _check_tables("pk_cross_fwd", rope, Lk, E, h, ck, sk)
    _nat.require_device(q, kv, bias, cq, sq, ck, sk)
    _contig(q, kv, bias, cq, sq, ck, sk)
    out = torch.empty(B, Lq, E, device=q.device, dtype=q.dtype)
    _nat.call("tabicl_pk_cross_fwd", q.data_ptr(), Bq, kv.data_ptr(), _bias_ptr(bias), _bias_rows(bias),
              cq.data_ptr(), sq.data_ptr(), ck.data_ptr(), sk.data_ptr(), out.data_ptr(), B, Lq, Lk, E, h,
              rope, half, rot, float(scale), _nat.dtype_code(q.dtype), _nat.stream_of(q))
    return out


@_pk_cross_fwd.register_fake
def _(q, kv, bias, cq, sq, ck, sk, h, lkp, bq, rope, half, rot, prec, scale):  # noqa: ANN001
    return q.new_empty(kv.shape[0], q.shape[1], q.shape[2])


def _q_len_arg(q_len: Tensor, B: int) -> Tensor:
    if q_len.dtype != torch.int32 or not q_len.is_contiguous() or q_len.numel() not in (1, B):
        raise ValueError(f"q_len must be a contiguous int32 tensor of 1 or {B} entries")
    return q_len


@torch.library.custom_op("tabicl_pk::pk_cross_fwd_ragged", mutates_args=())
def _pk_cross_fwd_ragged(q: Tensor, kv: Tensor, bias: Tensor, cq: Tensor, sq: Tensor, ck: Tensor, sk: Tensor,
                         q_len: Tensor, h: int, lkp: int, bq: int, rope: int, half: int, rot: int, prec: int,
                         scale: float) -> Tensor:
    """pk_cross_fwd over a ragged batch (inference only): rows below q_len[b] equal pk_cross_fwd's;
    the rows at or past it are padding whose contents are unspecified (the column ISAB-2 kernel skips
    them). No counterpart in the reference, whose bucketed runner computes its padding rows."""
    Bq, Lq, E = q.shape
    B, Lk, _ = kv.shape
    _check_tables("pk_cross_fwd_ragged", rope, Lq, E, h, cq, sq)
    _check_tables("pk_cross_fwd_ragged", rope, Lk, E, h, ck, sk)
    _nat.require_device(q, kv, bias, cq, sq, ck, sk, q_len)
    _contig(q, kv, bias, cq, sq, ck, sk)
    _q_len_arg(q_len, B)
    out = torch.empty(B, Lq, E, device=q.device, dtype=q.dtype)
    _nat.call("tabicl_pk_cross_fwd_ragged", q.data_ptr(), Bq, kv.data_ptr(), _bias_ptr(bias), _bias_rows(bias),
              cq.data_ptr(), sq.data_ptr(), ck.data_ptr(), sk.data_ptr(), out.data_ptr(), B, Lq, Lk, E, h,
              rope, half, rot, float(scale), _nat.dtype_code(q.dtype), q_len.data_ptr(), q_len.numel(),
              _nat.stream_of(q))
    return out


@_pk_cross_fwd_ragged.register_fake
def _(q, kv, bias, cq, sq, ck, sk, q_len, h, lkp, bq, rope, half, rot, prec, scale):  # noqa: ANN001
    return q.new_empty(kv.shape[0], q.shape[1], q.shape[2])


@torch.library.custom_op("tabicl_pk::hxf_fwd", mutates_args=())
def _hxf_fwd(valid: Tensor, q: Tensor, x: Tensor, bk: int, prec: int, key_bias: Optional[Tensor] = None) -> Tensor:
    """key_bias (extension): additive fp32 key mask [1|B, Lk] added to the scores."""
    _nat.require_device(valid, q, x, key_bias)
    _contig(valid, q, x)
    if valid.dtype != torch.int32:
        raise ValueError("valid must be int32")
    Bq, hq, E = q.shape
    B, Lk, _ = x.shape
    out = torch.empty(B, hq, E, device=x.device, dtype=x.dtype)
    code = _nat.dtype_code(x.dtype)
    key = ("hxf", B, hq, Lk, E, code, x.device.index)
    nbytes = _HXQ_WS_BYTES.get(key)
    if nbytes is None:
        nbytes = int(_nat.load().tabicl_hxf_workspace_bytes(B, hq, Lk, E, code))
        _HXQ_WS_BYTES[key] = max(nbytes, 0)
        nbytes = _HXQ_WS_BYTES[key]
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes > 0 else None
    wsp, wsn = (None, 0) if ws is None else (ws.data_ptr(), ws.numel())
    if key_bias is None:
        _nat.call("tabicl_hxf_fwd", valid.data_ptr(), valid.numel(), q.data_ptr(), Bq, x.data_ptr(), out.data_ptr(),
                  B, hq, Lk, E, code, wsp, wsn, _nat.stream_of(x))
        return out
    if key_bias.dtype != torch.float32 or key_bias.dim() != 2 or key_bias.shape[1] != Lk \
            or key_bias.shape[0] not in (1, B) or not key_bias.is_contiguous():
        raise ValueError(f"key_bias must be a contiguous float32 [1 or {B}, {Lk}] tensor, got "
                         f"{key_bias.dtype} {tuple(key_bias.shape)}")
    _nat.call("tabicl_hxf_fwd_masked", valid.data_ptr(), valid.numel(), key_bias.data_ptr(), key_bias.shape[0],
              q.data_ptr(), Bq, x.data_ptr(), out.data_ptr(), B, hq, Lk, E, code, wsp, wsn, _nat.stream_of(x))
    return out


@_hxf_fwd.register_fake
def _(valid, q, x, bk, prec, key_bias=None):  # noqa: ANN001
    return x.new_empty(x.shape[0], q.shape[1], q.shape[2])


# ---------------------------------------------------------------------------------------------
# backward ops and autograd (reference scripts/tabicl_tpu_pallas_attn.py:185-207, 618-671)
# ---------------------------------------------------------------------------------------------
_BWD_WS_BYTES: dict = {}


def _bwd_workspace(B: int, Lq: int, E: int, h: int, device) -> Tensor:
    """Scratch of one backward call (per-query softmax statistics and D), from torch's caching allocator."""
    key = (B, Lq, E, h)
    nbytes = _BWD_WS_BYTES.get(key)
    if nbytes is None:
        nbytes = int(_nat.load().tabicl_smallhead_bwd_workspace_bytes(B, Lq, E, h))
        if nbytes < 0:
            _nat.check(1, "tabicl_smallhead_bwd_workspace_bytes")
        _BWD_WS_BYTES[key] = nbytes
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


@torch.library.custom_op("tabicl_pk::hx_bwd", mutates_args=())
def _hx_bwd(q: Tensor, k: Tensor, v: Tensor, bias: Tensor, o: Tensor, do: Tensor, h: int, lkp: int, bq: int,
            prec: int) -> tuple[Tensor, Tensor, Tensor]:
    _nat.require_device(q, k, v, bias, o, do)
    _contig(q, k, v, bias, o, do)
    B, Lq, E = q.shape
    Lk = k.shape[1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = _bwd_workspace(B, Lq, E, h, q.device)
    _nat.call("tabicl_hx_bwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), _bias_ptr(bias), _bias_rows(bias),
              o.data_ptr(), do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, Lq, Lk, E, h,
              _nat.dtype_code(q.dtype), ws.data_ptr(), ws.numel(), _nat.stream_of(q))
    return dq, dk, dv


@_hx_bwd.register_fake
def _(q, k, v, bias, o, do, h, lkp, bq, prec):  # noqa: ANN001
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _hx_setup(ctx, inputs, output):  # noqa: ANN001
    q, k, v, bias, h, lkp, bq, prec = inputs
    ctx.save_for_backward(q, k, v, bias, output)
    ctx.cfg = (h, lkp, bq, prec)


def _hx_backward(ctx, do):  # noqa: ANN001
    q, k, v, bias, o = ctx.saved_tensors
    dq, dk, dv = torch.ops.tabicl_pk.hx_bwd(q, k, v, bias, o, do.to(o.dtype).contiguous(), *ctx.cfg)
    return dq, dk, dv, None, None, None, None, None


_hx_fwd.register_autograd(_hx_backward, setup_context=_hx_setup)


@torch.library.custom_op("tabicl_pk::pk_self_bwd", mutates_args=())
def _pk_self_bwd(qkv: Tensor, bias: Tensor, cos: Tensor, sin: Tensor, o: Tensor, do: Tensor, h: int, lkp: int,
                 rope: int, half: int, rot: int, prec: int, scale: float) -> Tensor:
    _nat.require_device(qkv, bias, cos, sin, o, do)
    _contig(qkv, bias, cos, sin, o, do)
    B, L, E3 = qkv.shape
    E = E3 // 3
    _check_tables("pk_self_bwd", rope, L, E, h, cos, sin)
    dqkv = torch.empty_like(qkv)
    ws = _bwd_workspace(B, L, E, h, qkv.device)
    _nat.call("tabicl_pk_self_bwd", qkv.data_ptr(), _bias_ptr(bias), _bias_rows(bias), cos.data_ptr(),
              sin.data_ptr(), o.data_ptr(), do.data_ptr(), dqkv.data_ptr(), B, L, E, h, rope, half, rot,
              float(scale), _nat.dtype_code(qkv.dtype), ws.data_ptr(), ws.numel(), _nat.stream_of(qkv))
    return dqkv


@_pk_self_bwd.register_fake
def _(qkv, bias, cos, sin, o, do, h, lkp, rope, half, rot, prec, scale):  # noqa: ANN001
    return torch.empty_like(qkv)


def _pk_self_setup(ctx, inputs, output):  # noqa: ANN001
    qkv, bias, cos, sin, *cfg = inputs
    ctx.save_for_backward(qkv, bias, cos, sin, output)
    ctx.cfg = tuple(cfg)


def _pk_self_backward(ctx, do):  # noqa: ANN001
    qkv, bias, cos, sin, o = ctx.saved_tensors
    dqkv = torch.ops.tabicl_pk.pk_self_bwd(qkv, bias, cos, sin, o, do.to(o.dtype).contiguous(), *ctx.cfg)
    return (dqkv,) + (None,) * (3 + len(ctx.cfg))


_pk_self_fwd.register_autograd(_pk_self_backward, setup_context=_pk_self_setup)


@torch.library.custom_op("tabicl_pk::pk_cross_bwd", mutates_args=())
def _pk_cross_bwd(q: Tensor, kv: Tensor, bias: Tensor, cq: Tensor, sq: Tensor, ck: Tensor, sk: Tensor, o: Tensor,
                  do: Tensor, h: int, lkp: int, bq: int, rope: int, half: int, rot: int, prec: int,
                  scale: float) -> tuple[Tensor, Tensor]:
    _nat.require_device(q, kv, bias, cq, sq, ck, sk, o, do)
    _contig(q, kv, bias, cq, sq, ck, sk, o, do)
    Bq, Lq, E = q.shape
    B, Lk, _ = kv.shape
    _check_tables("pk_cross_bwd", rope, Lq, E, h, cq, sq)
    _check_tables("pk_cross_bwd", rope, Lk, E, h, ck, sk)
    dq = torch.empty(B, Lq, E, device=q.device, dtype=q.dtype)
    dkv = torch.empty_like(kv)
    ws = _bwd_workspace(B, Lq, E, h, q.device)
    _nat.call("tabicl_pk_cross_bwd", q.data_ptr(), Bq, kv.data_ptr(), _bias_ptr(bias), _bias_rows(bias),
              cq.data_ptr(), sq.data_ptr(), ck.data_ptr(), sk.data_ptr(), o.data_ptr(), do.data_ptr(),
              dq.data_ptr(), dkv.data_ptr(), B, Lq, Lk, E, h, rope, half, rot, float(scale),
              _nat.dtype_code(q.dtype), ws.data_ptr(), ws.numel(), _nat.stream_of(q))
    if Bq != B:  # one query set broadcast over the batch: its gradient is the sum over the batch
        dq = dq.float().sum(dim=0, keepdim=True).to(q.dtype)
    return dq, dkv


@_pk_cross_bwd.register_fake
def _(q, kv, bias, cq, sq, ck, sk, o, do, h, lkp, bq, rope, half, rot, prec, scale):  # noqa: ANN001
    return torch.empty_like(q), torch.empty_like(kv)


def _pk_cross_setup(ctx, inputs, output):  # noqa: ANN001
    q, kv, bias, cq, sq, ck, sk, *cfg = inputs
    ctx.save_for_backward(q, kv, bias, cq, sq, ck, sk, output)
    ctx.cfg = tuple(cfg)


def _pk_cross_backward(ctx, do):  # noqa: ANN001
    q, kv, bias, cq, sq, ck, sk, o = ctx.saved_tensors
    dq, dkv = torch.ops.tabicl_pk.pk_cross_bwd(q, kv, bias, cq, sq, ck, sk, o, do.to(o.dtype).contiguous(),
                                               *ctx.cfg)
    return (dq, dkv) + (None,) * (5 + len(ctx.cfg))


_pk_cross_fwd.register_autograd(_pk_cross_backward, setup_context=_pk_cross_setup)


HX_FWD = torch.ops.tabicl_pk.hx_fwd
HXQ_FWD = torch.ops.tabicl_pk.hxq_fwd
PK_SELF = torch.ops.tabicl_pk.pk_self_fwd
PK_CROSS = torch.ops.tabicl_pk.pk_cross_fwd
PK_CROSS_RAGGED = torch.ops.tabicl_pk.pk_cross_fwd_ragged
HXF_FWD = torch.ops.tabicl_pk.hxf_fwd
HX_BWD = torch.ops.tabicl_pk.hx_bwd
PK_SELF_BWD = torch.ops.tabicl_pk.pk_self_bwd
PK_CROSS_BWD = torch.ops.tabicl_pk.pk_cross_bwd


# ---------------------------------------------------------------------------------------------
# Python wrappers (reference signatures)
# ---------------------------------------------------------------------------------------------
def hx_attention(q: Tensor, k: Tensor, v: Tensor, h: int, key_bias: Optional[Tensor] = None) -> Tensor:
    """q [..., Lq, E] (pre-scaled), k / v [..., Lk, E]; key_bias additive, broadcastable to [..., Lk]
    (reference scripts/tabicl_tpu_pallas_attn.py:767-790)."""
    lead = q.shape[:-2]
    Lq, E = q.shape[-2], q.shape[-1]
    Lk = k.shape[-2]
    lkp = -(-Lk // 128) * 128
    q3 = _flat(q, Lq, E)
    k3 = _flat(k, Lk, E)
    v3 = _flat(v, Lk, E)
    bias = _bias_arg(key_bias, lead, Lk, q.device)
    prec = _fp32_prec_code() if q.dtype == torch.float32 else 0
    out = HX_FWD(q3.contiguous(), k3.contiguous(), v3.contiguous(), bias, h, lkp, _pick_bq(Lq, lkp), prec)
    return out.reshape(*lead, Lq, E)


def hxq_attention(q: Tensor, kv: Tensor, valid_len: Optional[Tensor], h: int,
                  key_bias: Optional[Tensor] = None) -> Tensor:
    """Inference only. q [..., Lq, E] (pre-scaled), kv [..., Lk, 2E] packed (K = lanes [0, E),
    V = [E, 2E)); keys at positions >= valid_len are ignored (reference :323-336). valid_len may be
    a scalar or hold one entry per flattened batch element (ragged batches), or be None with a
    key_bias. key_bias (extension): additive key mask broadcastable to [..., Lk], e.g. the
    finfo.min train mask upstream builds from a tensor train size."""
    lead = q.shape[:-2]
    Lq, E = q.shape[-2], q.shape[-1]
    Lk = kv.shape[-2]
    q3 = _flat(q, Lq, E).contiguous()
    kv3 = _flat(kv, Lk, 2 * E).contiguous()
    if q3.shape[0] != kv3.shape[0]:
        q3 = q3.expand(kv3.shape[0], Lq, E).contiguous()
    if valid_len is None:
        valid = torch.full((1,), Lk, dtype=torch.int32, device=q.device)
    else:
        valid = torch.as_tensor(valid_len, device=q.device).to(dtype=torch.int32).reshape(-1).contiguous()
    kb = None
    if key_bias is not None:
        kb = _bias3(key_bias, kv.shape[:-2], Lk, q.device).reshape(-1, Lk)
    prec = _fp32_prec_code() if q.dtype == torch.float32 else 0
    out = HXQ_FWD(valid, q3, kv3, h, _pick_bk(Lk), prec, kb)
    return out.reshape(*lead, Lq, E) if len(lead) else out.reshape(Lq, E)


def pk_self_attention(qkv: Tensor, h: int, key_bias: Optional[Tensor], rope_mod, scale: float) -> Tensor:  # noqa: ANN001
    """qkv [..., L, 3E] (packed in-projection), RoPE (optional) on q and k, returns [..., L, E]
    (reference :722-732)."""
    lead = qkv.shape[:-2]
    L, E3 = qkv.shape[-2], qkv.shape[-1]
    E = E3 // 3
    lkp = -(-L // 128) * 128
    cos, sin, rc, half, rot = _tables(rope_mod, L, E, h, qkv.device)
    prec = _fp32_prec_code() if qkv.dtype == torch.float32 else 0
    out = PK_SELF(_flat(qkv, L, E3).contiguous(), _bias_arg(key_bias, lead, L, qkv.device), cos, sin, h, lkp, rc,
                  half, rot, prec, float(scale))
    return out.reshape(*lead, L, E)


ROPE_SHARED_TABLES = 0x10  # TABICL_ROPE_SHARED_TABLES of include/tabicl_attn.h


def _shared_tables(cos: Tensor, sin: Tensor, rc: int, d: int):
    """Shared-head form of rope_tables' output: its columns repeat every head (d columns), so one
    head's [L, d] slice serves all heads and the kernels read h times fewer table bytes (forward and
    backward kernels alike)."""
    return cos[:, :d].contiguous(), sin[:, :d].contiguous(), rc | ROPE_SHARED_TABLES


# Tables per rope module, built once per (L, E, h, device, form) and reused while the module's
# frequencies are unchanged: the row stage calls the kernels with the same module and length every
# layer, and building the tables takes ~8 small torch kernels (a fifth of a row-attention call).
_TABLES: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()
_NO_ROPE: dict = {}


def _freqs_stamp(rope_mod) -> tuple:  # noqa: ANN001
    f = getattr(rope_mod, "freqs", None)
    if not isinstance(f, Tensor):
        return (None,)
    return (f.data_ptr(), f._version, tuple(f.shape), f.dtype, getattr(rope_mod, "interpolate_factor", None))


def _tables(rope_mod, L: int, E: int, h: int, device):  # noqa: ANN001
    """The shared-head form of rope_tables(...), cached per rope module. Under torch.compile the tables
    are computed in the traced graph instead (the cache key holds the frequencies' storage address,
    which a trace cannot guard on), as the reference computes them at trace time."""
    if torch.compiler.is_compiling():
        if rope_mod is None:
            return torch.ones(1, E, device=device), torch.zeros(1, E, device=device), 0, 0, 0
        cos, sin, rc, half, rot = rope_tables(rope_mod, L, E, h, device)
        if rc:
            cos, sin, rc = _shared_tables(cos, sin, rc, E // h)
        return cos, sin, rc, half, rot
    if rope_mod is None:
        # rope code 0: the kernels never read the tables, so one cached row stands in for [L, E]
        key = (E, str(device))
        hit = _NO_ROPE.get(key)
        if hit is None:
            hit = _NO_ROPE[key] = (torch.ones(1, E, device=device), torch.zeros(1, E, device=device), 0, 0, 0)
        return hit
    try:
        per_mod = _TABLES.setdefault(rope_mod, {})
    except TypeError:  # not weak-referenceable: no cache
        per_mod = None
    key = (L, E, h, str(device), bool(rope_mod.interleaved), _freqs_stamp(rope_mod))
    hit = None if per_mod is None else per_mod.get(key)
    if hit is not None:
        return hit
    cos, sin, rc, half, rot = rope_tables(rope_mod, L, E, h, device)
    if rc:
        cos, sin, rc = _shared_tables(cos, sin, rc, E // h)
    out = (cos, sin, rc, half, rot)
    if per_mod is not None and not cos.requires_grad:  # learned frequencies under autograd: not cached
        if len(per_mod) > 64:
            per_mod.clear()
        per_mod[key] = out
    return out


def pk_cross_attention(q: Tensor, kv: Tensor, h: int, key_bias: Optional[Tensor], rope_mod,  # noqa: ANN001
                       scale: float, q_len: Optional[Tensor] = None) -> Tensor:
    """q [..., Lq, E], kv [..., Lk, 2E] (packed K | V projection); RoPE (optional) with positions
    0..L-1 each (reference :735-752). A q that is one query set broadcast over kv's batch (a single
    leading element, or an expanded view with batch stride 0) is read once by the kernel, not copied.
    q_len (extension, inference only): int32 tensor with 1 or one entry per flattened batch element
    giving the rows each one needs (a ragged batch padded to a row bucket); the contents of the rows
    at or past it are unspecified."""
    lead = q.shape[:-2]
    Lq, E = q.shape[-2], q.shape[-1]
    Lk = kv.shape[-2]
    lkp = -(-Lk // 128) * 128
    bq = _pick_bq(Lq, lkp)
    cq, sq, rc, half, rot = _tables(rope_mod, Lq, E, h, q.device)
    ck, sk, _, _, _ = _tables(rope_mod, Lk, E, h, q.device)
    prec = _fp32_prec_code() if q.dtype == torch.float32 else 0
    q3 = _flat(q, Lq, E)
    kv3 = _flat(kv, Lk, 2 * E)
    if q3.shape[0] == 1 or (q3.stride(0) == 0 and q3.shape[0] == kv3.shape[0]):
        q3 = q3[:1]
    elif q3.shape[0] != kv3.shape[0]:
        q3 = q3.expand(kv3.shape[0], Lq, E)
    out_lead = lead if q.shape[:-2].numel() == kv3.shape[0] else kv.shape[:-2]
    bias = _bias_arg(key_bias, out_lead, Lk, q.device)
    if q_len is not None:
        ql = q_len.to(device=q.device, dtype=torch.int32).reshape(-1).contiguous()
        out = PK_CROSS_RAGGED(q3.contiguous(), kv3.contiguous(), bias, cq, sq, ck, sk, ql, h, lkp, bq, rc, half, rot,
                              prec, float(scale))
    else:
        out = PK_CROSS(q3.contiguous(), kv3.contiguous(), bias, cq, sq, ck, sk, h, lkp, bq, rc, half, rot, prec,
                       float(scale))
    return out.reshape(*out_lead, Lq, E)


def hxf_attention(qf: Tensor, x: Tensor, valid_len: Optional[Tensor], key_bias: Optional[Tensor] = None) -> Tensor:
    """Inference only. qf [hq, E] (shared by every batch element) or [..., hq, E]: folded, pre-scaled
    queries; x [..., Lk, E]: the raw key/value rows (positions >= valid_len ignored). Returns
    softmax(qf x^T) x: [..., hq, E] (reference :429-442). valid_len may be a scalar or hold one
    length per flattened batch element, or be None with a key_bias (extension: additive key mask
    broadcastable to [..., Lk]); qf is computed in x's dtype."""
    lead = x.shape[:-2]
    Lk, E = x.shape[-2], x.shape[-1]
    hq = qf.shape[-2]
    x3 = _flat(x, Lk, E).contiguous()
    q3 = _flat(qf, hq, E).to(x.dtype)
    if q3.shape[0] not in (1, x3.shape[0]):
        q3 = q3.expand(x3.shape[0], hq, E)
    if valid_len is None:
        valid = torch.full((1,), Lk, dtype=torch.int32, device=x.device)
    else:
        valid = torch.as_tensor(valid_len, device=x.device).to(dtype=torch.int32).reshape(-1).contiguous()
    kb = None if key_bias is None else _bias3(key_bias, lead, Lk, x.device).reshape(-1, Lk)
    prec = _fp32_prec_code() if x.dtype == torch.float32 else 0
    out = HXF_FWD(valid, q3.contiguous(), x3, _pick_bk(Lk), prec, kb)
    return out.reshape(*lead, hq, E)
