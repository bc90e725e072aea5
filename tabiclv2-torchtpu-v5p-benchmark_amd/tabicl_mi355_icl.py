"""Dataset-wise in-context attention over a cached train-row K/V (8 heads x 64 dims) on MI355X.

Replaces the reference's Splash path for the ICL stage:
  * icl_sdpa(q, k, v, valid_kv_len) keeps the contract of the hook _tpu_pallas_splash_sdpa
    (results/tpu_patch.diff:123-155; knob version scripts/tabicl_tpu_bucketed.py:221-246): q, k, v
    [..., H, T, D], q not pre-scaled (D^-0.5 applied inside), keys at positions >= valid_kv_len
    ignored, output [..., H, Tq, D] in q's dtype. Unlike the reference nothing is padded: the kernel
    masks the key tail and any Tq works.
  * torch op tabicl::icl_cached_attn(q, k, v, valid, scale) is the registered kernel (the
    counterpart of tabicl::tpu_splash_sdpa_seg / _full, diff:95-120).
  * IclKVCache holds the fit-time cache in one [estimator, block, head, row, d] tensor per K and V
    (the reference keeps tuples of per-block [B, H, T, d] tensors, tabicl_tpu_bucketed.py:413-435),
    appended once per block at fit time and read per block at query time (:803-817).
    append_projected writes a block's K/V straight from the train rows and the packed in-projection;
    attention_layer runs one block's cached attention sub-layer (Q projection, attention over the
    cache, out-projection) around the kernel.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Optional, Union

import torch
import torch.nn.functional as F
from torch import Tensor

import tabicl_mi355_native as _nat


def _strides3(t: Tensor):
    """(n, h, row) element strides of a [N, H, T, D] view whose last dim is contiguous."""
    if t.stride(-1) != 1:
        raise ValueError("icl attention needs a contiguous last dimension")
    return t.stride(0), t.stride(1), t.stride(2)


_WS_BYTES: dict = {}


def _workspace(N: int, H: int, Tq: int, Tkv: int, D: int, code: int, device) -> Optional[Tensor]:
    """Scratch for the key-split path of the kernel (size from the library, per shape and device),
    taken from torch's caching allocator on the launch stream; None when the call does not split."""
    key = (N, H, Tq, Tkv, D, code, device.index)
    nbytes = _WS_BYTES.get(key)
    if nbytes is None:
        nbytes = int(_nat.load().tabicl_icl_workspace_bytes(N, H, Tq, Tkv, D, code))
        if nbytes < 0:
            raise RuntimeError(f"tabicl_icl_workspace_bytes: {_nat.last_error()}")
        _WS_BYTES[key] = nbytes
    return torch.empty(nbytes, dtype=torch.uint8, device=device) if nbytes > 0 else None


def _launch(q: Tensor, k: Tensor, v: Tensor, valid: Optional[Tensor], scale: float, out: Tensor,
            q_len: Optional[Tensor] = None, key_bias: Optional[Tensor] = None, plan_ws: Optional[Tensor] = None) -> None:
    _nat.require_device(q, k, v, valid, out, q_len, key_bias)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("icl_cached_attn expects [N, H, T, D] tensors")
    N, H, Tq, D = q.shape
    Tkv = k.shape[2]
    if k.shape != v.shape or k.shape[0] != N or k.shape[1] != H or k.shape[3] != D:
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if out.shape != q.shape:
        raise ValueError(f"out {tuple(out.shape)} must match q {tuple(q.shape)}")
    if q.dtype != k.dtype or k.dtype != v.dtype or out.dtype != q.dtype:
        raise ValueError("q, k, v and out must share a dtype (promote q to the cache dtype first)")
    vptr, vn = None, 0
    if valid is not None:
        if valid.dtype != torch.int32 or not valid.is_contiguous():
            raise ValueError("valid must be a contiguous int32 tensor")
        vptr, vn = valid.data_ptr(), valid.numel()
    code = _nat.dtype_code(q.dtype)
    if plan_ws is not None:
        if q_len is None or key_bias is not None:
            raise ValueError("a ragged plan serves ragged calls without a key mask")
        nbytes = _WS_BYTES.get((N, H, Tq, Tkv, D, code, q.device.index))
        if nbytes is None or plan_ws.numel() != nbytes or plan_ws.device != q.device:
            raise ValueError("the plan was made for other sizes, dtype or device")
    ws = plan_ws if plan_ws is not None else _workspace(N, H, Tq, Tkv, D, code, q.device)
    tail = (*_strides3(q), *_strides3(k), *_strides3(v), *_strides3(out), float(scale), code,
            None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _nat.stream_of(q))
    if q_len is not None and (q_len.dtype != torch.int32 or not q_len.is_contiguous() or q_len.numel() not in (1, N)):
        raise ValueError(f"q_len must be a contiguous int32 tensor of 1 or {N} entries")
    if key_bias is not None:
        if key_bias.dtype != torch.float32 or key_bias.dim() != 2 or key_bias.shape[1] != Tkv \
                or key_bias.shape[0] not in (1, N) or key_bias.stride(1) != 1:
            raise ValueError(f"key_bias must be a float32 [1 or {N}, {Tkv}] tensor with contiguous rows, got "
                             f"{key_bias.dtype} {tuple(key_bias.shape)}")
        _nat.call("tabicl_icl_fwd_masked", q.data_ptr(), k.data_ptr(), v.data_ptr(), vptr, vn, key_bias.data_ptr(),
                  key_bias.shape[0], key_bias.stride(0), None if q_len is None else q_len.data_ptr(),
                  0 if q_len is None else q_len.numel(), out.data_ptr(), N, H, Tq, Tkv, D, *tail)
        return
    if q_len is None:
        _nat.call("tabicl_icl_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), vptr, vn, out.data_ptr(),
                  N, H, Tq, Tkv, D, *tail)
        return
    _nat.call("tabicl_icl_fwd_ragged_listed" if plan_ws is not None else "tabicl_icl_fwd_ragged", q.data_ptr(),
              k.data_ptr(), v.data_ptr(), vptr, vn, q_len.data_ptr(), q_len.numel(), out.data_ptr(), N, H, Tq, Tkv, D,
              *tail)


@torch.library.custom_op("tabicl::icl_cached_attn", mutates_args=())
def _icl_cached_attn(q: Tensor, k: Tensor, v: Tensor, valid: Optional[Tensor], scale: float,
                     key_bias: Optional[Tensor] = None) -> Tensor:
    """key_bias: optional additive fp32 key mask [1 or N, Tkv] (the reference's masked path,
    results/tpu_patch.diff:263-270); a prefix mask (0 then <= -1e30) runs as a valid length on the
    pipelined kernel, any other mask on its masked instance (the mask terms start each score product;
    power-of-two scale) or on the exact kernel, which adds it tile by tile."""
    out = torch.empty(q.shape, device=q.device, dtype=q.dtype)
    _launch(q, k, v, valid, scale, out, None, key_bias)
    return out


@_icl_cached_attn.register_fake
def _(q, k, v, valid, scale, key_bias=None):  # noqa: ANN001
    return torch.empty_like(q)


@torch.library.custom_op("tabicl::icl_cached_attn_bwd", mutates_args=())
def _icl_cached_attn_bwd(q: Tensor, k: Tensor, v: Tensor, valid: Optional[Tensor], key_bias: Optional[Tensor],
                         out: Tensor, dout: Tensor, scale: float,
                         stat: Optional[Tensor] = None) -> tuple[Tensor, Tensor, Tensor]:
    """Gradients (dq, dk, dv) of icl_cached_attn for the upstream gradient dout, given the forward's
    inputs and its output `out` (tabicl_icl_bwd). The reference's calls with a gradient take autograd
    through its tiled online-softmax attention (results/tpu_patch.diff:158-193, chosen at :263-270);
    here both products and the softmax recompute run in the library's two backward kernels. Keys past
    the valid length get zero gradients; key_bias gets none (a mask, not a parameter). stat: the
    forward's softmax statistics [N, H, Tq, 2] (icl_cached_attn_train; calls without key_bias), which
    spare the backward its own sweep over the keys."""
    _nat.require_device(q, k, v, valid, key_bias, out, dout, stat)
    q, k, v, out, dout = (_nat.aligned16(t) for t in (q, k, v, out, dout))
    N, H, Tq, D = q.shape
    Tkv = k.shape[2]
    if k.shape != v.shape or k.shape[:2] != q.shape[:2] or k.shape[3] != D or out.shape != q.shape \
            or dout.shape != q.shape:
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)} "
                         f"out {tuple(out.shape)} dout {tuple(dout.shape)}")
    if not (q.dtype == k.dtype == v.dtype == out.dtype == dout.dtype):
        raise ValueError("q, k, v, out and dout must share a dtype")
    vptr, vn = None, 0
    if valid is not None:
        if valid.dtype != torch.int32 or not valid.is_contiguous():
            raise ValueError("valid must be a contiguous int32 tensor")
        vptr, vn = valid.data_ptr(), valid.numel()
    bptr, bn, bsn = None, 0, 0
    if key_bias is not None:
        if key_bias.dtype != torch.float32 or key_bias.dim() != 2 or key_bias.shape[1] != Tkv \
                or key_bias.shape[0] not in (1, N) or key_bias.stride(1) != 1:
            raise ValueError(f"key_bias must be a float32 [1 or {N}, {Tkv}] tensor with contiguous rows")
        bptr, bn, bsn = key_bias.data_ptr(), key_bias.shape[0], key_bias.stride(0)
    sptr = None
    if stat is not None:
        if stat.dtype != torch.float32 or stat.shape != (N, H, Tq, 2) or key_bias is not None:
            raise ValueError(f"stat must be the float32 [{N}, {H}, {Tq}, 2] statistics of a call without key_bias")
        stat = _nat.aligned16(stat)
        sptr = stat.data_ptr()
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    nbytes = int(_nat.load().tabicl_icl_bwd_workspace_bytes(N, H, Tq))
    if nbytes < 0:
        raise RuntimeError(f"tabicl_icl_bwd_workspace_bytes: {_nat.last_error()}")
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=q.device)
    _nat.call("tabicl_icl_bwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), vptr, vn, bptr, bn, bsn, out.data_ptr(),
              dout.data_ptr(), sptr, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), N, H, Tq, Tkv, D, float(scale),
              _nat.dtype_code(q.dtype), ws.data_ptr(), ws.numel(), _nat.stream_of(q))
    return dq, dk, dv


@_icl_cached_attn_bwd.register_fake
def _(q, k, v, valid, key_bias, out, dout, scale, stat=None):  # noqa: ANN001
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


@torch.library.custom_op("tabicl::icl_cached_attn_train", mutates_args=())
def _icl_cached_attn_train(q: Tensor, k: Tensor, v: Tensor, valid: Optional[Tensor],
                           scale: float) -> tuple[Tensor, Tensor]:
    """icl_cached_attn without a key mask for calls with a gradient: returns (out, stat), stat the
    softmax statistics [N, H, Tq, 2] (m, l) of each query row (tabicl_icl_fwd_stats), which its
    backward hands to icl_cached_attn_bwd. The forward of the reference's gradient path (autograd
    through _tiled_online_sdpa, results/tpu_patch.diff:158-193), whose saved tensors play this part."""
    _nat.require_device(q, k, v, valid)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("icl_cached_attn_train expects [N, H, T, D] tensors")
    N, H, Tq, D = q.shape
    Tkv = k.shape[2]
    if k.shape != v.shape or k.shape[0] != N or k.shape[1] != H or k.shape[3] != D:
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if q.dtype != k.dtype or k.dtype != v.dtype:
        raise ValueError("q, k and v must share a dtype")
    vptr, vn = None, 0
    if valid is not None:
        if valid.dtype != torch.int32 or not valid.is_contiguous():
            raise ValueError("valid must be a contiguous int32 tensor")
        vptr, vn = valid.data_ptr(), valid.numel()
    out = torch.empty(q.shape, device=q.device, dtype=q.dtype)
    stat = torch.empty((N, H, Tq, 2), device=q.device, dtype=torch.float32)
    code = _nat.dtype_code(q.dtype)
    ws = _workspace(N, H, Tq, Tkv, D, code, q.device)
    _nat.call("tabicl_icl_fwd_stats", q.data_ptr(), k.data_ptr(), v.data_ptr(), vptr, vn, out.data_ptr(),
              stat.data_ptr(), N, H, Tq, Tkv, D, *_strides3(q), *_strides3(k), *_strides3(v), *_strides3(out),
              float(scale), code, None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
              _nat.stream_of(q))
    return out, stat


@_icl_cached_attn_train.register_fake
def _(q, k, v, valid, scale):  # noqa: ANN001
    return torch.empty_like(q), q.new_empty((*q.shape[:3], 2), dtype=torch.float32)


def _icl_train_setup_context(ctx, inputs, output):  # noqa: ANN001
    q, k, v, valid, scale = inputs
    out, stat = output
    ctx.save_for_backward(q, k, v, valid, out, stat)
    ctx.scale = scale
    ctx.mark_non_differentiable(stat)


def _icl_train_backward(ctx, grad, grad_stat):  # noqa: ANN001
    q, k, v, valid, out, stat = ctx.saved_tensors
    dq, dk, dv = torch.ops.tabicl.icl_cached_attn_bwd(q, k, v, valid, None, out, grad, ctx.scale, stat)
    return dq, dk, dv, None, None


_icl_cached_attn_train.register_autograd(_icl_train_backward, setup_context=_icl_train_setup_context)


def _icl_setup_context(ctx, inputs, output):  # noqa: ANN001
    q, k, v, valid, scale, key_bias = inputs
    ctx.save_for_backward(q, k, v, valid, key_bias, output)
    ctx.scale = scale


def _icl_backward(ctx, grad):  # noqa: ANN001
    q, k, v, valid, key_bias, out = ctx.saved_tensors
    dq, dk, dv = torch.ops.tabicl.icl_cached_attn_bwd(q, k, v, valid, key_bias, out, grad, ctx.scale)
    return dq, dk, dv, None, None, None


_icl_cached_attn.register_autograd(_icl_backward, setup_context=_icl_setup_context)


@torch.library.custom_op("tabicl::icl_cached_attn_out", mutates_args=("out",))
def _icl_cached_attn_out(q: Tensor, k: Tensor, v: Tensor, valid: Optional[Tensor], scale: float,
                         out: Tensor, key_bias: Optional[Tensor] = None) -> None:
    """Same as icl_cached_attn, written into `out` (any [N, H, Tq, D] view with a contiguous last
    dim, e.g. one block of a [est, block, head, row, d] result buffer)."""
    _launch(q, k, v, valid, scale, out, None, key_bias)


@_icl_cached_attn_out.register_fake
def _(q, k, v, valid, scale, out, key_bias=None):  # noqa: ANN001
    return None


@torch.library.custom_op("tabicl::icl_cached_attn_ragged_out", mutates_args=("out",))
def _icl_cached_attn_ragged_out(q: Tensor, k: Tensor, v: Tensor, valid: Optional[Tensor], q_len: Tensor,
                                scale: float, out: Tensor, key_bias: Optional[Tensor] = None,
                                plan_ws: Optional[Tensor] = None) -> None:
    """icl_cached_attn_out over a ragged batch: rows at or past q_len[n] (1 or N entries) are neither
    computed nor written (out keeps what it held). No counterpart in the reference, whose bucketed
    runner attends with the padding rows of each table's test bucket too. plan_ws: the workspace of an
    IclRaggedPlan for these sizes and q_len (IclRaggedPlan.workspace): the list of live work items is
    taken from it instead of being computed by this call."""
    _launch(q, k, v, valid, scale, out, q_len, key_bias, plan_ws)


@_icl_cached_attn_ragged_out.register_fake
def _(q, k, v, valid, q_len, scale, out, key_bias=None, plan_ws=None):  # noqa: ANN001
    return None


ICL_FWD = torch.ops.tabicl.icl_cached_attn
ICL_FWD_TRAIN = torch.ops.tabicl.icl_cached_attn_train
ICL_FWD_OUT = torch.ops.tabicl.icl_cached_attn_out
ICL_FWD_RAGGED_OUT = torch.ops.tabicl.icl_cached_attn_ragged_out


class IclRaggedPlan:
    """The list of live work items of one ragged ICL call shape, computed once on the current stream
    (tabicl_icl_ragged_plan) into a workspace that the calls then share: pass `plan.workspace` as
    ICL_FWD_RAGGED_OUT's plan_ws for every call with the same N, H, Tq, Tkv, head dim, dtype and the
    same q_len contents, e.g. the 12 ICL blocks of one bucket. The calls must follow each other on one
    stream (they share the workspace); a q_len changed after the plan leaves rows unwritten. No
    counterpart in the reference (its runner has no ragged calls)."""

    def __init__(self, q_len: Tensor, N: int, H: int, Tq: int, Tkv: int, D: int = 64,
                 dtype: torch.dtype = torch.bfloat16):
        _nat.require_device(q_len)
        if q_len.dtype != torch.int32 or not q_len.is_contiguous() or q_len.numel() not in (1, N):
            raise ValueError(f"q_len must be a contiguous int32 tensor of 1 or {N} entries")
        code = _nat.dtype_code(dtype)
        ws = _workspace(N, H, Tq, Tkv, D, code, q_len.device)
        self.workspace = ws if ws is not None else torch.empty(0, dtype=torch.uint8, device=q_len.device)
        self.q_len = q_len
        _nat.call("tabicl_icl_ragged_plan", q_len.data_ptr(), q_len.numel(), N, H, Tq, Tkv, D, code,
                  None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _nat.stream_of(q_len))


@torch.library.custom_op("tabicl::tpu_splash_sdpa_seg", mutates_args=())
def splash_sdpa_seg_op(q_in: Tensor, k_in: Tensor, v_in: Tensor, valid_kv_t: Tensor, bq: int, bkv: int) -> Tensor:
    """The reference's Splash op under its own name and schema (results/tpu_patch.diff:95-102), on the
    HIP ICL kernel: q_in [N, H, Tq, D] already scaled by D^-0.5 (the caller pads and scales,
    diff:133-139), k_in / v_in [N, H, Tkv, D], keys >= valid_kv_t (an int32 scalar tensor) masked. bq and
    bkv are the TPU kernel's block sizes and are ignored: the library picks its own tiling, and needs no
    padding of Tq or Tkv. Bound to the upstream attention module's `_tpu_splash_sdpa_seg_op` by
    install(), so code that calls that attribute (the reference's knob hook,
    scripts/tabicl_tpu_bucketed.py:236-242) reaches this kernel."""
    valid = valid_kv_t.to(device=q_in.device, dtype=torch.int32).reshape(1).contiguous()
    out = torch.empty(q_in.shape, device=q_in.device, dtype=q_in.dtype)
    _launch(q_in, k_in, v_in, valid, 1.0, out)
    return out


@splash_sdpa_seg_op.register_fake
def _(q_in, k_in, v_in, valid_kv_t, bq, bkv):  # noqa: ANN001
    return torch.empty_like(q_in)


@torch.library.custom_op("tabicl::tpu_splash_sdpa_full", mutates_args=())
def splash_sdpa_full_op(q_in: Tensor, k_in: Tensor, v_in: Tensor, bq: int, bkv: int) -> Tensor:
    """tpu_splash_sdpa_seg with every key valid (results/tpu_patch.diff:110-115)."""
    out = torch.empty(q_in.shape, device=q_in.device, dtype=q_in.dtype)
    _launch(q_in, k_in, v_in, None, 1.0, out)
    return out


@splash_sdpa_full_op.register_fake
def _(q_in, k_in, v_in, bq, bkv):  # noqa: ANN001
    return torch.empty_like(q_in)


def icl_supported(Tq: int, Tkv: int, D: int, dtype: torch.dtype) -> bool:
    return dtype in (torch.bfloat16, torch.float32) and _nat.supported(_nat.OP_ICL, Tq, Tkv, D, 1, dtype)


def icl_sdpa(q: Tensor, k: Tensor, v: Tensor, valid_kv_len: Optional[Union[int, Tensor]] = None,
             key_bias: Optional[Tensor] = None) -> Tensor:
    """softmax(q k^T * D^-0.5 + key mask) v for q [..., H, Tq, D], k/v [..., H, Tkv, D]; keys at
    positions >= valid_kv_len are masked (a tensor may hold one length per flattened batch entry).
    Contract of the reference hook _tpu_pallas_splash_sdpa (results/tpu_patch.diff:123-155).
    key_bias (extension): an additive key mask with one row for all flattened batch entries or one
    per entry ([Tkv], [1, Tkv] or [N, Tkv]; any leading shape that flattens to those), e.g. the train
    mask upstream builds from a tensor train size (diff:1526-1542)."""
    D = q.shape[-1]
    lead = q.shape[:-3]
    H, Tq = q.shape[-3], q.shape[-2]
    Tkv = k.shape[-2]
    n = math.prod(lead)  # explicit: reshape(-1, ...) is ambiguous with no query rows
    q4 = q.reshape(n, H, Tq, D)
    k4 = k.reshape(n, H, Tkv, D)
    v4 = v.reshape(n, H, Tkv, D)
    valid = None
    if isinstance(valid_kv_len, Tensor):
        valid = valid_kv_len.to(device=q.device, dtype=torch.int32).reshape(-1).contiguous()
    elif valid_kv_len is not None and int(valid_kv_len) < Tkv:
        valid = torch.full((1,), int(valid_kv_len), dtype=torch.int32, device=q.device)
    kb = None
    if key_bias is not None:
        kb = key_bias.to(device=q.device, dtype=torch.float32).reshape(-1, Tkv)
        if kb.shape[0] not in (1, q4.shape[0]):
            raise ValueError(f"key_bias rows {kb.shape[0]} must be 1 or the flattened batch {q4.shape[0]}")
        kb = _nat.aligned16(kb)
    if kb is None and torch.is_grad_enabled() and (q4.requires_grad or k4.requires_grad or v4.requires_grad):
        out = ICL_FWD_TRAIN(q4, k4, v4, valid, float(D) ** -0.5)[0]  # keeps the statistics for the backward
    else:
        out = ICL_FWD(q4, k4, v4, valid, float(D) ** -0.5, kb)
    return out.reshape(*lead, H, Tq, D)


class IclKVCache:
    """Fit-time K/V cache of the ICL stage, one tensor per K and V of shape
    [estimators, blocks, heads, capacity, head_dim].

    append(block, k, v, row0) writes rows [row0, row0 + T) of one block from k/v [E, H, T, d]
    (the per-block K/V the prefill produces, reference scripts/tabicl_tpu_bucketed.py:659-692);
    block_kv(block) returns the [E, H, capacity, d] views the query reads (:803-817).

    Each block records which rows appends have written (merged row intervals); `length(block)` is the
    contiguous run from row 0. A query without an explicit valid length attends over exactly that run,
    so the unwritten rows of the cache (torch.empty memory) are never read; querying a block whose row 0
    was never written raises."""

    def __init__(self, estimators: int, blocks: int, heads: int, capacity: int, head_dim: int,
                 dtype: torch.dtype = torch.bfloat16, device: Union[str, torch.device] = "cuda"):
        shape = (estimators, blocks, heads, capacity, head_dim)
        self.keys = torch.empty(shape, dtype=dtype, device=device)
        self.values = torch.empty(shape, dtype=dtype, device=device)
        self.capacity = capacity
        self.written = [[] for _ in range(blocks)]  # per block: sorted, disjoint [start, end) row intervals
        self._len_t: dict = {}  # length -> int32 device tensor handed to the kernels

    def length(self, block: int) -> int:
        """Rows [0, length) of `block` hold appended K/V."""
        iv = self.written[block]
        return iv[0][1] if iv and iv[0][0] == 0 else 0

    def _record(self, block: int, row0: int, T: int) -> None:
        if T <= 0:
            return
        merged = []
        lo, hi = row0, row0 + T
        for a, b in self.written[block]:
            if b < lo or a > hi:
                merged.append((a, b))
            else:
                lo, hi = min(lo, a), max(hi, b)
        merged.append((lo, hi))
        self.written[block] = sorted(merged)

    def default_valid(self, block: int) -> Tensor:
        """The block's filled length from row 0 as the int32 device tensor the kernels take."""
        n = self.length(block)
        if n <= 0:
            raise ValueError(f"block {block} of the cache has no rows from row 0: append before querying")
        t = self._len_t.get(n)
        if t is None:
            t = self._len_t[n] = torch.full((1,), n, dtype=torch.int32, device=self.keys.device)
        return t

    @property
    def shape(self):
        return tuple(self.keys.shape)

    def nbytes(self) -> int:
        return 2 * self.keys.numel() * self.keys.element_size()

    def append(self, block: int, k: Tensor, v: Tensor, row0: int = 0) -> None:
        E, NB, H, cap, D = self.keys.shape
        if k.shape != v.shape or k.dim() != 4 or k.shape[0] != E or k.shape[1] != H or k.shape[3] != D:
            raise ValueError(f"append expects k/v [{E}, {H}, T, {D}], got {tuple(k.shape)} / {tuple(v.shape)}")
        if k.stride() != v.stride():
            raise ValueError("k and v must share strides")
        if k.dtype != self.keys.dtype or v.dtype != self.keys.dtype:
            raise ValueError(f"append expects {self.keys.dtype} (cast before appending)")
        if not 0 <= block < NB:
            raise ValueError(f"block {block} out of range [0, {NB})")
        _nat.require_device(k, v, self.keys)
        T = k.shape[2]
        if row0 < 0 or row0 + T > cap:
            raise ValueError(f"rows [{row0}, {row0 + T}) exceed the capacity {cap}")
        kc = self.keys[:, block]
        vc = self.values[:, block]
        _nat.call("tabicl_icl_cache_append", kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), row0, cap,
                  k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.stride(2), E, H, T, D,
                  _nat.dtype_code(k.dtype), _nat.stream_of(k))
        self._record(block, row0, T)

    def append_projected(self, block: int, x: Tensor, in_proj_weight: Tensor, in_proj_bias: Optional[Tensor] = None,
                         row0: int = 0) -> None:
        """Fit-time K/V of one block straight from its train rows x [E, T, width] (the rows the block's
        attention projects, after its pre-norm): k = x W_k^T + b_k, v = x W_v^T + b_v with W_k, W_v the
        second and third thirds of the packed in-projection [3 width, width] (the query takes the first,
        results/tpu_patch.diff:308-310; need_kv returns the K/V projections, diff:1569-1575, 989), split
        into heads and written to rows [row0, row0 + T) of the block. One GEMM [E T, width] x [width,
        2 width] (torch / hipBLASLt) produces K|V interleaved per row; the append kernel reads the heads
        out of it through strides, so no permuted copy is made."""
        E, NB, H, cap, D = self.keys.shape
        width = H * D
        if x.dim() != 3 or x.shape[0] != E or x.shape[2] != width:
            raise ValueError(f"append_projected expects x [{E}, T, {width}], got {tuple(x.shape)}")
        if tuple(in_proj_weight.shape) != (3 * width, width):
            raise ValueError(f"in_proj_weight must be [{3 * width}, {width}], got {tuple(in_proj_weight.shape)}")
        if in_proj_bias is not None and tuple(in_proj_bias.shape) != (3 * width,):
            raise ValueError(f"in_proj_bias must be [{3 * width}], got {tuple(in_proj_bias.shape)}")
        _nat.require_device(x, in_proj_weight)
        T = x.shape[1]
        kv = F.linear(x, in_proj_weight[width:], None if in_proj_bias is None else in_proj_bias[width:])
        if kv.dtype != self.keys.dtype:
            kv = kv.to(self.keys.dtype)  # the reference stores k_l.to(cache_dtype) (tabicl_tpu_bucketed.py:676, 688)
        kv = kv.view(E, T, 2, H, D)
        self.append(block, kv[:, :, 0].permute(0, 2, 1, 3), kv[:, :, 1].permute(0, 2, 1, 3), row0)

    def attention_layer(self, block: int, x: Tensor, in_proj_weight: Tensor, in_proj_bias: Optional[Tensor],
                        out_proj_weight: Tensor, out_proj_bias: Optional[Tensor],
                        valid_kv_len: Optional[Union[int, Tensor]] = None,
                        q_transform: Optional[Callable[[Tensor], Tensor]] = None) -> Tensor:
        """One block's cached attention sub-layer for test rows x [E, Tq, width] (after the block's
        pre-norm): q = x W_q^T + b_q split into heads [E, H, Tq, D] (diff:308-312), q_transform applied
        to it if given (the caller's RoPE on q and SSMax scaling with n = the train length, modules of
        the upstream model: diff:312-313, 251-254), attention over block `block` of the cache with keys
        >= valid_kv_len (default: the block's filled length) masked and q promoted to the cache dtype
        (diff:314-317), heads merged and the
        out-projection applied (diff:383-393). Returns [E, Tq, width] in the promoted dtype; the residual and the
        feed-forward part of the block stay with the caller."""
        E, NB, H, cap, D = self.keys.shape
        width = H * D
        if x.dim() != 3 or x.shape[0] != E or x.shape[2] != width:
            raise ValueError(f"attention_layer expects x [{E}, Tq, {width}], got {tuple(x.shape)}")
        Tq = x.shape[1]
        q = F.linear(x, in_proj_weight[:width], None if in_proj_bias is None else in_proj_bias[:width])
        q = q.view(E, Tq, H, D).transpose(1, 2)  # heads as a strided view: the kernel takes row strides
        if q_transform is not None:
            q = q_transform(q)
        attn_dtype = torch.promote_types(q.dtype, self.keys.dtype)
        merged = torch.empty(E, Tq, H, D, dtype=attn_dtype, device=x.device)
        self.query(block, q, valid_kv_len, out=merged.transpose(1, 2))  # written in merged-head order
        o = merged.view(E, Tq, width)
        return F.linear(o, out_proj_weight.to(o.dtype), None if out_proj_bias is None else out_proj_bias.to(o.dtype))

    def query_blocks(self, x: Tensor, blocks, valid_kv_len: Optional[Union[int, Tensor]] = None,  # noqa: ANN001
                     q_transform: Optional[Callable[[Tensor], Tensor]] = None,
                     activation: Callable[[Tensor], Tensor] = F.gelu) -> Tensor:
        """The cached ICL query loop of the reference (scripts/tabicl_tpu_bucketed.py:803-817): test-row
        representations x [E, Tq, width] through every block of the cache, each a pre-norm transformer
        block (results/tpu_patch.diff:1454-1462, norm_first; SafeLayerNorm :1385-1397 normalises in its
        weights' dtype and returns the input dtype) whose attention reads the block's cached K/V:
            x = x + attention_layer(LN1(x)),   x = x + W2 act(W1 LN2(x) + b1) + b2.
        blocks: one IclBlockWeights per cache block, in order. The GEMMs run in the weights' dtype (bf16
        weights: the reference's bf16 autocast of the ICL stage) and the residual stream keeps x's dtype.
        q_transform (RoPE / SSMax on q: upstream modules) is applied to every block's head-split q."""
        if len(blocks) > self.keys.shape[1]:
            raise ValueError(f"{len(blocks)} blocks of weights for a cache of {self.keys.shape[1]} blocks")
        for b, w in enumerate(blocks):
            h = _safe_layer_norm(x, w.ln1_w, w.ln1_b, w.eps, w.in_w.dtype)
            a = self.attention_layer(b, h, w.in_w, w.in_b, w.out_w, w.out_b, valid_kv_len, q_transform).to(x.dtype)
            x, h = add_layer_norm(x, a, w.ln2_w, w.ln2_b, w.eps, w.ff1_w.dtype)  # x + attention, then norm2
            x = x + F.linear(activation(F.linear(h, w.ff1_w, w.ff1_b)), w.ff2_w, w.ff2_b).to(x.dtype)
        return x

    def estimators(self, start: int, stop: int) -> "IclKVCache":
        """Estimators [start, stop) of this cache as a cache of their own: views of the same storage and
        the same per-block row record (appends through either are seen by both). The per-chunk caches
        of a query whose batch is cut into ICL calls (query_chunked)."""
        E = self.keys.shape[0]
        if not 0 <= start < stop <= E:
            raise ValueError(f"estimators [{start}, {stop}) out of range [0, {E})")
        view = object.__new__(IclKVCache)
        view.keys = self.keys[start:stop]
        view.values = self.values[start:stop]
        view.capacity = self.capacity
        view.written = self.written
        view._len_t = self._len_t
        return view

    def query_chunked(self, x: Tensor, blocks, chunks, valid_kv_len: Optional[Union[int, Tensor]] = None,  # noqa: ANN001
                      q_transform: Optional[Callable[[Tensor], Tensor]] = None,
                      activation: Callable[[Tensor], Tensor] = F.gelu) -> Tensor:
        """query_blocks run once per batch chunk [start, stop) of x [E, Tq, width] (each against those
        estimators of the cache) and concatenated: the reference runner's ICL call pattern for a batch
        cut by its memory rule (scripts/tabicl_tpu_bucketed.py:1329-1375; chunks from
        BucketPlan.chunks()). Every row's result is that of one query_blocks call over the whole batch."""
        if not chunks or chunks[0][0] != 0 or chunks[-1][1] != x.shape[0] or any(
                a[1] != b[0] for a, b in zip(chunks, chunks[1:])):
            raise ValueError(f"chunks {chunks} do not cover the batch [0, {x.shape[0]}) in order")
        parts = [self.estimators(a, b).query_blocks(x[a:b], blocks, valid_kv_len, q_transform, activation)
                 for a, b in chunks]
        return parts[0] if len(parts) == 1 else torch.cat(parts, dim=0)

    def block_kv(self, block: int):
        return self.keys[:, block], self.values[:, block]

    def query(self, block: int, q: Tensor, valid_kv_len: Optional[Union[int, Tensor]] = None,
              out: Optional[Tensor] = None) -> Tensor:
        """Attention of q [E, H, Tq, D] (any row / head / estimator strides, contiguous head dim) over
        block `block` of the cache (keys >= valid_kv_len masked; default: the block's filled length, never
        the unwritten rows past it); into `out` (any [E, H, Tq, D] view with a contiguous head dim) if given."""
        if valid_kv_len is None:
            valid_kv_len = self.default_valid(block)
        k, v = self.block_kv(block)
        # promote_types(q, cache) as in the reference's cached branch (results/tpu_patch.diff:314-317)
        attn_dtype = torch.promote_types(q.dtype, k.dtype)
        q, k, v = q.to(attn_dtype), k.to(attn_dtype), v.to(attn_dtype)
        if out is None:
            return icl_sdpa(q, k, v, valid_kv_len)
        if q.stride(-1) != 1:
            q = q.contiguous()
        ICL_FWD_OUT(q, k, v, _valid_arg(valid_kv_len, k.shape[-2], q.device), float(q.shape[-1]) ** -0.5, out)
        return out


@dataclass
class IclBlockWeights:
    """Parameters of one ICL block (a pre-norm transformer encoder layer, results/tpu_patch.diff:1454-1462):
    norm1 / norm2 LayerNorm weight and bias [width] (fp32 in the reference, SafeLayerNorm :1385-1397), the
    packed in-projection [3 width, width] and bias, the out-projection [width, width] and bias, and the
    feed-forward linear1 [ff, width] / linear2 [width, ff] with biases (ff = ff_factor x width; the
    reference trains with ff_factor 2, scripts/train_stage1_optimized.py:205). Biases may be None."""
    ln1_w: Tensor
    ln1_b: Optional[Tensor]
    in_w: Tensor
    in_b: Optional[Tensor]
    out_w: Tensor
    out_b: Optional[Tensor]
    ln2_w: Tensor
    ln2_b: Optional[Tensor]
    ff1_w: Tensor
    ff1_b: Optional[Tensor]
    ff2_w: Tensor
    ff2_b: Optional[Tensor]
    eps: float = 1e-5


_LN_WIDTHS = (128, 512)
_LN_DTYPES = (torch.bfloat16, torch.float32)


def _ln_native(x: Tensor, w: Tensor, b: Optional[Tensor], eps: float, out_dtype: torch.dtype,
               r: Optional[Tensor] = None) -> bool:
    """Whether the library's row LayerNorm (tabicl_layer_norm) takes this call: GPU tensors, rows of 128
    or 512 contiguous values in bf16 / fp32, fp32 weights, an output dtype of bf16 / fp32."""
    W = x.shape[-1]
    return (x.device.type == "cuda" and W in _LN_WIDTHS and x.dtype in _LN_DTYPES and out_dtype in _LN_DTYPES
            and w.dtype == torch.float32 and w.is_contiguous() and w.numel() == W
            and (b is None or (b.dtype == torch.float32 and b.is_contiguous() and b.numel() == W))
            and (r is None or (r.dtype == x.dtype and r.shape == x.shape)))


def _ln_call(x: Tensor, r: Optional[Tensor], w: Tensor, b: Optional[Tensor], eps: float,
             out_dtype: torch.dtype):
    x = _nat.aligned16(x)
    r = None if r is None else _nat.aligned16(r)
    out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    xs = torch.empty_like(x) if r is not None else None
    _nat.call("tabicl_layer_norm", x.data_ptr(), None if r is None else r.data_ptr(),
              None if xs is None else xs.data_ptr(), w.data_ptr(), None if b is None else b.data_ptr(),
              out.data_ptr(), x.numel() // x.shape[-1], x.shape[-1], float(eps), _nat.dtype_code(x.dtype),
              _nat.dtype_code(out_dtype), _nat.stream_of(x))
    return xs, out


def _safe_layer_norm(x: Tensor, w: Tensor, b: Optional[Tensor], eps: float, out_dtype: torch.dtype) -> Tensor:
    """LayerNorm over the last dim computed in the weights' dtype (results/tpu_patch.diff:1385-1397), the
    result cast to the next GEMM's dtype. On the GPU for rows of 128 / 512 values: the library's row
    kernel (fp32 statistics, one pass over HBM); otherwise torch."""
    if _ln_native(x, w, b, eps, out_dtype):
        return _ln_call(x, None, w, b, eps, out_dtype)[1]
    return F.layer_norm(x.to(w.dtype), (x.shape[-1],), w, b, eps).to(out_dtype)


def add_layer_norm(x: Tensor, r: Tensor, w: Tensor, b: Optional[Tensor], eps: float, out_dtype: torch.dtype):
    """(s, LayerNorm(s)) with s = x + r in x's dtype: a residual add and the next pre-norm in one pass
    over HBM on the GPU (tabicl_layer_norm with a residual); otherwise torch, the same two steps."""
    if _ln_native(x, w, b, eps, out_dtype, r):
        return _ln_call(x, r, w, b, eps, out_dtype)
    s = x + r
    return s, _safe_layer_norm(s, w, b, eps, out_dtype)


def _valid_arg(valid_kv_len, Tkv: int, device) -> Optional[Tensor]:  # noqa: ANN001
    if isinstance(valid_kv_len, Tensor):
        return valid_kv_len.to(device=device, dtype=torch.int32).reshape(-1).contiguous()
    if valid_kv_len is not None and int(valid_kv_len) < Tkv:
        return torch.full((1,), int(valid_kv_len), dtype=torch.int32, device=device)
    return None
