"""CPU oracle for the small-head and cached-KV attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only as the checker (or, for the CPU baseline, as the timed CPU restatement). The product path
(the tabicl_mi355_* modules and libtabicl_attn.so) never calls it.

It restates, in plain numpy (float64) and CPU torch (float32), the arithmetic of the reference:
  ref_attn                scripts/tests/test_pallas_attn.py:21-31   (the fp32 oracle the metric names)
  attention_f64           per-head softmax(q k^T + bias) v, the math of every kernel
                          (scripts/tabicl_tpu_pallas_attn.py:67-85, tabicl_tpu_mha.py:189-197)
  rope_tables_ref         scripts/tabicl_tpu_pallas_attn.py:681-698 (textbook inv_freq, see below)
  rope_merged_ref         scripts/tabicl_tpu_mha.py:201-248 ("roll" form) / pallas_attn.py:465-473
  hx/hxq/pk_self/pk_cross reference wrappers scripts/tabicl_tpu_pallas_attn.py:323-336,722-790
  splash_sdpa_ref         results/tpu_patch.diff:123-155 (q * D^-0.5, keys >= valid masked)
  tiled_online_sdpa_ref   results/tpu_patch.diff:158-193 (online-softmax recurrence)
  combined_mask_ref       scripts/tabicl_tpu_mha.py:251-290 (additive mask normalisation)
  attention_bwd_f64       scripts/tabicl_tpu_pallas_attn.py:87-122 (P, dP, D, dS; dq, dk, dv)
  rope_bwd_ref            pallas_attn.py:446-447, 476-477 (y cos - R(y sin))
  hx/pk_self/pk_cross_bwd_ref  pallas_attn.py:185-188, 512-560, 618-637 (packed gradients)
  hxf_ref, folded_mab1_ref     pallas_attn.py:345-404, 429-442; tests/test_pallas_attn.py:300-318

Pinning (tests/test_oracle.py): every function is checked against closed forms, invariants and
brute force (two-key sigmoid, one key, key permutation, row shift, masked keys, q = 0 mean, convex
hull, valid_len == slicing, chunked == one-shot, RoPE rotation closed form / norm / relative
position); the backward restatements against torch.autograd of the forward definitions and central
finite differences. Parity unpinned: the reference's RotaryEmbedding.freqs initialisation lives in upstream
tabicl (absent here); rope_tables_ref takes the frequencies as an input, and the textbook
inv_freq_i = base^(-2i/rot) used by tests and bench is an assumption, not a reference fact.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

NEG = -1e30  # reference sentinel for padded / invalid keys (scripts/tabicl_tpu_pallas_attn.py:31)


# -------------------------------------------------------------------------------------------
# core per-head attention
# -------------------------------------------------------------------------------------------
def ref_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, h: int, bias: Optional[torch.Tensor] = None):
    """fp32 oracle of scripts/tests/test_pallas_attn.py:21-31: head split, matmul, additive bias
    [B, Lk], softmax, matmul, merge. q [B, Lq, E] (pre-scaled), k/v [B, Lk, E]."""
    B, Lq, E = q.shape
    d = E // h
    qh = q.float().reshape(B, Lq, h, d).transpose(1, 2)
    kh = k.float().reshape(B, -1, h, d).transpose(1, 2)
    vh = v.float().reshape(B, -1, h, d).transpose(1, 2)
    s = qh @ kh.transpose(-1, -2)
    if bias is not None:
        s = s + bias.float().reshape(bias.shape[0], 1, 1, -1)
    p = torch.softmax(s, dim=-1)
    return (p @ vh).transpose(1, 2).reshape(B, Lq, E)


def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, h: int, bias: Optional[np.ndarray] = None,
                  valid=None) -> np.ndarray:
    """float64 per-head attention in merged layout. q [B, Lq, E], k/v [B, Lk, E], bias [1|B, Lk],
    valid: None, int or [B] ints (keys >= valid dropped; a row with no valid key -> 0)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Lq, E = q.shape
    Lk = k.shape[1]
    d = E // h
    out = np.zeros((B, Lq, E))
    for b in range(B):
        nv = Lk
        if valid is not None:
            vb = np.asarray(valid).reshape(-1)
            nv = int(min(max(vb[0 if vb.size == 1 else b], 0), Lk))
        if nv == 0:
            continue
        for g in range(h):
            sl = slice(g * d, (g + 1) * d)
            s = q[b, :, sl] @ k[b, :nv, sl].T
            if bias is not None:
                bb = np.asarray(bias, np.float64).reshape(-1, Lk)
                s = s + bb[0 if bb.shape[0] == 1 else b, :nv][None, :]
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b, :, sl] = p @ v[b, :nv, sl]
    return out


def attention_loops(q, k, v, h, bias=None):
    """Scalar-loop brute force (tiny inputs only): the definition written out element by element."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, Lq, E = q.shape
    Lk = k.shape[1]
    d = E // h
    out = np.zeros((B, Lq, E))
    for b in range(B):
        for g in range(h):
            for i in range(Lq):
                s = []
                for j in range(Lk):
                    acc = 0.0
                    for c in range(d):
                        acc += q[b, i, g * d + c] * k[b, j, g * d + c]
                    if bias is not None:
                        bb = np.asarray(bias, np.float64).reshape(-1, Lk)
                        acc += bb[0 if bb.shape[0] == 1 else b, j]
                    s.append(acc)
                m = max(s)
                e = [np.exp(x - m) for x in s]
                z = sum(e)
                for c in range(d):
                    out[b, i, g * d + c] = sum(e[j] * v[b, j, g * d + c] for j in range(Lk)) / z
    return out


# -------------------------------------------------------------------------------------------
# RoPE (merged-head layout)
# -------------------------------------------------------------------------------------------
def textbook_freqs(rot: int, base: float) -> np.ndarray:
    """inv_freq_i = base^(-2i/rot), i < rot/2 (textbook RoPE; upstream's init is unpinned)."""
    return base ** (-np.arange(0, rot, 2, dtype=np.float64) / rot)


def rope_tables_ref(freqs: np.ndarray, L: int, E: int, h: int, interleaved: bool, positions=None):
    """cos/sin [L, E] float64 tiled per head, cos=1 / sin=0 past rot, plus (code, half, rot)
    (scripts/tabicl_tpu_pallas_attn.py:681-698). freqs: [rot/2] inverse frequencies; halves repeat
    them as cat(f, f), pairs (interleaved) repeat each frequency twice."""
    d = E // h
    pos = np.arange(L, dtype=np.float64) if positions is None else np.asarray(positions, np.float64)
    f = pos[:, None] * np.asarray(freqs, np.float64)[None, :]
    ang = np.repeat(f, 2, axis=1) if interleaved else np.concatenate([f, f], axis=1)
    rot = ang.shape[1]
    cos, sin = np.cos(ang), np.sin(ang)
    if rot < d:
        cos = np.concatenate([cos, np.ones((L, d - rot))], axis=1)
        sin = np.concatenate([sin, np.zeros((L, d - rot))], axis=1)
    return np.tile(cos, (1, h)), np.tile(sin, (1, h)), (1 if interleaved else 2), rot // 2, rot


def rotate_merged(x: np.ndarray, h: int, code: int, half: int, rot: int) -> np.ndarray:
    """R(x) per head in merged layout: pairs out[2i] = -x[2i+1], out[2i+1] = x[2i]; halves
    out[j] = -x[j+half] (j < half), x[j-half] (half <= j < rot); 0 past rot
    (scripts/tabicl_tpu_mha.py:241-248)."""
    E = x.shape[-1]
    d = E // h
    out = np.zeros_like(x, dtype=np.float64)
    for g in range(h):
        for j in range(d):
            c = g * d + j
            if j >= rot:
                continue
            if code == 1:
                out[..., c] = -x[..., c + 1] if j % 2 == 0 else x[..., c - 1]
            else:
                out[..., c] = -x[..., c + half] if j < half else x[..., c - half]
    return out


def rope_merged_ref(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, h: int, code: int, half: int, rot: int):
    """x * cos + R(x) * sin over [..., L, E] (float64)."""
    x = np.asarray(x, np.float64)
    if code == 0:
        return x
    return x * cos + rotate_merged(x, h, code, half, rot) * sin


# -------------------------------------------------------------------------------------------
# op-level oracles (conventions of the reference wrappers)
# -------------------------------------------------------------------------------------------
def _f64(t) -> np.ndarray:
    return t.detach().double().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t, np.float64)


def hx_ref(q, k, v, h, bias=None):
    """hx_attention (q pre-scaled) - reference scripts/tabicl_tpu_pallas_attn.py:767-790."""
    return attention_f64(_f64(q), _f64(k), _f64(v), h, None if bias is None else _f64(bias))


def hxq_ref(q, kv, valid, h):
    """hxq_attention - reference :323-336 (test oracle: ref_attn(q, kv[:, :valid, :E], kv[:, :valid, E:]),
    scripts/tests/test_pallas_attn.py:167)."""
    q = _f64(q)
    kv = _f64(kv)
    E = q.shape[-1]
    return attention_f64(q, kv[..., :E], kv[..., E:], h, valid=_f64(valid).astype(np.int64))


def _cast(x: np.ndarray, dtype) -> np.ndarray:
    """x rounded as the reference's packed kernels round their operands: to fp32, then to `dtype`
    (`(rope(q) * scale).astype(dt)`, `rope(k).astype(dt)`, scripts/tabicl_tpu_pallas_attn.py:500-501);
    dtype None: unrounded."""
    if dtype is None:
        return x
    return torch.from_numpy(np.ascontiguousarray(x)).to(torch.float32).to(dtype).double().numpy()


def pk_self_ref(qkv, h, bias, rope, scale, cast=None):
    """pk_self_attention - reference :722-732; rope = None or (cos, sin, code, half, rot). cast (a torch
    dtype): q' = rope(q) scale and k' = rope(k) rounded to it, the reference kernel's rounding points."""
    x = _f64(qkv)
    E = x.shape[-1] // 3
    q, k, v = x[..., :E], x[..., E:2 * E], x[..., 2 * E:]
    if rope is not None:
        cos, sin, code, half, rot = rope
        q = rope_merged_ref(q, _f64(cos), _f64(sin), h, code, half, rot)
        k = rope_merged_ref(k, _f64(cos), _f64(sin), h, code, half, rot)
    return attention_f64(_cast(q * scale, cast), _cast(k, cast), v, h, None if bias is None else _f64(bias))


def pk_cross_ref(q, kv, h, bias, rope_q, rope_k, scale, cast=None):
    """pk_cross_attention - reference :735-752 (RoPE positions 0..L-1 on q and on k); cast as in
    pk_self_ref."""
    q = _f64(q)
    kv = _f64(kv)
    E = q.shape[-1]
    k, v = kv[..., :E], kv[..., E:]
    if rope_q is not None:
        q = rope_merged_ref(q, _f64(rope_q[0]), _f64(rope_q[1]), h, *rope_q[2:])
        k = rope_merged_ref(k, _f64(rope_k[0]), _f64(rope_k[1]), h, *rope_k[2:])
    if q.shape[0] != k.shape[0]:
        q = np.broadcast_to(q, (k.shape[0],) + q.shape[1:])
    return attention_f64(_cast(q * scale, cast), _cast(k, cast), v, h, None if bias is None else _f64(bias))


# -------------------------------------------------------------------------------------------
# backward (training): the reference's bwd kernels, scripts/tabicl_tpu_pallas_attn.py:87-122 (hx)
# and :512-560 (packed: RoPE and scale on q / k)
# -------------------------------------------------------------------------------------------
def attention_bwd_f64(q, k, v, h: int, do, bias=None, o=None):
    """(dq, dk, dv) of per-head softmax(q k^T + bias) v in merged layout, float64, as the reference's
    kernels form them: P recomputed; dP = dO V^T; D_g = sum over head g's dims of dO * O (O = the
    forward output `o` when given, else the exact one); dS = P (dP - D_g); dq = dS K, dk = dS^T Q,
    dv = P^T dO (pallas_attn.py:104-115). q [B, Lq, E], k/v [B, Lk, E], do [B, Lq, E], bias [1|B, Lk]."""
    q, k, v, do = _f64(q), _f64(k), _f64(v), _f64(do)
    B, Lq, E = q.shape
    Lk = k.shape[1]
    d = E // h
    if o is None:
        o = attention_f64(q, k, v, h, bias)
    o = _f64(o)
    bb = None if bias is None else _f64(bias).reshape(-1, Lk)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for b in range(B):
        for g in range(h):
            sl = slice(g * d, (g + 1) * d)
            s = q[b, :, sl] @ k[b, :, sl].T
            if bb is not None:
                s = s + bb[0 if bb.shape[0] == 1 else b][None, :]
            s = s - s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            dp = do[b, :, sl] @ v[b, :, sl].T
            dg = (do[b, :, sl] * o[b, :, sl]).sum(axis=1, keepdims=True)
            ds = p * (dp - dg)
            dq[b, :, sl] = ds @ k[b, :, sl]
            dk[b, :, sl] = ds.T @ q[b, :, sl]
            dv[b, :, sl] = p.T @ do[b, :, sl]
    return dq, dk, dv


def rope_bwd_ref(y, cos, sin, h: int, code: int, half: int, rot: int):
    """Gradient through x -> x cos + R(x) sin: y cos - R(y sin), since R^T = -R
    (scripts/tabicl_tpu_pallas_attn.py:446-447, 476-477)."""
    y = np.asarray(y, np.float64)
    if code == 0:
        return y
    return y * cos - rotate_merged(y * sin, h, code, half, rot)


def hx_bwd_ref(q, k, v, h, do, bias=None, o=None):
    """tabicl_pk::hx_bwd (reference :87-122, 185-188): q pre-scaled, no RoPE."""
    return attention_bwd_f64(q, k, v, h, do, bias, o)


def pk_self_bwd_ref(qkv, h, bias, rope, scale, do, o=None):
    """tabicl_pk::pk_self_bwd (reference :512-531, 554-560): d(qkv) [B, L, 3E] packed like qkv."""
    x = _f64(qkv)
    E = x.shape[-1] // 3
    q, k, v = x[..., :E], x[..., E:2 * E], x[..., 2 * E:]
    if rope is not None:
        cos, sin, code, half, rot = _f64(rope[0]), _f64(rope[1]), rope[2], rope[3], rope[4]
        q = rope_merged_ref(q, cos, sin, h, code, half, rot)
        k = rope_merged_ref(k, cos, sin, h, code, half, rot)
    dq, dk, dv = attention_bwd_f64(q * scale, k, v, h, do, bias, o)
    dq = dq * scale
    if rope is not None:
        dq = rope_bwd_ref(dq, cos, sin, h, code, half, rot)
        dk = rope_bwd_ref(dk, cos, sin, h, code, half, rot)
    return np.concatenate([dq, dk, dv], axis=-1)


def pk_cross_bwd_ref(q, kv, h, bias, rope_q, rope_k, scale, do, o=None):
    """tabicl_pk::pk_cross_bwd (reference :512-553): (dq, d(kv) packed like kv). A q with one
    leading element broadcast over kv's batch gets the sum of the per-element gradients."""
    q = _f64(q)
    kv = _f64(kv)
    E = q.shape[-1]
    k, v = kv[..., :E], kv[..., E:]
    if rope_q is not None:
        cq, sq = _f64(rope_q[0]), _f64(rope_q[1])
        ck, sk = _f64(rope_k[0]), _f64(rope_k[1])
        q = rope_merged_ref(q, cq, sq, h, *rope_q[2:])
        k = rope_merged_ref(k, ck, sk, h, *rope_k[2:])
    shared = q.shape[0] != k.shape[0]
    qb = np.broadcast_to(q, (k.shape[0],) + q.shape[1:]) if shared else q
    dq, dk, dv = attention_bwd_f64(qb * scale, k, v, h, do, bias, o)
    dq = dq * scale
    if rope_q is not None:
        dq = rope_bwd_ref(dq, cq, sq, h, *rope_q[2:])
        dk = rope_bwd_ref(dk, ck, sk, h, *rope_k[2:])
    if shared:
        dq = dq.sum(axis=0, keepdims=True)
    return dq, np.concatenate([dk, dv], axis=-1)


def hxf_ref(qf, x, valid):
    """hxf_attention (reference scripts/tabicl_tpu_pallas_attn.py:345-404, 429-442): U = softmax(qf x^T) x
    over the keys < valid, one head of width E; qf [1|B, hq, E] (1: shared), x [B, Lk, E]; a row with
    no valid key -> 0. float64."""
    qf = _f64(qf)
    x = _f64(x)
    if qf.shape[0] != x.shape[0]:
        qf = np.broadcast_to(qf, (x.shape[0],) + qf.shape[1:])
    return attention_f64(qf, x, x, 1, valid=np.asarray(valid).astype(np.int64))


def folded_mab1_ref(ind, x, valid, h: int, W, b):
    """The first ISAB attention before its output projection, unfolded: q = ind W_q^T + b_q (pre-scaled by
    hd^-0.5), K = x W_k^T + b_k, V = x W_v^T + b_v, per-head softmax(q K^T) V over keys < valid
    (reference check_hxf, scripts/tests/test_pallas_attn.py:300-318). ind [Lq, E], x [B, Lk, E]."""
    ind, x, W, b = _f64(ind), _f64(x), _f64(W), _f64(b)
    E = ind.shape[-1]
    hd = E // h
    q = (ind @ W[:E].T + b[:E]) * hd ** -0.5
    k = x @ W[E:2 * E].T + b[E:2 * E]
    v = x @ W[2 * E:].T + b[2 * E:]
    q = np.broadcast_to(q, (x.shape[0],) + q.shape)
    return attention_f64(q, k, v, h, valid=np.asarray(valid).astype(np.int64))


def splash_sdpa_ref(q, k, v, valid=None, bias=None):
    """ICL attention, reference hook _tpu_pallas_splash_sdpa (results/tpu_patch.diff:123-155):
    q, k, v [N, H, T, D] float, q scaled by D^-0.5, keys >= valid masked. float64 result.
    bias: optional additive key mask [1|N, Tkv] (the reference's masked paths, diff:158-193, 263-282:
    `scores.float() + attn_mask.float()`), added to the scores in float32 as there, so a mask entry of
    finfo.min absorbs the score and a row masked everywhere gets equal weights."""
    q = _f64(q)
    k = _f64(k)
    v = _f64(v)
    N, H, Tq, D = q.shape
    Tkv = k.shape[2]
    out = np.zeros((N, H, Tq, D))
    vl = None if valid is None else np.asarray(_f64(valid)).reshape(-1).astype(np.int64)
    bb = None if bias is None else np.asarray(_f64(bias), np.float32).reshape(-1, Tkv)
    for n in range(N):
        nv = Tkv if vl is None else int(min(max(vl[0 if vl.size == 1 else n], 0), Tkv))
        if nv == 0:
            continue
        s = np.einsum("htd,hsd->hts", q[n] * D ** -0.5, k[n, :, :nv])
        if bb is not None:
            s = (s.astype(np.float32) + bb[0 if bb.shape[0] == 1 else n, :nv]).astype(np.float64)
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[n] = np.einsum("hts,hsd->htd", p, v[n, :, :nv])
    return out


def splash_sdpa_bwd_ref(q, k, v, do, valid=None, bias=None, o=None):
    """Gradients (dq, dk, dv) of splash_sdpa_ref's attention, float64 (the quantities the reference's
    autograd fallback _tiled_online_sdpa, results/tpu_patch.diff:158-193, differentiates): with
    S = D^-0.5 q k^T + bias over the visible keys, P = softmax(S), dP = dO V^T, D_row = sum over the
    head dims of dO * O (O = `o` when given, else the exact output), dS = P (dP - D_row),
    dq = D^-0.5 dS k, dk = D^-0.5 dS^T q, dv = P^T dO; keys at or past valid get zero gradients."""
    q, k, v, do = _f64(q), _f64(k), _f64(v), _f64(do)
    N, H, Tq, D = q.shape
    Tkv = k.shape[2]
    sc = D ** -0.5
    if o is None:
        o = splash_sdpa_ref(q, k, v, valid, bias)
    o = _f64(o)
    vl = None if valid is None else np.asarray(_f64(valid)).reshape(-1).astype(np.int64)
    bb = None if bias is None else np.asarray(_f64(bias), np.float32).reshape(-1, Tkv)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    for n in range(N):
        nv = Tkv if vl is None else int(min(max(vl[0 if vl.size == 1 else n], 0), Tkv))
        if nv == 0:
            continue
        s = np.einsum("htd,hsd->hts", q[n] * sc, k[n, :, :nv])
        if bb is not None:
            s = (s.astype(np.float32) + bb[0 if bb.shape[0] == 1 else n, :nv]).astype(np.float64)
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        dp = np.einsum("htd,hsd->hts", do[n], v[n, :, :nv])
        drow = (do[n] * o[n]).sum(axis=-1, keepdims=True)
        ds = p * (dp - drow)
        dq[n] = sc * np.einsum("hts,hsd->htd", ds, k[n, :, :nv])
        dk[n, :, :nv] = sc * np.einsum("hts,htd->hsd", ds, q[n])
        dv[n, :, :nv] = np.einsum("hts,htd->hsd", p, do[n])
    return dq, dk, dv


def splash_sdpa_torch(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, valid: Optional[int] = None):
    """The same ICL attention as splash_sdpa_ref in CPU torch float32 (head split, matmul, fp32
    softmax, matmul) -- the CPU baseline the bench times."""
    D = q.shape[-1]
    kk = k if valid is None else k[..., :valid, :]
    vv = v if valid is None else v[..., :valid, :]
    s = (q.float() * D ** -0.5) @ kk.float().transpose(-1, -2)
    return torch.softmax(s, dim=-1) @ vv.float()


def tiled_online_sdpa_ref(q, k, v, chunk: int, valid=None):
    """Online-softmax recurrence over key chunks (results/tpu_patch.diff:158-193), float64:
    m_new = max(m, rowmax); alpha = exp(m - m_new); l = l alpha + sum p; acc = acc alpha + p v."""
    q = _f64(q)
    k = _f64(k)
    v = _f64(v)
    D = q.shape[-1]
    Tkv = k.shape[-2] if valid is None else valid
    qs = q * D ** -0.5
    m = np.full(q.shape[:-1] + (1,), -np.inf)
    l = np.zeros(q.shape[:-1] + (1,))
    acc = np.zeros(q.shape)
    for s0 in range(0, Tkv, chunk):
        e = min(s0 + chunk, Tkv)
        sc = qs @ np.swapaxes(k[..., s0:e, :], -1, -2)
        new_m = np.maximum(m, sc.max(axis=-1, keepdims=True))
        alpha = np.exp(m - new_m)
        p = np.exp(sc - new_m)
        l = l * alpha + p.sum(axis=-1, keepdims=True)
        acc = acc * alpha + p @ v[..., s0:e, :]
        m = new_m
    return acc / np.maximum(l, 1e-20)


def combined_mask_ref(attn_mask, key_padding_mask, batch_shape, nh: int, Lq: int, Lk: int):
    """Additive mask broadcastable to (*batch, nh, Lq, Lk), or None; False for unsupported forms
    (bool masks, shapes that do not broadcast) - scripts/tabicl_tpu_mha.py:251-290."""
    nb = len(batch_shape)
    correct = (*batch_shape, nh, Lq, Lk)
    m = None
    if attn_mask is not None:
        a = np.asarray(attn_mask)
        if a.dtype == np.bool_:
            return False
        if a.ndim == 2:
            if a.shape != (Lq, Lk):
                return False
            m = a.reshape((1,) * nb + (1, Lq, Lk))
        elif a.ndim == 4 and nb != 1 and a.shape[:3] == (1, 1, 1) and a.shape[-1] == Lk:
            m = a.reshape((1,) * nb + (1, 1, Lk))
        elif a.ndim == len(correct):
            if any(g not in (1, e) for g, e in zip(a.shape, correct)):
                return False
            m = a
        else:
            return False
    if key_padding_mask is not None:
        kp = np.asarray(key_padding_mask)
        if kp.dtype == np.bool_:
            return False
        if kp.shape == (1, Lk) or (kp.ndim == nb + 1 and kp.shape[-1] == Lk):
            if any(g not in (1, e) for g, e in zip(kp.shape[:-1], batch_shape)):
                return False
            if kp.ndim == 2 and nb != 1:
                kpm = kp.reshape((1,) * nb + (1, 1, Lk))
            else:
                kpm = kp.reshape(kp.shape[:-1] + (1, 1, Lk))
        else:
            return False
        m = kpm if m is None else m + kpm
    return None if m is None else np.asarray(m, np.float32)
