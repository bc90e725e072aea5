"""GPU tests of the ragged-batch entry points (tabicl_icl_fwd_ragged, tabicl_pk_cross_fwd_ragged).

A ragged call takes per-batch query-row counts q_len. Bar (written here): rows below q_len[b] are
bit-identical to the plain call on the same inputs (same kernels, same key splits), and the plain
call itself is checked against the fp64 oracle on a subset of rows (tests/parity.py bars: 2e-2 bf16,
1e-4 fp32, and 2e-2 / 1e-3 times max |ref|), so the
ragged rows are pinned to the oracle through it. The ICL kernels never write the rows at or past
q_len (checked with a NaN sentinel); for pk_cross their contents are unspecified (the resident
kernel skips them, the others compute them). Cases: whole work items past q_len, a work item cut
inside, q_len = 0, q_len >= Lq, one q_len for the whole batch, key splits, the fp32 kernel, many
work items (the pipelined kernel's list of live work items), q_len with an additive key mask (prefix
and scattered), and for
pk_cross the resident kernel (short runs, long runs, the exact-scale long runs of the column ISAB-2)
plus the streaming and fp32 kernels.
"""
import numpy as np
import pytest
import torch

from oracle import attention as O
from parity import check

pytestmark = pytest.mark.gpu


def _check_rows(out, ref, q_len, row_dim, untouched=False):
    """out/ref: device tensors with the query-row axis at row_dim and the batch axis 0. untouched:
    the rows past q_len must still hold the NaN the output was filled with."""
    B = out.shape[0]
    for b in range(B):
        n = max(0, min(int(q_len[b if len(q_len) > 1 else 0]), out.shape[row_dim]))
        live = out[b].narrow(row_dim - 1, 0, n)
        assert torch.equal(live, ref[b].narrow(row_dim - 1, 0, n)), f"batch {b}: live rows differ"
        if untouched:
            dead = out[b].narrow(row_dim - 1, n, out.shape[row_dim] - n)
            assert bool(torch.isnan(dead).all()), f"batch {b}: rows past q_len were written"


@pytest.mark.parametrize("name,N,H,Tq,Tkv,valid,q_len,dtype", [
    # key splits (few work items): item 0 cut at 37 rows, items past q_len skipped, q_len = 0
    ("split_bf16", 3, 8, 520, 3000, [3000, 1500, 700], [37, 0, 300], torch.bfloat16),
    # one split (Tkv too short to split): q_len past Tq, exactly a work-item edge, one row
    ("nosplit_bf16", 4, 8, 700, 900, None, [700, 999, 256, 1], torch.bfloat16),
    ("shared_qlen_bf16", 2, 4, 600, 2000, [2000], [300], torch.bfloat16),
    ("split_fp32", 3, 2, 300, 2500, [2500, 100, 1], [129, 300, 64], torch.float32),
    # one or two full key tiles (with and without a crossing tile) in work items whose later waves
    # hold no live row: the idle waves' joins match the single-tile path's
    ("short_keys_idle_waves_bf16", 3, 8, 600, 300, [100, 64, 130], [70, 200, 1], torch.bfloat16),
    # many work items (the live work-item list of the pipelined kernel, a count that is not a multiple
    # of the 8 XCDs): per-element valid lengths and row counts across work-item edges, 0 and past Tq
    ("list_bf16", 37, 8, 1024, 2500, "random", "random", torch.bfloat16),
    # heads not a multiple of 8: one list section, each XCD an equal contiguous share (with remainders)
    ("list_h12_bf16", 21, 12, 1024, 2500, "random", "random", torch.bfloat16),
])
def test_icl_ragged(dev, name, N, H, Tq, Tkv, valid, q_len, dtype):
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(11)
    q = torch.randn(N, H, Tq, 64, generator=g).to(dtype)
    k = torch.randn(N, H, Tkv, 64, generator=g).to(dtype)
    v = torch.randn(N, H, Tkv, 64, generator=g).to(dtype)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    if valid == "random":
        valid = [int(x) for x in np.random.default_rng(5).integers(1, Tkv + 1, N)]
    if q_len == "random":
        q_len = [int(x) for x in np.random.default_rng(6).choice([0, 1, 100, 255, 256, 257, 700, 1024, 2000], N)]
        q_len[0] = 300
    vt = None if valid is None else torch.tensor(valid, dtype=torch.int32, device=dev)
    ql = torch.tensor(q_len, dtype=torch.int32, device=dev)
    ref = torch.empty_like(qd)
    icl.ICL_FWD_OUT(qd, kd, vd, vt, 64 ** -0.5, ref)
    out = torch.full_like(qd, float("nan"))
    icl.ICL_FWD_RAGGED_OUT(qd, kd, vd, vt, ql, 64 ** -0.5, out)
    torch.cuda.synchronize()
    _check_rows(out, ref, q_len, 2, untouched=True)
    # the plain call on the live rows of batch 0, head 0 against the oracle
    n0 = min(q_len[0], Tq)
    if n0 > 0:
        vl = Tkv if valid is None else valid[0]
        exp = O.splash_sdpa_ref(q[:1, :1], k[:1, :1], v[:1, :1], [vl])
        check(out[0, 0, :n0], exp[0, 0, :n0], dtype, name)


@pytest.mark.parametrize("name,mask,dtype", [
    ("prefix_bf16", "prefix", torch.bfloat16),      # prefix masks: the pipelined kernel at their lengths
    ("scattered_bf16", "scattered", torch.bfloat16),  # any other mask: the exact kernel adds it
    ("scattered_fp32", "scattered", torch.float32),
])
def test_icl_ragged_key_mask(dev, name, mask, dtype):
    # q_len together with an additive key mask (tabicl_icl_fwd_masked with q_len): the live rows equal
    # the plain masked call's bit for bit, the rows past q_len are left as they were, and the masked
    # call is checked against the oracle on batch 0
    import tabicl_mi355_icl as icl
    print(f"[ragged] key mask {name}", flush=True)
    N, H, Tq, Tkv = 3, 8, 600, 2000
    g = torch.Generator().manual_seed(12)
    q = torch.randn(N, H, Tq, 64, generator=g).to(dtype)
    k = torch.randn(N, H, Tkv, 64, generator=g).to(dtype)
    v = torch.randn(N, H, Tkv, 64, generator=g).to(dtype)
    bias = torch.zeros(N, Tkv)
    if mask == "prefix":
        for n, L in enumerate((2000, 1300, 41)):
            bias[n, L:] = torch.finfo(torch.float32).min
    else:
        bias = -3 * torch.rand(N, Tkv, generator=g)
        bias[:, ::5] = -1e30
    q_len = [37, 600, 0]
    qd, kd, vd, bd = q.to(dev), k.to(dev), v.to(dev), bias.to(dev)
    ql = torch.tensor(q_len, dtype=torch.int32, device=dev)
    ref = torch.empty_like(qd)
    icl.ICL_FWD_OUT(qd, kd, vd, None, 64 ** -0.5, ref, bd)
    out = torch.full_like(qd, float("nan"))
    icl.ICL_FWD_RAGGED_OUT(qd, kd, vd, None, ql, 64 ** -0.5, out, bd)
    torch.cuda.synchronize()
    _check_rows(out, ref, q_len, 2, untouched=True)
    exp = O.splash_sdpa_ref(q[:1], k[:1], v[:1], None, bias[:1].numpy())
    check(ref[0], exp[0], dtype, name)


@pytest.mark.parametrize("name,N,H,Tq,Tkv,dtype", [
    ("c5_bucket_shape_bf16", 80, 8, 1024, 2048, torch.bfloat16),  # 10 tables x 8 estimators, 1k test bucket
    ("split_bf16", 3, 8, 520, 6000, torch.bfloat16),              # few work items: the keys split
    ("fp32", 4, 2, 300, 900, torch.float32),                      # no list: the plan does nothing
])
def test_icl_ragged_plan_reused_across_blocks(dev, name, N, H, Tq, Tkv, dtype):
    # one plan (the live work-item list, computed once) serves several calls with the same sizes and
    # q_len, as the 12 ICL blocks of a bucket do; each equals the call that builds its own list, bit for bit
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(13)
    rng = np.random.default_rng(7)
    q_len = torch.tensor([int(x) for x in rng.integers(0, Tq + 1, N)], dtype=torch.int32, device=dev)
    valid = torch.tensor([int(x) for x in rng.integers(1, Tkv + 1, N)], dtype=torch.int32, device=dev)
    plan = icl.IclRaggedPlan(q_len, N, H, Tq, Tkv, 64, dtype)
    print(f"[ragged plan] {name}", flush=True)
    for blk in range(3):
        q = torch.randn(N, H, Tq, 64, generator=g).to(dtype).to(dev)
        k = torch.randn(N, H, Tkv, 64, generator=g).to(dtype).to(dev)
        v = torch.randn(N, H, Tkv, 64, generator=g).to(dtype).to(dev)
        want = torch.full_like(q, float("nan"))
        got = torch.full_like(q, float("nan"))
        icl.ICL_FWD_RAGGED_OUT(q, k, v, valid, q_len, 64 ** -0.5, want)
        icl.ICL_FWD_RAGGED_OUT(q, k, v, valid, q_len, 64 ** -0.5, got, None, plan.workspace)
        torch.cuda.synchronize()
        assert torch.equal(torch.nan_to_num(got, nan=7.0), torch.nan_to_num(want, nan=7.0)), (name, blk)
        n0 = int(q_len[0])
        if n0 > 0 and blk == 0:
            exp = O.splash_sdpa_ref(q[:1, :1].cpu(), k[:1, :1].cpu(), v[:1, :1].cpu(), valid[:1].cpu().numpy())
            check(got[0, 0, :n0], exp[0, 0, :n0], dtype, name)


def _pk_cross_case(dev, B, Lq, Lk, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Lq, 128, generator=g) * 0.5).to(dtype).to(dev)
    kv = torch.randn(B, Lk, 256, generator=g).to(dtype).to(dev)
    return q, kv


@pytest.mark.parametrize("name,B,Lq,Lk,dtype,q_len", [
    # resident kernel, one 16-row block per workgroup: cut blocks, empty rows, full rows
    ("resident_short", 6, 300, 128, torch.bfloat16, [0, 1, 15, 16, 17, 300]),
    ("resident_shared", 3, 104, 104, torch.bfloat16, [50]),
    # resident kernel with runs of 2 blocks (40 x 250 blocks > 8192 workgroups)
    ("resident_runs", 40, 4000, 128, torch.bfloat16, "random"),
    # runs of 9 blocks: the exact-scale form (column ISAB-2 at C5's buckets)
    ("resident_exact", 70, 16000, 128, torch.bfloat16, "random"),
    # the other kernels compute every row
    ("stream_bf16", 4, 200, 300, torch.bfloat16, [0, 77, 200, 5000]),
    ("fp32", 4, 200, 128, torch.float32, [3, 0, 199, 64]),
])
def test_pk_cross_ragged(dev, name, B, Lq, Lk, dtype, q_len):
    import tabicl_mi355_attn as pk
    q, kv = _pk_cross_case(dev, B, Lq, Lk, dtype, 12)
    if q_len == "random":
        rng = np.random.default_rng(5)
        q_len = [int(x) for x in rng.integers(0, Lq + 1, B)]
        q_len[0], q_len[1] = Lq, 16 * (Lq // 32)
    ql = torch.tensor(q_len, dtype=torch.int32, device=dev)
    ref = pk.pk_cross_attention(q, kv, 8, None, None, 0.25)
    out = pk.pk_cross_attention(q, kv, 8, None, None, 0.25, q_len=ql)
    torch.cuda.synchronize()
    _check_rows(out, ref, q_len, 1)
    # the plain call against the oracle on a few live rows of batch 0
    n0 = min(q_len[0], Lq, 64)
    if n0 > 0:
        exp = O.pk_cross_ref(q[:1, :n0], kv[:1], 8, None, None, None, 0.25)
        check(out[:1, :n0], exp, dtype, name)
