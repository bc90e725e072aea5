"""GPU parity of the cached-KV in-context attention (head dim 64) against the CPU oracle.

Bars (tests/parity.py, written there): max abs error <= 2e-2 for bf16 inputs with fp32 accumulation
and <= 1e-4 in the fp32-input validation mode, and max abs error <= 2e-2 (bf16) / 1e-3 (fp32) times
max |ref|, against the fp64 restatement of the reference's Splash hook. The scale-aware bar is what
discriminates at 45,000 keys, where N(0,1) inputs give outputs ~0.03; the full C4 shape also runs
with sharpened queries (q x 4, outputs O(1)).
At the full C4 shape a subset of (estimator, head) slices and query rows is compared and the whole
output is checked for NaN/Inf and for the convex-hull property (every output lies within the
per-dim range of the visible values).
"""
import pytest
import torch

from oracle import attention as O
from parity import check

pytestmark = pytest.mark.gpu


def _icl():
    import tabicl_mi355_icl as icl
    return icl


@pytest.mark.parametrize("name,N,H,Tq,Tkv,valid,dtype", [
    ("tiny_bf16", 1, 1, 7, 5, None, torch.bfloat16),
    ("tiny_fp32", 1, 2, 33, 70, None, torch.float32),
    ("valid_scalar_bf16", 2, 8, 300, 1000, 777, torch.bfloat16),
    ("valid_scalar_fp32", 2, 8, 300, 1000, 777, torch.float32),
    ("valid_tile_edge", 1, 8, 128, 256, 64, torch.bfloat16),
    ("one_full_tile_and_tail", 2, 8, 300, 256, 100, torch.bfloat16),
    ("two_full_tiles", 1, 8, 300, 256, 128, torch.bfloat16),
    ("valid_one_key", 1, 4, 64, 128, 1, torch.float32),
    ("odd_sizes", 3, 2, 1000, 4099, None, torch.bfloat16),
])
def test_icl_parity(dev, name, N, H, Tq, Tkv, valid, dtype):
    icl = _icl()
    g = torch.Generator().manual_seed(3)
    q = torch.randn(N, H, Tq, 64, generator=g).to(dtype)
    k = torch.randn(N, H, Tkv, 64, generator=g).to(dtype)
    v = torch.randn(N, H, Tkv, 64, generator=g).to(dtype)
    print(f"[icl] {name}", flush=True)
    vt = None if valid is None else torch.tensor(valid, dtype=torch.int32).to(dev)
    out = icl.icl_sdpa(q.to(dev), k.to(dev), v.to(dev), vt)
    torch.cuda.synchronize()
    ref = O.splash_sdpa_ref(q, k, v, valid)
    assert out.shape == q.shape and out.dtype == dtype
    check(out, ref, dtype, name)


def test_icl_int_valid_and_per_batch_valid(dev):
    icl = _icl()
    g = torch.Generator().manual_seed(4)
    q = torch.randn(3, 2, 50, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(3, 2, 500, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(3, 2, 500, 64, generator=g).to(torch.bfloat16)
    out = icl.icl_sdpa(q.to(dev), k.to(dev), v.to(dev), 321)
    check(out, O.splash_sdpa_ref(q, k, v, 321), torch.bfloat16, "int valid")
    vn = torch.tensor([500, 17, 0], dtype=torch.int32)
    out = icl.icl_sdpa(q.to(dev), k.to(dev), v.to(dev), vn.to(dev))
    check(out, O.splash_sdpa_ref(q, k, v, vn.numpy()), torch.bfloat16, "per-batch valid")
    assert torch.all(out[2] == 0)


def test_icl_strided_cache_views_and_padding_garbage(dev):
    # q/k/v as views of a [est, block, head, row, d] cache, rows past valid hold NaN
    icl = _icl()
    g = torch.Generator().manual_seed(5)
    E_, NB, H, cap, D = 2, 3, 8, 600, 64
    kc = torch.randn(E_, NB, H, cap, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(E_, NB, H, cap, D, generator=g).to(torch.bfloat16)
    kc[..., 450:, :] = float("nan")
    vc[..., 450:, :] = float("inf")
    qa = torch.randn(E_, NB, H, 90, D, generator=g).to(torch.bfloat16)
    kd, vd, qd = kc.to(dev), vc.to(dev), qa.to(dev)
    for blk in range(NB):
        out = icl.icl_sdpa(qd[:, blk], kd[:, blk], vd[:, blk], torch.tensor(450, dtype=torch.int32).to(dev))
        ref = O.splash_sdpa_ref(qa[:, blk], kc[:, blk], vc[:, blk], 450)
        assert torch.isfinite(out.float()).all()
        check(out, ref, torch.bfloat16, f"strided block {blk}")


def test_icl_cache_append_and_query(dev):
    icl = _icl()
    g = torch.Generator().manual_seed(6)
    E_, NB, H, cap, D = 2, 2, 8, 1000, 64
    cache = icl.IclKVCache(E_, NB, H, cap, D, torch.bfloat16, dev)
    ks = [torch.randn(E_, H, 700, D, generator=g).to(torch.bfloat16) for _ in range(NB)]
    vs = [torch.randn(E_, H, 700, D, generator=g).to(torch.bfloat16) for _ in range(NB)]
    for b in range(NB):
        # append in two chunks, the second from a non-contiguous (row-strided) view
        kd, vd = ks[b].to(dev), vs[b].to(dev)
        cache.append(b, kd[:, :, :300], vd[:, :, :300], row0=0)
        cache.append(b, kd[:, :, 300:], vd[:, :, 300:], row0=300)
    torch.cuda.synchronize()
    for b in range(NB):
        assert torch.equal(cache.keys[:, b, :, :700].cpu(), ks[b])
        assert torch.equal(cache.values[:, b, :, :700].cpu(), vs[b])
    q = torch.randn(E_, H, 200, D, generator=g).to(torch.bfloat16)
    out = cache.query(1, q.to(dev), torch.tensor(700, dtype=torch.int32).to(dev))
    check(out, O.splash_sdpa_ref(q, ks[1], vs[1], 700), torch.bfloat16, "cache query")
    with pytest.raises(ValueError):
        cache.append(0, ks[0].to(dev), vs[0].to(dev), row0=400)  # past capacity


def test_icl_split_choice(dev):
    # the launcher splits keys only when the grid would leave CUs idle (workspace = flags + prefix view +
    # live work-item list, plus fp32 partials [S][N*H*Tq][66] when S > 1): a C4 block launch (8 x 8
    # heads x 20 query blocks = 1280 work items on 256 CUs) runs unsplit; one estimator's 160 work
    # items over 45k keys split
    import tabicl_mi355_native as nat
    lib = nat.load()

    def head(items):  # flags, prefix view, list (count + items), each 256-byte aligned
        return (items * 4 + 255) // 256 * 256 + 256 + ((items + 1) * 4 + 255) // 256 * 256

    c4 = lib.tabicl_icl_workspace_bytes(8, 8, 5000, 45000, 64, 0)
    assert c4 == head(1280)  # no partials
    one = lib.tabicl_icl_workspace_bytes(1, 8, 5000, 45000, 64, 0)
    split = {s: head(160 * s) + s * 8 * 5000 * 66 * 4 for s in (2, 3, 4)}
    assert one in split.values(), (one, split)


def test_icl_split_matches_unsplit(dev):
    # the key-split path (workspace given) and the single-pass path (no workspace) agree; ragged
    # valid lengths leave some splits empty
    import tabicl_mi355_native as nat
    icl = _icl()
    g = torch.Generator().manual_seed(8)
    N, H, Tq, Tkv, D = 3, 4, 200, 3000, 64
    q = torch.randn(N, H, Tq, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(N, H, Tkv, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(N, H, Tkv, D, generator=g).to(torch.bfloat16).to(dev)
    valid = torch.tensor([3000, 700, 64], dtype=torch.int32, device=dev)
    assert nat.load().tabicl_icl_workspace_bytes(N, H, Tq, Tkv, D, 0) > 0
    split = icl.icl_sdpa(q, k, v, valid)
    single = torch.empty_like(q)
    nat.call("tabicl_icl_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), valid.data_ptr(), N, single.data_ptr(),
             N, H, Tq, Tkv, D, *q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *single.stride()[:3],
             D ** -0.5, 0, None, 0, nat.stream_of(q))
    torch.cuda.synchronize()
    assert float((split.float() - single.float()).abs().max()) <= 1e-2
    ref = O.splash_sdpa_ref(q.cpu(), k.cpu(), v.cpu(), valid.cpu().numpy())
    check(split, ref, torch.bfloat16, "split")


@pytest.mark.parametrize("qscale", [1.0, 4.0], ids=["normal_q", "sharp_q"])
def test_icl_full_c4_slice(dev, qscale):
    # BASELINE config 4 at full size for one block: 8 est x 8 heads, 5000 q over 45000 cached keys.
    # Oracle on 2 (est, head) slices x 256 query rows; whole output finite and in the value hull.
    # qscale 4: scores ~N(0, 16), a few hundred keys carry the weight and outputs are O(1)
    icl = _icl()
    g = torch.Generator(device="cpu").manual_seed(3)
    N, H, Tq, Tkv, D = 8, 8, 5000, 45000, 64
    q = (torch.randn(N, H, Tq, D, generator=g) * qscale).to(torch.bfloat16)
    k = torch.randn(N, H, Tkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(N, H, Tkv, D, generator=g).to(torch.bfloat16)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    print(f"[icl] full c4 qscale={qscale}", flush=True)
    out = icl.icl_sdpa(qd, kd, vd, torch.tensor(Tkv, dtype=torch.int32).to(dev))
    assert torch.isfinite(out.float()).all()
    vmax = vd.float().amax(dim=2, keepdim=True)
    vmin = vd.float().amin(dim=2, keepdim=True)
    assert bool((out.float() <= vmax + 1e-2).all()) and bool((out.float() >= vmin - 1e-2).all())
    rows = torch.arange(0, Tq, Tq // 256)[:256]
    for n, h in ((0, 0), (3, 2), (7, 5)):
        ref = O.splash_sdpa_ref(q[n:n + 1, h:h + 1, rows], k[n:n + 1, h:h + 1], v[n:n + 1, h:h + 1])
        check(out[n:n + 1, h:h + 1, rows], ref, torch.bfloat16, f"c4 ({n},{h}) qscale={qscale}")


@pytest.mark.parametrize("form", ["seg", "full"])
def test_reference_splash_op_names(dev, form):
    # the reference's call pattern around its Splash ops (results/tpu_patch.diff:123-155): q scaled by
    # D^-0.5 in the input dtype and padded to a multiple of bq, k/v padded with zeros to a multiple of
    # bkv, then tabicl::tpu_splash_sdpa_seg with the valid length (or _full when every padded key is
    # valid), the padded query rows sliced off
    import torch.nn.functional as F

    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(14)
    N, H, Tq, Tkv, D = 2, 8, 700, 3000 if form == "seg" else 4096, 64
    bq, bkv = 512, 1024
    q = torch.randn(N, H, Tq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(N, H, Tkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(N, H, Tkv, D, generator=g).to(torch.bfloat16)
    tq, tk = -(-Tq // bq) * bq, -(-Tkv // bkv) * bkv
    q_in = F.pad((q.to(dev) * D ** -0.5).contiguous(), (0, 0, 0, tq - Tq))
    k_in = F.pad(k.to(dev), (0, 0, 0, tk - Tkv))
    v_in = F.pad(v.to(dev), (0, 0, 0, tk - Tkv))
    if form == "seg":
        out = torch.ops.tabicl.tpu_splash_sdpa_seg(q_in, k_in, v_in, torch.tensor(2500, dtype=torch.int32, device=dev),
                                                   bq, bkv)
        ref = O.splash_sdpa_ref(q, k, v, 2500)
    else:
        assert tk == Tkv
        out = icl.splash_sdpa_full_op(q_in, k_in, v_in, bq, bkv)
        ref = O.splash_sdpa_ref(q, k, v)
    torch.cuda.synchronize()
    assert out.shape == q_in.shape
    check(out[:, :, :Tq], ref, torch.bfloat16, f"splash op {form}")


def _native_icl(q, k, v, valid, ws):
    import tabicl_mi355_native as nat
    out = torch.empty_like(q)
    N, H, Tq, D = q.shape
    nat.call("tabicl_icl_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), valid.data_ptr(), valid.numel(),
             out.data_ptr(), N, H, Tq, k.shape[2], D, *q.stride()[:3], *k.stride()[:3], *v.stride()[:3],
             *out.stride()[:3], D ** -0.5, 0, ws.data_ptr(), ws.numel(), nat.stream_of(q))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("name,qscale,expect_flag", [
    ("ordinary_scores", 1.0, False),
    ("scores_far_above_first_keys", 80.0, True),  # ~120 nats above the first 32 keys' maximum
])
def test_icl_fixed_reference_and_exact_recompute(dev, name, qscale, expect_flag):
    # bf16 with a workspace runs the pipelined kernel with a fixed softmax reference; work items
    # whose scores leave its range are flagged (first 256 workspace bytes) and recomputed exactly
    import tabicl_mi355_native as nat
    g = torch.Generator().manual_seed(13)
    N, H, Tq, Tkv, D = 2, 2, 300, 4000, 64
    q = (torch.randn(N, H, Tq, D, generator=g) * qscale).to(torch.bfloat16)
    k = torch.randn(N, H, Tkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(N, H, Tkv, D, generator=g).to(torch.bfloat16)
    valid = torch.tensor([3900, 2500], dtype=torch.int32)
    nbytes = int(nat.load().tabicl_icl_workspace_bytes(N, H, Tq, Tkv, D, 0))
    assert nbytes >= 256
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    print(f"[icl] {name}", flush=True)
    out = _native_icl(q.to(dev), k.to(dev), v.to(dev), valid.to(dev), ws)
    flags = ws[:256].view(torch.int32).cpu()
    assert bool((flags != 0).any()) == expect_flag, flags
    assert torch.isfinite(out.float()).all()
    ref = O.splash_sdpa_ref(q, k, v, valid.numpy())
    check(out, ref, torch.bfloat16, name)
