"""GPU parity of the ICL attention's backward (tabicl_icl_bwd, through the autograd formula of
tabicl::icl_cached_attn) against the float64 oracle oracle.attention.splash_sdpa_bwd_ref, the gradients
the reference's autograd fallback _tiled_online_sdpa gives (results/tpu_patch.diff:158-193), which its
attention takes for calls with a gradient (diff:263-270).

Cases: key counts and query counts off the 64-row tiles, a valid length (one for the batch, one per
entry, including 0), an additive key mask (per entry, with a row masked everywhere: uniform attention),
mask and valid length together, NaN in the keys past the valid length (never read: gradients there are exact
zeros), a cache view that is not contiguous, and the ICL hook on an upstream
stand-in under autograd with SSMax (gradients to q, k and v through the whole call, against the
stand-in's torch float32 math on the same GPU). The upstream gradient is N(0, 1) in the output dtype;
the oracle gets the same rounded inputs. Bars (written here): max abs error <= 2e-2 * max(1, max |grad|)
for bf16 inputs and <= 1e-4 * max(1, max |grad|) for fp32, and the scale-aware bar max abs error <=
2e-2 (bf16) / 1e-4 (fp32) times max |grad|, which is what discriminates where gradients are small (long
key rows, diffuse softmax). Keys past the valid length must get exact zeros.
"""
import numpy as np
import pytest
import torch

from oracle import attention as O

pytestmark = pytest.mark.gpu
ABS = {torch.bfloat16: 2e-2, torch.float32: 1e-4}
REL = {torch.bfloat16: 2e-2, torch.float32: 1e-4}


def _icl():
    import tabicl_mi355_icl as icl
    return icl


def _check(name, got, ref, dtype):
    got = got.detach().double().cpu().numpy()
    mx = float(np.abs(ref).max())
    err = float(np.abs(got - ref).max())
    print(f"  {name}: max abs err {err:.3e} (ref max {mx:.3e}, err/max {err / max(mx, 1e-300):.2e})", flush=True)
    assert np.isfinite(got).all(), name
    assert err <= ABS[dtype] * max(1.0, mx), (name, err, mx)
    assert err <= REL[dtype] * mx or err == 0.0, (name, err, mx)


def _inputs(seed, N, H, Tq, Tkv, dtype, qscale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(N, H, Tq, 64, generator=g) * qscale).to(dtype)
    k = torch.randn(N, H, Tkv, 64, generator=g).to(dtype)
    v = torch.randn(N, H, Tkv, 64, generator=g).to(dtype)
    do = torch.randn(N, H, Tq, 64, generator=g).to(dtype)
    return q, k, v, do


def _run(dev, q, k, v, do, valid=None, bias=None):
    icl = _icl()
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    vt = None if valid is None else torch.as_tensor(valid, dtype=torch.int32).to(dev)
    out = icl.icl_sdpa(qd, kd, vd, vt, None if bias is None else bias.to(dev))
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    return out, qd.grad, kd.grad, vd.grad


@pytest.mark.parametrize("name,N,H,Tq,Tkv,valid,dtype", [
    ("tiny_bf16", 1, 1, 7, 5, None, torch.bfloat16),
    ("tiny_fp32", 1, 2, 33, 70, None, torch.float32),
    ("one_tile_bf16", 2, 8, 64, 64, None, torch.bfloat16),
    ("valid_scalar_bf16", 2, 8, 300, 1000, 777, torch.bfloat16),
    ("valid_scalar_fp32", 2, 8, 300, 1000, 777, torch.float32),
    ("valid_tile_edge", 1, 8, 128, 256, 64, torch.bfloat16),
    ("valid_per_entry_with_zero_bf16", 3, 2, 100, 200, [0, 130, 200], torch.bfloat16),
    ("valid_per_entry_with_zero_fp32", 3, 2, 100, 200, [0, 1, 129], torch.float32),
    ("long_keys_bf16", 1, 8, 200, 4099, None, torch.bfloat16),
    ("many_queries_bf16", 1, 4, 1500, 700, 650, torch.bfloat16),
])
def test_icl_bwd_parity(dev, name, N, H, Tq, Tkv, valid, dtype):
    print(f"[icl_bwd] {name}", flush=True)
    q, k, v, do = _inputs(7, N, H, Tq, Tkv, dtype)
    if valid is not None:  # keys past the valid length are never read: NaN there must not reach anything
        vl = np.broadcast_to(np.asarray(valid), (N,))
        for n in range(N):
            k[n, :, vl[n]:] = float("nan")
            v[n, :, vl[n]:] = float("nan")
    out, dq, dk, dv = _run(dev, q, k, v, do, valid)
    rdq, rdk, rdv = O.splash_sdpa_bwd_ref(q, k, v, do, valid, None, out.detach().cpu())
    _check("dq", dq, rdq, dtype)
    _check("dk", dk, rdk, dtype)
    _check("dv", dv, rdv, dtype)
    if valid is not None:
        vl = np.broadcast_to(np.asarray(valid), (N,))
        for n in range(N):
            if vl[n] < Tkv:
                assert float(dk[n, :, vl[n]:].abs().max()) == 0.0 and float(dv[n, :, vl[n]:].abs().max()) == 0.0
            if vl[n] == 0:
                assert float(dq[n].abs().max()) == 0.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_icl_bwd_key_mask(dev, dtype):
    # a per-entry additive key mask with -1e30 / finfo.min entries, entry 2 masked everywhere (uniform
    # attention over every key, as the reference's finite fill gives it), and the mask with a valid length
    print(f"[icl_bwd] key mask {dtype}", flush=True)
    N, H, Tq, Tkv = 3, 4, 65, 300
    q, k, v, do = _inputs(8, N, H, Tq, Tkv, dtype)
    g = torch.Generator().manual_seed(9)
    bias = -torch.rand(N, Tkv, generator=g) * 3
    bias[0, 250:] = -1e30
    bias[1, ::7] = torch.finfo(torch.float32).min
    bias[2] = torch.finfo(torch.float32).min
    out, dq, dk, dv = _run(dev, q, k, v, do, None, bias)
    rdq, rdk, rdv = O.splash_sdpa_bwd_ref(q, k, v, do, None, bias.numpy(), out.detach().cpu())
    _check("dq", dq, rdq, dtype)
    _check("dk", dk, rdk, dtype)
    _check("dv", dv, rdv, dtype)
    assert float(dv[0, :, 250:].abs().max()) == 0.0 and float(dv[1, :, ::7].abs().max()) == 0.0
    assert float(dv[2].abs().min()) > 0.0  # every key carries weight 1/Tkv
    valid = [280, 100, 0]
    out, dq, dk, dv = _run(dev, q, k, v, do, valid, bias[:1].clone())
    rdq, rdk, rdv = O.splash_sdpa_bwd_ref(q, k, v, do, valid, bias[:1].numpy(), out.detach().cpu())
    _check("dq (mask + valid)", dq, rdq, dtype)
    _check("dk (mask + valid)", dk, rdk, dtype)
    _check("dv (mask + valid)", dv, rdv, dtype)


def test_icl_bwd_sharp_and_cache_view(dev):
    # sharpened queries (q x 4: peaked softmax, large dq) on a K/V cache view [E, block, H, T, d] ->
    # [E, H, T, d] that is not contiguous over the batch (the fit-time cache's layout)
    print("[icl_bwd] sharp, cache view", flush=True)
    icl = _icl()
    dtype = torch.bfloat16
    E_, B_, H, Tq, Tkv = 2, 3, 8, 257, 1100
    g = torch.Generator().manual_seed(10)
    q = (torch.randn(E_, H, Tq, 64, generator=g) * 4).to(dtype)
    kc = torch.randn(E_, B_, H, Tkv, 64, generator=g).to(dtype)
    vc = torch.randn(E_, B_, H, Tkv, 64, generator=g).to(dtype)
    do = torch.randn(E_, H, Tq, 64, generator=g).to(dtype)
    qd = q.to(dev).requires_grad_()
    kcd, vcd = kc.to(dev).requires_grad_(), vc.to(dev).requires_grad_()
    out = icl.icl_sdpa(qd, kcd[:, 1], vcd[:, 1], 1000)
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    rdq, rdk, rdv = O.splash_sdpa_bwd_ref(q, kc[:, 1], vc[:, 1], do, 1000, None, out.detach().cpu())
    _check("dq", qd.grad, rdq, dtype)
    _check("dk", kcd.grad[:, 1], rdk, dtype)
    _check("dv", vcd.grad[:, 1], rdv, dtype)
    assert float(kcd.grad[:, 0].abs().max()) == 0.0 and float(vcd.grad[:, 2].abs().max()) == 0.0


def test_icl_bwd_empty(dev):
    # no query rows: dq empty, dk and dv zero; no batch entries: empty gradients
    icl = _icl()
    for N, Tq in ((2, 0), (0, 5)):
        print(f"[icl_bwd] empty N={N} Tq={Tq}", flush=True)
        q = torch.randn(N, 8, Tq, 64, device=dev, dtype=torch.bfloat16, requires_grad=True)
        k = torch.randn(N, 8, 100, 64, device=dev, dtype=torch.bfloat16, requires_grad=True)
        v = torch.randn(N, 8, 100, 64, device=dev, dtype=torch.bfloat16, requires_grad=True)
        out = icl.icl_sdpa(q, k, v, 50)
        out.backward(torch.ones_like(out))
        torch.cuda.synchronize()
        assert q.grad.shape == q.shape and k.grad.shape == k.shape
        if N:
            assert float(k.grad.abs().max()) == 0.0 and float(v.grad.abs().max()) == 0.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_icl_hook_gradients(dev, dtype, monkeypatch):
    # the ICL hook installed on an upstream stand-in, called the way upstream's attention calls it with
    # a tensor train size (additive finfo.min key mask) and SSMax, under autograd: q, k and v gradients
    # against the stand-in's own torch math (float32 softmax) on the same GPU
    import upstream_stub as U
    import tabicl_mi355_icl as icl
    import tabicl_mi355_mha as mha
    print(f"[icl_bwd] hook {dtype}", flush=True)
    seen = []
    fn = icl.icl_sdpa

    def spy(*a, **k):
        seen.append("icl_sdpa")
        return fn(*a, **k)

    monkeypatch.setattr(icl, "icl_sdpa", spy)
    mod, ref_mod = U.make_module(), U.make_module()
    assert mha.install(mod, None, mode="pk")
    g = torch.Generator().manual_seed(11)
    N, H, Tq, Tkv, train = 2, 4, 90, 700, 610
    q = torch.randn(N, H, Tq, 64, generator=g).to(dev, dtype)
    k = torch.randn(N, H, Tkv, 64, generator=g).to(dev, dtype)
    v = torch.randn(N, H, Tkv, 64, generator=g).to(dev, dtype)
    do = torch.randn(N, H, Tq, 64, generator=g).to(dev, dtype)
    mask = torch.zeros(N, 1, 1, Tkv, device=dev, dtype=dtype)
    mask[..., train:] = torch.finfo(dtype).min
    ssm = U.SSMaxStub(H).to(dev)
    grads = []
    for m in (mod, ref_mod):
        qd, kd, vd = (t.clone().requires_grad_() for t in (q, k, v))
        out = m.sdpa_with_flattened_batch(qd, kd, vd, mask, ssmax_layer=ssm, src_len_override=torch.tensor(train))
        out.backward(do)
        grads.append((out, qd.grad, kd.grad, vd.grad))
    torch.cuda.synchronize()
    assert seen == ["icl_sdpa"]
    for name, a, b in zip(("out", "dq", "dk", "dv"), grads[0], grads[1]):
        b = b.detach().double().cpu().numpy()
        _check(name, a, b, dtype)
    assert float(grads[0][2][:, :, train:].abs().max()) == 0.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_icl_train_forward_statistics(dev, dtype):
    # tabicl::icl_cached_attn_train: the output equals the inference op's, and each row's statistics
    # (m, l) give its log2-sum-exp: m + log2 l = log2 sum over visible keys of exp2(scale log2(e) q.k)
    # (float64 from the same rounded inputs); rows with no visible key hold l = 0. Bar: bf16 sums the
    # bf16-rounded probabilities (the ones its O is made of), each within half a bf16 ulp (2^-8
    # relative), so log2 l is within 2^-8 / ln 2 < 6e-3: <= 8e-3 in log2 units; fp32 1e-4 x max(1, |lse|)
    import tabicl_mi355_icl as icl
    print(f"[icl_bwd] train forward statistics {dtype}", flush=True)
    N, H, Tq, Tkv = 3, 4, 150, 700
    q, k, v, _ = _inputs(12, N, H, Tq, Tkv, dtype, qscale=3.0)
    valid = torch.tensor([700, 333, 0], dtype=torch.int32)
    qd, kd, vd, vt = q.to(dev), k.to(dev), v.to(dev), valid.to(dev)
    out, stat = icl.ICL_FWD_TRAIN(qd, kd, vd, vt, 0.125)
    ref_out = icl.ICL_FWD(qd, kd, vd, vt, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out) or float((out.float() - ref_out.float()).abs().max()) <= ABS[dtype]
    s = torch.einsum("nhqd,nhkd->nhqk", q.double(), k.double()) * 0.125 * np.log2(np.e)
    keep = torch.arange(Tkv)[None, :] < valid[:, None].long()
    s = s.masked_fill(~keep[:, None, None, :], float("-inf"))
    lse = torch.logsumexp(s * np.log(2.0), dim=-1) / np.log(2.0)
    st = stat.double().cpu()
    for n in range(2):
        got = st[n, ..., 0] + torch.log2(st[n, ..., 1])
        err = float((got - lse[n]).abs().max())
        print(f"  n={n}: max |lse err| {err:.3e} (log2 units)", flush=True)
        assert err <= (8e-3 if dtype == torch.bfloat16 else 1e-4 * max(1.0, float(lse[n].abs().max()))), err
    assert float(st[2, ..., 1].abs().max()) == 0.0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_icl_bwd_without_forward_statistics(dev, dtype):
    # the inference op under autograd (no statistics from the forward: the backward takes its own)
    # against the oracle, and against the statistics path on the same inputs
    import tabicl_mi355_icl as icl
    print(f"[icl_bwd] own statistics {dtype}", flush=True)
    N, H, Tq, Tkv = 2, 8, 200, 900
    q, k, v, do = _inputs(13, N, H, Tq, Tkv, dtype)
    valid = torch.tensor([900, 450], dtype=torch.int32)
    grads = []
    for train in (False, True):
        qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
        if train:
            out = icl.ICL_FWD_TRAIN(qd, kd, vd, valid.to(dev), 0.125)[0]
        else:
            out = icl.ICL_FWD(qd, kd, vd, valid.to(dev), 0.125, None)
        out.backward(do.to(dev))
        torch.cuda.synchronize()
        grads.append((out.detach(), qd.grad, kd.grad, vd.grad))
    rdq, rdk, rdv = O.splash_sdpa_bwd_ref(q, k, v, do, valid, None, grads[0][0].cpu())
    for name, g, r in (("dq", grads[0][1], rdq), ("dk", grads[0][2], rdk), ("dv", grads[0][3], rdv)):
        _check(name, g, r, dtype)
    for name, a, b in zip(("dq", "dk", "dv"), grads[0][1:], grads[1][1:]):
        d = float((a.float() - b.float()).abs().max())
        print(f"  {name}: own vs forward statistics max diff {d:.3e}", flush=True)
        assert d <= ABS[dtype] * max(1.0, float(b.float().abs().max()))


def test_icl_bwd_bench_shape_sampled(dev):
    # the bench's training shape (8 tables x 8 heads, 1024 q over 16384 keys, bf16, q x 2): three (n, h)
    # slices against the float64 oracle, and over every slice two identities of the exact gradients:
    # sum over keys of dv = sum over queries of dO (each P row sums to 1) and sum over keys of dk = 0
    # (each dS row sums to 0: the -D term), both within 2e-3 of the sums' magnitudes (measured ~1.5e-4;
    # a dropped -D term leaves sum dk = scale sum_i q_i D_i, ~3% of them here)
    print("[icl_bwd] bench shape, sampled slices and identities", flush=True)
    icl = _icl()
    dtype = torch.bfloat16
    N, H, Tq, Tkv = 8, 8, 1024, 16384
    g = torch.Generator(device=dev).manual_seed(21)
    q = (torch.randn(N, H, Tq, 64, generator=g, device=dev) * 2).to(dtype).requires_grad_()
    k = torch.randn(N, H, Tkv, 64, generator=g, device=dev).to(dtype).requires_grad_()
    v = torch.randn(N, H, Tkv, 64, generator=g, device=dev).to(dtype).requires_grad_()
    do = torch.randn(N, H, Tq, 64, generator=g, device=dev).to(dtype)
    out = icl.icl_sdpa(q, k, v)
    out.backward(do)
    torch.cuda.synchronize()
    for t in (q.grad, k.grad, v.grad):
        assert bool(torch.isfinite(t.float()).all())
    sdv = v.grad.double().sum(dim=2)
    sdo = do.double().sum(dim=2)
    err_v = float((sdv - sdo).abs().max())
    sdk = k.grad.double().sum(dim=2)
    err_k = float(sdk.abs().max())
    mag_k = float(k.grad.double().abs().sum(dim=2).max())
    print(f"  sum dv - sum dO: {err_v:.3e} (max |sum dO| {float(sdo.abs().max()):.3e}); "
          f"max |sum dk| {err_k:.3e} (sum |dk| up to {mag_k:.3e})", flush=True)
    assert err_v <= 2e-3 * max(1.0, float(sdo.abs().max()))
    assert err_k <= 2e-3 * mag_k
    for n, h in ((0, 0), (3, 5), (7, 7)):
        sl = (slice(n, n + 1), slice(h, h + 1))
        args = [t[sl].detach().cpu() for t in (q, k, v, do)]
        rdq, rdk, rdv = O.splash_sdpa_bwd_ref(*args, None, None, out[sl].detach().cpu())
        _check(f"dq[{n},{h}]", q.grad[sl], rdq, dtype)
        _check(f"dk[{n},{h}]", k.grad[sl], rdk, dtype)
        _check(f"dv[{n},{h}]", v.grad[sl], rdv, dtype)


@pytest.mark.parametrize("seed", range(8))
def test_icl_bwd_random_shapes(dev, seed):
    # seeded shapes: batch 1-4, heads 1-8, 1-700 queries over 1-1500 keys, a valid length per entry or
    # none, a scattered key mask or none, bf16 or fp32, q scaled 0.5-3
    rng = np.random.default_rng(1000 + seed)
    N, H = int(rng.integers(1, 5)), int(rng.integers(1, 9))
    Tq, Tkv = int(rng.integers(1, 701)), int(rng.integers(1, 1501))
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float32
    valid = [int(x) for x in rng.integers(0, Tkv + 1, N)] if rng.random() < 0.5 else None
    bias = None
    if rng.random() < 0.4:
        bias = torch.tensor(-2 * rng.random((N, Tkv)), dtype=torch.float32)
        bias[torch.tensor(rng.random((N, Tkv)) < 0.2)] = -1e30
    qscale = float(rng.uniform(0.5, 3.0))
    print(f"[icl_bwd] random seed={seed}: N={N} H={H} Tq={Tq} Tkv={Tkv} {dtype} valid={valid} "
          f"bias={bias is not None} qscale={qscale:.2f}", flush=True)
    q, k, v, do = _inputs(2000 + seed, N, H, Tq, Tkv, dtype, qscale)
    out, dq, dk, dv = _run(dev, q, k, v, do, valid, bias)
    rdq, rdk, rdv = O.splash_sdpa_bwd_ref(q, k, v, do, valid, None if bias is None else bias.numpy(),
                                          out.detach().cpu())
    _check("dq", dq, rdq, dtype)
    _check("dk", dk, rdk, dtype)
    _check("dv", dv, rdv, dtype)
