"""GPU test of the allocation-free ICL entry point tabicl_icl_fwd_noalloc, called through the C ABI:
its output must match tabicl_icl_fwd's (with a workspace from torch) on two calls in a row, the second
with a smaller input, to the kernel's bar (bit-identical when both split the keys the same way; within
2e-2 bf16 / 1e-4 fp32 otherwise), plus a key-masked call and the refusal of an oversized call."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib():
    import tabicl_mi355_native as nat
    return nat, nat.load()


def _strides(t):
    return t.stride(0), t.stride(1), t.stride(2)


def _call_noalloc(nat, lib, q, k, v, out, valid=None, bias=None, qlen=None):
    N, H, Tq, D = q.shape
    st = lib.tabicl_icl_fwd_noalloc(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), None if valid is None else valid.data_ptr(),
        0 if valid is None else valid.numel(), None if bias is None else bias.data_ptr(),
        0 if bias is None else bias.shape[0], 0 if bias is None else bias.stride(0),
        None if qlen is None else qlen.data_ptr(), 0 if qlen is None else qlen.numel(), out.data_ptr(),
        N, H, Tq, k.shape[2], D, *_strides(q), *_strides(k), *_strides(v), *_strides(out), D ** -0.5,
        nat.dtype_code(q.dtype), nat.stream_of(q))
    nat.check(st, "tabicl_icl_fwd_noalloc")


def _call_ws(q, k, v, valid=None, bias=None):
    import tabicl_mi355_icl as icl
    out = torch.empty_like(q)
    icl.ICL_FWD_OUT(q, k, v, valid, q.shape[-1] ** -0.5, out, bias)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry(dev, dtype):
    nat, lib = _lib()
    assert lib.tabicl_icl_noalloc_scratch_bytes() == 32 << 20
    g = torch.Generator().manual_seed(70)
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-4
    for (N, H, Tq, Tkv, valid) in ((4, 8, 1300, 20000, 19000), (2, 3, 257, 900, 800)):  # second call smaller
        print(f"[noalloc] {dtype} N={N} H={H} Tq={Tq} Tkv={Tkv}", flush=True)
        q = torch.randn(N, H, Tq, 64, generator=g).to(dtype).to(dev)
        k = torch.randn(N, H, Tkv, 64, generator=g).to(dtype).to(dev)
        v = torch.randn(N, H, Tkv, 64, generator=g).to(dtype).to(dev)
        vt = torch.tensor([valid], dtype=torch.int32, device=dev)
        out = torch.full_like(q, float("nan"))
        _call_noalloc(nat, lib, q, k, v, out, vt)
        want = _call_ws(q, k, v, vt)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all()
        assert float((out.float() - want.float()).abs().max()) <= tol
    # a ragged call (per-element row counts: the live work-item list goes to the scratch array too)
    N, H, Tq, Tkv = 9, 8, 1024, 2000
    q = torch.randn(N, H, Tq, 64, generator=g).to(dtype).to(dev)
    k = torch.randn(N, H, Tkv, 64, generator=g).to(dtype).to(dev)
    v = torch.randn(N, H, Tkv, 64, generator=g).to(dtype).to(dev)
    vt = torch.randint(1, Tkv + 1, (N,), generator=g).to(torch.int32).to(dev)
    ql = torch.tensor([0, 1, 100, 256, 257, 700, 1024, 5000, 33], dtype=torch.int32, device=dev)
    out = torch.zeros_like(q)
    _call_noalloc(nat, lib, q, k, v, out, vt, qlen=ql)
    import tabicl_mi355_icl as icl
    want = torch.zeros_like(q)
    icl.ICL_FWD_RAGGED_OUT(q, k, v, vt, ql, 64 ** -0.5, want)
    torch.cuda.synchronize()
    assert float((out.float() - want.float()).abs().max()) <= tol
    # a key-masked call (prefix rows and a row with scattered masked keys)
    N, H, Tq, Tkv = 3, 4, 300, 3000
    q = torch.randn(N, H, Tq, 64, generator=g).to(dtype).to(dev)
    k = torch.randn(N, H, Tkv, 64, generator=g).to(dtype).to(dev)
    v = torch.randn(N, H, Tkv, 64, generator=g).to(dtype).to(dev)
    b = torch.zeros(N, Tkv)
    b[0, 2000:] = torch.finfo(torch.float32).min
    b[1] = torch.randn(Tkv, generator=g)
    b = b.to(dev)
    out = torch.empty_like(q)
    _call_noalloc(nat, lib, q, k, v, out, None, b)
    want = _call_ws(q, k, v, None, b)
    torch.cuda.synchronize()
    assert float((out.float() - want.float()).abs().max()) <= tol


def test_noalloc_refuses_oversized_call(dev):
    # 1024 x 8 x 1100 = 9.0M work items of 256 query rows need 36 MB of flags even unsplit, more than the
    # 32 MiB array (the grid itself, 18M workgroups of 128 rows, is within limits): refused before any launch
    nat, lib = _lib()
    a = torch.empty(16, dtype=torch.bfloat16, device=dev)
    p = a.data_ptr()
    st = lib.tabicl_icl_fwd_noalloc(p, p, p, None, 0, None, 0, 0, None, 0, p, 1024, 8, 256 * 1100, 64, 64,
                                    *([64] * 12), 0.125, 0, nat.stream_of(a))
    assert st == 1 and "scratch" in nat.last_error()
