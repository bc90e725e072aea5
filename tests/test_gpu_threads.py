"""Host-thread safety of the C ABI (reentrant entry points, thread-local error messages, no global
mutable state): two host threads, each with its own HIP stream (default priority), launch the ICL
attention (forward and backward) and the row-stage small-head attention on their own inputs at the same
time; every result must be bit-identical to the same call made alone (the per-thread error message is
tested on the CPU, tests/test_abi.py).
"""
import threading

import pytest
import torch

pytestmark = pytest.mark.gpu


class _Rope:
    interleaved = False
    freqs = 100000.0 ** (-torch.arange(0, 16, 2, dtype=torch.float32) / 16)

    def get_seq_pos(self, n, device=None, dtype=torch.float32):
        return torch.arange(n, device=device, dtype=dtype)


def _work(dev, seed):
    import tabicl_mi355_attn as pk
    import tabicl_mi355_icl as icl
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(2, 8, 400, 64, generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    k = torch.randn(2, 8, 3000, 64, generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    v = torch.randn(2, 8, 3000, 64, generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    do = torch.randn(2, 8, 400, 64, generator=g, device=dev).to(torch.bfloat16)
    x = torch.randn(64, 104, 384, generator=g, device=dev).to(torch.bfloat16)
    rope = _Rope()

    def run():
        q.grad = k.grad = v.grad = None
        out = icl.icl_sdpa(q, k, v, 2500)
        out.backward(do)
        row = pk.pk_self_attention(x, 8, None, rope, 0.25)
        return [out.detach().clone(), q.grad.clone(), k.grad.clone(), v.grad.clone(), row]

    return run


def test_two_host_threads_two_streams(dev):
    print("[threads] two host threads, two streams", flush=True)
    runs = [_work(dev, 90), _work(dev, 91)]
    want = []
    for r in runs:  # alone, one after the other
        want.append(r())
        torch.cuda.synchronize()
    got = [None, None]
    errors = []

    def body(i):
        try:
            s = torch.cuda.Stream(device=dev)
            with torch.cuda.stream(s):
                res = None
                for _ in range(5):
                    res = runs[i]()
                s.synchronize()
            got[i] = res
        except Exception as exc:  # reported in the main thread
            errors.append(exc)

    ts = [threading.Thread(target=body, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i in range(2):
        for a, b in zip(got[i], want[i]):
            assert torch.equal(a, b)
