"""HIP graph capture of the HIP ops (torch.cuda.CUDAGraph on ROCm): the kernels of this library
allocate nothing, record no memset and never synchronise with the host, so a caller can capture a
step into a graph and replay it (serving loops, the reference's static-shape compiled steps).

Each case captures one call on static input tensors, then replays the graph three times; before
each replay the inputs are rewritten in place by eager work, and after it the graph's output must
equal (bit for bit) an eager call of the same op on the same inputs, with a synchronisation in
between. Cases: the cached ICL attention with a valid length (pipelined kernel, trust-flag gate, key
split merge), the same with a prefix key mask (device-side prefix reduction) and with masks that are
not prefix masks (the pipelined kernel's masked instance, the gate's exact recompute), the ragged ICL entry
point (device-built list of live work items, row counts rewritten between replays), the persistent
row-stage kernel (pk_self, RoPE), the few-query streaming hxq with a key mask, and a training step of
the ICL attention (forward with statistics, autograd backward through the dq and dk/dv kernels).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
H, E = 8, 128


def _replays(dev, fn, inputs, refresh):
    """Capture fn() (inputs are the static tensors it reads), then 3 x: refresh inputs eagerly, replay,
    compare with an eager fn()."""
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()  # warm-up on the side stream (caches, first-call set-up) before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    for step in range(3):
        refresh(step)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = fn()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {step} differs from the eager call"
        assert torch.isfinite(out.float()).all()


def test_graph_icl_valid_length(dev):
    import tabicl_mi355_icl as icl
    g = torch.Generator(device=dev).manual_seed(70)
    q = torch.randn(8, 8, 1000, 64, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(8, 8, 20000, 64, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(8, 8, 20000, 64, generator=g, device=dev).to(torch.bfloat16)
    valid = torch.tensor([18000], dtype=torch.int32, device=dev)

    def refresh(step):
        q.copy_(torch.randn(q.shape, generator=g, device=dev).to(torch.bfloat16))
        valid.fill_(17000 + 1000 * step)

    print("[graph] icl valid", flush=True)
    _replays(dev, lambda: icl.icl_sdpa(q, k, v, valid), (q, k, v, valid), refresh)


def test_graph_icl_prefix_key_mask(dev):
    import tabicl_mi355_icl as icl
    g = torch.Generator(device=dev).manual_seed(71)
    q = torch.randn(4, 8, 600, 64, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(4, 8, 9000, 64, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(4, 8, 9000, 64, generator=g, device=dev).to(torch.bfloat16)
    bias = torch.zeros(4, 9000, device=dev)

    def refresh(step):
        bias.zero_()
        for n in range(4):
            bias[n, 5000 + 700 * n + 300 * step:] = torch.finfo(torch.float32).min

    refresh(0)
    print("[graph] icl key mask", flush=True)
    _replays(dev, lambda: icl.icl_sdpa(q, k, v, None, bias), (q, k, v, bias), refresh)


def test_graph_icl_scattered_key_mask(dev):
    # masks that are not prefix masks (the pipelined kernel's masked instance), rewritten between
    # replays: every row scattered, then rows 0-1 prefix masks and rows 2-3 scattered, then row 3
    # masked everywhere (its work items recomputed by the gated exact kernel inside the graph)
    import tabicl_mi355_icl as icl
    g = torch.Generator(device=dev).manual_seed(74)
    q = torch.randn(4, 8, 600, 64, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(4, 8, 9000, 64, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(4, 8, 9000, 64, generator=g, device=dev).to(torch.bfloat16)
    bias = torch.zeros(4, 9000, device=dev)
    fmin = torch.finfo(torch.float32).min

    def refresh(step):
        bias.copy_(torch.where(torch.rand(4, 9000, generator=g, device=dev) < 0.1, fmin, 0.0))
        if step >= 1:
            bias[:2] = 0.0
            bias[0, 7000:] = fmin
            bias[1, 4000:] = fmin
        if step == 2:
            bias[3] = fmin

    refresh(0)
    print("[graph] icl scattered key mask", flush=True)
    _replays(dev, lambda: icl.icl_sdpa(q, k, v, None, bias), (q, k, v, bias), refresh)


def test_graph_icl_ragged(dev):
    # the ragged entry point: the live work-item list is rebuilt on the device at every replay from the
    # row counts the eager work rewrote (rows past them are not written: the output starts at zero)
    import tabicl_mi355_icl as icl
    g = torch.Generator(device=dev).manual_seed(74)
    N = 24
    q = torch.randn(N, 8, 1024, 64, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(N, 8, 3000, 64, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(N, 8, 3000, 64, generator=g, device=dev).to(torch.bfloat16)
    valid = torch.randint(1, 3001, (N,), generator=g, device=dev).to(torch.int32)
    qlen = torch.randint(0, 1100, (N,), generator=g, device=dev).to(torch.int32)

    def fn():
        out = torch.zeros_like(q)  # a fill kernel, not a memset node
        icl.ICL_FWD_RAGGED_OUT(q, k, v, valid, qlen, 64 ** -0.5, out)
        return out

    def refresh(step):
        qlen.copy_(torch.randint(0, 1100, (N,), generator=g, device=dev).to(torch.int32))
        valid.copy_(torch.randint(1, 3001, (N,), generator=g, device=dev).to(torch.int32))

    print("[graph] icl ragged", flush=True)
    _replays(dev, fn, (q, k, v, valid, qlen), refresh)


def test_graph_row_stage_persistent(dev):
    import tabicl_mi355_attn as pk

    class _Rope:
        interleaved = False
        freqs = 10000.0 ** (-torch.arange(0, 16, 2, dtype=torch.float32) / 16)

        def get_seq_pos(self, n, device=None, dtype=torch.float32):
            return torch.arange(n, device=device, dtype=dtype)

    g = torch.Generator(device=dev).manual_seed(72)
    qkv = torch.randn(2048, 104, 3 * E, generator=g, device=dev).to(torch.bfloat16)
    rope = _Rope()

    def refresh(step):
        qkv.mul_(0.5 + 0.25 * step)

    def fn():
        with torch.no_grad():
            return pk.pk_self_attention(qkv, H, None, rope, 0.25)

    print("[graph] row stage", flush=True)
    _replays(dev, fn, (qkv,), refresh)


def test_graph_hxq_key_mask(dev):
    import tabicl_mi355_attn as pk
    g = torch.Generator(device=dev).manual_seed(73)
    q = (torch.randn(24, 128, E, generator=g, device=dev) * 0.25).to(torch.bfloat16)
    kv = torch.randn(24, 6000, 2 * E, generator=g, device=dev).to(torch.bfloat16)
    bias = torch.zeros(1, 6000, device=dev)

    def refresh(step):
        bias.zero_()
        bias[0, 4000 + 500 * step:] = torch.finfo(torch.float32).min

    refresh(0)
    print("[graph] hxq key mask", flush=True)
    _replays(dev, lambda: pk.hxq_attention(q, kv, None, H, bias), (q, kv, bias), refresh)


def test_graph_icl_forward_backward(dev):
    # forward + backward captured together (gradients allocated from the graph's pool inside the
    # capture); q and the valid length rewritten between replays
    import tabicl_mi355_icl as icl
    g = torch.Generator(device=dev).manual_seed(75)
    q = torch.randn(4, 8, 700, 64, generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    k = torch.randn(4, 8, 5000, 64, generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    v = torch.randn(4, 8, 5000, 64, generator=g, device=dev).to(torch.bfloat16).requires_grad_()
    go = torch.randn(4, 8, 700, 64, generator=g, device=dev).to(torch.bfloat16)
    valid = torch.tensor([4500, 5000, 3000, 1], dtype=torch.int32, device=dev)

    def step():
        q.grad = k.grad = v.grad = None
        out = icl.icl_sdpa(q, k, v, valid)
        out.backward(go)
        return torch.cat([out.detach().flatten(), q.grad.flatten(), k.grad.flatten(), v.grad.flatten()])

    def refresh(i):
        with torch.no_grad():
            q.copy_(torch.randn(q.shape, generator=g, device=dev).to(torch.bfloat16))
            valid[0] = 4000 + 300 * i

    print("[graph] icl forward + backward", flush=True)
    _replays(dev, step, (q, k, v, go, valid), refresh)
