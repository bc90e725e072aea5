"""torch.compile (fullgraph=True, backend aot_eager) over the HIP ops on the GPU: the compiled step runs
the same kernels as the eager one, so outputs and gradients must be bit-identical to eager calls. Cases:
the row stage's pk_self with RoPE (tables computed inside the traced graph) and the ICL attention's
training step (forward with statistics, backward kernels). The reference checks that its wrapper traces
as one graph (scripts/tests/test_mha_cpu.py:106-124).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


class _Rope:
    interleaved = False
    freqs = 100000.0 ** (-torch.arange(0, 16, 2, dtype=torch.float32) / 16)

    def get_seq_pos(self, n, device=None, dtype=torch.float32):
        return torch.arange(n, device=device, dtype=dtype)


def _step(fn, leaves, g_out):
    for t in leaves:
        t.grad = None
    out = fn(*leaves)
    out.backward(g_out)
    torch.cuda.synchronize()
    return [out.detach().clone()] + [t.grad.clone() for t in leaves]


@pytest.mark.parametrize("case", ["pk_self_rope", "icl_train"])
def test_compiled_matches_eager(dev, case):
    import tabicl_mi355_attn as pk
    import tabicl_mi355_icl as icl
    torch._dynamo.reset()
    print(f"[compile] {case}", flush=True)
    g = torch.Generator(device=dev).manual_seed(80)
    if case == "pk_self_rope":
        leaves = [torch.randn(64, 104, 384, generator=g, device=dev).to(torch.bfloat16).requires_grad_()]
        rope = _Rope()

        def fn(x):
            return pk.pk_self_attention(x, 8, None, rope, 0.25)
        g_out = torch.randn(64, 104, 128, generator=g, device=dev).to(torch.bfloat16)
    else:
        leaves = [torch.randn(2, 8, 300, 64, generator=g, device=dev).to(torch.bfloat16).requires_grad_(),
                  torch.randn(2, 8, 2000, 64, generator=g, device=dev).to(torch.bfloat16).requires_grad_(),
                  torch.randn(2, 8, 2000, 64, generator=g, device=dev).to(torch.bfloat16).requires_grad_()]
        valid = torch.tensor([1500, 2000], dtype=torch.int32, device=dev)

        def fn(q, k, v):
            return icl.icl_sdpa(q, k, v, valid)
        g_out = torch.randn(2, 8, 300, 64, generator=g, device=dev).to(torch.bfloat16)
    eager = _step(fn, leaves, g_out)
    compiled_fn = torch.compile(fn, backend="aot_eager", fullgraph=True)
    for _ in range(2):
        got = _step(compiled_fn, leaves, g_out)
        for a, b in zip(got, eager):
            assert torch.equal(a, b)
