"""GPU parity of the row LayerNorm kernel (tabicl_layer_norm: the pre-norms, out-norm and final norm of
the cached-KV query's blocks) against a float64 restatement of LayerNorm on the same inputs: mean and
biased variance per row, (x - mean) / sqrt(var + eps) * w + b.

Bars (tests/parity.py): fp32 output max abs error <= 1e-4 and <= 1e-3 x max |ref|; bf16 output 2e-2 and
2e-2 x max |ref| (the output rounding). With a residual, the written sum equals torch's `x + r` in the
input dtype bit for bit, and the norm is taken of that rounded sum. Widths 128 (column / row stages) and
512 (ICL stage), row counts that do not fill the kernel's row groups, a row of constant values
(variance 0: the output is the bias).
"""
import pytest
import torch

from parity import check

pytestmark = pytest.mark.gpu


def _ref(s: torch.Tensor, w, b, eps):
    s = s.double()
    mean = s.mean(-1, keepdim=True)
    var = ((s - mean) ** 2).mean(-1, keepdim=True)
    y = (s - mean) / torch.sqrt(var + eps)
    return y * w.double() + (0.0 if b is None else b.double())


@pytest.mark.parametrize("W", [128, 512])
@pytest.mark.parametrize("din,dout", [(torch.float32, torch.float32), (torch.float32, torch.bfloat16),
                                      (torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("rows", [1, 7, 4099])
@pytest.mark.parametrize("residual", [False, True])
def test_layer_norm(dev, W, din, dout, rows, residual):
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(W + rows)
    x = (torch.randn(rows, W, generator=g) * 3 + 1).to(din)
    r = (torch.randn(rows, W, generator=g)).to(din)
    x[0] = 2.5  # constant row: variance 0
    if residual:
        r[0] = 0.0
    w = 1 + 0.1 * torch.randn(W, generator=g)
    b = 0.1 * torch.randn(W, generator=g)
    xd, rd, wd, bd = x.to(dev), r.to(dev), w.to(dev), b.to(dev)
    print(f"[layernorm] W={W} {din}->{dout} rows={rows} residual={residual}", flush=True)
    if residual:
        s, out = icl.add_layer_norm(xd, rd, wd, bd, 1e-5, dout)
        torch.cuda.synchronize()
        want_s = xd + rd
        assert torch.equal(s, want_s)
        ref = _ref(want_s.cpu(), w, b, 1e-5)
    else:
        out = icl._safe_layer_norm(xd, wd, bd, 1e-5, dout)
        torch.cuda.synchronize()
        ref = _ref(x, w, b, 1e-5)
    assert out.dtype == dout and out.shape == x.shape
    check(out, ref, dout, f"layernorm W={W} {din}->{dout}")
    assert torch.allclose(out[0].double().cpu(), b.double(), atol=1e-2 if dout == torch.bfloat16 else 1e-5)


def test_layer_norm_leading_dims_and_no_bias(dev):
    # [est, column, row, 128] rows as the column stage hands them, no bias: the same as the flat rows
    import tabicl_mi355_icl as icl
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 13, 300, 128, generator=g)
    w = 1 + 0.1 * torch.randn(128, generator=g)
    out = icl._safe_layer_norm(x.to(dev), w.to(dev), None, 1e-5, torch.float32)
    flat = icl._safe_layer_norm(x.reshape(-1, 128).to(dev), w.to(dev), None, 1e-5, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(out.reshape(-1, 128), flat)
    check(out, _ref(x, w, None, 1e-5), torch.float32, "layernorm 4-D no bias")
