"""GPU checks at BASELINE's full sizes for the row (C2) and column ISAB-2 (C3) attention, the two d = 16
configs that the other GPU tests run at reduced batch: the fp64 oracle on sampled sequences, and over
the whole output the size-independent properties of softmax attention: every output is finite and,
per head and dimension, lies between the smallest and largest value of V over the keys (a convex
combination), and a bit-identical rerun. Inputs come from a device generator (the CPU oracle gets
copies of the sampled sequences only).

Bar (written here): max abs error <= 2e-2 against the oracle (bf16 inputs); hull with 2e-2 slack for
the bf16 rounding of the output.
"""
import pytest
import torch

from oracle import attention as O

pytestmark = pytest.mark.gpu
H, E = 8, 128


class _Rope:
    interleaved = False

    def __init__(self):
        self.freqs = 10000.0 ** (-torch.arange(0, 16, 2, dtype=torch.float32) / 16)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)


def _hull_ok(out, v, tol=2e-2):
    # out [B, Lq, E], v [B, Lk, E]: per (batch, dim) the output lies within V's range over the keys
    vmax = v.float().amax(dim=1, keepdim=True)
    vmin = v.float().amin(dim=1, keepdim=True)
    return bool((out.float() <= vmax + tol).all()) and bool((out.float() >= vmin - tol).all())


def test_c2_row_stage_full_size(dev):
    import numpy as np

    import tabicl_mi355_attn as pk
    g = torch.Generator(device=dev).manual_seed(1)
    B, L = 16384, 104
    qkv = torch.randn(B, L, 3 * E, generator=g, device=dev).to(torch.bfloat16)
    rope = _Rope()
    print("[fullsize] c2", flush=True)
    with torch.no_grad():
        out = pk.pk_self_attention(qkv, H, None, rope, 0.25)
        again = pk.pk_self_attention(qkv, H, None, rope, 0.25)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out, again)
    assert _hull_ok(out, qkv[..., 2 * E:])
    tables = O.rope_tables_ref(rope.freqs.double().numpy(), L, E, H, False)
    for b in (0, 1, 4097, 9999, B - 1):
        ref = O.pk_self_ref(qkv[b:b + 1].cpu(), H, None, tables, 0.25)
        err = float(np.abs(out[b:b + 1].double().cpu().numpy() - ref).max())
        assert err <= 2e-2, (b, err)


def test_c3_isab2_full_size(dev):
    import numpy as np

    import tabicl_mi355_attn as pk
    g = torch.Generator(device=dev).manual_seed(2)
    B, T, NI = 800, 50000, 128
    q = torch.randn(B, T, E, generator=g, device=dev).to(torch.bfloat16)
    kv = torch.randn(B, NI, 2 * E, generator=g, device=dev).to(torch.bfloat16)
    print("[fullsize] c3 isab2", flush=True)
    with torch.no_grad():
        out = pk.pk_cross_attention(q, kv, H, None, None, 0.25)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert _hull_ok(out, kv[..., E:])
    rows = torch.arange(0, T, 997)
    for b in (0, 399, B - 1):
        ref = O.pk_cross_ref(q[b:b + 1, rows].cpu(), kv[b:b + 1].cpu(), H, None, None, None, 0.25)
        err = float(np.abs(out[b:b + 1, rows].double().cpu().numpy() - ref).max())
        assert err <= 2e-2, (b, err)
    del q, out
