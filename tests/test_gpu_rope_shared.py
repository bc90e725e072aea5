"""GPU check of the shared-table RoPE form (TABICL_ROPE_SHARED_TABLES): the forward kernels given one
head's [L, 16] columns of rope_tables' output must return exactly (bit for bit) what they return for
the tiled [L, 128] tables, for every forward kernel that reads tables: the resident bf16 kernel (row
stage, 104 tokens; CLS cross attention), the general bf16 kernel (keys past the resident limit, and a
partial-rotary form) and the fp32 kernel. The tiled-table results are checked against the oracle by
test_gpu_smallhead.py; the wrappers use the shared form whenever no gradient is needed.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


class _Rope:
    def __init__(self, interleaved, rot=16):
        import numpy as np

        from oracle import attention as O
        self.interleaved = interleaved
        self.freqs = torch.tensor(np.asarray(O.textbook_freqs(rot, 10000.0)), dtype=torch.float32)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)

    def forward(self, seq, seq_len=None):
        f = (seq.float().unsqueeze(-1) * self.freqs.to(seq.device))
        return f.repeat_interleave(2, dim=-1) if self.interleaved else torch.cat([f, f], dim=-1)


@pytest.mark.parametrize("name,B,L,dtype,interleaved,rot", [
    ("row_resident_halves", 64, 104, torch.bfloat16, False, 16),
    ("row_resident_pairs", 16, 104, torch.bfloat16, True, 16),
    ("long_general_bf16", 4, 300, torch.bfloat16, False, 16),
    ("partial_rotary_bf16", 8, 104, torch.bfloat16, False, 8),
    ("fp32", 8, 104, torch.float32, False, 16),
])
def test_pk_self_shared_tables(dev, name, B, L, dtype, interleaved, rot):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(21)
    qkv = torch.randn(B, L, 384, generator=g).to(dtype).to(dev)
    bias = torch.zeros(B, 1, L, device=dev)
    bias[:, :, L - 3:] = -1e30
    rope = _Rope(interleaved, rot)
    cos, sin, rc, half, r = pk.rope_tables(rope, L, 128, 8, dev)
    lkp = -(-L // 128) * 128
    full = pk.PK_SELF(qkv, bias, cos, sin, 8, lkp, rc, half, r, 0, 0.25)
    cs, sn, rcs = pk._shared_tables(cos, sin, rc, 16)
    shared = pk.PK_SELF(qkv, bias, cs, sn, 8, lkp, rcs, half, r, 0, 0.25)
    torch.cuda.synchronize()
    assert torch.equal(full, shared), name


def test_pk_cross_shared_tables_cls(dev):
    import tabicl_mi355_attn as pk
    g = torch.Generator().manual_seed(22)
    q = torch.randn(256, 4, 128, generator=g).to(torch.bfloat16).to(dev)
    kv = torch.randn(256, 104, 256, generator=g).to(torch.bfloat16).to(dev)
    rope = _Rope(False)
    cq, sq, rc, half, r = pk.rope_tables(rope, 4, 128, 8, dev)
    ck, sk, _, _, _ = pk.rope_tables(rope, 104, 128, 8, dev)
    none = torch.empty(0, device=dev)
    full = pk.PK_CROSS(q, kv, none, cq, sq, ck, sk, 8, 128, 4, rc, half, r, 0, 0.25)
    cqs, sqs, _ = pk._shared_tables(cq, sq, rc, 16)
    cks, sks, rcs = pk._shared_tables(ck, sk, rc, 16)
    shared = pk.PK_CROSS(q, kv, none, cqs, sqs, cks, sks, 8, 128, 4, rcs, half, r, 0, 0.25)
    torch.cuda.synchronize()
    assert torch.equal(full, shared)
