"""CPU checks of the C ABI and the host logic: the library loads, exports every symbol that
include/tabicl_attn.h declares, rejects bad arguments before any device work, and the Python host
helpers keep the reference's semantics. No kernel is launched here."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as O

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tabicl_attn.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tabicl_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import tabicl_mi355_native as nat
    lib = nat.load()
    names = _declared()
    assert set(names) == set(nat.SIGNATURES), sorted(set(names) ^ set(nat.SIGNATURES))
    for name in names:
        assert hasattr(lib, name), name
        assert name in nat.SIGNATURES, name
    assert nat.version().startswith("tabicl_attn")


def test_supported_predicate():
    import tabicl_mi355_native as nat
    bf, f32 = torch.bfloat16, torch.float32
    assert nat.supported(nat.OP_HX, 1024, 128, 128, 8, bf)
    assert nat.supported(nat.OP_HXQ, 128, 53248, 128, 8, f32)
    assert not nat.supported(nat.OP_HX, 16, 16, 256, 16, bf)  # head dim 16 but 16 heads: not built
    assert not nat.supported(nat.OP_HX, 16, 0, 128, 8, bf)
    assert not nat.supported(nat.OP_HX, 16, 16, 128, 8, torch.float16)
    assert nat.supported(nat.OP_ICL, 5000, 45000, 64, 8, bf)
    assert not nat.supported(nat.OP_ICL, 5000, 45000, 128, 8, bf)


def test_bad_arguments_rejected_before_launch():
    import tabicl_mi355_native as nat
    lib = nat.load()
    # E != 128 -> status 1 and a message, with NULL pointers (nothing is dereferenced or launched)
    st = lib.tabicl_hx_fwd(None, None, None, None, 1, None, 2, 3, 4, 64, 8, 0, None)
    assert st == 1 and "E == 128" in nat.last_error()
    st = lib.tabicl_icl_fwd(None, None, None, None, 0, None, 1, 1, 1, 1, 32, *([64] * 12), 1.0, 0, None, 0, None)
    assert st == 1 and "head dim" in nat.last_error()
    st = lib.tabicl_pk_self_fwd(None, None, 1, None, None, None, 1, 8, 128, 8, 2, 3, 16, 0.25, 0, None)
    assert st == 1 and "rope" in nat.last_error()
    st = lib.tabicl_icl_cache_append(None, None, 64, 64, 10, 12, None, None, 64, 64, 64, 1, 1, 5, 64, 0, None)
    assert st == 1 and "capacity" in nat.last_error()
    # rope codes other than none / pairs / halves (with or without the shared-table flag) are refused by
    # the backward entry points too
    a = 0x1000  # 16-byte aligned placeholder address: the rope code is refused before any use
    for code in (3, 3 | 0x10, 0x20 | 2):
        st = lib.tabicl_pk_self_bwd(a, None, 1, a, a, a, a, a, 1, 8, 128, 8, code, 8, 16, 0.25, 0, a, 1 << 20, None)
        assert st == 1 and "rope code" in nat.last_error()
    # ragged entry points: a q_len array of neither 1 nor N (B) entries is refused before any launch
    qlen = ctypes.c_int32(3)
    st = lib.tabicl_icl_fwd_ragged(None, None, None, None, 0, ctypes.byref(qlen), 2, None, 3, 1, 1, 1, 64,
                                   *([64] * 12), 1.0, 0, None, 0, None)
    assert st == 1 and "q_len" in nat.last_error()
    st = lib.tabicl_pk_cross_fwd_ragged(None, 1, None, None, 1, None, None, None, None, None, 4, 8, 8, 128, 8, 0, 0,
                                        0, 0.25, 0, ctypes.byref(qlen), 2, None)
    assert st == 1 and "q_len" in nat.last_error()
    # RoPE tables of the cross entry points must be 16-byte aligned (float4 loads)
    st = lib.tabicl_pk_cross_fwd_ragged(a, 1, a, None, 1, a + 4, a, a, a, a, 4, 8, 8, 128, 8, 2, 8, 16, 0.25, 0,
                                        None, 0, None)
    assert st == 1 and "aligned" in nat.last_error()
    st = lib.tabicl_pk_cross_fwd(a, 1, a, None, 1, a, a, a, a + 8, a, 4, 8, 8, 128, 8, 2, 8, 16, 0.25, 0, None)
    assert st == 1 and "aligned" in nat.last_error()
    # masked entry points: key-mask rows must be 1 or N (B)
    st = lib.tabicl_icl_fwd_masked(a, a, a, None, 0, a, 3, 64, None, 0, a, 2, 1, 1, 64, 64, *([64] * 12), 0.125, 0,
                                   None, 0, None)
    assert st == 1 and "key_bias" in nat.last_error()
    st = lib.tabicl_icl_fwd_masked(a, a, a, None, 0, a, 1, 64, None, 0, a, 2, 1, 1, 64, 64, *([64] * 12), 0.0, 0,
                                   None, 0, None)
    assert st == 1 and "scale" in nat.last_error()
    st = lib.tabicl_hxq_fwd_masked(None, 0, a, 3, a, a, a, 2, 8, 300, 128, 8, 0, None, 0, None)
    assert st == 1 and "key_bias" in nat.last_error()
    st = lib.tabicl_hxf_fwd_masked(None, 0, a, 3, a, 1, a, a, 2, 64, 300, 128, 0, None, 0, None)
    assert st == 1 and "key_bias" in nat.last_error()
    # ICL gradient path: the statistics forward needs its stat array; the backward takes forward
    # statistics only without a key mask, needs a positive scale and a workspace of the size it names
    st = lib.tabicl_icl_fwd_stats(a, a, a, None, 0, a, None, 2, 1, 3, 64, 64, *([64] * 12), 0.125, 0, None, 0, None)
    assert st == 1 and "stat" in nat.last_error()
    bwd = lambda bias, stat, scale, ws, wsb: lib.tabicl_icl_bwd(  # noqa: E731
        a, a, a, None, 0, bias, 1, 64, a, a, stat, a, a, a, 2, 1, 3, 64, 64, scale, 0, ws, wsb, None)
    st = bwd(a, a, 0.125, a, 1 << 20)
    assert st == 1 and "key mask" in nat.last_error()
    st = bwd(None, None, -0.125, a, 1 << 20)
    assert st == 1 and "scale" in nat.last_error()
    need = lib.tabicl_icl_bwd_workspace_bytes(2, 1, 3)
    assert need > 0 and lib.tabicl_icl_bwd_workspace_bytes(-1, 1, 3) < 0
    st = bwd(None, a, 0.125, a, need - 1)
    assert st == 1 and "workspace" in nat.last_error()
    st = bwd(None, a, 0.125, None, need)
    assert st == 1 and "workspace" in nat.last_error()
    with pytest.raises(nat.UnsupportedShapeError):
        nat.check(1, "x")


def test_empty_calls_return_before_launch():
    # no batch element or no query row: status 0 with nothing dereferenced or launched (NULL pointers,
    # no stream), the key count then allowed to be 0 (an empty self-attention); keys are still required
    # when there is work
    import tabicl_mi355_native as nat
    lib = nat.load()
    assert lib.tabicl_pk_self_fwd(None, None, 1, None, None, None, 3, 0, 128, 8, 0, 8, 16, 0.25, 0, None) == 0
    assert lib.tabicl_hx_fwd(None, None, None, None, 1, None, 3, 0, 0, 128, 8, 0, None) == 0
    assert lib.tabicl_hx_fwd(None, None, None, None, 1, None, 0, 40, 0, 128, 8, 0, None) == 0
    st = lib.tabicl_hx_fwd(None, None, None, None, 1, None, 3, 40, 0, 128, 8, 0, None)
    assert st == 1 and "bad sizes" in nat.last_error()


@pytest.mark.parametrize("shared", [False, True])
def test_rope_table_shapes_refused_before_launch(shared):
    # a table of the wrong width, length or dtype is refused before any pointer reaches the library
    import tabicl_mi355_attn as pk
    import tabicl_mi355_native as nat
    rc = 2 | (pk.ROPE_SHARED_TABLES if shared else 0)
    cols = 16 if shared else 128
    qkv = torch.zeros(2, 10, 384)
    empty_bias = torch.empty(0, 1, 10)
    good = torch.zeros(10, cols)
    for bad in (torch.zeros(10, 128 if shared else 16), torch.zeros(9, cols), torch.zeros(10, cols, dtype=torch.float64)):
        with pytest.raises(ValueError, match="table"):
            torch.ops.tabicl_pk.pk_self_fwd(qkv, empty_bias, bad, good, 8, 128, rc, 8, 16, 0, 0.25)
        with pytest.raises(ValueError, match="table"):
            torch.ops.tabicl_pk.pk_cross_fwd(qkv[..., :128], qkv[..., :256], empty_bias, good, good, good, bad, 8, 128,
                                             10, rc, 8, 16, 0, 0.25)
    # right tables: the shape checks pass and the op then refuses CPU tensors (no CPU path)
    with pytest.raises(nat.NativeLibraryError):
        torch.ops.tabicl_pk.pk_self_fwd(qkv, empty_bias, good, good, 8, 128, rc, 8, 16, 0, 0.25)


def test_rope_tables_cached_per_module():
    import tabicl_mi355_attn as pk
    rope = torch.nn.Module()
    rope.interleaved = False
    rope.freqs = torch.nn.Parameter(torch.tensor(O.textbook_freqs(16, 10000.0), dtype=torch.float32),
                                    requires_grad=False)
    rope.get_seq_pos = lambda L, device=None, dtype=torch.float32: torch.arange(L, device=device, dtype=dtype)
    a = pk._tables(rope, 104, 128, 8, "cpu")
    b = pk._tables(rope, 104, 128, 8, "cpu")
    assert a[0] is b[0] and a[2] == 2 | pk.ROPE_SHARED_TABLES and tuple(a[0].shape) == (104, 16)
    full = pk.rope_tables(rope, 104, 128, 8, "cpu")
    assert tuple(full[0].shape) == (104, 128) and full[2] == 2
    for hd in range(8):  # the shared table is every head's columns of the full one
        np.testing.assert_array_equal(a[0].numpy(), full[0][:, 16 * hd:16 * hd + 16].numpy())
        np.testing.assert_array_equal(a[1].numpy(), full[1][:, 16 * hd:16 * hd + 16].numpy())
    with torch.no_grad():
        rope.freqs.mul_(2.0)  # in-place change of the frequencies: the cached tables are not reused
    c = pk._tables(rope, 104, 128, 8, "cpu")
    assert c[0] is not a[0] and not torch.allclose(c[1], a[1])
    n1, n2 = pk._tables(None, 50, 128, 8, "cpu"), pk._tables(None, 70, 128, 8, "cpu")
    assert n1[2] == 0 and n1[0] is n2[0]  # no RoPE: one stand-in row, never read by the kernels


def test_icl_cache_fill_bookkeeping():
    import tabicl_mi355_icl as icl
    cache = icl.IclKVCache(2, 3, 8, 1000, 64, torch.bfloat16, "cpu")
    with pytest.raises(ValueError, match="no rows"):
        cache.default_valid(0)
    cache._record(0, 300, 200)  # rows [300, 500) first: row 0 not written yet, no default length
    assert cache.length(0) == 0
    with pytest.raises(ValueError, match="no rows"):
        cache.default_valid(0)
    cache._record(0, 0, 300)  # now [0, 500) is contiguous
    cache._record(0, 100, 50)  # rewriting rows inside it keeps the length
    cache._record(0, 700, 10)  # a later island does not extend it
    assert cache.length(0) == 500 and cache.length(1) == 0
    assert cache.written[0] == [(0, 500), (700, 710)]
    t = cache.default_valid(0)
    assert t.dtype == torch.int32 and t.tolist() == [500] and cache.default_valid(0) is t
    cache._record(0, 500, 200)  # closes the gap: [0, 710)
    assert cache.length(0) == 710


def test_icl_cache_estimator_views():
    import tabicl_mi355_icl as icl
    cache = icl.IclKVCache(4, 2, 8, 100, 64, torch.bfloat16, "cpu")
    v = cache.estimators(1, 3)
    assert v.shape == (2, 2, 8, 100, 64) and v.keys.data_ptr() == cache.keys[1].data_ptr()
    v.keys.fill_(1.0)
    assert float(cache.keys[1:3].float().sum()) == 2 * 2 * 8 * 100 * 64  # same storage
    v._record(0, 0, 40)  # the row record is shared with the whole cache
    assert cache.length(0) == 40 and v.length(0) == 40
    for bad in ((0, 0), (3, 5), (-1, 2)):
        with pytest.raises(ValueError, match="out of range"):
            cache.estimators(*bad)
    x = torch.zeros(4, 5, 512)
    for chunks in ([], [(0, 2)], [(0, 2), (3, 4)], [(1, 4)]):
        with pytest.raises(ValueError, match="do not cover"):
            cache.query_chunked(x, [], chunks)


def test_ops_refuse_cpu_tensors():
    import tabicl_mi355_attn as pk
    import tabicl_mi355_native as nat
    q = torch.zeros(1, 4, 128)
    with pytest.raises(nat.NativeLibraryError):
        pk.hx_attention(q, q, q, 8)


def test_pick_blocks_match_reference_rules():
    import tabicl_mi355_attn as pk
    assert pk._pick_bq(1024, 128) == 512
    assert pk._pick_bq(104, 128) == 104
    assert pk._pick_bq(53248, 128) == 512
    assert pk._pick_bq(4, 128) == 4
    assert pk._pick_bq(1001, 1024) == 0
    assert pk._pick_bk(53248) == 512
    assert pk._pick_bk(1024) == 512
    assert pk._pick_bk(384) == 128
    assert pk._pick_bk(100) == 0


def test_bias3_forms():
    import tabicl_mi355_attn as pk
    assert pk._bias3(None, (4, 2), 7, "cpu").shape == (1, 1, 7)
    b = torch.arange(7.0)
    assert torch.equal(pk._bias3(b, (4, 2), 7, "cpu"), b.reshape(1, 1, 7))
    b2 = torch.randn(4, 1, 7)
    out = pk._bias3(b2, (4, 2), 7, "cpu")
    assert out.shape == (8, 1, 7)
    assert torch.equal(out[3], b2[1])


def test_key_bias_alignment_fixup():
    # a contiguous view that starts off a 16-byte boundary (here 1 float in) is copied into a fresh,
    # aligned allocation by _bias3 and by the ICL wrapper's helper; aligned contiguous rows pass through
    import tabicl_mi355_attn as pk
    import tabicl_mi355_native as nat
    base = torch.randn(1, 66)
    view = base[:, 1:65]
    assert view.is_contiguous() and view.data_ptr() % 16 != 0
    fixed = nat.aligned16(view)
    assert fixed.data_ptr() % 16 == 0 and torch.equal(fixed, view)
    out = pk._bias3(view[0], (3,), 64, "cpu")
    assert out.data_ptr() % 16 == 0 and torch.equal(out[0, 0], view[0])
    rows = torch.randn(3, 65)[:, 1:]  # non-contiguous rows
    out = pk._bias3(rows, (3,), 64, "cpu")
    assert out.is_contiguous() and out.data_ptr() % 16 == 0 and torch.equal(out[:, 0], rows)
    ok = torch.randn(64)
    assert nat.aligned16(ok) is ok


class _Rope:
    def __init__(self, interleaved):
        self.interleaved = interleaved
        self.freqs = torch.tensor(O.textbook_freqs(16, 10000.0), dtype=torch.float32)

    def get_seq_pos(self, L, device=None, dtype=torch.float32):
        return torch.arange(L, device=device, dtype=dtype)

    def forward(self, seq, seq_len=None):
        return (seq.float().unsqueeze(-1) * self.freqs).repeat_interleave(2, dim=-1)


@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_tables_match_oracle(interleaved):
    import tabicl_mi355_attn as pk
    cos, sin, code, half, rot = pk.rope_tables(_Rope(interleaved), 104, 128, 8, "cpu")
    c2, s2, code2, half2, rot2 = O.rope_tables_ref(O.textbook_freqs(16, 10000.0), 104, 128, 8, interleaved)
    assert (code, half, rot) == (code2, half2, rot2)
    np.testing.assert_allclose(cos.numpy(), c2, atol=1e-5)
    np.testing.assert_allclose(sin.numpy(), s2, atol=1e-5)
    c0, s0, code0, _, _ = pk.rope_tables(None, 4, 128, 8, "cpu")
    assert code0 == 0 and torch.all(c0 == 1) and torch.all(s0 == 0)


def test_error_message_is_per_thread():
    # the library's last-error message is thread-local: a refusal in another host thread leaves this
    # thread's message as it was
    import threading
    import tabicl_mi355_native as nat
    lib = nat.load()
    st = lib.tabicl_icl_fwd(None, None, None, None, 0, None, 1, 1, 1, 1, 32, *([64] * 12), 1.0, 0, None, 0, None)
    assert st == 1 and "head dim" in nat.last_error()
    other = {}

    def refuse():
        other["st"] = lib.tabicl_hx_fwd(None, None, None, None, 1, None, 2, 3, 4, 64, 8, 0, None)
        other["msg"] = nat.last_error()

    t = threading.Thread(target=refuse)
    t.start()
    t.join()
    assert other["st"] == 1 and "E == 128" in other["msg"]
    assert "head dim" in nat.last_error()
