"""Pins the CPU oracle (oracle/attention.py) with closed forms, invariants and brute force, so that a
dropped term, a wrong sign or index, or a transposed operand in the oracle fails one of these."""
import numpy as np
import pytest
import torch

from oracle import attention as O

H = 8
E = 128


def _rand(rng, *shape, scale=1.0):
    return rng.standard_normal(shape) * scale


def test_loops_vs_vectorised_vs_torch_fp32():
    rng = np.random.default_rng(0)
    q, k, v = _rand(rng, 2, 5, 16, scale=0.5), _rand(rng, 2, 7, 16), _rand(rng, 2, 7, 16)
    bias = _rand(rng, 2, 7)
    a = O.attention_loops(q, k, v, 2, bias)
    b = O.attention_f64(q, k, v, 2, bias)
    c = O.ref_attn(torch.tensor(q), torch.tensor(k), torch.tensor(v), 2, torch.tensor(bias)).double().numpy()
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)
    np.testing.assert_allclose(b, c, rtol=0, atol=1e-5)


def test_two_keys_closed_form():
    # p(key0) = sigmoid(s0 - s1); out = p v0 + (1 - p) v1, per head
    rng = np.random.default_rng(1)
    q, k, v = _rand(rng, 1, 3, E), _rand(rng, 1, 2, E), _rand(rng, 1, 2, E)
    out = O.attention_f64(q, k, v, H)
    d = E // H
    for g in range(H):
        sl = slice(g * d, (g + 1) * d)
        s0 = q[0, :, sl] @ k[0, 0, sl]
        s1 = q[0, :, sl] @ k[0, 1, sl]
        p0 = 1.0 / (1.0 + np.exp(-(s0 - s1)))
        want = p0[:, None] * v[0, 0, sl] + (1 - p0)[:, None] * v[0, 1, sl]
        np.testing.assert_allclose(out[0, :, sl], want, atol=1e-12)


def test_one_key_gives_value_row():
    rng = np.random.default_rng(2)
    q, k, v = _rand(rng, 2, 4, E), _rand(rng, 2, 1, E), _rand(rng, 2, 1, E)
    out = O.attention_f64(q, k, v, H)
    np.testing.assert_allclose(out, np.broadcast_to(v, out.shape), atol=1e-12)


def test_key_permutation_invariance_and_row_shift():
    rng = np.random.default_rng(3)
    q, k, v = _rand(rng, 2, 6, E, scale=0.3), _rand(rng, 2, 9, E), _rand(rng, 2, 9, E)
    bias = _rand(rng, 2, 9)
    base = O.attention_f64(q, k, v, H, bias)
    perm = rng.permutation(9)
    np.testing.assert_allclose(O.attention_f64(q, k[:, perm], v[:, perm], H, bias[:, perm]), base, atol=1e-12)
    # a constant added to every key's bias shifts every score of a row equally -> no change
    np.testing.assert_allclose(O.attention_f64(q, k, v, H, bias + 7.5), base, atol=1e-12)


def test_masked_keys_equal_slicing_and_valid_len():
    rng = np.random.default_rng(4)
    q, k, v = _rand(rng, 3, 5, E, scale=0.3), _rand(rng, 3, 11, E), _rand(rng, 3, 11, E)
    bias = np.zeros((3, 11))
    bias[:, 8:] = O.NEG
    masked = O.attention_f64(q, k, v, H, bias)
    sliced = O.attention_f64(q, k[:, :8], v[:, :8], H)
    np.testing.assert_allclose(masked, sliced, atol=1e-12)
    np.testing.assert_allclose(O.attention_f64(q, k, v, H, valid=8), sliced, atol=1e-12)
    # ragged valid lengths, one per batch element; 0 valid keys -> output 0 (defined behaviour)
    got = O.attention_f64(q, k, v, H, valid=np.array([11, 3, 0]))
    np.testing.assert_allclose(got[0], O.attention_f64(q[:1], k[:1], v[:1], H)[0], atol=1e-12)
    np.testing.assert_allclose(got[1], O.attention_f64(q[1:2], k[1:2, :3], v[1:2, :3], H)[0], atol=1e-12)
    assert np.all(got[2] == 0)


def test_zero_query_is_mean_and_convex_hull():
    rng = np.random.default_rng(5)
    q, k, v = np.zeros((1, 2, E)), _rand(rng, 1, 13, E), _rand(rng, 1, 13, E)
    out = O.attention_f64(q, k, v, H)
    np.testing.assert_allclose(out[0, 0], v[0].mean(axis=0), atol=1e-12)
    q2 = _rand(rng, 1, 20, E)
    out2 = O.attention_f64(q2, k, v, H)
    assert np.all(out2 <= v.max(axis=1, keepdims=True) + 1e-12)
    assert np.all(out2 >= v.min(axis=1, keepdims=True) - 1e-12)


def test_heads_are_independent_column_blocks():
    # changing head 3's keys must leave every other head's output unchanged
    rng = np.random.default_rng(6)
    q, k, v = _rand(rng, 1, 4, E), _rand(rng, 1, 6, E), _rand(rng, 1, 6, E)
    base = O.attention_f64(q, k, v, H)
    k2 = k.copy()
    k2[..., 48:64] = _rand(rng, 1, 6, 16)
    alt = O.attention_f64(q, k2, v, H)
    same = np.ones(E, bool)
    same[48:64] = False
    np.testing.assert_allclose(alt[..., same], base[..., same], atol=1e-12)
    assert np.abs(alt[..., 48:64] - base[..., 48:64]).max() > 1e-3


def test_splash_ref_scale_and_valid():
    rng = np.random.default_rng(7)
    q, k, v = _rand(rng, 2, 2, 5, 64), _rand(rng, 2, 2, 9, 64), _rand(rng, 2, 2, 9, 64)
    got = O.splash_sdpa_ref(q, k, v, valid=np.array([9, 4]))
    # same thing through the merged-layout oracle: one head per [N*H] slice, q pre-scaled by 1/8
    for n, nv in ((0, 9), (1, 4)):
        for hh in range(2):
            want = O.attention_f64(q[n, hh][None] / 8.0, k[n, hh, :nv][None], v[n, hh, :nv][None], 1)[0]
            np.testing.assert_allclose(got[n, hh], want, atol=1e-12)
    qt, kt, vt = (torch.tensor(x, dtype=torch.float32) for x in (q, k, v))
    np.testing.assert_allclose(O.splash_sdpa_torch(qt[:1], kt[:1], vt[:1]).double().numpy(),
                               O.splash_sdpa_ref(q[:1], k[:1], v[:1]), atol=2e-5)


@pytest.mark.parametrize("chunk", [1, 3, 4, 64])
def test_online_softmax_equals_one_shot(chunk):
    rng = np.random.default_rng(8)
    q, k, v = _rand(rng, 1, 2, 6, 64), _rand(rng, 1, 2, 10, 64), _rand(rng, 1, 2, 10, 64)
    np.testing.assert_allclose(O.tiled_online_sdpa_ref(q, k, v, chunk), O.splash_sdpa_ref(q, k, v), atol=1e-12)
    np.testing.assert_allclose(O.tiled_online_sdpa_ref(q, k, v, chunk, valid=7), O.splash_sdpa_ref(q, k, v, 7),
                               atol=1e-12)


@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_closed_form_norm_and_relative_position(interleaved):
    rng = np.random.default_rng(9)
    h, d = 8, 16
    freqs = O.textbook_freqs(16, 10000.0)
    L = 7
    cos, sin, code, half, rot = O.rope_tables_ref(freqs, L, h * d, h, interleaved)
    assert (code, half, rot) == ((1 if interleaved else 2), 8, 16)
    x = _rand(rng, L, h * d)
    y = O.rope_merged_ref(x, cos, sin, h, code, half, rot)
    # position 0 is the identity
    np.testing.assert_allclose(y[0], x[0], atol=1e-12)
    # explicit 2-D rotation of each (a, b) pair by angle pos * freq_i
    for pos in range(L):
        for g in range(h):
            for i in range(d // 2):
                a_i, b_i = (g * d + 2 * i, g * d + 2 * i + 1) if interleaved else (g * d + i, g * d + i + 8)
                th = pos * freqs[i]
                a, b = x[pos, a_i], x[pos, b_i]
                assert abs(y[pos, a_i] - (a * np.cos(th) - b * np.sin(th))) < 1e-12
                assert abs(y[pos, b_i] - (b * np.cos(th) + a * np.sin(th))) < 1e-12
    # rotation preserves each head's norm
    np.testing.assert_allclose(np.linalg.norm(y.reshape(L, h, d), axis=-1),
                               np.linalg.norm(x.reshape(L, h, d), axis=-1), atol=1e-12)
    # <R_m q, R_n k> depends only on m - n
    qv, kv = _rand(rng, 1, h * d), _rand(rng, 1, h * d)
    def rot_at(vec, pos):
        c, s_, *_ = O.rope_tables_ref(freqs, 1, h * d, h, interleaved, positions=[pos])
        return O.rope_merged_ref(vec, c, s_, h, code, half, rot)
    d1 = (rot_at(qv, 5) * rot_at(kv, 2)).reshape(h, d).sum(-1)
    d2 = (rot_at(qv, 9) * rot_at(kv, 6)).reshape(h, d).sum(-1)
    np.testing.assert_allclose(d1, d2, atol=1e-10)


def test_rope_partial_rotary_dims_pass_through():
    rng = np.random.default_rng(10)
    freqs = O.textbook_freqs(8, 100000.0)  # rot = 8 < d = 16
    cos, sin, code, half, rot = O.rope_tables_ref(freqs, 4, E, H, False)
    assert (half, rot) == (4, 8)
    x = _rand(rng, 4, E)
    y = O.rope_merged_ref(x, cos, sin, H, code, half, rot)
    for g in range(H):
        np.testing.assert_allclose(y[:, g * 16 + 8:(g + 1) * 16], x[:, g * 16 + 8:(g + 1) * 16], atol=1e-12)


def test_op_oracles_compose():
    rng = np.random.default_rng(11)
    B, L = 2, 6
    qkv = _rand(rng, B, L, 3 * E)
    freqs = O.textbook_freqs(16, 10000.0)
    cos, sin, code, half, rot = O.rope_tables_ref(freqs, L, E, H, False)
    got = O.pk_self_ref(qkv, H, None, (cos, sin, code, half, rot), 0.25)
    q = O.rope_merged_ref(qkv[..., :E], cos, sin, H, code, half, rot) * 0.25
    k = O.rope_merged_ref(qkv[..., E:2 * E], cos, sin, H, code, half, rot)
    np.testing.assert_allclose(got, O.attention_f64(q, k, qkv[..., 2 * E:], H), atol=1e-12)
    kv = _rand(rng, B, 9, 2 * E)
    qq = _rand(rng, 1, 3, E)
    got = O.pk_cross_ref(qq, kv, H, None, None, None, 0.25)
    np.testing.assert_allclose(got[1], O.attention_f64(qq * 0.25, kv[1:, :, :E], kv[1:, :, E:], H)[0], atol=1e-12)
    np.testing.assert_allclose(O.hxq_ref(qq.repeat(2, 0), kv, np.array([5]), H),
                               O.attention_f64(qq.repeat(2, 0), kv[:, :5, :E], kv[:, :5, E:], H), atol=1e-12)


def test_combined_mask_forms():
    m = O.combined_mask_ref(np.zeros((3, 5), np.float32), None, (2,), 8, 3, 5)
    assert m.shape == (1, 1, 3, 5)
    kp = np.zeros((2, 5), np.float32)
    kp[1, 3:] = -np.inf
    m = O.combined_mask_ref(None, kp, (2,), 8, 3, 5)
    assert m.shape == (2, 1, 1, 5) and np.isneginf(m[1, 0, 0, 4])
    assert O.combined_mask_ref(np.zeros((3, 5), bool), None, (2,), 8, 3, 5) is False
    assert O.combined_mask_ref(np.zeros((4, 5), np.float32), None, (2,), 8, 3, 5) is False
    assert O.combined_mask_ref(None, None, (2,), 8, 3, 5) is None


# --- backward restatements -------------------------------------------------------------------

def _attn_torch(q, k, v, h, bias=None):
    """The forward definition in float64 torch (autograd gives the gradients the restatement must
    match): per-head softmax(q k^T + bias) v, merged layout."""
    B, Lq, Em = q.shape
    d = Em // h
    qh = q.reshape(B, Lq, h, d).transpose(1, 2)
    kh = k.reshape(k.shape[0], -1, h, d).transpose(1, 2)
    vh = v.reshape(v.shape[0], -1, h, d).transpose(1, 2)
    s = qh @ kh.transpose(-1, -2)
    if bias is not None:
        s = s + bias.reshape(bias.shape[0], 1, 1, -1)
    return (torch.softmax(s, dim=-1) @ vh).transpose(1, 2).reshape(B, Lq, Em)


def _rot_matrix(h, code, half, rot):
    """R as an explicit [E, E] matrix (R(x) = x @ M^T), built column by column from unit vectors."""
    eye = np.eye(E)
    return O.rotate_merged(eye, h, code, half, rot).T


def _rope_torch(x, cos, sin, M):
    return x * cos + (x @ M.T) * sin


@pytest.mark.parametrize("with_bias", [False, True])
def test_attention_bwd_matches_autograd(with_bias):
    rng = np.random.default_rng(20)
    q, k, v = _rand(rng, 2, 6, E, scale=0.25), _rand(rng, 2, 9, E), _rand(rng, 2, 9, E)
    do = _rand(rng, 2, 6, E)
    bias = None
    if with_bias:
        bias = _rand(rng, 2, 9)
        bias[:, -2:] = -1e30  # masked keys get zero gradient
    dq, dk, dv = O.attention_bwd_f64(q, k, v, H, do, bias)
    qt, kt, vt = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    out = _attn_torch(qt, kt, vt, H, None if bias is None else torch.tensor(bias))
    out.backward(torch.tensor(do))
    np.testing.assert_allclose(dq, qt.grad.numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(dk, kt.grad.numpy(), rtol=0, atol=1e-12)
    np.testing.assert_allclose(dv, vt.grad.numpy(), rtol=0, atol=1e-12)
    if with_bias:
        assert np.abs(dk[:, -2:]).max() == 0 and np.abs(dv[:, -2:]).max() == 0


def test_attention_bwd_finite_differences():
    # central differences of <dO, O> on a tiny case (one head of width 16 so that d = 16 holds)
    rng = np.random.default_rng(21)
    q, k, v = _rand(rng, 1, 2, 16, scale=0.5), _rand(rng, 1, 3, 16), _rand(rng, 1, 3, 16)
    do = _rand(rng, 1, 2, 16)
    dq, dk, dv = O.attention_bwd_f64(q, k, v, 1, do)
    f = lambda q_, k_, v_: float((O.attention_loops(q_, k_, v_, 1) * do).sum())  # noqa: E731
    eps = 1e-6
    for grad, which in ((dq, 0), (dk, 1), (dv, 2)):
        for idx in [(0, 0, 0), (0, 1, 5), (0, 0, 15)]:
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += eps
            up = f(*args)
            args[which][idx] -= 2 * eps
            dn = f(*args)
            assert abs((up - dn) / (2 * eps) - grad[idx]) < 1e-6


def test_bwd_uses_given_forward_output_for_d():
    # D comes from the stored output: a perturbed O shifts dq/dk by dS changes, dv not at all
    rng = np.random.default_rng(22)
    q, k, v = _rand(rng, 1, 4, E, scale=0.25), _rand(rng, 1, 5, E), _rand(rng, 1, 5, E)
    do = _rand(rng, 1, 4, E)
    o = O.attention_f64(q, k, v, H)
    a = O.attention_bwd_f64(q, k, v, H, do, o=o)
    b = O.attention_bwd_f64(q, k, v, H, do, o=o + 0.01)
    np.testing.assert_allclose(a[2], b[2], rtol=0, atol=0)
    assert np.abs(a[0] - b[0]).max() > 1e-6


@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_bwd_is_transpose_of_rope(interleaved):
    rng = np.random.default_rng(23)
    L = 7
    cos, sin, code, half, rot = O.rope_tables_ref(O.textbook_freqs(16, 1e4), L, E, H, interleaved)
    y = _rand(rng, L, E)
    x = torch.tensor(_rand(rng, L, E), requires_grad=True)
    M = torch.tensor(_rot_matrix(H, code, half, rot))
    _rope_torch(x, torch.tensor(cos), torch.tensor(sin), M).backward(torch.tensor(y))
    np.testing.assert_allclose(O.rope_bwd_ref(y, cos, sin, H, code, half, rot), x.grad.numpy(), rtol=0,
                               atol=1e-12)


def test_pk_self_bwd_matches_autograd():
    rng = np.random.default_rng(24)
    B, L, scale = 2, 6, 0.25
    rope = O.rope_tables_ref(O.textbook_freqs(16, 1e4), L, E, H, False)
    cos, sin, code, half, rot = rope
    x = _rand(rng, B, L, 3 * E)
    do = _rand(rng, B, L, E)
    bias = _rand(rng, 1, L)
    got = O.pk_self_bwd_ref(x, H, bias, rope, scale, do)
    xt = torch.tensor(x, requires_grad=True)
    M = torch.tensor(_rot_matrix(H, code, half, rot))
    c, s_ = torch.tensor(cos), torch.tensor(sin)
    q, k, v = xt[..., :E], xt[..., E:2 * E], xt[..., 2 * E:]
    out = _attn_torch(_rope_torch(q, c, s_, M) * scale, _rope_torch(k, c, s_, M), v, H, torch.tensor(bias))
    out.backward(torch.tensor(do))
    np.testing.assert_allclose(got, xt.grad.numpy(), rtol=0, atol=1e-11)


@pytest.mark.parametrize("shared_q", [False, True])
def test_pk_cross_bwd_matches_autograd(shared_q):
    rng = np.random.default_rng(25)
    B, Lq, Lk, scale = 3, 4, 6, 0.25
    rq = O.rope_tables_ref(O.textbook_freqs(16, 1e4), Lq, E, H, True)
    rk = O.rope_tables_ref(O.textbook_freqs(16, 1e4), Lk, E, H, True)
    q = _rand(rng, 1 if shared_q else B, Lq, E)
    kv = _rand(rng, B, Lk, 2 * E)
    do = _rand(rng, B, Lq, E)
    dq, dkv = O.pk_cross_bwd_ref(q, kv, H, None, rq, rk, scale, do)
    qt = torch.tensor(q, requires_grad=True)
    kvt = torch.tensor(kv, requires_grad=True)
    M = torch.tensor(_rot_matrix(H, *rq[2:]))
    qr = _rope_torch(qt, torch.tensor(rq[0]), torch.tensor(rq[1]), M)
    kr = _rope_torch(kvt[..., :E], torch.tensor(rk[0]), torch.tensor(rk[1]), M)
    out = _attn_torch(qr.expand(B, Lq, E) * scale, kr, kvt[..., E:], H)
    out.backward(torch.tensor(do))
    assert dq.shape == q.shape
    np.testing.assert_allclose(dq, qt.grad.numpy(), rtol=0, atol=1e-11)
    np.testing.assert_allclose(dkv, kvt.grad.numpy(), rtol=0, atol=1e-11)


def test_folding_identity_matches_unfolded_attention():
    # the algebra the folded first ISAB attention rests on (reference scripts/tabicl_tpu_mha.py:60-92):
    # softmax(q_g K_g^T) V_g == softmax((q_g W_k,g) x^T) x W_v,g^T + b_v,g  (q_g . b_k,g drops out of
    # the softmax; rows of P sum to 1)
    rng = np.random.default_rng(26)
    B, Lq, Lk, valid, hd = 2, 5, 11, 8, E // H
    ind = _rand(rng, Lq, E, scale=0.5)
    x = _rand(rng, B, Lk, E)
    W = _rand(rng, 3 * E, E, scale=E ** -0.5)
    b = _rand(rng, 3 * E, scale=0.1)
    ref = O.folded_mab1_ref(ind, x, valid, H, W, b)
    q = (ind @ W[:E].T + b[:E]) * hd ** -0.5
    qf = np.concatenate([q[:, g * hd:(g + 1) * hd] @ W[E + g * hd:E + (g + 1) * hd] for g in range(H)])  # [H*Lq, E]
    u = O.hxf_ref(qf[None], x, valid)  # [B, H*Lq, E]
    out = np.zeros((B, Lq, E))
    for g in range(H):
        wv = W[2 * E + g * hd:2 * E + (g + 1) * hd]
        out[..., g * hd:(g + 1) * hd] = u[:, g * Lq:(g + 1) * Lq] @ wv.T + b[2 * E + g * hd:2 * E + (g + 1) * hd]
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-10)


def test_hxf_ref_valid_and_shared_query():
    rng = np.random.default_rng(27)
    qf = _rand(rng, 1, 6, E, scale=0.1)
    x = _rand(rng, 3, 9, E)
    got = O.hxf_ref(qf, x, np.array([9, 4, 0]))
    np.testing.assert_allclose(got[1], O.hxf_ref(qf, x[1:2, :4], 4)[0], rtol=0, atol=1e-12)
    assert np.abs(got[2]).max() == 0
    np.testing.assert_allclose(got[0], O.attention_loops(qf, x[:1], x[:1], 1)[0], rtol=0, atol=1e-12)


def test_splash_ref_key_bias():
    # the key-mask parameter of the ICL oracle, pinned by closed forms and invariants
    g = torch.Generator().manual_seed(31)
    q = torch.randn(2, 3, 5, 64, generator=g)
    k = torch.randn(2, 3, 40, 64, generator=g)
    v = torch.randn(2, 3, 40, 64, generator=g)
    base = O.splash_sdpa_ref(q, k, v)
    # (with a mask the scores are summed in float32, as the reference does: agreement to fp32 rounding)
    np.testing.assert_allclose(O.splash_sdpa_ref(q, k, v, bias=np.zeros((1, 40))), base, atol=1e-6)
    # one constant per row (and per n) shifts every score of the row: softmax unchanged
    np.testing.assert_allclose(O.splash_sdpa_ref(q, k, v, bias=np.array([[3.0] * 40, [-7.0] * 40])), base, atol=1e-6)
    # a prefix mask (0, then finfo.min or -inf) is the valid length
    for fill in (float(np.finfo(np.float32).min), -np.inf):
        b = np.zeros((2, 40))
        b[0, 17:] = fill
        b[1, 33:] = fill
        np.testing.assert_allclose(O.splash_sdpa_ref(q, k, v, bias=b), O.splash_sdpa_ref(q, k, v, np.array([17, 33])),
                                   atol=1e-6)
    # every key at finfo.min: the fp32 sum absorbs the scores, weights are equal -> mean of V
    allm = np.full((1, 40), float(np.finfo(np.float32).min))
    np.testing.assert_allclose(O.splash_sdpa_ref(q, k, v, bias=allm),
                               np.broadcast_to(v.double().numpy().mean(axis=2, keepdims=True), (2, 3, 5, 64)), atol=1e-12)
    # two keys, bias b on key 1: weight of key 1 = sigmoid(s1 + b - s0)
    q2, k2, v2 = q[:1, :1, :1], k[:1, :1, :2], v[:1, :1, :2]
    s = (q2[0, 0, 0].double() @ k2[0, 0].double().T).numpy() * 0.125
    w1 = 1.0 / (1.0 + np.exp(-(np.float64(np.float32(s[1]) + np.float32(1.5)) - np.float32(s[0]))))
    want = (1 - w1) * v2[0, 0, 0].double().numpy() + w1 * v2[0, 0, 1].double().numpy()
    np.testing.assert_allclose(O.splash_sdpa_ref(q2, k2, v2, bias=np.array([[0.0, 1.5]]))[0, 0, 0], want, atol=1e-6)


@pytest.mark.parametrize("case", ["plain", "valid", "bias"])
def test_splash_bwd_matches_autograd(case):
    # the ICL attention's gradients against torch autograd in float64 through an independent forward
    # (scaled scores, masked keys as -inf, softmax, product)
    rng = np.random.default_rng(40)
    N, Hh, Tq, Tkv, D = 2, 3, 5, 11, 64
    q, k, v, do = _rand(rng, N, Hh, Tq, D), _rand(rng, N, Hh, Tkv, D), _rand(rng, N, Hh, Tkv, D), _rand(rng, N, Hh, Tq, D)
    valid = np.array([7, 11]) if case == "valid" else None
    bias = None
    if case == "bias":
        bias = _rand(rng, N, Tkv).astype(np.float32)
        bias[:, -3:] = -1e30  # masked by the mask: zero gradients there
    dq, dk, dv = O.splash_sdpa_bwd_ref(q, k, v, do, valid, bias)
    qt, kt, vt = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    s = (qt * D ** -0.5) @ kt.transpose(-1, -2)
    if valid is not None:
        keep = torch.arange(Tkv)[None, :] < torch.tensor(valid)[:, None]
        s = s.masked_fill(~keep[:, None, None, :], float("-inf"))
    if bias is not None:
        # the kernel adds the bias to float32 scores; the rounded value enters with an identity gradient
        b32 = torch.tensor(bias)[:, None, None, :]
        s = s + ((s.detach().float() + b32).double() - s.detach())
    out = torch.softmax(s, dim=-1) @ vt
    out.backward(torch.tensor(do))
    for got, t in ((dq, qt), (dk, kt), (dv, vt)):
        np.testing.assert_allclose(got, t.grad.numpy(), rtol=0, atol=1e-10)
    if valid is not None:
        assert np.abs(dk[0, :, 7:]).max() == 0 and np.abs(dv[0, :, 7:]).max() == 0
    if bias is not None:
        assert np.abs(dk[:, :, -3:]).max() < 1e-300 and np.abs(dv[:, :, -3:]).max() < 1e-300


def test_splash_bwd_finite_differences():
    # central differences of <dO, O> through splash_sdpa_ref on a tiny case
    rng = np.random.default_rng(41)
    q, k, v, do = _rand(rng, 1, 1, 2, 64), _rand(rng, 1, 1, 3, 64), _rand(rng, 1, 1, 3, 64), _rand(rng, 1, 1, 2, 64)
    dq, dk, dv = O.splash_sdpa_bwd_ref(q, k, v, do)
    f = lambda q_, k_, v_: float((O.splash_sdpa_ref(q_, k_, v_) * do).sum())  # noqa: E731
    eps = 1e-6
    for grad, which in ((dq, 0), (dk, 1), (dv, 2)):
        for idx in [(0, 0, 0, 0), (0, 0, 1, 33), (0, 0, 0, 63)]:
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += eps
            up = f(*args)
            args[which][idx] -= 2 * eps
            dn = f(*args)
            assert abs((up - dn) / (2 * eps) - grad[idx]) < 1e-6


def test_operand_rounding_points():
    # the packed ops' oracle option that rounds q' = rope(q) scale and k' = rope(k) to the input dtype
    # where the reference's kernel casts them (scripts/tabicl_tpu_pallas_attn.py:500-501)
    g = torch.Generator().manual_seed(91)
    x = torch.randn(3, 40, 384, generator=g).double().numpy() * 3.0
    r = O._cast(x, torch.bfloat16)
    assert np.array_equal(O._cast(r, torch.bfloat16), r)  # representable: rounding again changes nothing
    assert np.all(np.abs(r - x) <= 2.0 ** -8 * np.abs(x))  # within half a bf16 ulp: 8 significant bits
    assert np.array_equal(O._cast(x, None), x)
    # without RoPE and with a power-of-two scale the operands are exact in bf16: rounding changes nothing
    qkv = torch.randn(2, 30, 384, generator=g).to(torch.bfloat16)
    a = O.pk_self_ref(qkv, 8, None, None, 0.25)
    b = O.pk_self_ref(qkv, 8, None, None, 0.25, cast=torch.bfloat16)
    assert np.array_equal(a, b)
    # with RoPE the rotated operands are not bf16 values: rounding moves the result, by ~2^-9 relative
    rope = O.rope_tables_ref(O.textbook_freqs(16, 100000.0), 30, 128, 8, False)
    a = O.pk_self_ref(qkv, 8, None, rope, 0.25)
    b = O.pk_self_ref(qkv, 8, None, rope, 0.25, cast=torch.bfloat16)
    d = float(np.abs(a - b).max()) / float(np.abs(a).max())
    assert 1e-5 < d < 2e-2, d
    y = torch.randn(2, 30, 256, generator=g).to(torch.bfloat16)
    qc = torch.randn(1, 7, 128, generator=g).to(torch.bfloat16)
    assert np.array_equal(O.pk_cross_ref(qc, y, 8, None, None, None, 0.25),
                          O.pk_cross_ref(qc, y, 8, None, None, None, 0.25, cast=torch.bfloat16))
