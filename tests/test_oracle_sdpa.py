"""Pins the oracle's sdpa_decode / causal prefill (forward_cpu.rs:424-510)
against the reference's known-answer tests (engine-core/tests/sdpa_cpu_tests.rs)
and an independent dense float64 attention written with numpy."""
import numpy as np
import pytest

from oracle import orc


def dense_attention(k, v, q, n_head, n_kv, hd, gqa=lambda qh, group, n_kv: qh // group):
    """Textbook softmax attention in float64 over dense K/V [T, n_kv, hd]."""
    group = n_head // n_kv
    out = np.zeros((n_head, hd))
    for qh in range(n_head):
        hk = gqa(qh, group, n_kv)
        s = (k[:, hk, :].astype(np.float64) @ q[qh].astype(np.float64)) / np.sqrt(hd)
        w = np.exp(s - s.max())
        w /= w.sum()
        out[qh] = w @ v[:, hk, :].astype(np.float64)
    return out


def dense_from_pool(pool, table, bt, n_tok, n_kv, hd):
    rl = n_kv * hd
    k = np.zeros((n_tok, n_kv, hd), np.float32)
    v = np.zeros((n_tok, n_kv, hd), np.float32)
    for t in range(n_tok):
        base = int(table[t // bt]) * bt * 2 * rl + (t % bt) * 2 * rl
        k[t] = pool[base:base + rl].reshape(n_kv, hd)
        v[t] = pool[base + rl:base + 2 * rl].reshape(n_kv, hd)
    return k, v


def test_sequential_blocks_match_hand_computed():
    # sdpa_cpu_tests.rs:89-175 (seed 0x55AA, q = [0.8, -0.4], tol 1e-5)
    bt, nb = 2, 2
    pool = np.zeros(nb * bt * 4, np.float32)
    orc.fill_pool_paged(pool, [0, 1], bt, 1, 2, 0x55AA, 3)
    q = np.array([0.8, -0.4], np.float32)
    got = orc.sdpa_decode(pool, [0, 1], bt, 3, q, 1, 1, 2, False, 3)
    k, v = dense_from_pool(pool, [0, 1], bt, 3, 1, 2)
    exp = dense_attention(k, v, q[None], 1, 1, 2)[0]
    assert np.max(np.abs(got - exp)) < 1e-5


def test_scattered_blocks_match_contiguous():
    # sdpa_cpu_tests.rs:180-277
    bt, n_head, n_kv, hd, seq = 2, 2, 1, 3, 7
    size = 4 * bt * 2 * n_kv * hd
    pc, ps = np.zeros(size, np.float32), np.zeros(size, np.float32)
    orc.fill_pool_paged(pc, [0, 1, 2, 3], bt, n_kv, hd, 0x12345678, seq)
    orc.fill_pool_paged(ps, [3, 0, 2, 1], bt, n_kv, hd, 0x12345678, seq)
    q = orc.xorshift_a(0xABCD, n_head * hd)
    a = orc.sdpa_decode(pc, [0, 1, 2, 3], bt, seq, q, n_head, n_kv, hd, False, seq)
    b = orc.sdpa_decode(ps, [3, 0, 2, 1], bt, seq, q, n_head, n_kv, hd, False, seq)
    assert np.array_equal(a, b)
    assert np.all(np.isfinite(a)) and np.linalg.norm(a) > 0


def test_causal_masks_upper_triangle():
    # sdpa_cpu_tests.rs:282-352
    pool = np.zeros(4 * 2 * 4, np.float32)
    orc.fill_pool_paged(pool, [0, 1, 2, 3], 2, 1, 2, 0xCAFE, 8)
    q = np.array([0.6, 0.9], np.float32)
    c = orc.sdpa_decode(pool, [0, 1, 2, 3], 2, 8, q, 1, 1, 2, True, 3)
    r = orc.sdpa_decode(pool, [0, 1, 2, 3], 2, 4, q, 1, 1, 2, False, 4)
    assert np.max(np.abs(c - r)) < 1e-5


def test_single_token_returns_value_row():
    pool = np.zeros(4 * 4 * 2 * 4, np.float32)
    orc.fill_pool_paged(pool, [3, 0, 2, 1], 4, 1, 4, 0x1234, 1)
    q = orc.xorshift_a(0x1234 ^ 0xF00D, 2 * 4)
    out = orc.sdpa_decode(pool, [3, 0, 2, 1], 4, 1, q, 2, 1, 4, False, 1)
    vrow = pool[3 * 4 * 8 + 4: 3 * 4 * 8 + 8]
    assert np.array_equal(out[:4], vrow) and np.array_equal(out[4:], vrow)


def test_zero_sizes_return_zeros():
    out = orc.sdpa_decode(np.zeros(8, np.float32), [0], 2, 0, np.ones(4, np.float32), 2, 1, 2,
                          False, 0)
    assert np.array_equal(out, np.zeros(4, np.float32))


@pytest.mark.parametrize("n_head,n_kv,hd,bt", [(4, 1, 64, 16), (8, 2, 32, 16), (4, 4, 16, 8),
                                              (2, 1, 8, 4), (14, 2, 64, 16), (12, 2, 128, 16)])
@pytest.mark.parametrize("causal", [False, True])
def test_matches_dense_float64(n_head, n_kv, hd, bt, causal):
    rng = np.random.default_rng(n_head * 1000 + hd)
    n_tok = 3 * bt + 3
    nb = (n_tok + bt - 1) // bt + 2
    table = rng.permutation(nb)[: (n_tok + bt - 1) // bt].astype(np.uint32)
    pool = rng.standard_normal(nb * bt * 2 * n_kv * hd).astype(np.float32)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    qp = n_tok - 4 if causal else n_tok
    got = orc.sdpa_decode(pool, table, bt, n_tok, q, n_head, n_kv, hd, causal, qp)
    used = qp + 1 if causal else n_tok
    k, v = dense_from_pool(pool, table, bt, used, n_kv, hd)
    exp = dense_attention(k, v, q.reshape(n_head, hd), n_head, n_kv, hd)
    assert np.max(np.abs(got.reshape(n_head, hd) - exp)) < 1e-6
    if n_kv > 1 and n_head // n_kv > 1:
        # A plausible mistake (interleaved instead of blocked GQA mapping)
        # planted in the independent model must be detected.
        wrong = dense_attention(k, v, q.reshape(n_head, hd), n_head, n_kv, hd,
                                gqa=lambda qh, group, nk: qh % nk)
        assert np.max(np.abs(got.reshape(n_head, hd) - wrong)) > 1e-3


def test_prefill_equals_per_query_decode_and_dense_causal():
    rng = np.random.default_rng(7)
    n_head, n_kv, hd, bt = 4, 2, 16, 4
    pos_offset, q_tokens = 9, 6
    total = pos_offset + q_tokens
    nb = (total + bt - 1) // bt
    table = rng.permutation(nb + 3)[:nb].astype(np.uint32)
    pool = rng.standard_normal((nb + 3) * bt * 2 * n_kv * hd).astype(np.float32)
    q = rng.standard_normal((q_tokens, n_head, hd)).astype(np.float32)
    out = orc.prefill_causal(pool, table, bt, q, q_tokens, pos_offset, n_head, n_kv, hd)
    for i in range(q_tokens):
        k, v = dense_from_pool(pool, table, bt, pos_offset + i + 1, n_kv, hd)
        exp = dense_attention(k, v, q[i], n_head, n_kv, hd)
        assert np.max(np.abs(out[i] - exp)) < 1e-6


def test_batched_driver_matches_single():
    rng = np.random.default_rng(3)
    n_head, n_kv, hd, bt = 6, 2, 32, 8
    lens = np.array([5, 17, 1, 0, 24], np.uint32)
    stride = 4
    nb = 32
    pool = rng.standard_normal(nb * bt * 2 * n_kv * hd).astype(np.float32)
    tab = rng.permutation(nb)[: len(lens) * stride].reshape(len(lens), stride).astype(np.uint32)
    q = rng.standard_normal((len(lens), n_head, hd)).astype(np.float32)
    out = orc.sdpa_decode_batched(pool, tab, lens, bt, q, n_head, n_kv, hd)
    for b, n in enumerate(lens):
        exp = orc.sdpa_decode(pool, tab[b], bt, int(n), q[b].ravel(), n_head, n_kv, hd, True,
                              max(int(n) - 1, 0))
        assert np.array_equal(out[b].ravel(), exp)
