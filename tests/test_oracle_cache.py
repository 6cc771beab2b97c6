"""Pins the oracle's PagedKvCache restatement against the reference's own
known-answer tests (engine-kvcache/src/cache.rs:258-472,
engine-cuda/tests/paged_kv_gpu.rs:64-141, paged_kv_parity.rs:68-225) and the
closed-form page layout."""
import numpy as np
import pytest

from oracle import orc


def test_create_pool_reports_blocks_total():
    # cache.rs:262-275
    c = orc.Cache(8, 16, 4, 6)
    assert c.blocks_total() == 8 and c.blocks_used() == 0
    assert c.row_len * 2 == 2 * 4 * 6


def test_append_single_token_reads_back_exact_floats():
    # cache.rs:278-302
    c = orc.Cache(8, 16, 2, 3)
    s = c.new_sequence()
    key = [1.5, -2.25, 0.5, 3.0, -4.0, 6.0]
    val = [4.0, 8.0, -16.0, 1.0, 2.0, 3.0]
    c.append(s, key, val)
    assert c.read_key(s, 0).tolist() == key
    assert c.read_value(s, 0).tolist() == val


def test_append_spanning_scattered_blocks():
    # cache.rs:305-370.  The reference comment expects seq_a's second page at
    # id 3, but seq_b's 4 tokens fill a single 4-token page, so the code
    # (which the reference test does not check for ids) yields [0, 2].
    c = orc.Cache(4, 4, 1, 2)
    a, b = c.new_sequence(), c.new_sequence()
    for k in range(4):
        c.append(a, [k, k * 10.0], [0, 0])
    for v in (9.0, 8.0, 7.0, 6.0):
        c.append(b, [v, v], [v, v])
    for t in range(4, 8):
        c.append(a, [t, t * 10.0], [0, 0])
    assert c.token_count(a) == 8
    assert c.seq_block_table(a).tolist() == [0, 2]
    assert c.seq_block_table(b).tolist() == [1]
    keys = c.read_keys(a)
    for t in range(8):
        assert keys[2 * t] == t and keys[2 * t + 1] == t * 10.0


def test_pool_exhaustion_returns_typed_error():
    # cache.rs:373-405
    c = orc.Cache(1, 2, 1, 2)
    s = c.new_sequence()
    c.append(s, [0.5, 1.5], [0.5, 1.5])
    c.append(s, [0.5, 1.5], [0.5, 1.5])
    with pytest.raises(orc.KvCacheError) as e:
        c.append(s, [0.5, 1.5], [0.5, 1.5])
    assert e.value.kind == "PoolExhausted"
    assert (e.value.blocks_used, e.value.blocks_total) == (1, 1)
    assert c.blocks_used() == 1 and c.token_count(s) == 2


def test_free_then_realloc_succeeds():
    # cache.rs:408-444
    c = orc.Cache(2, 2, 1, 2)
    s = c.new_sequence()
    for _ in range(4):
        c.append(s, [1.0, 2.0], [1.0, 2.0])
    with pytest.raises(orc.KvCacheError):
        c.append(s, [1.0, 2.0], [1.0, 2.0])
    first = c.seq_block_table(s).tolist()
    c.free_sequence(s)
    assert c.blocks_used() == 0 and c.token_count(s) == 0
    for _ in range(3):
        c.append(s, [1.0, 2.0], [1.0, 2.0])
    assert c.token_count(s) == 3 and c.blocks_used() == 2
    # cache.rs:131: freed pages are reused in their original order.
    assert c.seq_block_table(s).tolist() == first
    assert c.read_keys(s).size == 6


def test_budget_capacity_matches_config_total():
    # cache.rs:447-472
    c = orc.Cache(3, 4, 2, 3)
    a, b = c.new_sequence(), c.new_sequence()
    row = [0.1] * 6
    while c.blocks_used() < c.blocks_total():
        c.append(a, row, row)
        assert c.blocks_used() <= c.blocks_total()
    with pytest.raises(orc.KvCacheError) as e:
        c.append(b, row, row)
    assert e.value.kind == "PoolExhausted"


@pytest.mark.parametrize("args,msg", [
    ((0, 16, 1, 1), "n_blocks must be non-zero"),
    ((1, 0, 1, 1), "block_tokens must be non-zero"),
    ((1, 1, 0, 1), "heads and head_dim must be non-zero"),
    ((1, 1, 1, 0), "heads and head_dim must be non-zero"),
])
def test_invalid_config(args, msg):
    # cache.rs:65-76
    with pytest.raises(orc.KvCacheError) as e:
        orc.Cache(*args)
    assert e.value.kind == "InvalidArgs" and e.value.msg == msg


def test_invalid_append_and_read():
    c = orc.Cache(2, 2, 1, 2)
    s = c.new_sequence()
    with pytest.raises(orc.KvCacheError) as e:
        c.append(s, [1.0], [1.0, 2.0])
    assert e.value.msg == "key/value length must equal heads * head_dim"
    with pytest.raises(orc.KvCacheError) as e:
        c.append(7, [1.0, 2.0], [1.0, 2.0])
    assert e.value.msg == "unknown sequence id"
    with pytest.raises(orc.KvCacheError) as e:
        c.read_key(s, 0)
    assert e.value.msg == "token out of range"


def test_closed_form_layout_and_gather_identity():
    """Page bytes follow b*fpb + s*fpt (+row_len for V) exactly, and
    read_all(append(x)) == x, on the paged_kv_parity.rs scenario."""
    heads, hd, bt, nb = 2, 8, 6, 9
    rl = heads * hd
    c = orc.Cache(nb, bt, heads, hd)
    a, b = c.new_sequence(), c.new_sequence()
    ka, va = orc.generate_rows_b(0xDEADBEEF, 5 * bt, rl)
    for t in range(5 * bt):
        c.append(a, ka[t * rl:(t + 1) * rl], va[t * rl:(t + 1) * rl])
    nb_tok = 3 * bt + 4
    kb, vb = orc.generate_rows_b(0x12345678, nb_tok, rl)
    for t in range(nb_tok):
        c.append(b, kb[t * rl:(t + 1) * rl], vb[t * rl:(t + 1) * rl])
    table = c.seq_block_table(b).tolist()
    assert table == [5, 6, 7, 8]   # seq_b after seq_a took pages 0-4
    assert np.array_equal(c.read_keys(b), kb) and np.array_equal(c.read_values(b), vb)
    buf = c.buffer()
    fpt, fpb = 2 * rl, bt * 2 * rl
    for t in range(nb_tok):
        base = table[t // bt] * fpb + (t % bt) * fpt
        assert np.array_equal(buf[base:base + rl], kb[t * rl:(t + 1) * rl])
        assert np.array_equal(buf[base + rl:base + 2 * rl], vb[t * rl:(t + 1) * rl])


def test_seeded_free_list_order():
    c = orc.Cache(6, 2, 1, 2)
    c.seed_free_list([4, 1, 5, 0, 3, 2])
    s = c.new_sequence()
    for _ in range(5):
        c.append(s, [1.0, 2.0], [3.0, 4.0])
    assert c.seq_block_table(s).tolist() == [4, 1, 5]
    assert c.blocks_used() == 3


def test_f16_elements_copied_verbatim():
    c = orc.Cache(4, 4, 1, 4, dtype=np.float16)
    s = c.new_sequence()
    k = np.array([1.0, -0.0, 65504.0, 6e-8], dtype=np.float16)
    v = np.array([np.inf, -2.5, 0.1, 3.0], dtype=np.float16)
    c.append(s, k, v)
    assert c.read_key(s, 0).view(np.uint16).tolist() == k.view(np.uint16).tolist()
    assert c.read_value(s, 0).view(np.uint16).tolist() == v.view(np.uint16).tolist()


def test_xorshift_generators_known_values():
    # xorshift32 from state 1 produces 270369 first (13/17/5 shifts).
    a = orc.xorshift_a(1, 1)
    assert a[0] == np.float32(270369 / 2 ** 32 * 2 - 1)
    k, v = orc.generate_rows_b(1, 1, 1)
    assert k[0] == np.float32((270369 & 0xFFFFFF) / 2 ** 23 - 1)
    # seed 0 maps to 0x6D2B79F5 for generator A (tests/common/mod.rs:19-21).
    assert np.array_equal(orc.xorshift_a(0, 8), orc.xorshift_a(0x6D2B79F5, 8))
