"""Pins the CPU oracle (oracle/attention.py) against facts that do not come from it.

Independent sources used here:
* the paged layout is built from *logical* per-sequence K/V with the
  engine's block-slice cache write (a page of 16 consecutive tokens per table
  entry, femtovllm/models/qwen/qwen3.py:322-366), not with the oracle's
  per-key index map;
* torch's ``scaled_dot_product_attention`` on the logical K/V (a library
  routine) and a pure-Python triple loop (oracle/brute.py);
* closed forms: kv_len == 1 returns the V row; q == 0 returns the mean of
  the visible V rows; a dominant "spike" key returns its V row;
* invariants: a permutation of the physical blocks changes nothing.

The ``planted`` tests swap one decision of the oracle for a plausible
mistake and show that one of these checks fails.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle.attention as oa
from oracle import brute, sdpa_path

PAGE = 16


# ---------------------------------------------------------------------------
# Construction helpers (independent of the oracle's gather).
# ---------------------------------------------------------------------------


def write_pages(pool, table, logical):
    """Block-slice cache write: page i of the table receives tokens [16i, 16i+16)."""
    length = logical.shape[1]
    for i, blk in enumerate(table):
        lo, hi = i * PAGE, min(length, (i + 1) * PAGE)
        if lo >= hi:
            break
        pool[blk, :, : hi - lo] = logical[:, lo:hi]


def build_paged(rng, kv_lens, n_kv, dim, num_blocks, gen=None):
    """Random logical K/V per sequence placed through random block tables.

    Returns pools (NaN where unused), -1 padded tables, logical K and V lists.
    """
    gen = gen or (lambda shape: rng.standard_normal(shape))
    perm = [int(x) for x in rng.permutation(num_blocks)]
    k_pool = np.full((num_blocks, n_kv, PAGE, dim), np.nan)
    v_pool = np.full((num_blocks, n_kv, PAGE, dim), np.nan)
    tables, ks, vs, cursor = [], [], [], 0
    for L in kv_lens:
        npages = -(-L // PAGE)
        t = perm[cursor : cursor + npages]
        cursor += npages
        k, v = gen((n_kv, L, dim)), gen((n_kv, L, dim))
        write_pages(k_pool, t, k)
        write_pages(v_pool, t, v)
        tables.append(t)
        ks.append(k)
        vs.append(v)
    width = max(len(t) for t in tables)
    padded = np.array([t + [-1] * (width - len(t)) for t in tables], dtype=np.int64)
    return k_pool, v_pool, padded, ks, vs


def chunk_positions(kv_lens, q_lens):
    cu, pos = [0], []
    for L, n in zip(kv_lens, q_lens):
        pos.extend(range(L - n, L))
        cu.append(cu[-1] + n)
    return cu, np.array(pos)


def sdpa_logical(q_rows, k, v, positions, n_rep):
    """torch SDPA (float64) on logical K/V with the mask j <= position."""
    L = k.shape[1]
    qt = torch.from_numpy(q_rows)  # (H, n, D)
    kt = torch.from_numpy(k).repeat_interleave(n_rep, dim=0)
    vt = torch.from_numpy(v).repeat_interleave(n_rep, dim=0)
    mask = torch.arange(L)[None, :] <= torch.from_numpy(np.asarray(positions))[:, None]
    return F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask).numpy()


# ---------------------------------------------------------------------------
# Checks (plain functions so the planted tests can reuse them).
# ---------------------------------------------------------------------------


def check_prefill_vs_sdpa(seed=0):
    rng = np.random.default_rng(seed)
    H, KVH, D = 8, 4, 32
    kv_lens, q_lens = [59, 44, 16, 1], [8, 16, 16, 1]
    k_pool, v_pool, tables, ks, vs = build_paged(rng, kv_lens, KVH, D, 24)
    cu, pos = chunk_positions(kv_lens, q_lens)
    q = rng.standard_normal((H, cu[-1], D))
    got = oa.paged_prefill(q, k_pool, v_pool, cu, tables, kv_lens, pos)
    for b in range(len(kv_lens)):
        lo, hi = cu[b], cu[b + 1]
        want = sdpa_logical(q[:, lo:hi], ks[b], vs[b], pos[lo:hi], H // KVH)
        np.testing.assert_allclose(got[:, lo:hi], want, rtol=0, atol=1e-12)


def check_decode_vs_sdpa(seed=1):
    rng = np.random.default_rng(seed)
    H, KVH, D = 16, 8, 16
    kv_lens = [17, 64, 200, 511]
    k_pool, v_pool, tables, ks, vs = build_paged(rng, kv_lens, KVH, D, 64)
    q = rng.standard_normal((H, len(kv_lens), D))
    got = oa.paged_decode(q, k_pool, v_pool, tables, kv_lens)
    for b, L in enumerate(kv_lens):
        want = sdpa_logical(q[:, b : b + 1], ks[b], vs[b], [L - 1], H // KVH)
        np.testing.assert_allclose(got[:, b : b + 1], want, rtol=0, atol=1e-12)


def check_gather_spike_scan():
    """A dominant key at every logical index j* must return V[j*] (decode)."""
    rng = np.random.default_rng(2)
    D, KVH, H = 8, 2, 2
    L = 53
    for jstar in range(L):
        def gen(shape, _c=[0]):
            return np.zeros(shape)
        k_pool, v_pool, tables, ks, vs = build_paged(rng, [L], KVH, D, 8, gen=gen)
        k_log = np.zeros((KVH, L, D))
        k_log[:, jstar, 0] = 1.0
        v_log = rng.standard_normal((KVH, L, D))
        write_pages(k_pool, [int(t) for t in tables[0] if t >= 0], k_log)
        write_pages(v_pool, [int(t) for t in tables[0] if t >= 0], v_log)
        q = np.zeros((H, 1, D))
        q[:, 0, 0] = 400.0 * math.sqrt(D)
        out = oa.paged_decode(q, k_pool, v_pool, tables, [L])
        for h in range(H):
            np.testing.assert_allclose(out[h, 0], v_log[h, jstar], rtol=0, atol=1e-12)


def check_causal_boundary():
    """Spike at j = position must be seen; spike at position + 1 must not."""
    rng = np.random.default_rng(3)
    D, KVH, H = 8, 1, 1
    L, n = 40, 12
    cu, pos = chunk_positions([L], [n])
    for i in range(n):
        p = int(pos[i])
        for jstar, seen in ((p, True), (p + 1, False)):
            if jstar >= L:
                continue
            k_pool, v_pool, tables, _, _ = build_paged(rng, [L], KVH, D, 4, gen=np.zeros)
            k_log = np.zeros((KVH, L, D))
            k_log[0, jstar, 0] = 1.0
            v_log = rng.standard_normal((KVH, L, D))
            t = [int(x) for x in tables[0] if x >= 0]
            write_pages(k_pool, t, k_log)
            write_pages(v_pool, t, v_log)
            q = np.zeros((H, n, D))
            q[0, i, 0] = 400.0 * math.sqrt(D)
            out = oa.paged_prefill(q, k_pool, v_pool, cu, tables, [L], pos, rows=[i])
            want = v_log[0, jstar] if seen else v_log[0, : p + 1].mean(axis=0)
            np.testing.assert_allclose(out[0, i], want, rtol=0, atol=1e-12)


def check_gqa_mapping():
    """Query heads 0..n_rep-1 read kv head 0, the next n_rep read kv head 1, ..."""
    rng = np.random.default_rng(4)
    D, KVH, H, L = 8, 2, 4, 20
    k_pool, v_pool, tables, _, _ = build_paged(rng, [L], KVH, D, 4, gen=np.zeros)
    k_log = np.zeros((KVH, L, D))
    k_log[0, 3, 0] = 1.0
    k_log[1, 11, 0] = 1.0
    v_log = rng.standard_normal((KVH, L, D))
    t = [int(x) for x in tables[0] if x >= 0]
    write_pages(k_pool, t, k_log)
    write_pages(v_pool, t, v_log)
    q = np.zeros((H, 1, D))
    q[:, 0, 0] = 400.0 * math.sqrt(D)
    out = oa.paged_decode(q, k_pool, v_pool, tables, [L])
    for h in range(H):
        g = h // (H // KVH)
        want = v_log[0, 3] if g == 0 else v_log[1, 11]
        np.testing.assert_allclose(out[h, 0], want, rtol=0, atol=1e-12)


def check_brute_force():
    rng = np.random.default_rng(5)
    H, KVH, D = 4, 2, 6
    kv_lens, q_lens = [21, 7], [5, 7]
    k_pool, v_pool, tables, _, _ = build_paged(rng, kv_lens, KVH, D, 6)
    cu, pos = chunk_positions(kv_lens, q_lens)
    q = rng.standard_normal((H, cu[-1], D))
    got = oa.paged_prefill(q, k_pool, v_pool, cu, tables, kv_lens, pos)
    want = brute.paged_prefill(q.tolist(), np.nan_to_num(k_pool).tolist(), np.nan_to_num(v_pool).tolist(),
                               cu, tables.tolist(), kv_lens, pos.tolist())
    np.testing.assert_allclose(got, np.array(want), rtol=0, atol=1e-12)


# ---------------------------------------------------------------------------
# The oracle passes every check.
# ---------------------------------------------------------------------------


def test_prefill_matches_torch_sdpa():
    check_prefill_vs_sdpa()


def test_decode_matches_torch_sdpa():
    check_decode_vs_sdpa()


def test_gather_spike_scan_every_logical_index():
    check_gather_spike_scan()


def test_causal_boundary_is_inclusive():
    check_causal_boundary()


def test_gqa_consecutive_replication():
    check_gqa_mapping()


def test_prefill_matches_brute_force():
    check_brute_force()


def test_kv_len_one_returns_v_row():
    rng = np.random.default_rng(6)
    k_pool, v_pool, tables, ks, vs = build_paged(rng, [1, 1], 2, 16, 4)
    q = rng.standard_normal((4, 2, 16))
    out = oa.paged_decode(q, k_pool, v_pool, tables, [1, 1])
    for b in range(2):
        for h in range(4):
            assert np.array_equal(out[h, b], vs[b][h // 2, 0])


def test_zero_query_is_mean_of_visible_rows():
    rng = np.random.default_rng(7)
    kv_lens, q_lens = [45], [13]
    k_pool, v_pool, tables, ks, vs = build_paged(rng, kv_lens, 1, 8, 4)
    cu, pos = chunk_positions(kv_lens, q_lens)
    q = np.zeros((2, cu[-1], 8))
    out = oa.paged_prefill(q, k_pool, v_pool, cu, tables, kv_lens, pos)
    for i, p in enumerate(pos):
        np.testing.assert_allclose(out[:, i], np.broadcast_to(vs[0][0, : p + 1].mean(0), (2, 8)), atol=1e-13)


def test_block_permutation_invariance():
    rng = np.random.default_rng(8)
    kv_lens, q_lens = [37, 50], [5, 9]
    k_pool, v_pool, tables, _, _ = build_paged(rng, kv_lens, 2, 8, 10)
    cu, pos = chunk_positions(kv_lens, q_lens)
    q = rng.standard_normal((4, cu[-1], 8))
    base = oa.paged_prefill(q, k_pool, v_pool, cu, tables, kv_lens, pos)
    perm = rng.permutation(10)
    inv = np.argsort(perm)
    t2 = np.where(tables >= 0, inv[np.maximum(tables, 0)], -1)
    got = oa.paged_prefill(q, k_pool[perm], v_pool[perm], cu, t2, kv_lens, pos)
    assert np.array_equal(base, got)


def test_edge_conventions():
    rng = np.random.default_rng(9)
    k_pool, v_pool, tables, _, _ = build_paged(rng, [5], 1, 8, 2)
    # decode with an empty context returns zeros (the GEMV's untouched accumulator)
    q = rng.standard_normal((2, 2, 8))
    out = oa.paged_decode(q, k_pool, v_pool, np.vstack([tables, tables]), [5, 0])
    assert np.all(out[:, 1] == 0)
    # prefill with kv_len == 0 is 0 / 0 = NaN
    out = oa.paged_prefill(q[:, :1], k_pool, v_pool, [0, 1], tables, [0], [0])
    assert np.all(np.isnan(out))


def test_sdpa_path_restatement_matches_oracle():
    """The torch restatement of the reference CPU path agrees with the oracle."""
    rng = np.random.default_rng(10)
    kv_lens, q_lens = [59, 44], [8, 16]
    k_pool, v_pool, tables, _, _ = build_paged(rng, kv_lens, 4, 32, 12)
    cu, pos = chunk_positions(kv_lens, q_lens)
    q = rng.standard_normal((8, cu[-1], 32))
    want = oa.paged_prefill(q, k_pool, v_pool, cu, tables, kv_lens, pos)
    got = sdpa_path.paged_prefill(torch.from_numpy(q), torch.from_numpy(k_pool), torch.from_numpy(v_pool), cu,
                                  tables.tolist(), kv_lens, torch.from_numpy(pos))
    np.testing.assert_allclose(got.numpy(), want, atol=1e-12)


def test_dense_matches_torch_sdpa():
    rng = np.random.default_rng(11)
    q = rng.standard_normal((2, 4, 9, 16))
    k = rng.standard_normal((2, 2, 13, 16))
    v = rng.standard_normal((2, 2, 13, 16))
    got = oa.dense_attention(q, k, v)
    want = F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k).repeat_interleave(2, 1),
                                          torch.from_numpy(v).repeat_interleave(2, 1)).numpy()
    np.testing.assert_allclose(got, want, atol=1e-12)


def test_cache_write_matches_block_slice_write():
    rng = np.random.default_rng(12)
    kv_lens, q_lens = [37, 20], [14, 20]
    k_pool, v_pool, tables, ks, vs = build_paged(rng, kv_lens, 2, 8, 8)
    cu, pos = chunk_positions(kv_lens, q_lens)
    k_new = np.concatenate([ks[b][:, -n:].transpose(1, 0, 2) for b, n in enumerate(q_lens)])
    v_new = np.concatenate([vs[b][:, -n:].transpose(1, 0, 2) for b, n in enumerate(q_lens)])
    blank_k = k_pool.copy()
    blank_v = v_pool.copy()
    for b, (L, n) in enumerate(zip(kv_lens, q_lens)):
        for blk in tables[b]:
            if blk >= 0:
                blank_k[blk] = np.nan
                blank_v[blk] = np.nan
        t = [int(x) for x in tables[b] if x >= 0]
        write_pages(blank_k, t, ks[b][:, : L - n])
        write_pages(blank_v, t, vs[b][:, : L - n])
    got_k, got_v = oa.cache_write(blank_k, blank_v, k_new, v_new, tables, cu, pos)
    np.testing.assert_array_equal(np.nan_to_num(got_k, nan=-7), np.nan_to_num(k_pool, nan=-7))
    np.testing.assert_array_equal(np.nan_to_num(got_v, nan=-7), np.nan_to_num(v_pool, nan=-7))


def _written(pool):
    """{(block, row): value} of the non-zero entries of a (NB, 1, 16, 1) pool."""
    return {(int(b), int(r)): int(pool[b, 0, r, 0]) for b, _, r, _ in zip(*np.nonzero(pool))}


@pytest.mark.parametrize("case", ["stop_at_minus_one", "past_table_width", "block_outside_pool",
                                  "first_position_rules", "decode_layout", "shared_block_rewrite"])
def test_cache_write_known_answers(case):
    """Hand-computed placements of the reference loop (qwen3.py:322-366, 240-264).

    Values are token ids + 1 in a (6 blocks, 1 head, 16 rows, 1 dim) pool.
    """
    nb = 6
    if case == "stop_at_minus_one":      # p0 = 14: rows 14, 15 of block 3, then column 1 is -1
        tables, cu, pos, n = [[3, -1, 5]], [0, 5], [14, 15, 16, 17, 18], 5
        want = {(3, 14): 1, (3, 15): 2}
    elif case == "past_table_width":     # p0 = 30: block 4 rows 14-15, block 0 rows 0-15, column 3 missing
        tables, cu, pos, n = [[2, 4, 0]], [0, 20], list(range(30, 50)), 20
        want = {(4, 14): 1, (4, 15): 2, **{(0, r): r + 3 for r in range(16)}}
    elif case == "block_outside_pool":   # column 1 holds 99 >= 6 blocks: the walk stops there
        tables, cu, pos, n = [[1, 99]], [0, 3], [15, 16, 17], 3
        want = {(1, 15): 1}
    elif case == "first_position_rules":  # tokens follow positions[q_begin], not their own positions
        tables, cu, pos, n = [[5]], [0, 3], [5, 40, 2], 3
        want = {(5, 5): 1, (5, 6): 2, (5, 7): 3}
    elif case == "decode_layout":        # cu_seqlens=None: token b at positions[b]
        tables, cu, pos, n = [[1, 2], [3, -1]], None, [17, 0], 2
        want = {(2, 1): 1, (3, 0): 2}
    else:                                # two sequences share block 2; both write row 4 of it
        tables, cu, pos, n = [[2, 1], [2, 3]], [0, 2, 3], [3, 4, 4], 3
        want = {(2, 3): 1, (2, 4): 3}    # the later sequence's token lands last
    k_new = (np.arange(n, dtype=np.float64) + 1).reshape(n, 1, 1)
    blank = np.zeros((nb, 1, 16, 1))
    got_k, got_v = oa.cache_write(blank, blank, k_new, k_new, tables, cu, pos)
    assert _written(got_k) == want
    assert _written(got_v) == want


# ---------------------------------------------------------------------------
# Planted mistakes in the oracle are caught.
# ---------------------------------------------------------------------------


def test_planted_wrong_gqa_map_is_caught(monkeypatch):
    monkeypatch.setattr(oa, "kv_head_of", lambda h, n_heads, n_kv: h % n_kv)
    with pytest.raises(AssertionError):
        check_gqa_mapping()


def test_planted_strict_causal_is_caught(monkeypatch):
    monkeypatch.setattr(oa, "visible", lambda j, kv_len, pos: (j < kv_len) & (j < pos))
    with pytest.raises(AssertionError):
        check_causal_boundary()


def test_planted_shifted_page_row_is_caught(monkeypatch):
    monkeypatch.setattr(oa, "page_slot", lambda j, ps=16: (j // ps, (j + 1) % ps))
    with pytest.raises(AssertionError):
        check_gather_spike_scan()


def test_planted_page_index_without_table_is_caught(monkeypatch):
    # reading logical page j // 16 as if it were the physical block
    real = oa.gather_seq_kv

    def no_table(pool, table_row, kv_len):
        return real(pool, list(range(len([p for p in table_row if p >= 0]))), kv_len)

    monkeypatch.setattr(oa, "gather_seq_kv", no_table)
    with pytest.raises(AssertionError):
        check_decode_vs_sdpa()


def test_planted_missing_scale_is_caught(monkeypatch):
    monkeypatch.setattr(oa, "softmax_scale", lambda dim: 1.0)
    with pytest.raises(AssertionError):
        check_prefill_vs_sdpa()


def test_planted_wrong_row_in_cache_write_is_caught(monkeypatch):
    monkeypatch.setattr(oa, "page_slot", lambda j, page_size=16: (j // page_size, (j + 1) % page_size))
    with pytest.raises(AssertionError):
        test_cache_write_known_answers("past_table_width")


# ---------------------------------------------------------------------------
# Prologue oracle (RMSNorm + RoPE), pinned by torch and by the complex form.
# ---------------------------------------------------------------------------


def test_rms_norm_matches_torch():
    import oracle.prologue as op
    rng = np.random.default_rng(41)
    x = rng.standard_normal((7, 3, 128)) * 3
    w = rng.standard_normal(128)
    got = op.rms_norm(x, w, 1e-6)
    want = F.rms_norm(torch.from_numpy(x), (128,), torch.from_numpy(w), 1e-6).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_rope_is_a_complex_rotation():
    """RoPE pairs (x_i, x_{i+64}) and rotates them by theta_i = p * base**(-2i/D): as complex numbers,
    (x_i + j x_{i+64}) * exp(j theta_i).  Checked against that form, with the tables' own theta."""
    import oracle.prologue as op
    rng = np.random.default_rng(42)
    T, Hh, D = 9, 2, 128
    x = rng.standard_normal((T, Hh, D))
    pos = rng.integers(0, 5000, size=T)
    cos, sin = op.rope_tables(6000, D)
    got = op.rope(x, cos, sin, pos)
    inv = (1.0 / 1000000.0) ** (2.0 * np.arange(D // 2) / D)
    theta = pos[:, None] * inv[None, :]
    z = (x[..., :64] + 1j * x[..., 64:]) * np.exp(1j * theta)[:, None, :]
    want = np.concatenate([z.real, z.imag], axis=-1)
    np.testing.assert_allclose(got, want, atol=5e-3)  # float32 tables vs float64 angles
    np.testing.assert_allclose(op.rope(x, cos, sin, np.zeros(T, dtype=np.int64)), x, atol=0)  # position 0
    pair_norm = lambda a: a[..., :64] ** 2 + a[..., 64:] ** 2
    np.testing.assert_allclose(pair_norm(got), pair_norm(x), rtol=1e-6)


def test_planted_wrong_rope_half_is_caught(monkeypatch):
    import oracle.prologue as op

    def bad_rope(x, cos, sin, positions):  # rotates the wrong way (sign of the swapped half)
        x = np.asarray(x, dtype=np.float64)
        rot = np.concatenate([x[..., 64:], -x[..., :64]], axis=-1)
        pos = np.asarray(positions)
        return np.asarray(cos, dtype=np.float64)[pos][:, None, :] * x + np.asarray(sin, dtype=np.float64)[pos][:, None, :] * rot

    monkeypatch.setattr(op, "rope", bad_rope)
    with pytest.raises(AssertionError):
        test_rope_is_a_complex_rotation()


def test_rope_tables_match_float64_angles():
    """femtovllm.rope.rope_tables (torch, the operator's callers) and the oracle's numpy tables both
    follow theta = p * base**(-2i/D) (qwen3.py:35-52): checked against float64 angles, within the
    float32 angle error (~4e-7 * p) that both constructions carry."""
    import oracle.prologue as op
    from femtovllm.rope import rope_tables
    P, D = 4096, 128
    inv = (1.0 / 1000000.0) ** (2.0 * np.arange(D // 2) / D)
    theta = np.arange(P)[:, None] * inv[None, :]
    theta = np.concatenate([theta, theta], axis=1)
    bound = 1e-6 + 4e-7 * np.arange(P)[:, None]
    for cos, sin in (tuple(t.numpy() for t in rope_tables(P, D)), op.rope_tables(P, D)):
        assert np.all(np.abs(cos - np.cos(theta)) <= bound)
        assert np.all(np.abs(sin - np.sin(theta)) <= bound)


def test_sdpa_path_decode_matches_oracle():
    """The torch restatement of the reference CPU decode path agrees with the oracle."""
    rng = np.random.default_rng(12)
    kv_lens = [17, 64, 200, 1]
    k_pool, v_pool, tables, _, _ = build_paged(rng, kv_lens, 4, 32, 24)
    q = rng.standard_normal((8, len(kv_lens), 32))
    want = oa.paged_decode(q, k_pool, v_pool, tables, kv_lens)
    got = sdpa_path.paged_decode(torch.from_numpy(q), torch.from_numpy(k_pool), torch.from_numpy(v_pool),
                                 tables.tolist(), kv_lens)
    np.testing.assert_allclose(got.numpy(), want, atol=1e-12)


def test_sdpa_path_dense_matches_oracle():
    """The torch restatement of the dense entry (GQA, non-causal) agrees with the oracle."""
    rng = np.random.default_rng(13)
    q = rng.standard_normal((2, 8, 9, 16))
    k = rng.standard_normal((2, 2, 13, 16))
    v = rng.standard_normal((2, 2, 13, 16))
    got = sdpa_path.dense_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v))
    np.testing.assert_allclose(got.numpy(), oa.dense_attention(q, k, v), atol=1e-12)


def test_row_bound_has_power_at_131072_keys():
    """At 131,072 keys the outputs are small (RMS ~ 1/sqrt(keys)), so max-abs 1e-2
    alone accepts an answer scaled by 0.9 (or 0.5); the per-row scale-aware bound
    of the parity helper rejects it, and accepts the bf16 rounding of the answer."""
    from femtovllm import workloads
    from helpers import assert_close, np32, np64, np_tables

    L = 131072
    w = workloads.make_paged_workload("row_bound", [(L - 1, 1)], 4, 1, seed=31)
    q, meta = w.gemv_call()
    want = oa.paged_decode(np64(q), np32(w.k_pool), np32(w.v_pool), np_tables(meta), meta.kv_lens.tolist())
    assert np.abs(want).max() < 0.05  # the regime where max-abs 1e-2 is weak
    rounded = torch.from_numpy(want).to(torch.bfloat16)
    assert_close(rounded, want, torch.bfloat16, "bf16 rounding of the oracle")
    for factor in (0.9, 0.5):
        scaled = torch.from_numpy(want * factor).to(torch.bfloat16)
        assert np.abs(np64(scaled) - want).max() <= 1e-2  # max-abs alone would pass
        with pytest.raises(AssertionError, match="per-row bound"):
            assert_close(scaled, want, torch.bfloat16, f"oracle x {factor}")


def test_agree_allows_the_sum_of_two_bounds():
    """Two results 0.9 of a row bound from the exact value on opposite sides each pass
    assert_close and pass assert_agree (1.8 bounds apart); results 1.1 bounds from it on
    opposite sides (2.2 apart) fail both."""
    from helpers import assert_agree, assert_close, row_bound

    rng = np.random.default_rng(5)
    want = rng.standard_normal((4, 64, 128)) * 0.01
    rb = row_bound(want, torch.float32)
    for k, ok in ((0.9, True), (1.1, False)):
        a, b = want + k * rb, want - k * rb
        if ok:
            assert_close(a, want, torch.float32, "a")
            assert_close(b, want, torch.float32, "b")
            assert_agree(a, b, torch.float32, "a vs b")
        else:
            with pytest.raises(AssertionError):
                assert_close(a, want, torch.float32, "a")
            with pytest.raises(AssertionError, match="per-row bound"):
                assert_agree(a, b, torch.float32, "a vs b")


# ---------------------------------------------------------------------------
# The reference kernel's own precision (oracle/ref_arith.py) and the max-abs
# bound of the parity helper.
# ---------------------------------------------------------------------------


def _bf16_values(rng, shape, sigma=1.0):
    """Random values that are exact bf16 numbers, as float32."""
    from oracle.ref_arith import bf16_round

    return bf16_round(rng.standard_normal(shape) * sigma)


def test_ref_arith_equal_scores_give_the_rounded_mean():
    """q == 0: every weight is exp(0) = 1 (exact in bf16), so the reference's
    arithmetic returns the bf16 rounding of the exact mean of the V rows
    (2 and 4 keys: sums and the division are exact in fp32)."""
    from oracle.ref_arith import bf16_round, prefill_row_bf16

    rng = np.random.default_rng(5)
    for L in (1, 2, 4):
        k = _bf16_values(rng, (L, 128))
        v = _bf16_values(rng, (L, 128), 3.0)
        got = prefill_row_bf16(np.zeros(128, np.float32), k, v, oa.softmax_scale(128))
        want = bf16_round(v.astype(np.float64).mean(axis=0))
        assert np.array_equal(got, want)


def test_ref_arith_needs_the_output_rounding_allowance():
    """The reference's arithmetic (fp32 softmax, weights cast to bf16 before
    P.V, bf16 output) on rows of a few visible keys with outputs of magnitude
    2-8: against the float64 oracle it exceeds a plain max-abs 1e-2 on some
    rows (the bf16 grid there is 2^-6 to 2^-5 wide), and it always stays
    within 1e-2 plus half a bf16 ulp of the exact value, the bound the parity
    helper uses."""
    from helpers import half_ulp
    from oracle.ref_arith import prefill_row_bf16

    rng = np.random.default_rng(11)
    scale = oa.softmax_scale(128)
    over, worst_excess = 0, 0.0
    for _ in range(3000):
        L = int(rng.integers(1, 4))
        q = _bf16_values(rng, (128,))
        k = _bf16_values(rng, (L, 128))
        v = _bf16_values(rng, (L, 128), 3.0)
        got = prefill_row_bf16(q, k, v, scale).astype(np.float64)
        want = oa._softmax_attend(q[None].astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                                  np.ones((1, L), bool), scale)[0]
        err = np.abs(got - want)
        over += int(np.any(err > 1e-2))
        worst_excess = max(worst_excess, float((err - 1e-2 - half_ulp(np.abs(want), torch.bfloat16)).max()))
    assert over > 0
    assert worst_excess <= 0.0
