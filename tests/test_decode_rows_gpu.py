"""Decode rows of a varlen prefill call run on the decode kernel.

femto_paged_attention_gemm hands every sequence of exactly one query token
to the decode kernel's wave workers (when its sizes allow such sequences and
a workspace is given) and the MFMA kernel skips them.  The result must be
the one the reference's single CUSTOM_GEMM call gives
(femtovllm/models/qwen/qwen3.py:575-580 -> paged_attention_gemm): token t of
sequence b sees keys j < kv_lens[b] with j <= positions[t], and a row with
no visible key is NaN.  Every row is checked against the oracle, with the
routing on, with it off (no workspace) and with a max_q_len that rules
decode rows out.
"""

import numpy as np
import pytest
import torch

import oracle.attention as oa
from femtovllm import workloads
from helpers import assert_close, np32, np64, np_tables

pytestmark = pytest.mark.gpu


def _gemm(ops, q, meta, wd, gpu, max_q_len=None, kv_lens=None, positions=None):
    out = ops.paged_attention_gemm(
        q.to(gpu), wd.k_pool, wd.v_pool, meta.cu_seqlens, meta.max_q_len if max_q_len is None else max_q_len,
        meta.Q_TILE_SIZE, meta.cu_q_tiles, meta.q_tile_to_seq_idx, meta.block_tables,
        meta.kv_lens if kv_lens is None else kv_lens, meta.positions if positions is None else positions,
    )
    torch.cuda.synchronize()
    return out


def _oracle(q, meta, w, kv_lens, positions):
    return oa.paged_prefill(np64(q), np32(w.k_pool), np32(w.v_pool), meta.raw_cu_seqlens, np_tables(meta),
                            list(kv_lens), np.asarray(positions))


def _no_workspace(monkeypatch):
    from femtovllm import _C

    monkeypatch.setattr(_C, "_prefill_workspace", lambda *args: (None, 0))


# (cached prefix, new tokens): one-token sequences between prefill chunks,
# an empty sequence, a one-token sequence with no prefix (kv_len 1), long
# and page-aligned contexts.
CHUNKS = [(100, 1), (0, 1), (500, 40), (37, 1), (2000, 1), (20, 0), (15, 1), (255, 1), (64, 70), (4095, 1)]


@pytest.fixture(scope="module")
def batch(gpu):
    w = workloads.make_paged_workload("decode_rows", CHUNKS, 32, 8, seed=31)
    q, meta = w.gemm_call(device=gpu)
    return w, w.to(gpu), q, meta


@pytest.mark.parametrize("routed", [True, False], ids=["routed", "no_workspace"])
def test_mixed_rows_match_oracle(ops, gpu, batch, routed, monkeypatch):
    w, wd, q, meta = batch
    if not routed:
        _no_workspace(monkeypatch)
    out = _gemm(ops, q, meta, wd, gpu)
    want = _oracle(q, meta, w, meta.kv_lens.tolist(), meta.raw_positions)
    assert_close(out, want, torch.bfloat16, f"mixed rows ({'routed' if routed else 'MFMA only'})")


def test_decode_row_positions_and_empty_contexts(ops, gpu, batch):
    """A one-token row sees min(kv_len, position + 1) keys: positions inside
    the context cut it, positions past it do not, and no visible key
    (kv_len 0 or position -1) gives NaN, as the MFMA kernel gives."""
    w, wd, q, meta = batch
    pos = list(meta.raw_positions)
    kv = meta.kv_lens.tolist()
    cu = meta.raw_cu_seqlens
    one = [b for b in range(len(CHUNKS)) if cu[b + 1] - cu[b] == 1]
    rng = np.random.default_rng(5)
    for b in one[:3]:
        pos[cu[b]] = int(rng.integers(0, kv[b]))  # cut inside the context
    pos[cu[one[3]]] = kv[one[3]] + 1000  # past the context: sees all of it
    pos[cu[one[4]]] = -1  # sees nothing
    kv[one[5]] = 0  # empty context
    positions = torch.tensor(pos, dtype=torch.int32, device=gpu)
    kv_lens = torch.tensor(kv, dtype=torch.int32, device=gpu)
    out = _gemm(ops, q, meta, wd, gpu, kv_lens=kv_lens, positions=positions)
    want = _oracle(q, meta, w, kv, pos)
    assert np.isnan(want[:, cu[one[4]]]).all() and np.isnan(want[:, cu[one[5]]]).all()
    assert_close(out, want, torch.bfloat16, "decode rows with cut / empty contexts")


def test_understated_max_q_len_keeps_rows_in_mfma_kernel(ops, gpu, monkeypatch):
    """With max_q_len below the longest chunk the size bound can rule decode
    rows out; the MFMA kernel then computes them itself."""
    chunks = [(300, 1), (200, 40), (100, 40)]
    w = workloads.make_paged_workload("understated", chunks, 16, 8, seed=32)
    q, meta = w.gemm_call(device=gpu)
    wd = w.to(gpu)
    want = _oracle(q, meta, w, meta.kv_lens.tolist(), meta.raw_positions)
    # 81 tokens, 3 sequences: max_q_len 39 bounds the one-token sequences by
    # (3 * 39 - 81) / 38 = 0
    out = _gemm(ops, q, meta, wd, gpu, max_q_len=39)
    assert_close(out, want, torch.bfloat16, "understated max_q_len")
    routed = _gemm(ops, q, meta, wd, gpu)
    assert_close(routed, want, torch.bfloat16, "true max_q_len")


def test_all_decode_rows_call(ops, gpu, monkeypatch):
    """A prefill call whose every sequence has one token (max_q_len 1) is all
    decode rows; with and without the workspace it matches the oracle and the
    decode entry point."""
    chunks = [(int(n) - 1, 1) for n in np.random.default_rng(33).integers(1, 3000, size=24)]
    w = workloads.make_paged_workload("all_decode", chunks, 16, 8, seed=33)
    q, meta = w.gemm_call(device=gpu)
    wd = w.to(gpu)
    want = _oracle(q, meta, w, meta.kv_lens.tolist(), meta.raw_positions)
    routed = _gemm(ops, q, meta, wd, gpu)
    assert_close(routed, want, torch.bfloat16, "all decode rows, routed")
    gemv = ops.paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens,
                                    meta.max_kv_len)
    torch.cuda.synchronize()
    assert_close(gemv, want, torch.bfloat16, "all decode rows, decode entry point")
    with monkeypatch.context() as m:
        _no_workspace(m)
        mfma = _gemm(ops, q, meta, wd, gpu)
    assert_close(mfma, want, torch.bfloat16, "all decode rows, MFMA kernel")
