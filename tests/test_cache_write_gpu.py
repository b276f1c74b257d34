"""Bit-exact parity of the HIP KV-cache write (femto_kv_cache_write) with the oracle.

Reference behaviour: the per-sequence slicing loops that write the new K/V
into the paged pools before the attention ops
(femtovllm/models/qwen/qwen3.py:240-264 decode, 322-366 prefill), restated
by oracle.attention.cache_write.  Every comparison is on the raw bits of
the whole pools, so untouched entries (NaN-poisoned) must stay as they were.
"""

import numpy as np
import pytest
import torch

import oracle.attention as oa
from femtovllm import workloads

pytestmark = pytest.mark.gpu


def bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int32 if t.element_size() == 4 else torch.int16)


def padded(tables):
    width = max(1, max(len(t) for t in tables))
    return torch.tensor([list(t) + [-1] * (width - len(t)) for t in tables], dtype=torch.int32)


def run_case(ops, gpu, pools, k_new, v_new, tables, cu, positions, max_q_len=None):
    """Write on the GPU and with the oracle; compare the pools bit for bit."""
    k_pool, v_pool = pools
    tab = tables if isinstance(tables, torch.Tensor) else padded(tables)
    kd, vd = k_pool.to(gpu), v_pool.to(gpu)
    cu_t = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=gpu)
    if max_q_len is None:
        max_q_len = 1 if cu is None else max(cu[i + 1] - cu[i] for i in range(len(cu) - 1))
    ops.kv_cache_write(k_new.to(gpu), v_new.to(gpu), kd, vd, torch.tensor(positions, dtype=torch.int32, device=gpu),
                       tab.to(gpu), cu_seqlens=cu_t, max_q_len=max_q_len)
    torch.cuda.synchronize()
    # The oracle moves values without arithmetic, so it runs on the raw bits
    # (NaN poison included) and the comparison is bit for bit.
    want_k, want_v = oa.cache_write(bits(k_pool).numpy(), bits(v_pool).numpy(), bits(k_new).numpy(),
                                    bits(v_new).numpy(), tab.tolist(), cu, positions)
    assert torch.equal(bits(kd), torch.from_numpy(want_k)), "k_pool differs from the oracle"
    assert torch.equal(bits(vd), torch.from_numpy(want_v)), "v_pool differs from the oracle"
    return kd, vd


def poisoned_pools(nb, kvh, d, dtype):
    k = torch.full((nb, kvh, 16, d), float("nan"), dtype=dtype)
    v = torch.full((nb, kvh, 16, d), float("nan"), dtype=dtype)
    return k, v


def fresh(rng, n, kvh, d, dtype):
    return (torch.from_numpy(rng.standard_normal((n, kvh, d))).to(dtype),
            torch.from_numpy(rng.standard_normal((n, kvh, d))).to(dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_prefill_chunks_bit_exact(ops, gpu, dtype):
    """8 chunks of ragged length after ragged cached prefixes, random block placement."""
    rng = np.random.default_rng(31)
    prefixes = [int(x) for x in rng.integers(0, 300, size=8)]
    lens = [int(x) for x in rng.integers(1, 200, size=8)]
    pages = [-(-(p + n) // 16) for p, n in zip(prefixes, lens)]
    nb = sum(pages) + 7
    perm = rng.permutation(nb)
    tables, at = [], 0
    for np_ in pages:
        tables.append([int(x) for x in perm[at:at + np_]])
        at += np_
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    positions = [p + i for p, n in zip(prefixes, lens) for i in range(n)]
    k_new, v_new = fresh(rng, cu[-1], 8, 128, dtype)
    run_case(ops, gpu, poisoned_pools(nb, 8, 128, dtype), k_new, v_new, tables, cu, positions)


def test_decode_layout_bit_exact(ops, gpu):
    """cu_seqlens=None: one token per sequence at positions[b] (the decode metadata)."""
    rng = np.random.default_rng(32)
    B = 64
    L = [int(x) for x in rng.integers(1, 4000, size=B)]
    pages = [-(-l // 16) for l in L]
    nb = sum(pages) + 3
    perm = rng.permutation(nb)
    tables, at = [], 0
    for np_ in pages:
        tables.append([int(x) for x in perm[at:at + np_]])
        at += np_
    k_new, v_new = fresh(rng, B, 8, 128, torch.bfloat16)
    run_case(ops, gpu, poisoned_pools(nb, 8, 128, torch.bfloat16), k_new, v_new, tables, None, [l - 1 for l in L])


def test_stop_rule_and_bad_block_ids(ops, gpu):
    """Writes stop at the first -1, at a block id outside the pool, and past the table width."""
    rng = np.random.default_rng(33)
    tables = [[3, -1, 5], [2, 4, 0], [1, 99], [6, 7, 8, 9]]
    chunks = [(14, 40), (30, 40), (15, 3), (0, 64)]  # (first position, tokens)
    cu = [0]
    for _, n in chunks:
        cu.append(cu[-1] + n)
    positions = [p + i for p, n in chunks for i in range(n)]
    k_new, v_new = fresh(rng, cu[-1], 4, 64, torch.float16)
    run_case(ops, gpu, poisoned_pools(12, 4, 64, torch.float16), k_new, v_new, tables, cu, positions)


def test_positions_follow_first_token(ops, gpu):
    """Tokens land at positions[q_begin] + i whatever the later positions say (qwen3.py:330-364)."""
    rng = np.random.default_rng(34)
    tables = [[0, 1, 2], [3, 4]]
    cu = [0, 20, 27]
    positions = [7] + [int(x) for x in rng.integers(0, 40, size=19)] + [16] + [0] * 6
    k_new, v_new = fresh(rng, 27, 2, 128, torch.bfloat16)
    run_case(ops, gpu, poisoned_pools(5, 2, 128, torch.bfloat16), k_new, v_new, tables, cu, positions)


def test_shared_block_idempotent_rewrite(ops, gpu):
    """Two sequences share their first blocks (prefix tree); both rewrite the shared last
    token with identical values, as the scheduler's (L-1) rule does
    (femtovllm/engine/scheduler/v3.py:370-400)."""
    rng = np.random.default_rng(35)
    shared = [4, 9]
    tables = [shared + [1, 2], shared + [7]]
    # sequence 0 re-runs token 31 (cached, in shared block 9) and adds 20 more;
    # sequence 1 re-runs the same token 31 only
    cu = [0, 21, 22]
    positions = list(range(31, 52)) + [31]
    k_new, v_new = fresh(rng, 22, 8, 128, torch.bfloat16)
    k_new[21], v_new[21] = k_new[0], v_new[0]  # the same token, the same K/V
    run_case(ops, gpu, poisoned_pools(10, 8, 128, torch.bfloat16), k_new, v_new, tables, cu, positions)


@pytest.mark.parametrize("shape", [(1, 64), (8, 128), (2, 256), (16, 128)])
def test_head_shapes_and_strided_source(ops, gpu, shape):
    """k and v as views of a fused (tokens, H + 2*KVH, D) projection (token stride != KVH*D)."""
    kvh, d = shape
    h = 2 * kvh
    rng = np.random.default_rng(36 + kvh * d)
    n = 45
    qkv = torch.from_numpy(rng.standard_normal((n, h + 2 * kvh, d))).to(torch.bfloat16).to(gpu)
    k_view, v_view = qkv[:, h:h + kvh], qkv[:, h + kvh:]
    assert not k_view.is_contiguous()
    tables = [[2, 0, 5], [1, 4]]
    cu = [0, 33, 45]
    positions = list(range(10, 43)) + list(range(20, 32))
    k_pool, v_pool = poisoned_pools(6, kvh, d, torch.bfloat16)
    kd, vd = k_pool.to(gpu), v_pool.to(gpu)
    ops.kv_cache_write(k_view, v_view, kd, vd, torch.tensor(positions, dtype=torch.int32, device=gpu),
                       padded(tables).to(gpu), cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=gpu),
                       max_q_len=33)
    torch.cuda.synchronize()
    want_k, want_v = oa.cache_write(bits(k_pool).numpy(), bits(v_pool).numpy(), bits(k_view).numpy(),
                                    bits(v_view).numpy(), padded(tables).tolist(), cu, positions)
    assert torch.equal(bits(kd), torch.from_numpy(want_k))
    assert torch.equal(bits(vd), torch.from_numpy(want_v))


def test_write_then_attend(ops, gpu):
    """Blank a prefill chunk's own K/V rows, write them back with the kernel, then attend.

    The pools must come back bit for bit, so the prefill attention over them
    gives the same bits as over the original pools."""
    w = workloads.make_paged_workload("wa", [(100, 60), (0, 40), (250, 9)], 16, 8, seed=37)
    q, meta = w.gemm_call(device=gpu)
    wd = w.to(gpu)
    # keep the cached prefix, blank the chunk's own rows, and write them back with the kernel
    k_new = torch.cat([w.k_pool.new_empty(0, 8, 128)] + [
        torch.stack([w.k_pool[w.raw_block_tables[b][p // 16], :, p % 16] for p in range(pre, pre + n)])
        for b, (pre, n) in enumerate(w.chunks)])
    v_new = torch.cat([
        torch.stack([w.v_pool[w.raw_block_tables[b][p // 16], :, p % 16] for p in range(pre, pre + n)])
        for b, (pre, n) in enumerate(w.chunks)])
    kd, vd = wd.k_pool.clone(), wd.v_pool.clone()
    for b, (pre, n) in enumerate(w.chunks):
        for p in range(pre, pre + n):
            kd[w.raw_block_tables[b][p // 16], :, p % 16] = float("nan")
            vd[w.raw_block_tables[b][p // 16], :, p % 16] = float("nan")
    ops.kv_cache_write(k_new.to(gpu), v_new.to(gpu), kd, vd, meta.positions, meta.block_tables,
                       cu_seqlens=meta.cu_seqlens, max_q_len=meta.max_q_len)
    torch.cuda.synchronize()
    assert torch.equal(bits(kd), bits(wd.k_pool)) and torch.equal(bits(vd), bits(wd.v_pool))
    args = (meta.cu_seqlens, meta.max_q_len, meta.Q_TILE_SIZE, meta.cu_q_tiles, meta.q_tile_to_seq_idx,
            meta.block_tables, meta.kv_lens, meta.positions)
    q = q.to(gpu)
    a = ops.paged_attention_gemm(q, kd, vd, *args)
    b = ops.paged_attention_gemm(q, wd.k_pool, wd.v_pool, *args)
    torch.cuda.synchronize()
    assert torch.equal(bits(a), bits(b))


def test_errors(ops, gpu):
    k = torch.zeros(4, 8, 128, dtype=torch.bfloat16, device=gpu)
    pool = torch.zeros(4, 8, 16, 128, dtype=torch.bfloat16, device=gpu)
    tab = torch.zeros(4, 1, dtype=torch.int32, device=gpu)
    pos = torch.zeros(4, dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError):
        ops.kv_cache_write(k.cpu(), k.cpu(), pool, pool, pos, tab)
    with pytest.raises(RuntimeError):
        ops.kv_cache_write(k, k.float(), pool, pool, pos, tab)
    with pytest.raises(RuntimeError):  # 4 tokens but 3 sequences and no cu_seqlens
        ops.kv_cache_write(k, k, pool, pool, pos[:3], tab[:3])
    with pytest.raises(RuntimeError):  # head count differs from the pools
        ops.kv_cache_write(k[:, :4], k[:, :4], pool, pool, pos, tab)


@pytest.mark.parametrize("max_q_len", [1, 5])
def test_max_q_len_below_chunk_lengths(ops, gpu, max_q_len):
    """max_q_len only sizes the grid: chunks longer than it are still written whole."""
    rng = np.random.default_rng(37)
    prefixes = [0, 17, 200, 5]
    lens = [70, 1, 33, 129]
    pages = [-(-(p + n) // 16) for p, n in zip(prefixes, lens)]
    nb = sum(pages) + 3
    perm = rng.permutation(nb)
    tables, at = [], 0
    for np_ in pages:
        tables.append([int(x) for x in perm[at:at + np_]])
        at += np_
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    positions = [p + i for p, n in zip(prefixes, lens) for i in range(n)]
    k_new, v_new = fresh(rng, cu[-1], 8, 128, torch.bfloat16)
    run_case(ops, gpu, poisoned_pools(nb, 8, 128, torch.bfloat16), k_new, v_new, tables, cu, positions,
             max_q_len=max_q_len)
