"""Parity of the fused QK-norm + RoPE + KV-cache write (femto_qk_norm_rope_cache_write).

Reference behaviour: q_norm / k_norm (torch.nn.RMSNorm, qwen3.py:181-183),
rotary_embd (QwenRotaryEmbedding, qwen3.py:17-138) and the cache-write loops
(qwen3.py:240-264, 322-366), restated by oracle.prologue and
oracle.attention.cache_write.  The kernel computes in fp32 and rounds each
output once, so q and the written k rows are compared with the float64
oracle within the storage type's rounding (plus 1e-2 absolute for bf16 and
1e-4 for f32, the attention ops' tolerances); v rows are copied and must match bit for bit, and
every pool byte the reference does not write must keep its (NaN) poison.
"""

import numpy as np
import pytest
import torch

import oracle.attention as oa
import oracle.prologue as op

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: (1e-2, 2.0 ** -8), torch.float16: (1e-2, 2.0 ** -11), torch.float32: (1e-4, 1e-6)}


def bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int32 if t.element_size() == 4 else torch.int16)


def close(got, want, dtype, what):
    atol, rel = TOL[dtype]
    got = got.detach().float().cpu().double().numpy()
    err = np.abs(got - want)
    bound = atol + rel * np.abs(want)
    assert np.all(err <= bound), f"{what}: max err {err.max():.3e} (bound {bound[np.argmax(err - bound)]:.3e})"


def make_case(rng, chunks, H, KVH, dtype, tables_extra=3):
    pages = [-(-(p + n) // 16) for p, n in chunks]
    nb = sum(pages) + tables_extra
    perm = rng.permutation(nb)
    tables, at = [], 0
    for np_ in pages:
        tables.append([int(x) for x in perm[at:at + np_]])
        at += np_
    width = max(len(t) for t in tables)
    tab = torch.tensor([t + [-1] * (width - len(t)) for t in tables], dtype=torch.int32)
    cu = [0]
    for _, n in chunks:
        cu.append(cu[-1] + n)
    positions = [p + i for p, n in chunks for i in range(n)]
    T = cu[-1]
    q = torch.from_numpy(rng.standard_normal((T, H, 128)) * 2).to(dtype)
    k = torch.from_numpy(rng.standard_normal((T, KVH, 128)) * 2).to(dtype)
    v = torch.from_numpy(rng.standard_normal((T, KVH, 128))).to(dtype)
    wq = torch.from_numpy(1 + 0.1 * rng.standard_normal(128)).to(dtype)
    wk = torch.from_numpy(1 + 0.1 * rng.standard_normal(128)).to(dtype)
    pool = torch.full((nb, KVH, 16, 128), float("nan"), dtype=dtype)
    return q, k, v, wq, wk, pool, tab, cu, positions


def run_and_check(ops, gpu, case, dtype, decode=False, eps=1e-6, in_place=False, max_q_len=None):
    q, k, v, wq, wk, pool, tab, cu, positions = case
    cos, sin = op.rope_tables(8192, 128)
    g = lambda t: t.to(gpu)
    kd, vd = g(pool), g(pool.clone())
    qd = g(q)
    out = ops.qk_norm_rope_cache_write(
        qd, g(k), g(v), g(wq), g(wk), eps, g(torch.from_numpy(cos)), g(torch.from_numpy(sin)),
        g(torch.tensor(positions, dtype=torch.int32)), kd, vd, g(tab),
        cu_seqlens=None if decode else g(torch.tensor(cu, dtype=torch.int32)),
        max_q_len=max_q_len if max_q_len is not None else
        (1 if decode else max(cu[i + 1] - cu[i] for i in range(len(cu) - 1))),
        out=qd if in_place else None)
    torch.cuda.synchronize()
    if in_place:
        assert out.data_ptr() == qd.data_ptr()
    f64 = lambda t: t.double().numpy()
    q_ref, k_ref = op.qk_norm_rope(f64(q), f64(k), f64(wq), f64(wk), eps, cos, sin, positions)
    close(out, q_ref, dtype, "q")
    # where the reference writes, and what: k_ref / exact v at the oracle's slots
    nanpool = np.full(pool.shape, np.nan)
    want_k, want_v = oa.cache_write(nanpool, nanpool, k_ref, f64(v), tab.tolist(), None if decode else cu, positions)
    written = ~np.isnan(want_k)
    assert np.array_equal(written, ~np.isnan(want_v))
    gk, gv = kd.cpu(), vd.cpu()
    wmask = torch.from_numpy(written)
    assert torch.equal(bits(gk)[~wmask], bits(pool)[~wmask]), "k_pool bytes outside the written rows changed"
    assert torch.equal(bits(gv)[~wmask], bits(pool)[~wmask]), "v_pool bytes outside the written rows changed"
    close(gk[wmask], want_k[written], dtype, "k in the pool")
    assert np.array_equal(gv.double().numpy()[written], want_v[written]), "v rows are not bit-exact"
    return out, kd, vd


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("heads", [(32, 8), (16, 8), (8, 1)])
def test_prefill_chunks(ops, gpu, dtype, heads):
    rng = np.random.default_rng(51 + heads[0])
    chunks = [(int(rng.integers(0, 3000)), int(rng.integers(1, 150))) for _ in range(5)] + [(0, 1), (7000, 33)]
    run_and_check(ops, gpu, make_case(rng, chunks, *heads, dtype), dtype)


@pytest.mark.parametrize("max_q_len", [1, 6])
def test_max_q_len_below_chunk_lengths(ops, gpu, max_q_len):
    """max_q_len only sizes the grid: chunks longer than it are still processed whole."""
    rng = np.random.default_rng(55)
    chunks = [(0, 70), (300, 1), (17, 129), (4000, 33)]
    run_and_check(ops, gpu, make_case(rng, chunks, 16, 8, torch.bfloat16), torch.bfloat16, max_q_len=max_q_len)


def test_decode_layout_in_place(ops, gpu):
    rng = np.random.default_rng(52)
    chunks = [(int(rng.integers(0, 8000)), 1) for _ in range(64)]
    run_and_check(ops, gpu, make_case(rng, chunks, 16, 8, torch.bfloat16), torch.bfloat16, decode=True, in_place=True)


def test_stop_rule_matches_cache_write(ops, gpu):
    """A -1 in the table stops a sequence's writes exactly as in kv_cache_write; q is still rotated."""
    rng = np.random.default_rng(53)
    case = list(make_case(rng, [(20, 60), (100, 40)], 16, 8, torch.bfloat16))
    tab = case[6].clone()
    tab[0, 3] = -1   # positions 48.. of sequence 0 are not written
    tab[1, 7] = 999  # block outside the pool
    case[6] = tab
    run_and_check(ops, gpu, tuple(case), torch.bfloat16)


def test_eps_and_large_rows(ops, gpu):
    rng = np.random.default_rng(54)
    case = list(make_case(rng, [(5, 40)], 8, 8, torch.float32))
    case[0] = case[0] * 1000.0
    case[1] = case[1] * 1e-3  # small rows: eps matters
    run_and_check(ops, gpu, tuple(case), torch.float32, eps=1e-2)


def test_position_outside_tables_is_nan(ops, gpu):
    q = torch.randn(2, 4, 128, device=gpu).to(torch.bfloat16)
    k = torch.randn(2, 4, 128, device=gpu).to(torch.bfloat16)
    w = torch.ones(128, device=gpu, dtype=torch.bfloat16)
    cos, sin = (torch.from_numpy(t).to(gpu) for t in op.rope_tables(64, 128))
    pool = torch.zeros(4, 4, 16, 128, device=gpu, dtype=torch.bfloat16)
    tab = torch.tensor([[0, 1, 2, 3], [1, 2, 3, 0]], dtype=torch.int32, device=gpu)
    pos = torch.tensor([10, 64], dtype=torch.int32, device=gpu)  # the second is past the 64-row tables
    out = ops.qk_norm_rope_cache_write(q, k, k, w, w, 1e-6, cos, sin, pos, pool, pool.clone(), tab)
    torch.cuda.synchronize()
    assert not torch.isnan(out[0].float()).any() and torch.isnan(out[1].float()).all()


def test_errors(ops, gpu):
    q = torch.randn(2, 4, 128, device=gpu).to(torch.bfloat16)
    w = torch.ones(128, device=gpu, dtype=torch.bfloat16)
    cos, sin = (torch.from_numpy(t).to(gpu) for t in op.rope_tables(64, 128))
    pool = torch.zeros(4, 4, 16, 128, device=gpu, dtype=torch.bfloat16)
    tab = torch.zeros(2, 1, dtype=torch.int32, device=gpu)
    pos = torch.zeros(2, dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError):
        ops.qk_norm_rope_cache_write(q.cpu(), q, q, w, w, 1e-6, cos, sin, pos, pool, pool, tab)
    with pytest.raises(RuntimeError):  # half-precision tables
        ops.qk_norm_rope_cache_write(q, q, q, w, w, 1e-6, cos.half(), sin.half(), pos, pool, pool, tab)
    with pytest.raises(RuntimeError):  # head_dim 64
        ops.qk_norm_rope_cache_write(q[..., :64], q[..., :64], q[..., :64], w[:64], w[:64], 1e-6, cos, sin, pos,
                                     pool[..., :64], pool[..., :64], tab)
