"""The bf16/f16 MFMA paged-prefill kernel (head_dim 128, GQA groups 1, 2, 4).

Every call here has head_dim 128 and a 16-bit dtype, so mi_paged_prefill
routes it to the MFMA kernel. Results are compared with the fp32 oracle
(restating microinfer/layer/paged_attention.py:22-67) at 2e-2 max-abs, the
decode/prefill tolerance for 16-bit inputs. The cases cover query blocks that
end inside a 32-row MFMA tile, 32-key tiles that end inside a cache block,
prefixes shorter and longer than a tile, single-row (decode) requests in the
same launch, every block size the kernel takes, invalid table entries and
poison in unused slots, contiguous K/V, and pools past 2^31 elements
(64-bit tile addressing) against the same blocks in a small pool.
"""

import math

import numpy as np
import pytest
import torch

from microinfer_amd.layer.hip_paged_attention import hip_paged_prefill
from oracle import dense_causal_attention_f64
from tests.support import as_f32, max_abs, oracle_prefill

pytestmark = pytest.mark.gpu
DEV = "cuda"
D = 128


def _paged_case(q_lens, prefixes, hq, hkv, block_size, dtype, seed, poison=False):
    """Random caches and shuffled block tables for requests with the given
    query lengths and cached prefixes (context = prefix + query length)."""
    gen = torch.Generator().manual_seed(seed)
    contexts = [p + q for p, q in zip(prefixes, q_lens)]
    nblk = [(c + block_size - 1) // block_size for c in contexts]
    width = max(nblk)
    pool = sum(nblk) + 3
    perm = torch.randperm(pool, generator=gen)
    tables = torch.full((len(q_lens), width), -1, dtype=torch.int32)
    used = 0
    for r, n in enumerate(nblk):
        tables[r, :n] = perm[used:used + n]
        used += n
    # poison: True puts +-1000 in unused slots, a float puts that value.
    fill = float(poison) if isinstance(poison, float) else (1000.0 if poison else 0.0)
    kc = torch.randn(pool, block_size, hkv, D, generator=gen)
    vc = torch.randn(pool, block_size, hkv, D, generator=gen)
    if poison:
        # Slots past each context hold +-1000: a kernel that reads them fails.
        for r, c in enumerate(contexts):
            last = tables[r, nblk[r] - 1]
            off = c - (nblk[r] - 1) * block_size
            kc[last, off:] = fill
            vc[last, off:] = -fill
        unused = perm[used:]
        kc[unused] = fill
        vc[unused] = -fill
    q = torch.randn(sum(q_lens), hq, D, generator=gen)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(contexts)]).astype(np.int32)
    return (q.to(dtype).to(DEV), kc.to(dtype).to(DEV), vc.to(dtype).to(DEV),
            tables.to(DEV), contexts, cu_q, cu_k)


def _run(q, kc, vc, tables, cu_q, cu_k):
    return hip_paged_prefill(q, kc, vc, torch.tensor(cu_q, device=DEV),
                             torch.tensor(cu_k, device=DEV), tables,
                             max_seqlen_q=int(np.diff(cu_q).max()),
                             scale=1 / math.sqrt(D))


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 8), (32, 8)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_group_sizes_and_tile_edges(hq, hkv, dtype):
    # Query lengths around the 32-row tile and the workgroup's row block;
    # prefixes around the 32-key tile and the 16-token block.
    q_lens = [1, 31, 32, 33, 70, 129]
    prefixes = [0, 1, 15, 16, 47, 300]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, hq, hkv, 16, dtype, 1)
    out = _run(q, kc, vc, tables, cu_q, cu_k)
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(out, expected) <= 2e-2


@pytest.mark.parametrize("block_size", [16, 32, 64, 128, 256])
def test_block_sizes(block_size):
    # The single row's context spans several blocks and ends mid-tile.
    q_lens = [5, 64, 100, 1]
    prefixes = [block_size - 3, 2 * block_size + 1, 0, 3 * block_size + 20]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, 32, 8, block_size,
                                                          torch.bfloat16, 2)
    out = _run(q, kc, vc, tables, cu_q, cu_k)
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(out, expected) <= 2e-2


def test_poison_in_unused_slots_is_never_read():
    q_lens = [17, 64, 1]
    prefixes = [10, 100, 250]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, 16, 8, 16,
                                                          torch.bfloat16, 3, poison=True)
    out = _run(q, kc, vc, tables, cu_q, cu_k)
    assert torch.isfinite(out).all()
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(out, expected) <= 2e-2


def test_nan_in_unused_slots_and_invalid_blocks_stays_out():
    """Slots past each context and blocks no table names hold NaN, as an
    uninitialised pool may: the reference's masked loads never read them
    (microinfer/layer/triton_paged_attention.py:176-218), so the output must
    stay finite and equal the oracle's. Tail tiles read those slots as whole
    rows; their weights are 0 and their V rows are zeroed before use."""
    q_lens = [17, 64, 1, 33, 5]
    prefixes = [10, 100, 250, 0, 31]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, 16, 8, 16,
                                                          torch.bfloat16, 5,
                                                          poison=float("nan"))
    assert not torch.isfinite(vc).all()
    out = _run(q, kc, vc, tables, cu_q, cu_k)
    assert torch.isfinite(out).all()
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(out, expected) <= 2e-2
    # Invalid ids inside the contexts read block 0 instead, and drop out of
    # the softmax; make block 0 an unused (NaN) block first.
    named = set(int(b) for b in tables.flatten().tolist() if b >= 0)
    spare = next(b for b in range(kc.shape[0]) if b not in named)
    if 0 in named:
        for cache in (kc, vc):
            keep = cache[0].clone()
            cache[0] = cache[spare]
            cache[spare] = keep
        tables = torch.where(tables == 0, torch.full_like(tables, spare), tables)
    assert not torch.isfinite(vc[0]).any()
    bad = tables.clone()
    bad[1, 2] = -1
    bad[2, 5] = -1  # a single-row request
    bad[3, 0] = 10 ** 6
    out = _run(q, kc, vc, bad, cu_q, cu_k)
    assert torch.isfinite(out).all()


def test_invalid_table_entries_are_masked():
    # A -1 and an out-of-range id inside the contexts: those blocks drop out
    # of the softmax (as in the decode kernel) and are never dereferenced.
    q_lens = [40, 20, 1]
    prefixes = [60, 10, 90]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, 16, 8, 16,
                                                          torch.bfloat16, 4)
    bad = tables.clone()
    bad[0, 1] = -1
    bad[1, 0] = 10 ** 6
    bad[2, 0] = -1  # the single row's first tile
    bad[2, 3] = 10 ** 6
    out = _run(q, kc, vc, bad, cu_q, cu_k)
    assert torch.isfinite(out).all()
    # Expected: the same attention with those blocks' keys excluded.
    host_t = bad.cpu().numpy()
    ref = np.zeros(as_f32(out).shape, dtype=np.float64)
    kf, vf, qf = as_f32(kc), as_f32(vc), as_f32(q)
    for r in range(3):
        c, ql = contexts[r], q_lens[r]
        pos = np.arange(c)
        blk = host_t[r, pos // 16]
        keep = (blk >= 0) & (blk < kc.shape[0])
        ks = np.where(keep[:, None, None], kf[np.clip(blk, 0, kc.shape[0] - 1), pos % 16], 0)
        vs = np.where(keep[:, None, None], vf[np.clip(blk, 0, kc.shape[0] - 1), pos % 16], 0)
        for i in range(ql):
            row = cu_q[r] + i
            visible = keep & (pos <= c - ql + i)
            for h in range(16):
                s = (ks[:, h // 2] @ qf[row, h]) / math.sqrt(D)
                s = np.where(visible, s, -np.inf)
                if not visible.any():
                    continue
                w = np.exp(s - s.max())
                ref[row, h] = (w / w.sum()) @ vs[:, h // 2]
    assert np.abs(as_f32(out) - ref).max() <= 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_contiguous_kv_matches_dense(dtype):
    torch.manual_seed(5)
    q_lens = [33, 1, 128, 7]
    total = sum(q_lens)
    q = torch.randn(total, 16, D, device=DEV).to(dtype)
    k = torch.randn(total, 8, D, device=DEV).to(dtype)
    v = torch.randn(total, 8, D, device=DEV).to(dtype)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_t = torch.tensor(cu, device=DEV)
    out = hip_paged_prefill(q, k, v, cu_t, cu_t, None, max_seqlen_q=max(q_lens))
    expected = np.concatenate([
        dense_causal_attention_f64(as_f32(q[a:b]), as_f32(k[a:b]), as_f32(v[a:b]),
                                   scale=1 / math.sqrt(D))
        for a, b in zip(cu[:-1], cu[1:])
    ])
    assert max_abs(out, expected) <= 2e-2


@pytest.mark.parametrize("hq", [8, 16, 32])
def test_single_rows_over_long_contexts(hq):
    # Single-row requests (the decode rows of a mixed step) take a path of
    # their own: 16-position tiles spread over the workgroup's four waves.
    # Contexts around multiples of 16 and 64 and up to 2 K positions.
    q_lens = [1] * 7 + [48]
    prefixes = [0, 15, 16, 63, 64, 1023, 2047, 200]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, hq, 8, 16,
                                                          torch.bfloat16, 6)
    out = _run(q, kc, vc, tables, cu_q, cu_k)
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(out, expected) <= 2e-2


def test_planned_launch_splits_merge_deterministically():
    # Long prefixes make the plan split (query block, KV head) items along
    # their keys (target 8-13 tiles here); the merged result must match the
    # unsplit launch to float rounding, the oracle to the usual bound, and
    # be the same bits on every call whatever order the partitions finish in.
    q_lens = [512, 96, 1, 200, 1, 33]
    prefixes = [2500, 1300, 3000, 0, 17, 700]
    for hq in (32, 16, 8):
        q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, hq, 8, 16,
                                                              torch.bfloat16, 8)
        args = (q, kc, vc, torch.tensor(cu_q, device=DEV), torch.tensor(cu_k, device=DEV),
                tables)
        kw = dict(max_seqlen_q=max(q_lens), scale=1 / math.sqrt(D))
        first = hip_paged_prefill(*args, **kw)
        for _ in range(3):
            assert torch.equal(hip_paged_prefill(*args, **kw), first)
        unplanned = hip_paged_prefill(*args, planned=False, **kw)
        assert max_abs(first, as_f32(unplanned)) <= 1e-2
        expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
        assert max_abs(first, expected) <= 2e-2
        assert max_abs(unplanned, expected) <= 2e-2


def test_one_plan_serves_many_calls():
    # A plan made once (per step) and passed to several calls gives the bits
    # of a call that plans for itself; a plan for other sizes is refused.
    from microinfer_amd.layer.hip_paged_attention import prefill_plan

    q_lens = [300, 1, 64, 1]
    prefixes = [2000, 900, 40, 5]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, 32, 8, 16,
                                                          torch.bfloat16, 9)
    cq, ck = torch.tensor(cu_q, device=DEV), torch.tensor(cu_k, device=DEV)
    kw = dict(max_seqlen_q=max(q_lens), scale=1 / math.sqrt(D))
    own = hip_paged_prefill(q, kc, vc, cq, ck, tables, **kw)
    plan = prefill_plan(cq, ck, num_tokens=q.shape[0], num_q_heads=32, num_kv_heads=8,
                        head_dim=D, dtype=q.dtype, block_size=16,
                        block_table_width=tables.shape[1])
    assert plan is not None
    for _ in range(3):
        assert torch.equal(hip_paged_prefill(q, kc, vc, cq, ck, tables, plan=plan, **kw), own)
    with pytest.raises(ValueError, match="prefill_plan"):
        hip_paged_prefill(q[:-1], kc, vc, cq, ck, tables, plan=plan, **kw)
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(own, expected) <= 2e-2


def test_long_prefix_chunk():
    # One 512-row chunk on a 3000-token prefix (one request of the mixed prefill step).
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case([512], [3000], 32, 8, 16,
                                                          torch.bfloat16, 6)
    out = _run(q, kc, vc, tables, cu_q, cu_k)
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(out, expected) <= 2e-2


def test_pool_beyond_int32_offsets_matches_small_pool():
    # A pool of more than 2^31 elements per cache (> 4 GiB each in bf16) takes
    # the 64-bit tile addressing; blocks near its top must give exactly what
    # the same blocks give in a small pool (32-bit addressing) and match the
    # oracle.
    hkv, bs = 8, 16
    big_blocks = (1 << 31) // (bs * hkv * D) + 64
    q_lens, prefixes = [40, 1, 96], [100, 700, 33]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, 32, hkv, bs,
                                                          torch.bfloat16, 7)
    top = big_blocks - kc.shape[0]  # small block b lives at big block top + b
    big_k = torch.empty(big_blocks, bs, hkv, D, dtype=torch.bfloat16, device=DEV)
    big_v = torch.empty_like(big_k)
    big_k[top:] = kc
    big_v[top:] = vc
    big_tables = torch.where(tables >= 0, tables + top, tables)
    small = _run(q, kc, vc, tables, cu_q, cu_k)
    big = _run(q, big_k, big_v, big_tables, cu_q, cu_k)
    del big_k, big_v
    assert torch.equal(small, big)
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(big, expected) <= 2e-2


def _read_plan(plan, num_tokens, num_requests, hq, hkv):
    """Items of a prefill plan, read back from its workspace (the layout
    mi_paged_prefill_workspace_bytes sizes: count, counters, items)."""
    r256 = lambda x: (x + 255) // 256 * 256  # noqa: E731
    part_cap = max(2, 1024 // hkv)
    counters = part_cap // 2 * hkv
    bm = 128 // (hq // hkv)
    max_entries = (num_tokens + bm - 1) // bm + num_requests + part_cap
    raw = plan.workspace.cpu()
    count = int(raw[:4].view(torch.int32)[0])
    assert 0 < count <= max_entries
    off = 256 + r256(counters * 4)
    items = raw[off:off + count * 32].view(torch.int32).reshape(count, 8).numpy()
    return items, part_cap, counters


def test_plan_items_cover_every_block_once_largest_first():
    # Few items on long contexts: the plan splits; every (request, row block)
    # must appear with key ranges that partition its tiles, each split with
    # its own partial slots and counter, listed by size, largest first.
    from microinfer_amd.layer.hip_paged_attention import prefill_plan

    q_lens = [64, 1, 40, 1]
    prefixes = [6000, 3000, 500, 20]
    hq, hkv = 32, 8
    _, _, _, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, hq, hkv, 16,
                                                        torch.bfloat16, 10)
    total = sum(q_lens)
    plan = prefill_plan(torch.tensor(cu_q, device=DEV), torch.tensor(cu_k, device=DEV),
                        num_tokens=total, num_q_heads=hq, num_kv_heads=hkv, head_dim=D,
                        dtype=torch.bfloat16, block_size=16, block_table_width=tables.shape[1])
    items, part_cap, counters = _read_plan(plan, total, len(q_lens), hq, hkv)
    bm = 32
    expected = {}
    for r, (ql, c) in enumerate(zip(q_lens, contexts)):
        for b in range((ql + bm - 1) // bm):
            kv_end = min(c, c - ql + min(ql, (b + 1) * bm))
            expected[(r, b)] = (kv_end + 31) // 32
    seen = {}
    slots, ctrs, sizes = set(), set(), []
    for req, qb, t0, t1, part, nparts, slot, ctr in items.tolist():
        assert (req, qb) in expected
        seen.setdefault((req, qb), []).append((part, nparts, t0, t1, slot, ctr))
        single = q_lens[req] == 1
        # the plan counts a single row as ceil(ctx / 48) tiles
        sizes.append(-(-contexts[req] // 48) if single else t1 - t0)
        if nparts > 1:
            assert not single
            assert slot + part < part_cap
            assert ctr * hkv < counters
            slots.add(slot + part)
            ctrs.add(ctr)
    assert set(seen) == set(expected)
    split = 0
    for key, parts in seen.items():
        n = parts[0][1]
        assert sorted(p[0] for p in parts) == list(range(n))
        assert all(p[1] == n for p in parts)
        if n > 1:
            split += 1
            assert len({(p[4], p[5]) for p in parts}) == 1  # one slot base, one counter
        ranges = sorted((p[2], p[3]) for p in parts)
        assert ranges[0][0] == 0 and ranges[-1][1] == expected[key]
        assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
        assert all(t1 > t0 for t0, t1 in ranges)
    assert split > 0  # the long request's blocks were split
    assert len(ctrs) == split
    assert sizes == sorted(sizes, reverse=True)


@pytest.mark.parametrize("hq,dtype", [(8, torch.bfloat16), (16, torch.bfloat16),
                                      (32, torch.float16)])
def test_split_launches_match_oracle_across_groups_and_dtypes(hq, dtype):
    # Few long items make the plan split; groups 1 and 2 have 128- and
    # 64-row blocks, f16 its own conversions.
    q_lens = [96, 1, 200]
    prefixes = [5000, 2000, 3000]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, hq, 8, 16, dtype,
                                                          11)
    args = (q, kc, vc, torch.tensor(cu_q, device=DEV), torch.tensor(cu_k, device=DEV), tables)
    kw = dict(max_seqlen_q=max(q_lens), scale=1 / math.sqrt(D))
    planned = hip_paged_prefill(*args, **kw)
    unplanned = hip_paged_prefill(*args, planned=False, **kw)
    assert max_abs(planned, as_f32(unplanned)) <= 1e-2
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(planned, expected) <= 2e-2


def _causal_f64(q, k, v, scale):
    """Causal GQA attention of one no-prefix prompt in float64 (numpy)."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    rows, hq, _ = q.shape
    group = hq // k.shape[1]
    out = np.empty_like(q)
    mask = np.tril(np.ones((rows, rows), dtype=bool))
    for h in range(hq):
        s = (q[:, h] @ k[:, h // group].T) * scale
        s = np.where(mask, s, -np.inf)
        w = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (w / w.sum(axis=1, keepdims=True)) @ v[:, h // group]
    return out


def test_contiguous_kv_split_matches_dense():
    # One long no-prefix prompt on one KV head: 32 row blocks, so the plan
    # splits the later blocks' keys on the contiguous path too.
    gen = torch.Generator().manual_seed(12)
    rows = 1024
    q = torch.randn(rows, 4, D, generator=gen).to(torch.bfloat16).to(DEV)
    k = torch.randn(rows, 1, D, generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn(rows, 1, D, generator=gen).to(torch.bfloat16).to(DEV)
    cu = torch.tensor([0, rows], dtype=torch.int32, device=DEV)
    kw = dict(max_seqlen_q=rows, scale=1 / math.sqrt(D))
    planned = hip_paged_prefill(q, k, v, cu, cu, None, **kw)
    assert torch.equal(hip_paged_prefill(q, k, v, cu, cu, None, **kw), planned)
    unplanned = hip_paged_prefill(q, k, v, cu, cu, None, planned=False, **kw)
    assert max_abs(planned, as_f32(unplanned)) <= 1e-2
    expected = _causal_f64(as_f32(q), as_f32(k), as_f32(v), 1 / math.sqrt(D))
    assert max_abs(planned, expected) <= 2e-2


def test_call_with_many_items_runs_unplanned():
    # 8 x 512 rows with 8 KV heads: 1088 (query block, KV head) items, more
    # than two per CU, so a call without a shared plan skips the plan kernel
    # and its output is the unplanned launch's, bit for bit.
    q_lens = [512] * 8
    prefixes = [0, 16, 100, 300, 40, 7, 512, 1]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, 32, 8, 16,
                                                          torch.bfloat16, 13)
    args = (q, kc, vc, torch.tensor(cu_q, device=DEV), torch.tensor(cu_k, device=DEV), tables)
    kw = dict(max_seqlen_q=512, scale=1 / math.sqrt(D))
    assert torch.equal(hip_paged_prefill(*args, **kw),
                       hip_paged_prefill(*args, planned=False, **kw))


@pytest.mark.parametrize("block_size", [32, 64, 256])
def test_split_launches_across_block_sizes(block_size):
    # Long contexts on few items (so the plan splits) with tiles spanning
    # part of a block or several blocks.
    q_lens = [70, 1, 33]
    prefixes = [4000 + block_size // 2, 2500, 3000 - 5]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, 32, 8, block_size,
                                                          torch.bfloat16, 14)
    args = (q, kc, vc, torch.tensor(cu_q, device=DEV), torch.tensor(cu_k, device=DEV), tables)
    kw = dict(max_seqlen_q=max(q_lens), scale=1 / math.sqrt(D))
    planned = hip_paged_prefill(*args, **kw)
    assert max_abs(planned, as_f32(hip_paged_prefill(*args, planned=False, **kw))) <= 1e-2
    expected = oracle_prefill(q, kc, vc, tables, contexts, cu_q, 1 / math.sqrt(D))
    assert max_abs(planned, expected) <= 2e-2


def test_split_launch_with_nan_pool_and_invalid_ids_stays_finite():
    # Split items whose ranges cross invalid table entries, over a pool whose
    # unused slots hold NaN: every partition masks what it cannot see, the
    # merge weighs empty partitions zero, and the result equals the unsplit
    # launch's to float rounding.
    q_lens = [64, 1, 40]
    prefixes = [3500, 2000, 2600]
    q, kc, vc, tables, contexts, cu_q, cu_k = _paged_case(q_lens, prefixes, 32, 8, 16,
                                                          torch.bfloat16, 15,
                                                          poison=float("nan"))
    bad = tables.clone()
    bad[0, 5] = -1
    bad[0, 150] = 10 ** 6
    bad[1, 70] = -1
    bad[2, 0] = -1
    args = (q, kc, vc, torch.tensor(cu_q, device=DEV), torch.tensor(cu_k, device=DEV), bad)
    kw = dict(max_seqlen_q=max(q_lens), scale=1 / math.sqrt(D))
    planned = hip_paged_prefill(*args, **kw)
    assert torch.isfinite(planned).all()
    unplanned = hip_paged_prefill(*args, planned=False, **kw)
    assert torch.isfinite(unplanned).all()
    assert max_abs(planned, as_f32(unplanned)) <= 1e-2
