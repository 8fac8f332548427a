"""Split decode under repetition: 200 graph replays, every output bit-identical.

The split partitions hand their partials to the last arrival with
agent-scope (L2-coherent) stores, a wait for those stores, and a relaxed
agent-scope counter; the last arrival reads them with agent-scope loads.
These tests put that hand-off under repetition at the two shapes where it
matters most: one 32768-token sequence (Qwen3-8B heads, 24 partitions per KV
head merged by one workgroup) and the 32-sequence Qwen3-0.6B decode batch
with contexts U[128, 2048] and the fused append (mixed one- and two-part
splits, early merges). Each graph holds the decode launch and a device-side
copy of its output into the next row of a history buffer, so the 200
replays run back to back with no host synchronisation between them; every
row must equal the first bit for bit (the first mismatch is reported), and
the first must match the oracle.
"""

import math

import numpy as np
import pytest
import torch

from microinfer_amd.layer.hip_paged_attention import decode_plan, hip_paged_decode
from microinfer_amd.runner import capture_graph
from microinfer_amd.worker.kv_cache import KVCache
from microinfer_amd.workloads import QWEN3_06B, make_decode_batch
from tests.support import as_f32, oracle_decode

pytestmark = pytest.mark.gpu
DEV = "cuda"
REPLAYS = 200


def replay_history(step, out_shape, dtype):
    """Capture ``step`` (returns the output) plus a copy of it into history
    row ``idx`` (then ``idx += 1``); replay REPLAYS times back to back."""
    history = torch.empty((REPLAYS, *out_shape), dtype=dtype, device=DEV)
    idx = torch.zeros(1, dtype=torch.long, device=DEV)
    one = torch.ones(1, dtype=torch.long, device=DEV)
    step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # per-stream library state made before capture
        step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph, stream=side):
        out = step()
        history.index_copy_(0, idx, out[None])
        idx.add_(one)
    torch.cuda.synchronize()
    for _ in range(REPLAYS):
        graph.replay()
    torch.cuda.synchronize()
    assert int(idx.item()) == REPLAYS  # capture records; only the replays run
    return history, graph


def assert_all_rows_equal(history):
    bits = history.view(torch.int16).reshape(REPLAYS, -1)
    same = (bits == bits[0]).all(dim=1).cpu().numpy()
    if not same.all():
        first_bad = int(np.argmin(same))
        diff = (history[first_bad].float() - history[0].float()).abs().max().item()
        raise AssertionError(f"replay {first_bad} differs from replay 0 (max abs {diff:.3g})")


def test_one_32k_sequence_replays_bit_identically():
    print("case: 1 x 32768, Qwen3-8B heads, 200 replays", flush=True)
    hq, hkv, d, bs, ctx = 32, 8, 128, 16, 32768
    nb = ctx // bs
    pool = nb + 64
    gen = torch.Generator(device=DEV).manual_seed(11)
    cache = KVCache(1, pool, bs, hkv, d, dtype=torch.bfloat16, device=DEV)
    kc, vc = cache.keys[0], cache.values[0]
    kc.copy_(torch.randn(kc.shape, generator=gen, device=DEV))
    vc.copy_(torch.randn(vc.shape, generator=gen, device=DEV))
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(11))[:nb]
    tables = perm.to(torch.int32).reshape(1, nb).to(DEV)
    lens = torch.tensor([ctx], dtype=torch.int32, device=DEV)
    q = torch.randn((1, hq, d), generator=gen, device=DEV).to(torch.bfloat16)
    scale = 1 / math.sqrt(d)

    def step():
        plan = decode_plan(lens, num_kv_heads=hkv, block_size=bs, block_table_width=nb)
        return hip_paged_decode(q, kc, vc, tables, lens, scale=scale, plan=plan)

    history, _ = replay_history(step, (1, hq, d), torch.bfloat16)
    assert_all_rows_equal(history)
    expected = oracle_decode(q, kc, vc, tables, lens, scale)
    np.testing.assert_allclose(as_f32(history[0]), expected, atol=2e-2, rtol=2e-2)


def test_decode_batch_with_append_replays_bit_identically():
    print("case: 32 x U[128,2048], Qwen3-0.6B heads, fused append, 200 replays", flush=True)
    batch = make_decode_batch(num_seqs=32, ctx_lo=128, ctx_hi=2048, pool_blocks=16384,
                              draw_pools=False, **QWEN3_06B)
    gen = torch.Generator(device=DEV).manual_seed(0)
    cache = KVCache(1, 16384, 16, 8, 128, dtype=torch.bfloat16, device=DEV)
    kc, vc = cache.keys[0], cache.values[0]
    kc.copy_(torch.randn(kc.shape, generator=gen, device=DEV))
    vc.copy_(torch.randn(vc.shape, generator=gen, device=DEV))
    q = torch.randn((32, 16, 128), generator=gen, device=DEV).to(torch.bfloat16)
    new_k = torch.randn((32, 8, 128), generator=gen, device=DEV).to(torch.bfloat16)
    new_v = torch.randn((32, 8, 128), generator=gen, device=DEV).to(torch.bfloat16)
    tables = torch.tensor(batch.block_tables, device=DEV)
    lens = torch.tensor(batch.context_lens, device=DEV)
    scale = 1 / math.sqrt(128)

    def step():
        # Rewriting the same new rows at the same slots is idempotent, so
        # every replay sees the same cache.
        plan = decode_plan(lens, num_kv_heads=8, block_size=16,
                           block_table_width=tables.shape[1])
        return hip_paged_decode(q, kc, vc, tables, lens, scale=scale, plan=plan,
                                new_keys=new_k, new_values=new_v)

    history, _ = replay_history(step, (32, 16, 128), torch.bfloat16)
    assert_all_rows_equal(history)
    expected = oracle_decode(q, kc, vc, tables, lens, scale)
    np.testing.assert_allclose(as_f32(history[0]), expected, atol=2e-2, rtol=2e-2)
