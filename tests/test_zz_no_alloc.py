"""The allocation-free decode entry point (mi_paged_decode_append_noalloc)
against mi_paged_decode_append, through the C ABI.

Both run the same kernels and, given the same context lengths, the same
partition plan, so outputs and appended cache rows must be bit-identical.
Two calls in a row share the library's static scratch: the second is
smaller (fewer sequences, shorter contexts) and must not see the first
call's leftovers. A captured call replays with new context lengths.
(Oversized calls are refused before any HIP call: tests/test_capi.py.)
"""

import math

import pytest
import torch

from microinfer_amd import _lib
from microinfer_amd.layer.hip_paged_attention import hip_paged_decode
from microinfer_amd.worker.kv_cache import KVCache
from microinfer_amd.workloads import QWEN3_06B, make_decode_batch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def noalloc_decode(new_k, new_v, q, kc, vc, tables, lens, scale):
    out = torch.empty_like(q)
    num_seqs, hq, d = q.shape
    num_blocks, block_size, hkv, _ = kc.shape
    lib = _lib.load()
    status = lib.mi_paged_decode_append_noalloc(
        new_k.data_ptr(), new_k.stride(0), new_k.stride(1),
        new_v.data_ptr(), new_v.stride(0), new_v.stride(1),
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
        kc.stride(0), kc.stride(1), kc.stride(2),
        tables.data_ptr(), tables.stride(0), tables.shape[1], lens.data_ptr(),
        out.data_ptr(), out.stride(0), out.stride(1),
        num_seqs, hq, hkv, d, block_size, num_blocks, 0, scale,
        _lib.dtype_code(q.dtype), _lib.stream_handle(q.device))
    _lib.check(status, "mi_paged_decode_append_noalloc")
    return out


def one_case(num_seqs, ctx_lo, ctx_hi, seed):
    pool = 4096
    batch = make_decode_batch(num_seqs=num_seqs, ctx_lo=ctx_lo, ctx_hi=ctx_hi, pool_blocks=pool,
                              draw_pools=False, seed=seed, **QWEN3_06B)
    print(f"case: {num_seqs} sequences, contexts U[{ctx_lo},{ctx_hi}], seed {seed}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    cache = KVCache(1, pool, 16, 8, 128, dtype=torch.bfloat16, device=DEV)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, generator=gen, device=DEV))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, generator=gen, device=DEV))
    kc, vc = cache.keys[0], cache.values[0]
    kc2, vc2 = kc.clone(), vc.clone()  # same layout (clone keeps strides)
    q = torch.randn((num_seqs, 16, 128), generator=gen, device=DEV).to(torch.bfloat16)
    new_k = torch.randn((num_seqs, 8, 128), generator=gen, device=DEV).to(torch.bfloat16)
    new_v = torch.randn((num_seqs, 8, 128), generator=gen, device=DEV).to(torch.bfloat16)
    tables = torch.tensor(batch.block_tables, device=DEV)
    lens = torch.tensor(batch.context_lens, device=DEV)
    scale = 1 / math.sqrt(128)
    expected = hip_paged_decode(q, kc, vc, tables, lens, scale=scale, new_keys=new_k,
                                new_values=new_v)
    got = noalloc_decode(new_k, new_v, q, kc2, vc2, tables, lens, scale)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), expected.view(torch.int16))
    assert torch.equal(kc2.view(torch.int16), kc.view(torch.int16))
    assert torch.equal(vc2.view(torch.int16), vc.view(torch.int16))


def test_noalloc_matches_the_workspace_entry_point_twice():
    one_case(32, 128, 2048, seed=0)  # the 0.6B decode batch (split sequences)
    one_case(5, 16, 700, seed=1)     # smaller: fewer sequences, shorter contexts


def test_noalloc_under_graph_capture_tracks_context_lens():
    # Captured once (after an eager call has looked up this device's scratch),
    # replayed with two different context_lens: the plan kernel inside the
    # graph re-plans from the new lengths and re-zeroes its counters, so each
    # replay equals the workspace entry point run eagerly on the same inputs,
    # bit for bit (output and appended cache rows).
    from microinfer_amd.runner import capture_graph

    pool, num_seqs, width = 2048, 12, 64
    gen = torch.Generator(device=DEV).manual_seed(5)
    cache = KVCache(1, pool, 16, 8, 128, dtype=torch.bfloat16, device=DEV)
    cache.keys[0].copy_(torch.randn(cache.keys[0].shape, generator=gen, device=DEV))
    cache.values[0].copy_(torch.randn(cache.values[0].shape, generator=gen, device=DEV))
    kc, vc = cache.keys[0], cache.values[0]
    ref_k, ref_v = kc.clone(), vc.clone()
    q = torch.randn((num_seqs, 16, 128), generator=gen, device=DEV).to(torch.bfloat16)
    new_k = torch.randn((num_seqs, 8, 128), generator=gen, device=DEV).to(torch.bfloat16)
    new_v = torch.randn((num_seqs, 8, 128), generator=gen, device=DEV).to(torch.bfloat16)
    tables = torch.randperm(pool, generator=torch.Generator().manual_seed(5))[
        :num_seqs * width].to(torch.int32).reshape(num_seqs, width).to(DEV)
    lens = torch.full((num_seqs,), 100, dtype=torch.int32, device=DEV)
    scale = 1 / math.sqrt(128)
    noalloc_decode(new_k, new_v, q, kc, vc, tables, lens, scale)  # eager: scratch looked up
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph, stream=side):
        out = noalloc_decode(new_k, new_v, q, kc, vc, tables, lens, scale)
    torch.cuda.synchronize()
    rng = torch.Generator().manual_seed(6)
    for lo, hi in ((900, 1024), (1, 300)):
        print(f"replay: contexts U[{lo},{hi}]", flush=True)
        lens.copy_(torch.randint(lo, hi + 1, (num_seqs,), generator=rng, dtype=torch.int32))
        ref_k.copy_(kc)
        ref_v.copy_(vc)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        expected = hip_paged_decode(q, ref_k, ref_v, tables, lens, scale=scale, new_keys=new_k,
                                    new_values=new_v)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), expected.view(torch.int16))
        assert torch.equal(kc.view(torch.int16), ref_k.view(torch.int16))
        assert torch.equal(vc.view(torch.int16), ref_v.view(torch.int16))
