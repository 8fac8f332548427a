"""The allocation-free decode entry point (mi_paged_decode_append_noalloc)
against mi_paged_decode_append, through the C ABI.

Both run the same kernels and, given the same context lengths, the same
partition plan, so outputs and appended cache rows must be bit-identical.
Two calls in a row share the library's static scratch: the second is
smaller (fewer sequences, shorter contexts) and must not see the first
call's leftovers. Oversized calls are refused before any launch.
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


def test_noalloc_refuses_calls_beyond_its_scratch():
    lib = _lib.load()
    room = lib.mi_paged_decode_noalloc_max_bytes()
    assert room > 0
    # 4096 sequences of a 128-query-head layer need far more than the scratch.
    assert lib.mi_paged_decode_workspace_bytes(4096, 128, 16, 256, 0) > room
    fake = 256
    status = lib.mi_paged_decode_append_noalloc(
        fake, 4096, 256, fake, 4096, 256, fake, 32768, 256, fake, fake, 65536, 4096, 256,
        fake, 1, 1, fake, fake, 32768, 256, 4096, 128, 16, 256, 16, 64, 0, 1.0, 2, None)
    assert status == 3 and "scratch" in _lib.last_error()
