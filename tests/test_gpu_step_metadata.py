"""Device-built step metadata (mi_step_metadata via microinfer_amd.runner).

Every tensor is compared bit for bit with the oracle's restatement of the
runner's host build (oracle/step_metadata.py, following
microinfer/runner.py:160-215, :298-385, :561-576): the reference's own known
answers (tests/components/test_runner.py:36-74), random prefill and decode
batches at several block sizes, graph pad rows at a [bucket, num_blocks + 1]
table width, and buffer reuse across steps. The graph runner is checked end to
end: replayed fused decode steps of padded buckets must match the same steps
run eagerly and the attention oracle.
"""

import math
import random

import numpy as np
import pytest
import torch

from microinfer_amd.layer.hip_paged_attention import hip_paged_decode
from microinfer_amd.runner import DecodeGraphRunner, StepMetadataBuilder
from oracle.step_metadata import decode_rows, prefill_rows
from tests.support import FakeSeq, max_abs, oracle_decode
from tests.test_oracle_step_metadata import random_batch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def host(t):
    return None if t is None else t.cpu().numpy()


def check_prefill(builder, seqs):
    ids, positions, m = builder.prepare_prefill(seqs)
    want = prefill_rows(seqs, builder.block_size)
    assert ids.dtype == positions.dtype == torch.int64
    assert m.slot_mapping.dtype == m.cu_seqlens_q.dtype == m.cu_seqlens_k.dtype == torch.int32
    assert (host(ids) == want["input_ids"]).all()
    assert (host(positions) == want["positions"]).all()
    assert (host(m.slot_mapping) == want["slot_mapping"]).all()
    assert (host(m.cu_seqlens_q) == want["cu_seqlens_q"]).all()
    assert (host(m.cu_seqlens_k) == want["cu_seqlens_k"]).all()
    assert (m.max_seqlen_q, m.max_seqlen_k) == (want["max_seqlen_q"], want["max_seqlen_k"])
    if want["block_tables"] is None:
        assert m.block_tables is None and m.direct_prefill
    else:
        assert m.block_tables.dtype == torch.int32
        assert np.array_equal(host(m.block_tables), want["block_tables"])
    return ids, positions, m


def test_known_answers():
    # test_runner.py:36-50
    a, b = FakeSeq([10, 11, 12, 13, 14, 15]), FakeSeq([24, 25])
    a.num_cached_tokens, a.num_scheduled_tokens, a.block_table = 3, 3, [2, 0]
    b.num_scheduled_tokens, b.block_table = 2, [5]
    builder = StepMetadataBuilder(4, DEV)
    ids, positions, m = check_prefill(builder, [a, b])
    assert ids.tolist() == [13, 14, 15, 24, 25]
    assert m.slot_mapping.tolist() == [11, 0, 1, 20, 21]
    assert m.block_tables.tolist() == [[2, 0], [5, -1]]
    assert m.context_lens is None and m.is_prefill
    # :53-58
    seq = FakeSeq([1, 2])
    seq.num_scheduled_tokens, seq.block_table = 2, [0]
    _, _, m = check_prefill(builder, [seq])
    assert m.block_tables is None and m.cu_seqlens_k.tolist() == [0, 2]
    # :61-74
    a, b = FakeSeq([1, 2, 3, 4, 5]), FakeSeq([7, 8])
    a.block_table, b.block_table = [2, 0], [1]
    ids, positions, m = builder.prepare_decode([a, b])
    assert ids.tolist() == [5, 8] and positions.tolist() == [4, 1]
    assert m.is_decode and m.cu_seqlens_q is None and m.cu_seqlens_k is None
    assert m.context_lens.tolist() == [5, 2]
    assert m.slot_mapping.tolist() == [0, 5]
    assert m.block_tables.tolist() == [[2, 0], [1, -1]]


@pytest.mark.parametrize("block_size", [1, 3, 16, 64])
def test_random_prefill_batches(block_size):
    rng = random.Random(block_size)
    builder = StepMetadataBuilder(block_size, DEV)
    kept = []
    for n in (1, 4, 17, 64):
        seqs = random_batch(rng, n, block_size, 5000, prefill=True)
        kept.append((seqs, check_prefill(builder, seqs)))
    # Earlier steps' tensors are not overwritten by later steps.
    for seqs, (ids, _, m) in kept:
        want = prefill_rows(seqs, block_size)
        assert (host(ids) == want["input_ids"]).all()
        assert (host(m.slot_mapping) == want["slot_mapping"]).all()


@pytest.mark.parametrize("block_size", [4, 16])
def test_random_decode_batches_reuse_buffers(block_size):
    rng = random.Random(100 + block_size)
    builder = StepMetadataBuilder(block_size, DEV)
    for n in (9, 33, 2, 128, 1):
        seqs = random_batch(rng, n, block_size, 20000, prefill=False)
        ids, positions, m = builder.prepare_decode(seqs)
        width = m.block_tables.shape[1]
        want = decode_rows(seqs, block_size, width=width)
        assert (host(ids) == want["input_ids"]).all()
        assert (host(positions) == want["positions"]).all()
        assert (host(m.slot_mapping) == want["slot_mapping"]).all()
        assert (host(m.context_lens) == want["context_lens"]).all()
        assert np.array_equal(host(m.block_tables), want["block_tables"])


def test_graph_bucket_rows_at_pool_width():
    # A [bucket, num_blocks + 1] table as the graph runner allocates it
    # (runner.py:217-218), with pad rows after the batch.
    num_blocks, block_size, bucket = 4096, 16, 64
    rng = random.Random(5)
    builder = StepMetadataBuilder(block_size, DEV, pad_block_id=num_blocks)
    buffers = builder.pad_buffers(bucket, num_blocks + 1)
    want = decode_rows([], block_size, rows=bucket, width=num_blocks + 1, pad_block=num_blocks)
    assert np.array_equal(host(buffers.block_tables), want["block_tables"])
    assert (host(buffers.slot_mapping) == want["slot_mapping"]).all()
    for n in (50, 64, 3):
        seqs = random_batch(rng, n, block_size, num_blocks, prefill=False)
        builder.fill_decode(buffers, seqs, rows=bucket)
        want = decode_rows(seqs, block_size, rows=bucket, width=num_blocks + 1,
                           pad_block=num_blocks)
        for key in ("input_ids", "positions", "slot_mapping", "context_lens", "block_tables"):
            assert np.array_equal(host(getattr(buffers, key)), want[key]), key


def _attention_forward(kc, vc, banks, num_kv_heads, block_size):
    qbank, kbank, vbank = banks

    def forward(input_ids, positions, metadata):
        q = qbank.index_select(0, input_ids)
        k = kbank.index_select(0, input_ids)
        v = vbank.index_select(0, input_ids)
        plan = metadata.decode_plan(num_kv_heads, block_size)
        return hip_paged_decode(q, kc, vc, metadata.block_tables, metadata.context_lens,
                                plan=plan, new_keys=k, new_values=v)

    return forward


def test_graph_runner_matches_eager_steps():
    torch.manual_seed(0)
    num_blocks, block_size, hq, hkv, d, vocab = 512, 16, 16, 8, 128, 64
    pool = num_blocks + 1  # plus the pad block
    kc = torch.randn(pool, block_size, hkv, d, device=DEV).to(torch.bfloat16)
    vc = torch.randn(pool, block_size, hkv, d, device=DEV).to(torch.bfloat16)
    banks = [torch.randn(vocab, h, d, device=DEV).to(torch.bfloat16) for h in (hq, hkv, hkv)]
    kc_e, vc_e = kc.clone(), vc.clone()

    builder = StepMetadataBuilder(block_size, DEV, pad_block_id=num_blocks)
    graphs = DecodeGraphRunner(builder, _attention_forward(kc, vc, banks, hkv, block_size),
                               max_num_seqs=8, table_width=num_blocks + 1)
    assert [b[0] for b in graphs.buckets] == [1, 2, 4, 8]
    eager_builder = StepMetadataBuilder(block_size, DEV)
    eager = _attention_forward(kc_e, vc_e, banks, hkv, block_size)

    rng = random.Random(1)
    perm = rng.sample(range(num_blocks), num_blocks)
    seqs = []
    for i in range(8):
        s = FakeSeq([rng.randrange(vocab) for _ in range(rng.randint(1, 200))])
        s.block_table = perm[40 * i:40 * i + 20]
        seqs.append(s)
    for step, n in enumerate((3, 5, 8, 1, 6)):
        batch = seqs[:n]
        out_g = graphs.run(batch).clone()
        ids, positions, m = eager_builder.prepare_decode(batch)
        out_e = eager(ids, positions, m)
        assert out_g.shape == (n, hq, d)
        # Pad rows change the step's partition plan, so the two may round
        # differently; both must agree with each other and the oracle.
        assert (out_g.float() - out_e.float()).abs().max().item() <= 2e-2, f"step {step}"
        expected = oracle_decode(banks[0].index_select(0, ids), kc_e, vc_e, m.block_tables,
                                 m.context_lens, 1 / math.sqrt(d))
        assert max_abs(out_g, expected) <= 2e-2
        # Real blocks hold the same rows in both caches; only the pad block differs.
        assert torch.equal(kc[:num_blocks], kc_e[:num_blocks])
        assert torch.equal(vc[:num_blocks], vc_e[:num_blocks])
        for s in batch:  # next step: one more token
            s.token_ids.append(rng.randrange(vocab))
            s.last_token = s.token_ids[-1]
    assert graphs.run(seqs + seqs) is None  # larger than every bucket
