"""Greedy token selection on the device (mi_greedy_argmax via
microinfer_amd.layer.hip_sampler), compared index for index with the oracle
(oracle/greedy.py) and torch.argmax on the CPU.

Rows are large enough to split into many chunks, so equal maxima and NaNs
are placed in different chunks (the first must win across workgroups); the
row state must be zero after every launch; a captured graph must select the
right tokens on every replay; the graph runner's greedy buckets return the
tokens of their own logits.
"""

import math
import random

import numpy as np
import pytest
import torch

from microinfer_amd.layer import hip_sampler
from microinfer_amd.layer.hip_sampler import greedy_argmax
from microinfer_amd.runner import DecodeGraphRunner, StepMetadataBuilder, capture_graph
from oracle.greedy import greedy_argmax as oracle_argmax
from tests.support import FakeSeq
from tests.test_gpu_step_metadata import _attention_forward

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _check(logits, tokens):
    host = logits.cpu()
    want = oracle_argmax(host.float().numpy())
    np.testing.assert_array_equal(tokens.cpu().numpy(), want)
    np.testing.assert_array_equal(want, torch.argmax(host, dim=-1).numpy())


def _state_is_clear():
    torch.cuda.synchronize()
    return all(int(s.abs().sum()) == 0 for s in hip_sampler._states.values())


def _with_ties(rows, vocab, dtype, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(rows, vocab, generator=gen, device=DEV).to(dtype)
    if vocab > 1:
        top = x.float().amax(-1) + 1
        for r in range(0, rows, 2):  # the same maximum early and late in the row
            i, j = sorted(random.Random(seed * 1000 + r).sample(range(vocab), 2))
            x[r, i] = top[r].to(dtype)
            x[r, j] = top[r].to(dtype)
    return x


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,vocab", [(1, 151936), (32, 151936), (3, 1000), (5, 7),
                                        (7, 4097), (64, 32000), (300, 1), (2, 262144 + 3)])
def test_matches_oracle(dtype, rows, vocab):
    x = _with_ties(rows, vocab, dtype, rows + vocab)
    _check(x, greedy_argmax(x))
    assert _state_is_clear()


@pytest.mark.parametrize("dtype", DTYPES)
def test_special_rows_across_chunks(dtype):
    vocab = 151936
    x = torch.randn(8, vocab, device=DEV).to(dtype)
    x[0] = -math.inf                       # all -inf: index 0
    x[1, 5] = 1000.0
    x[1, vocab - 2] = math.nan             # a late NaN beats an early maximum
    x[2, 140000] = math.nan
    x[2, 70000] = math.nan                 # the first NaN
    x[3] = 0.0
    x[3, :1000] = -0.0                     # -0 ties with +0: index 0
    x[4] = 1.0                             # all equal: index 0
    x[5, vocab - 1] = math.inf
    x[5, 3] = math.inf                     # equal infinities: the first
    x[6, 0] = math.nan                     # NaN at index 0
    x[7] = -math.inf
    x[7, vocab - 1] = -1e30 if dtype == torch.float32 else -60000.0
    tokens = greedy_argmax(x)
    _check(x, tokens)
    assert tokens.tolist()[:8] == [0, vocab - 2, 70000, 0, 0, 3, 0, vocab - 1]


@pytest.mark.parametrize("dtype", DTYPES)
def test_strided_and_misaligned_rows(dtype):
    base = torch.randn(40, 32000 + 72, device=DEV).to(dtype)
    aligned = base[:, :32000]              # row stride 32072 elements
    _check(aligned, greedy_argmax(aligned))
    shifted = base[:, 1:32001]             # rows start off the 16-byte grid
    _check(shifted, greedy_argmax(shifted))
    odd = base[:, 3:1003]
    _check(odd, greedy_argmax(odd))
    column = base[:, 5:6]
    _check(column, greedy_argmax(column))


def test_out_argument_and_shrinking_batches():
    out = torch.full((32,), -7, dtype=torch.int64, device=DEV)
    for rows in (32, 9, 1, 17):
        x = _with_ties(rows, 151936, torch.bfloat16, 100 + rows)
        res = greedy_argmax(x, out=out[:rows])
        assert res.data_ptr() == out.data_ptr()
        _check(x, out[:rows])
        assert _state_is_clear()
    with pytest.raises(ValueError):
        greedy_argmax(x, out=torch.empty(17, dtype=torch.int32, device=DEV))
    with pytest.raises(ValueError):
        greedy_argmax(torch.empty(3, 0, device=DEV))
    with pytest.raises(ValueError):
        greedy_argmax(torch.zeros(3, 4, dtype=torch.int32, device=DEV))
    assert greedy_argmax(torch.empty(0, 5, device=DEV)).shape == (0,)


def test_graph_replays_select_each_new_batch():
    rows, vocab = 32, 151936
    logits = torch.zeros(rows, vocab, dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        greedy_argmax(logits)              # creates this stream's row state
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph, stream=side):
        tokens = greedy_argmax(logits)
    for replay in range(5):
        fresh = _with_ties(rows, vocab, torch.bfloat16, 500 + replay)
        if replay == 3:
            fresh[7, 120000] = math.nan
        logits.copy_(fresh)
        eager = greedy_argmax(fresh)       # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _check(fresh, tokens)
        assert torch.equal(tokens, eager), f"replay {replay}"
    assert _state_is_clear()


def test_graph_runner_greedy_buckets_return_their_tokens():
    torch.manual_seed(0)
    num_blocks, block_size, hq, hkv, d, vocab = 512, 16, 16, 8, 128, 64
    kc = torch.randn(num_blocks + 1, block_size, hkv, d, device=DEV).to(torch.bfloat16)
    vc = torch.randn(num_blocks + 1, block_size, hkv, d, device=DEV).to(torch.bfloat16)
    banks = [torch.randn(vocab, h, d, device=DEV).to(torch.bfloat16) for h in (hq, hkv, hkv)]
    head = torch.randn(hq * d, 5000, device=DEV) / 32
    attend = _attention_forward(kc, vc, banks, hkv, block_size)

    def forward(ids, positions, metadata):  # attention, then logits over 5000 ids
        out = attend(ids, positions, metadata)
        return (out.reshape(out.shape[0], -1).float() @ head).to(torch.bfloat16)

    builder = StepMetadataBuilder(block_size, DEV, pad_block_id=num_blocks)
    graphs = DecodeGraphRunner(builder, forward, max_num_seqs=8,
                               table_width=num_blocks + 1, greedy=True)
    rng = random.Random(3)
    perm = rng.sample(range(num_blocks), num_blocks)
    seqs = []
    for i in range(8):
        s = FakeSeq([rng.randrange(vocab) for _ in range(rng.randint(1, 150))])
        s.block_table = perm[40 * i:40 * i + 20]
        seqs.append(s)
    for n in (3, 8, 1, 6):
        logits, tokens = graphs.run(seqs[:n])
        assert logits.shape == (n, 5000) and tokens.shape == (n,)
        _check(logits, tokens)
        for s in seqs[:n]:
            s.token_ids.append(int(tokens[0]) % vocab)
            s.last_token = s.token_ids[-1]
    assert graphs.run(seqs + seqs) is None
