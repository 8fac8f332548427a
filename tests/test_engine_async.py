"""The asynchronous frontend (microinfer_amd.engine.async_engine) on the CPU.

Restates the reference's async cases (tests/components/test_async_engine.py:
62-113: streaming to a length finish, abort of a running request, the
backpressure limit and release after collect) and its recovery cases
(tests/integration/test_engine_recovery.py:44-90: a failed step releases
every admitted request and the engine serves a new one afterwards; generation
stops at the cache's capacity; abort in the middle of a chunked prefill)
through the async layer, with a stand-in runner (no kernels).
"""

import asyncio
import threading

import pytest

from microinfer_amd.engine.async_engine import AsyncEngine, BackpressureError
from microinfer_amd.engine.config import SampleParameter
from microinfer_amd.engine.llm_engine import LLMEngine


class Runner:
    """Token 100 + length for every row; can fail on demand; records threads."""

    def __init__(self):
        self.fail = False
        self.threads = set()
        self.calls = 0

    def run(self, seqs, is_prefill):
        self.threads.add(threading.get_ident())
        self.calls += 1
        if self.fail:
            raise RuntimeError("injected device error")
        return [100 + len(s) for s in seqs]


def make_engine(scheduler_factory, **limits):
    scheduler, manager = scheduler_factory(**limits)
    runner = Runner()
    return LLMEngine(scheduler, runner), runner, manager


def params(n, **kw):
    return SampleParameter(max_tokens=n, ignore_eos=True, **kw)


def test_streams_to_length_and_aborts(scheduler_factory):
    engine, runner, manager = make_engine(scheduler_factory, num_blocks=16, max_model_len=64)

    async def scenario():
        frontend = AsyncEngine(engine, max_waiting=2)
        request = await frontend.add_request([1, 2], params(4))
        events = [e async for e in frontend.stream(request)]
        assert [len(e.token_ids) for e in events] == [1, 2, 3, 4]
        assert events[-1].finished and events[-1].finish_reason == "length"
        assert events[-1].token_ids == request.token_ids == (102, 103, 104, 105)
        assert not any(e.finished for e in events[:-1])

        long = await frontend.add_request([3], params(100))
        first = await anext(frontend.stream(long))
        assert not first.finished
        assert await frontend.abort(long.seq_id)
        terminal = await frontend.collect(long)
        assert terminal.finished and terminal.finish_reason == "abort"
        await frontend.stop()
        assert not manager.used_block_ids
        assert frontend.stats()["active_requests"] == 0

    asyncio.run(scenario())


def test_backpressure_and_release(scheduler_factory):
    engine, _, _ = make_engine(scheduler_factory)

    async def scenario():
        frontend = AsyncEngine(engine, max_waiting=1)
        request = await frontend.add_request([1], params(2))
        with pytest.raises(BackpressureError):
            await frontend.add_request([2], params(2))
        await frontend.collect(request)  # releases the finished request
        second = await frontend.add_request([2], params(1))
        out = await frontend.collect(second)
        assert out.token_ids == (101,) and out.finish_reason == "length"
        await frontend.stop()
        with pytest.raises(RuntimeError, match="stopping"):
            await frontend.add_request([3], params(1))

    asyncio.run(scenario())


def test_bad_arguments(scheduler_factory):
    engine, _, _ = make_engine(scheduler_factory)
    with pytest.raises(ValueError):
        AsyncEngine(engine, max_waiting=0)

    async def scenario():
        frontend = AsyncEngine(engine)
        with pytest.raises(TypeError):
            await frontend.add_request([1], {"max_tokens": 2})
        with pytest.raises(ValueError):
            await frontend.add_request([], params(1))
        await frontend.stop()

    asyncio.run(scenario())


def test_failed_step_aborts_every_stream_and_engine_recovers(scheduler_factory):
    # test_engine_recovery.py:44-67 through the async layer: the step fails,
    # every open stream ends with "abort", no block stays allocated, and a
    # new request is served once the runner works again.
    engine, runner, manager = make_engine(scheduler_factory, max_num_batched_tokens=2)

    async def scenario():
        frontend = AsyncEngine(engine, max_waiting=8)
        runner.fail = True
        a = await frontend.add_request([1, 2, 3], params(2))
        b = await frontend.add_request([4], params(2))
        outs = [await frontend.collect(a), await frontend.collect(b)]
        assert all(o.finished and o.finish_reason == "abort" for o in outs)
        assert "injected" in frontend.stats()["last_error"]
        assert engine.is_finished() and not manager.used_block_ids
        runner.fail = False
        again = await frontend.generate([1, 2, 3], params(2))
        assert again.token_ids == (103, 104) and again.finish_reason == "length"
        await frontend.stop()

    asyncio.run(scenario())


def test_generation_stops_at_cache_capacity(scheduler_factory):
    # test_engine_recovery.py:70-75: two 4-token blocks hold 8 tokens, so a
    # 3-token prompt gets 5 tokens whatever max_tokens asks for.
    engine, _, manager = make_engine(scheduler_factory, num_blocks=2, max_model_len=16)

    async def scenario():
        frontend = AsyncEngine(engine)
        out = await frontend.generate([1, 2, 3], params(100, greedy=True))
        assert len(out.token_ids) == 5 and out.finish_reason == "length"
        await frontend.stop()
        assert not manager.used_block_ids

    asyncio.run(scenario())


def test_abort_during_chunked_prefill(scheduler_factory):
    # test_engine_recovery.py:84-91: a 5-token prompt prefilled 2 tokens a
    # step is aborted after its first chunk; its blocks are freed and the
    # stream ends with "abort" without any sampled token.
    engine, runner, manager = make_engine(scheduler_factory, max_num_batched_tokens=2)

    async def scenario():
        frontend = AsyncEngine(engine)
        request = await frontend.add_request([1, 2, 3, 4, 5], params(3))
        while runner.calls == 0:
            await asyncio.sleep(0)
        assert await frontend.abort(request.seq_id)
        assert not await frontend.abort(request.seq_id)
        out = await frontend.collect(request)
        assert out.finish_reason == "abort" and out.token_ids == ()
        assert not manager.used_block_ids
        await frontend.stop()

    asyncio.run(scenario())


def test_concurrent_requests_match_the_synchronous_engine(scheduler_factory):
    # Requests admitted from concurrent coroutines get the completions the
    # synchronous loop gives the same prompts, and every step runs on the one
    # worker thread.
    prompts = [[1, 2, 3], [4], [5, 6, 7, 8, 9], [10, 11]]
    engine, _, _ = make_engine(scheduler_factory, num_blocks=16, max_num_batched_tokens=5)
    expected = engine.generate(prompts, params(3))
    engine, runner, manager = make_engine(scheduler_factory, num_blocks=16,
                                          max_num_batched_tokens=5)

    async def scenario():
        frontend = AsyncEngine(engine)
        outs = await asyncio.gather(*(frontend.generate(p, params(3)) for p in prompts))
        await frontend.stop()
        return outs

    outs = asyncio.run(scenario())
    assert [list(o.token_ids) for o in outs] == expected
    assert len(runner.threads) == 1 and threading.get_ident() not in runner.threads
    assert not manager.used_block_ids


def test_text_from_a_tokenizer(scheduler_factory):
    class Digits:
        def decode(self, ids):
            return "".join(str(i % 10) for i in ids)

    engine, _, _ = make_engine(scheduler_factory)

    async def scenario():
        frontend = AsyncEngine(engine, tokenizer=Digits())
        request = await frontend.add_request([1, 2], params(3))
        events = [e async for e in frontend.stream(request)]
        assert "".join(e.text for e in events) == "234"
        assert request.text == "234"
        await frontend.stop()

    asyncio.run(scenario())


class StepInterrupted(BaseException):
    """Not an Exception: what a cancellation or interrupt raising in a step looks like."""


def test_base_exception_in_a_step_ends_every_stream(scheduler_factory):
    # The engine thread catches BaseException too: every admitted request's
    # consumer gets a terminal "abort" event (none waits forever), the engine
    # is left empty, and the thread serves the next request.
    engine, runner, manager = make_engine(scheduler_factory, num_blocks=16)
    run = runner.run

    def interrupted(seqs, is_prefill):
        if runner.calls >= 1:
            runner.calls += 1
            raise StepInterrupted("interrupted mid-step")
        return run(seqs, is_prefill)

    runner.run = interrupted

    async def scenario():
        frontend = AsyncEngine(engine, max_waiting=8)
        a = await frontend.add_request([1, 2], params(5))
        b = await frontend.add_request([3], params(5))
        outs = await asyncio.wait_for(asyncio.gather(frontend.collect(a), frontend.collect(b)), 10)
        assert all(o.finished and o.finish_reason == "abort" for o in outs)
        assert "interrupted" in frontend.stats()["last_error"]
        assert engine.is_finished() and not manager.used_block_ids
        runner.run = run
        again = await asyncio.wait_for(frontend.generate([4], params(2)), 10)
        assert again.finish_reason == "length" and len(again.token_ids) == 2
        await frontend.stop()

    asyncio.run(scenario())


def test_stop_during_a_step_ends_every_stream(scheduler_factory):
    # stop() while the engine thread is inside a step: the step finishes, the
    # thread then aborts what is left, and every consumer gets "abort".
    engine, runner, manager = make_engine(scheduler_factory, num_blocks=16)
    armed, entered, release = threading.Event(), threading.Event(), threading.Event()
    run = runner.run

    def slow(seqs, is_prefill):
        if armed.is_set():  # the first step after every admission
            entered.set()
            release.wait(10)
        return run(seqs, is_prefill)

    runner.run = slow

    async def scenario():
        frontend = AsyncEngine(engine, max_waiting=8)
        requests = [await frontend.add_request([i + 1], params(50)) for i in range(3)]
        armed.set()
        consumers = [asyncio.ensure_future(frontend.collect(r)) for r in requests]
        await asyncio.get_running_loop().run_in_executor(None, entered.wait, 10)
        stopping = asyncio.ensure_future(frontend.stop())
        await asyncio.sleep(0.05)
        release.set()
        await asyncio.wait_for(stopping, 10)
        outs = await asyncio.wait_for(asyncio.gather(*consumers), 10)
        assert all(o.finished and o.finish_reason == "abort" for o in outs)
        assert engine.is_finished() and not manager.used_block_ids
        assert frontend.stats()["active_requests"] == 0

    asyncio.run(scenario())
