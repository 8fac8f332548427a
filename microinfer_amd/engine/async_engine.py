"""Asynchronous request frontend over the synchronous engine.

Counterpart of ``AsyncEngine`` (microinfer/engine/async_engine.py:46-231).
The behaviour its tests pin is kept: per-request event streams ending in one
terminal event, ``BackpressureError`` past ``max_waiting`` tracked requests,
``abort`` closing a stream with reason ``"abort"``, a failed step closing
every open stream with ``"abort"`` and leaving the error in
``stats()["last_error"]``, and ``stop``.

Design: an **engine thread** owns the ``LLMEngine`` for the frontend's
lifetime; no other thread calls into it. Coroutines never touch the engine:
admissions, aborts and the stop request are commands put in the thread's
inbox, each answered through an ``asyncio`` future, so scheduler mutation
cannot race with a step by construction (no lock is held across a step).
Between two steps the thread applies every queued command, then runs one
``step_events`` and hands the updates to the event loop
(``call_soon_threadsafe``). It starts the next step only after the loop has
published them and run one more iteration (a one-step credit), so callers
woken by an event get in before the next step, as in the reference, and the
thread never runs ahead of the consumers by more than a step.

* If ``stream`` is given, the engine thread makes it its current torch
  stream once, at start-up; the HIP library reads the current stream at call
  time, so every kernel of every step lands on that stream.
* A step that raises (any ``BaseException``) aborts every request the thread
  has admitted and not finished, so the engine is empty and consistent, and
  the thread keeps serving: the next admission runs normally.
* Text is produced only when a ``tokenizer`` with ``decode`` is given (the
  reference's incremental detokenizer is outside this path).
"""

from __future__ import annotations

import asyncio
import collections
import logging
import threading
from dataclasses import dataclass

from microinfer_amd.engine.config import SampleParameter
from microinfer_amd.engine.sequence import Sequence

logger = logging.getLogger(__name__)


class BackpressureError(RuntimeError):
    """Too many requests are tracked by the frontend already."""


@dataclass(frozen=True)
class StreamEvent:
    seq_id: int
    token_ids: tuple[int, ...]
    text: str
    finished: bool
    finish_reason: str | None


@dataclass(frozen=True)
class RequestOutput:
    seq_id: int
    token_ids: tuple[int, ...]
    finished: bool
    finish_reason: str | None


class RequestChannel:
    """Caller-side view of one request: the latest state and its event queue.

    Only the event loop's thread writes to it.
    """

    def __init__(self, seq_id: int, prompt_tokens: int):
        self.seq_id = seq_id
        self.prompt_tokens = prompt_tokens
        self.token_ids: tuple[int, ...] = ()
        self.text = ""
        self.finished = False
        self.finish_reason: str | None = None
        self.events: asyncio.Queue[StreamEvent] = asyncio.Queue()

    def push(self, token_ids: tuple[int, ...], finished: bool, reason: str | None,
             tokenizer) -> None:
        if self.finished:
            return
        if not finished and len(token_ids) == len(self.token_ids):
            return  # a prompt chunk: nothing sampled for this request yet
        delta = ""
        if tokenizer is not None:
            text = tokenizer.decode(list(token_ids))
            delta, self.text = text[len(self.text):], text
        self.token_ids, self.finished, self.finish_reason = token_ids, finished, reason
        self.events.put_nowait(StreamEvent(self.seq_id, token_ids, delta, finished, reason))

    def terminate(self, reason: str) -> None:
        """Post the terminal event with the tokens so far (once)."""
        self.push(self.token_ids, True, reason, None)

    async def events_until_done(self):
        while True:
            event = await self.events.get()
            yield event
            if event.finished:
                return


class _EngineThread(threading.Thread):
    """Runs the engine's commands and steps; reports through the event loop."""

    def __init__(self, frontend: AsyncEngine, loop: asyncio.AbstractEventLoop, stream):
        super().__init__(name="mi-engine", daemon=True)
        self.frontend, self.loop, self.stream = frontend, loop, stream
        self.engine = frontend.engine
        self.cv = threading.Condition()
        self.inbox: collections.deque = collections.deque()
        self.credit = True  # the loop has taken the previous step's updates
        self.live: set[int] = set()  # admitted here, not finished or aborted

    # -- called on the loop's thread -------------------------------------------
    def post(self, kind: str, arg, future: asyncio.Future) -> None:
        with self.cv:
            self.inbox.append((kind, arg, future))
            self.cv.notify()

    def grant(self) -> None:
        with self.cv:
            self.credit = True
            self.cv.notify()

    # -- the thread (the only caller of the engine) ----------------------------
    def report(self, fn, *args) -> bool:
        try:
            self.loop.call_soon_threadsafe(fn, *args)
            return True
        except RuntimeError:  # the loop is closed: nobody is listening any more
            return False

    def can_step(self) -> bool:
        return self.credit and not self.engine.is_finished()

    def run(self) -> None:
        if self.stream is not None:
            import torch

            torch.cuda.set_stream(self.stream)
        while True:
            with self.cv:
                while not self.inbox and not self.can_step():
                    self.cv.wait()
                commands = list(self.inbox)
                self.inbox.clear()
            # Every queued command before the next step.
            for kind, arg, future in commands:
                if kind == "stop":
                    self.shut_down(future)
                    return
                if not self.apply(kind, arg, future):
                    return
            with self.cv:
                ready = self.can_step()
            if ready and not self.step():
                return

    def apply(self, kind: str, arg, future: asyncio.Future) -> bool:
        try:
            if kind == "admit":
                self.engine.add_request(arg)
                self.live.add(arg.seq_id)
                result = arg.seq_id
            else:  # "abort"
                result = self.engine.abort(arg)
                self.live.discard(arg)
        except Exception as exc:  # a refused admission is raised to its caller
            return self.report(self.frontend._settle, future, None, exc, self.engine.stats())
        return self.report(self.frontend._settle, future, result, None, self.engine.stats())

    def step(self) -> bool:
        with self.cv:
            self.credit = False
        try:
            _, _, updates = self.engine.step_events()
        except BaseException as exc:  # noqa: BLE001 - every admitted stream must end
            logger.exception("engine step failed")
            dropped = sorted(self.live)
            for seq_id in dropped:
                self.engine.abort(seq_id)
            self.live.clear()
            with self.cv:
                self.credit = True
            return self.report(self.frontend._fail, exc, dropped, self.engine.stats())
        for seq_id, _, finished, _ in updates:
            if finished:
                self.live.discard(seq_id)
        return self.report(self.frontend._deliver, updates, self.engine.stats())

    def shut_down(self, future: asyncio.Future) -> None:
        for seq_id in sorted(self.live):
            self.engine.abort(seq_id)
        self.live.clear()
        self.report(self.frontend._settle, future, None, None, self.engine.stats())


class AsyncEngine:
    def __init__(self, engine, *, max_waiting: int = 128, stream=None, tokenizer=None):
        if type(max_waiting) is not int or max_waiting <= 0:
            raise ValueError("max_waiting must be a positive integer")
        self.engine = engine
        self.max_waiting = max_waiting
        self.tokenizer = tokenizer
        self._stream = stream
        self._thread: _EngineThread | None = None
        self._channels: dict[int, RequestChannel] = {}
        self._engine_stats = engine.stats()
        self._stopping = False
        self._error: BaseException | None = None

    # -- engine thread plumbing (loop side) ----------------------------------------
    def _thread_for(self, loop: asyncio.AbstractEventLoop) -> _EngineThread:
        if self._thread is None:
            self._thread = _EngineThread(self, loop, self._stream)
            self._thread.start()
        elif self._thread.loop is not loop:
            raise RuntimeError("AsyncEngine is bound to another event loop")
        return self._thread

    async def _command(self, kind: str, arg):
        loop = asyncio.get_running_loop()
        future = loop.create_future()
        self._thread_for(loop).post(kind, arg, future)
        return await future

    def _settle(self, future: asyncio.Future, result, exc, stats) -> None:
        """A command's answer from the engine thread, to its caller."""
        self._engine_stats = stats
        if future.cancelled():
            return
        if exc is not None:
            future.set_exception(exc)
        else:
            future.set_result(result)

    def _deliver(self, updates, stats) -> None:
        """A step's updates: publish them, then grant the next step."""
        self._engine_stats = stats
        for seq_id, token_ids, finished, reason in updates:
            channel = self._channels.get(seq_id)
            if channel is not None:
                channel.push(token_ids, finished, reason, self.tokenizer)
        # One loop iteration later, so the consumers woken above run first.
        asyncio.get_running_loop().call_soon(self._thread.grant)

    def _fail(self, exc: BaseException, dropped: list[int], stats) -> None:
        """A failed step: end the stream of every request it dropped."""
        self._engine_stats = stats
        self._error = exc
        for seq_id in dropped:
            channel = self._channels.get(seq_id)
            if channel is not None:
                channel.terminate("abort")

    # -- requests -------------------------------------------------------------------
    async def add_request(self, prompt, sampling_params: SampleParameter) -> RequestChannel:
        """Admit one request (a list of token ids) and return its stream handle."""
        if not isinstance(sampling_params, SampleParameter):
            raise TypeError("sampling_params must be a SampleParameter")
        if self._stopping:
            raise RuntimeError("AsyncEngine is stopping")
        if len(self._channels) >= self.max_waiting:
            raise BackpressureError(f"{len(self._channels)} requests already tracked "
                                    f"(max_waiting={self.max_waiting})")
        seq = Sequence(list(prompt), sampling_params)
        channel = RequestChannel(seq.seq_id, seq.num_prompt_tokens)
        self._channels[seq.seq_id] = channel  # counts against max_waiting at once
        try:
            await self._command("admit", seq)
        except BaseException:
            del self._channels[seq.seq_id]
            raise
        return channel

    async def abort(self, seq_id: int) -> bool:
        removed = await self._command("abort", seq_id)
        channel = self._channels.get(seq_id)
        if channel is not None:
            channel.terminate("abort")
        return removed

    async def release(self, seq_id: int) -> None:
        """Forget a finished request (after its consumer read the last event)."""
        channel = self._channels.get(seq_id)
        if channel is not None and channel.finished:
            del self._channels[seq_id]

    async def stream(self, request: RequestChannel):
        async for event in request.events_until_done():
            yield event
        await self.release(request.seq_id)

    async def collect(self, request: RequestChannel) -> RequestOutput:
        last = None
        async for event in self.stream(request):
            last = event
        if last is None:
            raise RuntimeError("request stream ended without an event")
        return RequestOutput(request.seq_id, last.token_ids, last.finished, last.finish_reason)

    async def generate(self, prompt, sampling_params: SampleParameter) -> RequestOutput:
        return await self.collect(await self.add_request(prompt, sampling_params))

    def stats(self) -> dict:
        """Engine counters as of the last command or step, plus the frontend's."""
        stats = dict(self._engine_stats)
        stats["active_requests"] = len(self._channels)
        stats["max_waiting"] = self.max_waiting
        stats["last_error"] = None if self._error is None else str(self._error)
        return stats

    async def stop(self) -> None:
        """Abort what is left, end every stream and the engine thread."""
        self._stopping = True
        thread = self._thread
        if thread is not None and thread.is_alive():
            await self._command("stop", None)
            await asyncio.get_running_loop().run_in_executor(None, thread.join)
        for channel in self._channels.values():
            channel.terminate("abort")
        self._channels.clear()
