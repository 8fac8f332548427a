"""Asynchronous request frontend over the synchronous engine.

Counterpart of ``AsyncEngine`` (microinfer/engine/async_engine.py:46-209):
callers admit requests from coroutines and read per-request event streams;
one background task drives ``LLMEngine.step_events``. Semantics kept:

* ``add_request`` admits under the same lock the step runs under, so the
  scheduler is never mutated while a step executes; ``BackpressureError``
  when ``max_waiting`` requests are already tracked (:67-89);
* every step's updates become ``StreamEvent``s on the owning request's queue,
  a terminal event (``finished=True``) closes a stream (:187-209);
* ``abort`` removes a request from the engine and closes its stream with
  reason ``"abort"`` (:91-107); ``release`` drops the bookkeeping of a
  finished request (:109-115), which ``stream`` / ``collect`` do themselves;
* a step that raises closes every open stream with an ``"abort"`` event and
  records the error in ``stats()["last_error"]`` (:173-185); the next
  ``add_request`` starts the loop again;
* ``stop`` ends the loop, aborts what is left and clears the bookkeeping.

Design here: the blocking step runs on ONE dedicated worker thread for the
engine's lifetime (not a pool thread per step), so the GPU work of every step
is issued from the same thread. If ``stream`` is given, the worker makes it
its current torch stream once, at start-up; the HIP library reads the current
stream at call time, so every kernel of every step lands on that stream.
After a failed step the requests that were not part of it are aborted in the
engine too, so a later request starts from an empty, consistent engine.
Token ids only: text is produced when a ``tokenizer`` with ``decode`` is
given (the reference's incremental detokenizer is outside this path).
"""

from __future__ import annotations

import asyncio
import logging
import time
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field

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


@dataclass
class AsyncRequest:
    seq_id: int
    prompt_tokens: int
    queue: asyncio.Queue = field(repr=False)
    created_at: float = field(default_factory=time.monotonic)
    token_ids: tuple[int, ...] = ()
    text: str = ""
    finished: bool = False
    finish_reason: str | None = None

    def close(self, reason: str) -> None:
        """Mark finished and post the terminal event (once)."""
        if self.finished:
            return
        self.finished = True
        self.finish_reason = reason
        self.queue.put_nowait(StreamEvent(self.seq_id, self.token_ids, "", True, reason))

    async def stream(self):
        while True:
            event = await self.queue.get()
            yield event
            if event.finished:
                return


class AsyncEngine:
    def __init__(self, engine, *, max_waiting: int = 128, stream=None, tokenizer=None):
        if type(max_waiting) is not int or max_waiting <= 0:
            raise ValueError("max_waiting must be a positive integer")
        self.engine = engine
        self.max_waiting = max_waiting
        self.tokenizer = tokenizer
        self._stream = stream
        self._worker: ThreadPoolExecutor | None = None
        self._lock = asyncio.Lock()
        self._wakeup = asyncio.Event()
        self._task: asyncio.Task | None = None
        self._requests: dict[int, AsyncRequest] = {}
        self._stopping = False
        self._error: BaseException | None = None

    # -- the worker thread ----------------------------------------------------
    def _start_worker(self) -> ThreadPoolExecutor:
        if self._worker is None:
            init = None
            if self._stream is not None:
                import torch

                stream = self._stream

                def init():
                    torch.cuda.set_stream(stream)

            self._worker = ThreadPoolExecutor(max_workers=1, thread_name_prefix="mi-engine",
                                              initializer=init)
        return self._worker

    def _ensure_loop(self) -> None:
        if self._task is None or self._task.done():
            self._task = asyncio.get_running_loop().create_task(self._run_loop())

    # -- requests -------------------------------------------------------------
    async def add_request(self, prompt, sampling_params: SampleParameter) -> AsyncRequest:
        """Admit one request (a list of token ids) and return its stream handle."""
        if not isinstance(sampling_params, SampleParameter):
            raise TypeError("sampling_params must be a SampleParameter")
        async with self._lock:
            if self._stopping:
                raise RuntimeError("AsyncEngine is stopping")
            if len(self._requests) >= self.max_waiting:
                raise BackpressureError(
                    f"{len(self._requests)} requests already active (max_waiting="
                    f"{self.max_waiting})")
            seq = Sequence(list(prompt), sampling_params)
            self.engine.add_request(seq)
            request = AsyncRequest(seq.seq_id, seq.num_prompt_tokens, asyncio.Queue())
            self._requests[seq.seq_id] = request
            self._wakeup.set()
            self._ensure_loop()
            return request

    async def abort(self, seq_id: int) -> bool:
        async with self._lock:
            removed = self.engine.abort(seq_id)
            request = self._requests.get(seq_id)
            if request is not None:
                request.close("abort")
            return removed

    async def release(self, seq_id: int) -> None:
        """Forget a finished request (after its consumer read the last event)."""
        async with self._lock:
            request = self._requests.get(seq_id)
            if request is not None and request.finished:
                del self._requests[seq_id]

    async def stream(self, request: AsyncRequest):
        async for event in request.stream():
            yield event
        await self.release(request.seq_id)

    async def collect(self, request: AsyncRequest) -> RequestOutput:
        last = None
        async for event in self.stream(request):
            last = event
        if last is None:
            raise RuntimeError("request stream ended without an event")
        return RequestOutput(request.seq_id, last.token_ids, last.finished, last.finish_reason)

    async def generate(self, prompt, sampling_params: SampleParameter) -> RequestOutput:
        return await self.collect(await self.add_request(prompt, sampling_params))

    def stats(self) -> dict:
        stats = self.engine.stats()
        stats["active_requests"] = len(self._requests)
        stats["max_waiting"] = self.max_waiting
        stats["last_error"] = None if self._error is None else str(self._error)
        return stats

    # -- the step loop ----------------------------------------------------------
    async def _run_loop(self) -> None:
        loop = asyncio.get_running_loop()
        worker = self._start_worker()
        try:
            while True:
                async with self._lock:
                    if self._stopping:
                        return
                    busy = not self.engine.is_finished()
                    if busy:
                        _, _, updates = await loop.run_in_executor(worker,
                                                                   self.engine.step_events)
                        self._publish(updates)
                    else:
                        # Cleared under the lock: an add_request after this
                        # point sets it again, so the wait below cannot miss it.
                        self._wakeup.clear()
                if busy:
                    await asyncio.sleep(0)  # let callers in between steps
                else:
                    await self._wakeup.wait()
        except Exception as exc:  # a failed step ends every open stream
            self._error = exc
            logger.exception("engine step failed")
            async with self._lock:
                for seq_id, request in self._requests.items():
                    self.engine.abort(seq_id)
                    request.close("abort")

    def _publish(self, updates) -> None:
        for seq_id, token_ids, finished, reason in updates:
            request = self._requests.get(seq_id)
            if request is None or request.finished:
                continue
            if not finished and token_ids == request.token_ids:
                continue  # a prompt chunk that sampled nothing
            delta = ""
            if self.tokenizer is not None:
                text = self.tokenizer.decode(list(token_ids))
                delta, request.text = text[len(request.text):], text
            request.token_ids = token_ids
            request.finished = finished
            request.finish_reason = reason
            request.queue.put_nowait(StreamEvent(seq_id, token_ids, delta, finished, reason))

    async def stop(self) -> None:
        self._stopping = True
        self._wakeup.set()
        if self._task is not None:
            await self._task
        async with self._lock:
            for seq_id, request in self._requests.items():
                if not request.finished:
                    self.engine.abort(seq_id)
                    request.close("abort")
            self._requests.clear()
        if self._worker is not None:
            self._worker.shutdown(wait=True)
            self._worker = None
