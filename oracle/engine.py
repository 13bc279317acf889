"""The reference's continuous-batching loop, restated on the CPU (test infrastructure).

Follows tokserve/batching/engine.py:65-131 with the scheduler of
tokserve/scheduler/scheduler.py:58-159, the plan of batching/plan.py:37-65 and
the per-request execution of batching/execution.py:21-101: each step admits
waiting requests FIFO while a slot is free and the unreserved pool holds
ceil((prompt + max_new_tokens) / BS) blocks, plans running requests into
prefill (not yet prefilled) and decode (decode-ready) lists, prefills each in
order (a new sequence allocating ceil(T / BS) blocks, lowest free ids first,
allocator.py:47-66), then decodes each in order (one more block when the new
position crosses a block boundary), selects greedy tokens, and completes
requests at EOS or max_new_tokens, releasing their blocks. The forward is
oracle.model with a contiguous per-sequence cache.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass, field

import torch

from oracle import model as oracle_model


@dataclass
class Request:
    request_id: str
    prompt: list[int]
    max_new_tokens: int
    eos_token_id: int | None = None
    generated: list[int] = field(default_factory=list)
    state: str = "waiting"
    prefilled: bool = False
    done: str | None = None
    blocks: list[int] = field(default_factory=list)
    kv: oracle_model.SequenceKV | None = None
    released_blocks: tuple[int, ...] = ()


@dataclass(frozen=True)
class Record:
    iteration: int
    admitted_ids: tuple[str, ...]
    prefill_ids: tuple[str, ...]
    decode_ids: tuple[str, ...]
    completed_ids: tuple[str, ...]
    active_ids: tuple[str, ...]


class Engine:
    def __init__(self, state: dict[str, torch.Tensor], config: dict, *, num_blocks: int,
                 block_size: int, max_running: int,
                 kv_quant: tuple[float, float] | str | None = None) -> None:
        self.state, self.config = state, config
        self.kv_quant = kv_quant
        self.block_size, self.num_blocks, self.max_running = block_size, num_blocks, max_running
        self.free = list(range(num_blocks))
        self.waiting: list[Request] = []
        self.running: dict[str, Request] = {}
        self.reserved: dict[str, int] = {}
        self.records: list[Record] = []
        self.finished: dict[str, Request] = {}
        # Metrics hook calls in the reference's order (batching/engine.py:70-72,101-104,
        # 124-128; batching/execution.py:39-61,95-96): (hook name, arguments...).
        self.events: list[tuple] = []

    def submit(self, request: Request) -> None:
        self.waiting.append(request)

    def _blocks_for(self, length: int) -> int:
        return (length + self.block_size - 1) // self.block_size

    def _grow(self, request: Request, new_length: int) -> None:
        for _ in range(self._blocks_for(new_length) - len(request.blocks)):
            if not self.free:
                raise RuntimeError("not enough free physical KV blocks remain")
            request.blocks.append(heapq.heappop(self.free))

    def _next_token(self, request: Request, tokens: list[int]) -> int:
        ids = torch.tensor([tokens], dtype=torch.int64)
        logits = oracle_model.forward(self.state, self.config, ids, request.kv, self.kv_quant)
        return int(torch.argmax(logits[0, -1]))

    def _append(self, request: Request, token: int) -> None:
        request.generated.append(token)
        if request.eos_token_id is not None and token == request.eos_token_id:
            request.done = "eos"
        elif len(request.generated) >= request.max_new_tokens:
            request.done = "max_new_tokens"

    def step(self) -> Record:
        slots = self.max_running - len(self.running)
        blocks = max(0, self.num_blocks - sum(self.reserved.values()))
        admitted = []
        while slots > 0 and self.waiting:
            request = self.waiting[0]
            need = 0 if request.max_new_tokens == 0 else self._blocks_for(
                len(request.prompt) + request.max_new_tokens)
            if need > blocks:
                break
            self.waiting.pop(0)
            request.state = "running"
            self.running[request.request_id] = request
            if need:
                self.reserved[request.request_id] = need
                blocks -= need
            admitted.append(request.request_id)
            slots -= 1
        self.events.extend(("request_admitted", rid) for rid in admitted)
        prefill = [r for r in self.running.values() if r.done is None and not r.prefilled]
        decode = [r for r in self.running.values()
                  if r.done is None and r.prefilled and r.generated]
        for request in prefill:
            if request.max_new_tokens == 0:
                request.prefilled = True
                request.done = "max_new_tokens"
                continue
            self.events.append(("prefill_started", request.request_id))
            request.kv = oracle_model.SequenceKV()
            self._grow(request, len(request.prompt))
            token = self._next_token(request, request.prompt)
            self.events.append(("prefill_finished", request.request_id))
            request.prefilled = True
            self._append(request, token)
            self.events.append(("token_produced", request.request_id))
        for request in decode:
            self._grow(request, len(request.prompt) + len(request.generated))
            token = self._next_token(request, [request.generated[-1]])
            self._append(request, token)
            self.events.append(("token_produced", request.request_id))
        completed = []
        for request in list(self.running.values()):
            if request.done is None:
                continue
            self.reserved.pop(request.request_id, None)
            request.released_blocks = tuple(request.blocks)
            for block in request.blocks:
                heapq.heappush(self.free, block)
            request.blocks = []
            request.state = "finished"
            del self.running[request.request_id]
            self.finished[request.request_id] = request
            completed.append(request.request_id)
            self.events.append(("complete_request", request.request_id, request.done))
        record = Record(len(self.records), tuple(admitted), tuple(r.request_id for r in prefill),
                        tuple(r.request_id for r in decode), tuple(completed),
                        tuple(self.running))
        self.records.append(record)
        self.events.append(("record_iteration", len(prefill), len(decode)))
        return record

    def run(self, max_iterations: int = 10_000) -> list[Record]:
        while self.waiting or self.running:
            if len(self.records) >= max_iterations:
                raise RuntimeError("continuous batching exceeded max_iterations")
            self.step()
        return self.records
