"""Requests and their lifecycle (tokserve/scheduler/request.py).

A request is a prompt, a generation config and a lifecycle: WAITING ->
RUNNING -> FINISHED, or CANCELLED from either of the first two. The allowed
source states of each transition are one table (`_SOURCES`); every state
change goes through `_move`, which raises the reference's messages. While
RUNNING, the request first completes its prefill, then takes one token per
step until EOS or max_new_tokens: the stop rule is one function of the token
just taken and the count.

The prompt is kept as a read-only int64 NumPy array (the packed metadata
builder concatenates prompts without conversion) and the generated tokens as a
host list of ints (the batched executor reads a whole iteration's tokens back
in one copy and appends plain ints); the (1, n) tensors the reference API
exposes are built on the prompt's device when asked for.
"""

from __future__ import annotations

from enum import Enum

import numpy as np
import torch

from tokserve_amd.generation.types import GenerationConfig, GenerationResult, StopReason

__all__ = ["RequestState", "ScheduledRequest"]

_INTEGER_DTYPES = frozenset((torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8))


class RequestState(str, Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"
    CANCELLED = "cancelled"

    def __str__(self) -> str:
        return self.value


_SOURCES = {
    RequestState.RUNNING: (RequestState.WAITING,),
    RequestState.FINISHED: (RequestState.RUNNING,),
    RequestState.CANCELLED: (RequestState.WAITING, RequestState.RUNNING),
}


def _stop_reason(token: int, produced: int, config: GenerationConfig) -> StopReason | None:
    """Why generation ends after taking `token` as the produced-th output, if it does."""

    if config.eos_token_id is not None and token == config.eos_token_id:
        return "eos"
    if produced >= config.max_new_tokens:
        return "max_new_tokens"
    return None


class ScheduledRequest:
    """One validated generation request managed by the scheduler."""

    def __init__(self, request_id: str, input_ids: torch.Tensor,
                 generation_config: GenerationConfig) -> None:
        for bad, message in (
            (not request_id, "request_id must be nonempty"),
            (input_ids.ndim != 2 or input_ids.shape[0] != 1, "input_ids must have shape (1, T)"),
        ):
            if bad:
                raise ValueError(message)
        if input_ids.shape[1] < 1:
            raise ValueError("input_ids must contain at least one token")
        if input_ids.dtype not in _INTEGER_DTYPES:
            raise TypeError("input_ids must contain integers")
        self.request_id = request_id
        self.generation_config = generation_config
        self._prompt_ids = input_ids.clone()
        self._prompt = input_ids[0].cpu().numpy().astype(np.int64)
        self._prompt.flags.writeable = False
        self._generated: list[int] = []
        self._state = RequestState.WAITING
        self._prefilled = False
        self._stop: StopReason | None = None
        self._result: GenerationResult | None = None
        self._generator: torch.Generator | None = None
        if generation_config.do_sample and generation_config.seed is not None:
            self._generator = torch.Generator(device=input_ids.device)
            self._generator.manual_seed(generation_config.seed)

    # ----------------------------------------------------------- reading

    @property
    def input_ids(self) -> torch.Tensor:
        return self._prompt_ids.clone()

    @property
    def prompt_array(self) -> np.ndarray:
        """The prompt as int64 (read-only)."""

        return self._prompt

    @property
    def prompt_tokens(self) -> tuple[int, ...]:
        return tuple(self._prompt.tolist())

    @property
    def generated_tokens(self) -> tuple[int, ...]:
        return tuple(self._generated)

    @property
    def generated_token_ids(self) -> torch.Tensor:
        return self._ids(self._generated)

    @property
    def last_token(self) -> int:
        """The most recently generated token (the next decode input)."""

        return self._generated[-1]

    @property
    def state(self) -> RequestState:
        return self._state

    @property
    def result(self) -> GenerationResult | None:
        return self._result

    @property
    def prefill_complete(self) -> bool:
        return self._prefilled

    @property
    def decode_ready(self) -> bool:
        return (self._state is RequestState.RUNNING and self._prefilled
                and bool(self._generated) and self._stop is None)

    @property
    def next_input_token(self) -> torch.Tensor:
        if not self.decode_ready:
            raise RuntimeError("request is not decode-ready")
        return self._ids(self._generated[-1:])

    @property
    def sequence_length(self) -> int:
        return self._prompt.size + len(self._generated)

    @property
    def num_generated_tokens(self) -> int:
        return len(self._generated)

    @property
    def completion_reason(self) -> StopReason | None:
        return self._stop

    @property
    def sampling_generator(self) -> torch.Generator | None:
        return self._generator

    # ------------------------------------------------------- transitions

    def mark_running(self) -> None:
        self._move(RequestState.RUNNING)

    def mark_prefill_complete(self) -> None:
        self._expect(RequestState.RUNNING)
        if self._prefilled:
            raise RuntimeError("prefill is already complete")
        self._prefilled = True
        if self.generation_config.max_new_tokens == 0:
            self._stop = "max_new_tokens"

    def append_generated_token(self, token: int | torch.Tensor) -> None:
        """Record one generated token: an int, or a (1, 1) tensor of the prompt's dtype
        and device."""

        self._expect(RequestState.RUNNING)
        if isinstance(token, torch.Tensor):
            token = self._token_from_tensor(token)
        if not self._prefilled:
            raise RuntimeError("prefill must complete before generating tokens")
        if self._stop is not None:
            raise RuntimeError("request has already completed generation")
        token = int(token)
        self._generated.append(token)
        self._stop = _stop_reason(token, len(self._generated), self.generation_config)

    def build_result(self) -> GenerationResult:
        self._expect(RequestState.RUNNING)
        if self._stop is None:
            raise RuntimeError("request has not reached a completion condition")
        generated = self.generated_token_ids
        return GenerationResult(token_ids=torch.cat((self._prompt_ids, generated), dim=1),
                                generated_token_ids=generated, stop_reason=self._stop)

    def mark_finished(self, result: GenerationResult | None = None) -> None:
        self._expect(RequestState.RUNNING)
        if result is not None:
            self._generated = [int(t) for t in result.generated_token_ids[0].tolist()]
            self._result = result
        self._move(RequestState.FINISHED)

    def cancel(self) -> None:
        if self._state not in _SOURCES[RequestState.CANCELLED]:
            raise RuntimeError(f"cannot cancel request in state {self._state.value}")
        self._move(RequestState.CANCELLED)

    # ----------------------------------------------------------- helpers

    def _move(self, target: RequestState) -> None:
        sources = _SOURCES[target]
        if self._state not in sources:
            self._expect(sources[0])
        self._state = target

    def _expect(self, state: RequestState) -> None:
        if self._state is not state:
            raise RuntimeError(f"request must be {state.value}, not {self._state.value}")

    def _token_from_tensor(self, token: torch.Tensor) -> int:
        if token.shape != (1, 1):
            raise ValueError("token_ids must have shape (1, 1)")
        if token.dtype != self._prompt_ids.dtype:
            raise TypeError("generated tokens must match the prompt dtype")
        if token.device != self._prompt_ids.device:
            raise ValueError("generated tokens must match the prompt device")
        return int(token.item())

    def _ids(self, tokens: list[int]) -> torch.Tensor:
        return torch.tensor([tokens], dtype=self._prompt_ids.dtype,
                            device=self._prompt_ids.device).view(1, len(tokens))
