"""Requests and their lifecycle (tokserve/scheduler/request.py).

The lifecycle and its checks follow the reference: WAITING -> RUNNING ->
FINISHED (or CANCELLED); a running request first completes its prefill, then
appends one generated token per decode step until EOS or max_new_tokens.
Generated tokens are kept as a host list (the batched executor reads every
iteration's tokens back in one copy) and exposed as (1, n) tensors on the
prompt's device.
"""

from __future__ import annotations

from enum import Enum

import numpy as np
import torch

from tokserve_amd.generation.types import GenerationConfig, GenerationResult, StopReason

__all__ = ["RequestState", "ScheduledRequest"]

_INTEGER_DTYPES = (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8)


class RequestState(str, Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"
    CANCELLED = "cancelled"

    def __str__(self) -> str:
        return self.value


class ScheduledRequest:
    """One validated generation request managed by the scheduler."""

    def __init__(self, request_id: str, input_ids: torch.Tensor,
                 generation_config: GenerationConfig) -> None:
        if not request_id:
            raise ValueError("request_id must be nonempty")
        if input_ids.ndim != 2 or input_ids.shape[0] != 1:
            raise ValueError("input_ids must have shape (1, T)")
        if input_ids.shape[1] < 1:
            raise ValueError("input_ids must contain at least one token")
        if input_ids.dtype not in _INTEGER_DTYPES:
            raise TypeError("input_ids must contain integers")
        self.request_id = request_id
        self.generation_config = generation_config
        self._input_ids = input_ids.clone()
        self._prompt: tuple[int, ...] = tuple(int(t) for t in input_ids[0].tolist())
        self._prompt_array = np.asarray(self._prompt, dtype=np.int64)
        self._generated: list[int] = []
        self._state = RequestState.WAITING
        self._result: GenerationResult | None = None
        self._prefill_complete = False
        self._completion_reason: StopReason | None = None
        self._generator: torch.Generator | None = None
        if generation_config.do_sample and generation_config.seed is not None:
            self._generator = torch.Generator(device=input_ids.device)
            self._generator.manual_seed(generation_config.seed)

    # ------------------------------------------------------------- properties

    @property
    def input_ids(self) -> torch.Tensor:
        return self._input_ids.clone()

    @property
    def prompt_tokens(self) -> tuple[int, ...]:
        return self._prompt

    @property
    def prompt_array(self) -> np.ndarray:
        """The prompt as an int64 NumPy array (read-only use)."""

        return self._prompt_array

    @property
    def last_token(self) -> int:
        """The most recently generated token (the next decode input)."""

        return self._generated[-1]

    @property
    def generated_tokens(self) -> tuple[int, ...]:
        return tuple(self._generated)

    @property
    def generated_token_ids(self) -> torch.Tensor:
        return self._as_ids(self._generated)

    @property
    def state(self) -> RequestState:
        return self._state

    @property
    def result(self) -> GenerationResult | None:
        return self._result

    @property
    def prefill_complete(self) -> bool:
        return self._prefill_complete

    @property
    def decode_ready(self) -> bool:
        return (self._state is RequestState.RUNNING and self._prefill_complete
                and bool(self._generated) and self._completion_reason is None)

    @property
    def next_input_token(self) -> torch.Tensor:
        if not self.decode_ready:
            raise RuntimeError("request is not decode-ready")
        return self._as_ids(self._generated[-1:])

    @property
    def sequence_length(self) -> int:
        return len(self._prompt) + len(self._generated)

    @property
    def num_generated_tokens(self) -> int:
        return len(self._generated)

    @property
    def completion_reason(self) -> StopReason | None:
        return self._completion_reason

    @property
    def sampling_generator(self) -> torch.Generator | None:
        return self._generator

    # ------------------------------------------------------------ transitions

    def mark_running(self) -> None:
        self._require_state(RequestState.WAITING)
        self._state = RequestState.RUNNING

    def mark_prefill_complete(self) -> None:
        self._require_state(RequestState.RUNNING)
        if self._prefill_complete:
            raise RuntimeError("prefill is already complete")
        self._prefill_complete = True
        if self.generation_config.max_new_tokens == 0:
            self._completion_reason = "max_new_tokens"

    def append_generated_token(self, token: int | torch.Tensor) -> None:
        """Record one generated token (an int, or a (1, 1) tensor of the prompt's dtype)."""

        self._require_state(RequestState.RUNNING)
        if isinstance(token, torch.Tensor):
            if token.shape != (1, 1):
                raise ValueError("token_ids must have shape (1, 1)")
            if token.dtype != self._input_ids.dtype:
                raise TypeError("generated tokens must match the prompt dtype")
            if token.device != self._input_ids.device:
                raise ValueError("generated tokens must match the prompt device")
            token = int(token.item())
        if not self._prefill_complete:
            raise RuntimeError("prefill must complete before generating tokens")
        if self._completion_reason is not None:
            raise RuntimeError("request has already completed generation")
        self._generated.append(int(token))
        eos = self.generation_config.eos_token_id
        if eos is not None and token == eos:
            self._completion_reason = "eos"
        elif len(self._generated) >= self.generation_config.max_new_tokens:
            self._completion_reason = "max_new_tokens"

    def build_result(self) -> GenerationResult:
        self._require_state(RequestState.RUNNING)
        if self._completion_reason is None:
            raise RuntimeError("request has not reached a completion condition")
        generated = self.generated_token_ids
        return GenerationResult(token_ids=torch.cat((self._input_ids, generated), dim=1),
                                generated_token_ids=generated,
                                stop_reason=self._completion_reason)

    def mark_finished(self, result: GenerationResult | None = None) -> None:
        self._require_state(RequestState.RUNNING)
        if result is not None:
            self._generated = [int(t) for t in result.generated_token_ids[0].tolist()]
            self._result = result
        self._state = RequestState.FINISHED

    def cancel(self) -> None:
        if self._state not in (RequestState.WAITING, RequestState.RUNNING):
            raise RuntimeError(f"cannot cancel request in state {self._state.value}")
        self._state = RequestState.CANCELLED

    def _require_state(self, expected: RequestState) -> None:
        if self._state is not expected:
            raise RuntimeError(f"request must be {expected.value}, not {self._state.value}")

    def _as_ids(self, tokens: list[int]) -> torch.Tensor:
        return torch.tensor([tokens], dtype=self._input_ids.dtype,
                            device=self._input_ids.device).view(1, len(tokens))
