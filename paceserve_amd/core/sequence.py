"""The parts of a sequence the KV migration path reads.

Mirrors paceserve/core/datatypes/sequence.py:73-93 (tokens fill logical
blocks left to right, a new block opening when the last is full) and
paceserve/core/datatypes/block.py:12-50 (LogicalTokenBlock).  The worker
reads seq_id, block_size, prompt_token_ids, logical_token_blocks and
state._preemption_count (paceserve/worker/base_worker.py:249-277).  Any object
with those attributes works with this package; this class is a light one for
callers that have no reference Sequence.
"""
from __future__ import annotations

from typing import List, Optional

_BLANK_TOKEN_ID = -1


class LogicalTokenBlock:
    def __init__(self, block_number: int, block_size: int) -> None:
        self.block_number = block_number
        self.block_size = block_size
        self.token_ids = [_BLANK_TOKEN_ID] * block_size
        self.num_tokens = 0

    def is_empty(self) -> bool:
        return self.num_tokens == 0

    def get_num_empty_slots(self) -> int:
        return self.block_size - self.num_tokens

    def is_full(self) -> bool:
        return self.num_tokens == self.block_size

    def append_tokens(self, token_ids: List[int]) -> None:
        if len(token_ids) > self.get_num_empty_slots():
            raise ValueError("more tokens than empty slots")
        self.token_ids[self.num_tokens:self.num_tokens + len(token_ids)] = token_ids
        self.num_tokens += len(token_ids)


class _State:
    def __init__(self) -> None:
        self._preemption_count = 0


class Sequence:
    def __init__(self, seq_id: str, prompt_token_ids: List[int], block_size: int,
                 output_token_ids: Optional[List[int]] = None) -> None:
        self.seq_id = seq_id
        self.prompt_token_ids = list(prompt_token_ids)
        self.output_token_ids: List[int] = []
        self.block_size = block_size
        self.logical_token_blocks: List[LogicalTokenBlock] = []
        self.state = _State()
        self._append_tokens_to_blocks(self.prompt_token_ids)
        for t in output_token_ids or []:
            self.append_token_id(t)

    @classmethod
    def of_length(cls, seq_id: str, num_prompt_tokens: int, block_size: int,
                  num_output_tokens: int = 0) -> "Sequence":
        return cls(seq_id, list(range(num_prompt_tokens)), block_size, list(range(num_output_tokens)))

    def _append_logical_block(self) -> None:
        self.logical_token_blocks.append(LogicalTokenBlock(len(self.logical_token_blocks), self.block_size))

    def _append_tokens_to_blocks(self, token_ids: List[int]) -> None:
        cursor = 0
        while cursor < len(token_ids):
            if not self.logical_token_blocks or self.logical_token_blocks[-1].is_full():
                self._append_logical_block()
            last = self.logical_token_blocks[-1]
            take = last.get_num_empty_slots()
            last.append_tokens(token_ids[cursor:cursor + take])
            cursor += take

    def append_token_id(self, token_id: int) -> None:
        self.output_token_ids.append(token_id)
        self._append_tokens_to_blocks([token_id])

    def get_len(self) -> int:
        return len(self.prompt_token_ids) + len(self.output_token_ids)

    def __repr__(self) -> str:
        return f"Sequence(seq_id={self.seq_id!r}, len={self.get_len()}, blocks={len(self.logical_token_blocks)})"
