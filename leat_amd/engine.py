"""Batched decoding over the cache's slots (leat/engine.py:124-189, 546-583): sequences in slots of
their own, prompts run in chunks, and decode steps of several sequences at once, each batch size
one captured HIP graph.

Decode steps take batches of up to BATCH sequences. Only some batch sizes have a graph: the
powers of 2 below the number of slots (at most BATCH) and that number itself, so a batch of 3
runs in the graph of 4 and one of 5 to 7 in that of 8. Their spare rows are padding: each writes
its key and value at position 0 of a spare cache slot no sequence uses, and attends over that
one key, so no sequence's cache or output changes.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from leat_amd.kernels import MATVEC_TOKENS
from leat_amd.model import GraphStep, LlamaConfig, Model, Weights

BATCH = MATVEC_TOKENS  # the most sequences a decode step runs (leat/engine.py:36)


def batch_sizes(slots: int) -> list[int]:
    """The decode batch sizes with a graph: powers of 2 below min(slots, BATCH), and that."""
    most = min(slots, BATCH)
    return sorted({1 << i for i in range(most.bit_length()) if 1 << i < most} | {most})


def padded_sizes(sizes: list[int]) -> set[int]:
    """The sizes that take padding: those more than one past the size before them."""
    return {n for n, before in zip(sizes[1:], sizes[:-1], strict=True) if n > before + 1}


def plan(count: int, sizes: list[int]) -> list[tuple[int, int]]:
    """A decode step of `count` sequences as batches: (first sequence, batch size) for each
    BATCH-long run of them, the size the smallest graph that holds the run."""
    out = []
    for first in range(0, count, BATCH):
        n = min(BATCH, count - first)
        out.append((first, next(s for s in sizes if s >= n)))
    return out


@dataclass
class Sequence:
    """A sequence in its cache slot: its tokens so far, and how many of them the cache holds."""

    slot: int
    tokens: list[int] = field(default_factory=list)
    cached: int = 0


class Engine:
    """A Llama-architecture decoder with `slots` sequences' caches and a graph per batch size."""

    def __init__(self, config: LlamaConfig, weights: Weights, slots: int = 1, prefill_chunk: int = 512):
        if slots < 1:
            raise ValueError(f"slots must be at least 1, got {slots}")
        self.sizes = batch_sizes(slots)
        self.padded = padded_sizes(self.sizes)
        self.slots, self.prefill_chunk = slots, prefill_chunk
        self.spare = slots  # the padding rows' slot, past the sequences'
        cache_slots = slots + bool(self.padded)
        self.model = Model(LlamaConfig(**{**config.__dict__, "slots": cache_slots}), weights)
        self.device = weights.output.data.device
        self._graphs: dict[int, GraphStep] = {}
        self._free = list(range(slots))

    def _graph(self, n: int) -> GraphStep:
        if n not in self._graphs:
            self._graphs[n] = GraphStep(self.model, n, advance=False)
        return self._graphs[n]

    def start(self, prompt: list[int]) -> Sequence:
        """A new sequence in a free slot with `prompt` run through the model chunk by chunk, and
        its first generated token appended (greedy)."""
        if not self._free:
            raise RuntimeError("every slot holds a sequence")
        if not prompt or len(prompt) >= self.model.config.context:
            raise ValueError(f"a prompt of {len(prompt)} tokens in a context of {self.model.config.context}")
        seq = Sequence(self._free.pop(0), list(prompt))
        nxt = None
        for at in range(0, len(prompt), self.prefill_chunk):
            chunk = prompt[at : at + self.prefill_chunk]
            n = len(chunk)
            ids = torch.tensor(chunk, dtype=torch.int32, device=self.device)
            slots = torch.full((n,), seq.slot, dtype=torch.int32, device=self.device)
            positions = torch.arange(at, at + n, dtype=torch.int32, device=self.device)
            nxt = self.model.step(ids, slots, positions, last=True)
            seq.cached = at + n
        seq.tokens.append(int(nxt[-1]))
        return seq

    def decode(self, sequences: list[Sequence]) -> list[int]:
        """One decode step of every sequence: its last token run at its next position; each gets
        its greedy next token appended, which is also returned."""
        out = []
        for first, n in plan(len(sequences), self.sizes):
            batch = sequences[first : first + BATCH]
            k = len(batch)
            full = [s.slot for s in batch if s.cached >= self.model.config.context]
            if full:
                raise RuntimeError(f"the sequences in slots {full} fill the context of {self.model.config.context}")
            step = self._graph(n)
            rows = [(s.tokens[-1], s.slot, s.cached) for s in batch] + [(0, self.spare, 0)] * (n - k)
            host = torch.tensor(rows, dtype=torch.int32).t().contiguous().pin_memory()
            step.tokens.copy_(host[0], non_blocking=True)
            step.slots.copy_(host[1], non_blocking=True)
            step.positions.copy_(host[2], non_blocking=True)
            step.replay(max_length=max(s.cached for s in batch) + 1)
            tokens = step.next[:k].tolist()
            for s, t in zip(batch, tokens, strict=True):
                s.cached += 1
                s.tokens.append(int(t))
            out += tokens
        return out

    def finish(self, seq: Sequence) -> None:
        """Frees the sequence's slot for another."""
        self._free.append(seq.slot)
