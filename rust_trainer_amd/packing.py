"""Shared-prompt packed batches (``Packed`` / ``pack``, src/model.rs:234-290).

Several examples that start with the same prompt are laid out as one sequence
``[shared prompt | rest of example 1 | rest of example 2 | ...]``.  Each token keeps its position in
its own example (for RoPE) and carries a segment: 0 for the shared prompt, ``k + 1`` for example
``k``.  A token may attend to the shared prompt and to earlier tokens of its own segment only
(``Rope::allowed``, src/ops.rs:160-167), so the batch gives the log-probs and gradients of running
the examples separately while the prompt is computed once.  ``GpuModel.forward_backward_packed``
runs such a batch on the device.
"""
from __future__ import annotations

import dataclasses

from .head import Target, answer_targets  # noqa: F401  (re-exported: targets are built per example)


@dataclasses.dataclass
class Packed:
    tokens: list[int]
    positions: list[int]
    segments: list[int]
    shared: int  # length of the shared prompt
    offsets: list[int]  # where each example's own tokens start in ``tokens``

    def index(self, k: int, pos: int) -> int:
        """Index in ``tokens`` of position ``pos`` of example ``k`` (src/model.rs:247-253)."""
        return pos if pos < self.shared else self.offsets[k] + pos - self.shared

    def map_targets(self, k: int, targets) -> list[Target]:
        """Example ``k``'s targets mapped into the packed sequence (src/model.rs:255-257)."""
        return [Target(self.index(k, t.pos), t.token) for t in targets]


def pack(seqs) -> Packed:
    """Pack sequences sharing a leading prompt (src/model.rs:263-290): the shared part is their
    longest common prefix, kept short enough that every sequence has a token of its own; a batch of
    one shares nothing."""
    seqs = [[int(v) for v in s] for s in seqs]
    if not seqs:
        raise ValueError("pack: no sequences")
    min_len = min(len(s) for s in seqs)
    shared = 0
    while shared + 1 < min_len and all(s[shared] == seqs[0][shared] for s in seqs):
        shared += 1
    if len(seqs) == 1:
        shared = 0
    tokens = list(seqs[0][:shared])
    positions = list(range(shared))
    segments = [0] * shared
    offsets = []
    for k, s in enumerate(seqs):
        offsets.append(len(tokens))
        tokens += s[shared:]
        positions += range(shared, len(s))
        segments += [k + 1] * (len(s) - shared)
    return Packed(tokens, positions, segments, shared, offsets)
