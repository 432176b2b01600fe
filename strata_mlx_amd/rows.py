"""The rows of the output layer a draft guess is worked out over: strata_mlx/rows.py on the file's blocks.

`rows_of` makes the listed rows of a layer a layer of their own (rows.py:30-42). The reference copies those rows
out (padded to fours); here the rows stay where they are and the matvec reads them by id (`strata_dense_matvec`
with `row_ids`), each listed row getting the bits it has in the full layer. `GuessRows` keeps the list as the
reference's does (rows.py:45-97): rows added from the largest logits of the trunk's rows, restarted past `most`.
"""

import numpy as np
import torch

from .dense import BlockLinear

TOP, START, MOST, PIECES = 256, 1000, 48_000, 4  # strata_mlx/rows.py:27


def rows_of(head: BlockLinear, ids) -> callable:
    """The rows `ids` of a layer as a layer of their own: x (1, in) -> (1, len(ids))."""
    at = torch.as_tensor(np.asarray(ids, dtype=np.int64), device=head.blocks.device).to(torch.int32)
    return lambda x: head(x, row_ids=at)


class GuessRows:
    def __init__(self, head: BlockLinear, vocab: int, top: int = TOP, start: int = START, most: int = MOST):
        self.head, self.vocab = head, vocab
        self.top, self.start, self.most = min(top, vocab - 1), start, most
        self.clear()

    def clear(self):
        self.listed = np.zeros(self.vocab, dtype=bool)
        self.pieces = []  # (ids, their rows as a layer) per call of `add`, joined now and then
        self.count = 0
        self.pending = None
        self._ids = None

    @property
    def ready(self) -> bool:
        return self.count >= self.start

    def add(self, ids):
        """List these rows."""
        ids = np.unique(np.asarray(ids, dtype=np.int64))
        new = ids[~self.listed[ids]]
        if not len(new):
            return
        if self.count + len(new) > self.most:
            pending = self.pending
            self.clear()
            self.pending = pending
        self.listed[new] = True
        self.count += len(new)
        self.pieces.append((new, rows_of(self.head, new)))
        if len(self.pieces) > PIECES:
            everything = np.concatenate([i for i, _ in self.pieces])
            self.pieces = [(everything, rows_of(self.head, everything))]
        self._ids = None

    def note(self, logits: torch.Tensor):
        """logits (rows, vocab) the trunk has worked out: their largest are listed by the next call of this."""
        self.collect()
        self.pending = torch.topk(logits, self.top, dim=-1).indices

    def collect(self):
        if self.pending is not None:
            pending, self.pending = self.pending, None
            self.add(pending.reshape(-1).cpu().numpy())

    def logits(self, x: torch.Tensor):
        """x (1, in) -> (the listed rows' logits (1, count), the token of each)."""
        if self._ids is None:
            self._ids = torch.as_tensor(np.concatenate([i for i, _ in self.pieces]), device=x.device)
        parts = [layer(x) for _, layer in self.pieces]
        return (parts[0] if len(parts) == 1 else torch.cat(parts, dim=1)), self._ids
