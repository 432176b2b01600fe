"""Listed rows of an output layer, read where they lie: the row gather of strata_mlx/rows.py:30-42.

`rows_of` makes the listed rows of a layer a layer of its own. The reference copies those rows out into a new
layer (padded to a multiple of four); here they stay in the layer's blocks and the matvec reads each one by its id
(`strata_dense_matvec` with `row_ids`), so a listed row gets exactly the bits it has in the full layer and no
bytes are copied. Which rows to list (the reference's draft-guess policy) is the caller's business.
"""

import numpy as np
import torch

from .dense import BlockLinear


def rows_of(head: BlockLinear, ids) -> callable:
    """The rows `ids` of a layer as a layer of their own: x (1, in) -> (1, len(ids)). An id past the layer's rows
    gives NaN."""
    at = torch.as_tensor(np.asarray(ids, dtype=np.int64), device=head.blocks.device).to(torch.int32)
    return lambda x: head(x, row_ids=at)
