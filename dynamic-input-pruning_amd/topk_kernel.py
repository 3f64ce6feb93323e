"""Top-k channel selection (drop-in for the reference's topk_kernel.py:1-40).

``select_topk(s, k)`` returns int64 [k] indices identical to the reference's
topk_ops::topk_select followed by ``.to(torch.long)``: the threshold
bisection's tier |s| > t_strict in ascending index, then the tie band in
ascending index.  There is no torch.topk fallback (it picks a different set on
ties); the HIP library is required."""
import torch

import dip_ops  # noqa: F401  (registers torch.ops.topk_ops.topk_select)

_use_topk = True


def select_topk(s, k):
    """Select k channels by |s|; int64 [k] (topk_kernel.py:29-40)."""
    return torch.ops.topk_ops.topk_select(s.contiguous(), k).to(torch.long)
