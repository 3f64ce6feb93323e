"""int4 g128 symmetric quantizer (the reference's scripts/quantize.py:28-64).

Device tensors go through the HIP quantize kernel (IEEE division and
round-half-even, bit-exact with the reference's CPU torch code); host tensors
use torch ops as the reference does.  The synthetic benchmark stacks quantize
their N(0, 0.02) weights with it on the GPU; tests pin both routes bit for bit
against the CPU oracle."""
from __future__ import annotations

import torch

GROUP_SIZE = 128
QMAX = 7


def quantize_tensor_int4_groupwise(w: torch.Tensor):
    """w [out, in] -> (packed int8 [out, in/2], scales bf16 [out, in/128]).

    s = clamp(max|w_g| / 7, min=1e-8) in fp32; q = clamp(round(w / s), -8, 7)
    with round-half-even and the fp32 s; scales are cast to bf16 afterwards
    (scripts/quantize.py:43-63)."""
    out_f, in_f = w.shape
    assert in_f % GROUP_SIZE == 0, f"in_features {in_f} not divisible by {GROUP_SIZE}"
    if w.is_cuda:
        from _dip_hip import quantize_int4
        return quantize_int4(w)
    w = w.float()
    wg = w.reshape(out_f, in_f // GROUP_SIZE, GROUP_SIZE)
    scales = (wg.abs().amax(dim=2, keepdim=True) / QMAX).clamp(min=1e-8)
    q = torch.round(wg / scales).clamp(-8, 7).to(torch.int8).reshape(out_f, in_f)
    packed = pack_int4(q)
    return packed, scales.squeeze(-1).to(torch.bfloat16)


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """int8 [R, C] in [-8, 7] -> packed int8 [R, C/2]; low nibble = even
    column (dip_stream_predispatch.py:93-97)."""
    lo = (q[:, 0::2] & 0x0F).to(torch.uint8)
    hi = (q[:, 1::2] & 0x0F).to(torch.uint8)
    return (lo | (hi << 4)).view(torch.int8)
