"""int4 g128 symmetric format (drop-in for the reference's qlinear.py format
helpers, qlinear.py:25-88).

    qweight : int8 [out_features, in_features // 2]   two int4 per byte,
              low nibble = even column, high nibble = odd column
    scales  : bf16 [out_features, in_features // 128]

``dequantize`` on device tensors runs the HIP dequant kernel (bf16(q*s), the
same rounding as the reference); on host tensors it uses torch ops, which is
how the reference uses it at load time (e.g. the one-time down transpose).
``QuantLinear`` is the dense dequant + F.linear layer the reference uses for
prefill (qlinear.py:67-88).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

GROUP_SIZE = 128


def _unpack_int4(qweight: torch.Tensor) -> torch.Tensor:
    """int8 [R, C/2] -> int8 [R, C] in [-8, 7] (qlinear.py:28-50)."""
    q = qweight.view(torch.uint8) if qweight.dtype == torch.int8 else qweight.to(torch.uint8)
    low = (q & 0x0F).to(torch.int8)
    high = ((q >> 4) & 0x0F).to(torch.int8)
    low = torch.where(low >= 8, low - 16, low)
    high = torch.where(high >= 8, high - 16, high)
    return torch.stack((low, high), dim=-1).reshape(q.shape[0], q.shape[1] * 2)


def dequantize(qweight: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """bf16 [R, C] = bf16(q * s) (qlinear.py:53-64)."""
    if qweight.is_cuda:
        from _dip_hip import dequant_rows
        return dequant_rows(qweight, scales, mode=1)
    q = _unpack_int4(qweight)
    out_f, in_f = q.shape
    qf = q.float().reshape(out_f, in_f // GROUP_SIZE, GROUP_SIZE)
    s = scales.float().reshape(out_f, in_f // GROUP_SIZE, 1)
    return (qf * s).reshape(out_f, in_f).to(torch.bfloat16)


class QuantLinear(nn.Module):
    """INT4 g128 symmetric linear; dequantizes then calls F.linear
    (qlinear.py:67-88)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        assert in_features % GROUP_SIZE == 0
        self.register_buffer("qweight",
                             torch.empty(out_features, in_features // 2, dtype=torch.int8))
        self.register_buffer("scales",
                             torch.empty(out_features, in_features // GROUP_SIZE,
                                         dtype=torch.bfloat16))
        self.bias = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w = dequantize(self.qweight, self.scales)
        return F.linear(x, w.to(x.dtype))
