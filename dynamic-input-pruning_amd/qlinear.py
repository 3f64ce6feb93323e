"""int4 g128 symmetric format (drop-in for the reference's qlinear.py format
helpers, qlinear.py:25-88).

    qweight : int8 [out_features, in_features // 2]   two int4 per byte,
              low nibble = even column, high nibble = odd column
    scales  : bf16 [out_features, in_features // 128]

``dequantize`` on device tensors runs the HIP dequant kernel (bf16(q*s), the
same rounding as the reference); on host tensors it uses torch ops, which is
how the reference uses it at load time (e.g. the one-time down transpose).
``QuantLinear`` is the reference's projection layer (qlinear.py:67-88).  On
the GPU it reads the packed weight once instead of writing and re-reading a
bf16 copy: the int4 GEMV for one token, the int4 MFMA GEMM for prompts of up
to GEMM_MAX_TOKENS tokens; longer prompts take the reference's dequant +
F.linear route.  Both kernels take the weights as exact fp32 q*s (the
reference rounds them to bf16 first), so they differ from dequant + F.linear
by rounding only.
``_replace_linears_with_quant`` and ``load_quantized_qwen3`` build the
reference's int4 baseline model (qlinear.py:91-166) with every weight
resident on one device.
"""
from __future__ import annotations

from pathlib import Path

import torch
import torch.nn as nn
import torch.nn.functional as F

GROUP_SIZE = 128
_QUANT_SUBSTRINGS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
# Input widths the int4 GEMV kernel is built for (its dispatch table:
# 32-column chunks split over 4..32 lanes per row).
_GEMV_COLS = frozenset((128, 256, 512, 1024, 1536, 2048, 2560, 3072, 4096, 5120, 6144, 8192))
# Prompts of up to this many tokens run the int4 MFMA GEMM (weights read
# once as nibbles); longer ones dequantize once and use the library GEMM,
# which wins once the bf16 copy is amortised over enough tokens.
GEMM_MAX_TOKENS = 64


def int4_linear(x: torch.Tensor, qweight: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """x @ (q*s)^T for x [..., in] on the device, in x's dtype: the int4
    GEMV for one token, the int4 MFMA GEMM for up to GEMM_MAX_TOKENS, else
    dequantize + F.linear (the reference's route, qlinear.py:86-88)."""
    import _dip_hip as K
    in_f = qweight.shape[1] * 2
    rows = x.numel() // in_f
    if rows == 1 and in_f in _GEMV_COLS:
        y = K.int4_gemv(qweight, scales, x.reshape(-1).to(torch.bfloat16))
        return y.to(x.dtype).reshape(*x.shape[:-1], qweight.shape[0])
    if 1 < rows <= GEMM_MAX_TOKENS:
        y = K.int4_gemm(qweight, scales, x.reshape(rows, in_f).to(torch.bfloat16))
        return y.to(x.dtype).reshape(*x.shape[:-1], qweight.shape[0])
    return F.linear(x, dequantize(qweight, scales).to(x.dtype))


def int4_linear_t(x: torch.Tensor, qweight_t: torch.Tensor, scales_t: torch.Tensor) -> torch.Tensor:
    """x @ bf16(q*s) for a matrix stored as rows of the input dimension (the
    transposed down matrix) on the device, in x's dtype: the int4 MFMA GEMM
    for up to GEMM_MAX_TOKENS rows of x, else x @ dequantize (the reference's
    route, dip_stream_predispatch.py:213-215)."""
    import _dip_hip as K
    rows = x.numel() // x.shape[-1]
    if rows <= GEMM_MAX_TOKENS:
        return K.int4_gemm_t(qweight_t, scales_t, x.to(torch.bfloat16)).to(x.dtype)
    return x @ dequantize(qweight_t, scales_t).to(x.dtype)


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
        if x.is_cuda and self.out_features > 0:
            return int4_linear(x, self.qweight, self.scales)
        w = dequantize(self.qweight, self.scales)
        return F.linear(x, w.to(x.dtype))


def _replace_linears_with_quant(model: nn.Module) -> list:
    """Swap every nn.Linear whose qualified name contains one of the seven
    projection names for an empty QuantLinear of the same shape
    (qlinear.py:91-106); returns the swapped names.  lm_head and the
    embeddings stay as they are."""
    swapped = []
    for parent_name, parent in list(model.named_modules()):
        for child_name, child in list(parent.named_children()):
            full = f"{parent_name}.{child_name}" if parent_name else child_name
            if isinstance(child, nn.Linear) and any(s in full for s in _QUANT_SUBSTRINGS):
                setattr(parent, child_name, QuantLinear(child.in_features, child.out_features))
                swapped.append(full)
    return swapped


def load_quantized_qwen3(ckpt_dir, gpu_mem_gib: int = 13, cpu_mem_gib: int = 60,
                         device="cuda:0"):
    """The reference's int4 baseline (qlinear.py:109-166): the model of
    `ckpt_dir/config.json` with QuantLinear projections and the weights of
    model_int4.safetensors.  Returns (model, tokenizer or None).

    The reference splits the model between a small GPU and host memory with
    accelerate's offload hooks (gpu_mem_gib / cpu_mem_gib); one MI355X holds
    a whole int4 Qwen3-32B in HBM, so every tensor is placed on `device` and
    the two sizes are accepted for call compatibility only."""
    from dip_model import build_empty_model, load_tensors, load_tokenizer
    from dip_checkpoint import ST_NAME, read_quant_config
    ckpt_dir = Path(ckpt_dir)
    read_quant_config(ckpt_dir)
    model = build_empty_model(ckpt_dir)
    load_tensors(model, ckpt_dir / ST_NAME, device)
    return model, load_tokenizer(ckpt_dir)
