"""Gate projection on the int4 GEMV kernel (drop-in for the reference's
gate_kernel.py:1-33).  ``_use_gate`` is always True here: the HIP library is
required and importing fails loudly without it."""
import torch

import dip_ops  # noqa: F401  (registers torch.ops.int4_ops.int4_gemv)
import _dip_hip as K

_use_gate = True


def gate_gemv(qweight, scales, x):
    """gate_proj(x) for a decode vector x [in]; returns bf16 [out]
    (gate_kernel.py:29-33)."""
    return torch.ops.int4_ops.int4_gemv(qweight, scales, x.to(torch.bfloat16).contiguous())


def gate_silu(qweight, scales, x):
    """bf16(silu(gate_proj(x))) in one kernel (the gate + F.silu of
    dip_stream_predispatch.py:182)."""
    return K.int4_gemv(qweight, scales, x.to(torch.bfloat16), act=1)
