"""The reference's torch.library op schemas, backed by libdip_hip.so.

The reference registers five ops from its CUDA extensions (TORCH_LIBRARY
blocks) and a ``register_fake`` for each in Python.  This module registers the
same namespaces, names and schemas so ``torch.ops.<ns>.<op>(...)`` call sites
work unchanged:

  int4_ops::int4_gemv(Tensor qweight, Tensor scales, Tensor x) -> Tensor
      kernels/int4_gemv/int4_gemv.cu:110-115, fake at gate_kernel.py:21-23
  int4_gather_ops::int4_gather_gemv(Tensor qweight, Tensor scales, Tensor x,
                                    Tensor indices) -> Tensor
      kernels/int4_gather/int4_gather_gemv.cu:110-115,
      fake at dip_stream_predispatch.py:59-61
  int4_down_ops::int4_gather_down(Tensor down_t_sel, Tensor scales,
                                  Tensor h_sel) -> Tensor
      kernels/int4_down/int4_gather_down.cu:97-102,
      fake at dip_stream_predispatch.py:68-71
  topk_ops::topk_select(Tensor s, int k) -> Tensor        (int32)
      kernels/topk_select/topk_select.cu:166-171, fake at topk_kernel.py:21-23
  ca_fused_ops::ca_fused_gemv(Tensor res_qw, Tensor res_sc, Tensor str_qw,
                              Tensor str_sc, Tensor x, Tensor src,
                              Tensor row) -> Tensor
      kernels/ca_fused/ca_fused_gemv.cu:107-112, fake at dip_ca.py:50-52

Differences on purpose: outputs are produced on torch's current stream (the
reference launches on the legacy default stream) and invalid inputs raise
before any launch (the reference does not check).
"""
from __future__ import annotations

import torch

import _dip_hip as K

_LIBS = []


def _define(ns: str, schema: str, impl, fake):
    name = schema.split("(", 1)[0]
    if hasattr(torch.ops, ns) and hasattr(getattr(torch.ops, ns), name):
        return  # already registered in this process
    lib = torch.library.Library(ns, "DEF")
    lib.define(schema)
    lib.impl(name, impl, "CUDA")
    torch.library.register_fake(f"{ns}::{name}", fake, lib=lib)
    _LIBS.append(lib)


def _int4_gemv(qweight, scales, x):
    return K.int4_gemv(qweight, scales, x)


def _int4_gemv_fake(qweight, scales, x):
    return torch.empty(qweight.shape[0], dtype=torch.bfloat16, device=x.device)


def _gather_gemv(qweight, scales, x, indices):
    return K.int4_gather_gemv(qweight, scales, x, indices)


def _gather_gemv_fake(qweight, scales, x, indices):
    return torch.empty(indices.shape[0], dtype=torch.bfloat16, device=x.device)


def _gather_down(down_t_sel, scales, h_sel):
    return K.int4_gather_down(down_t_sel, scales, h_sel)


def _gather_down_fake(down_t_sel, scales, h_sel):
    return torch.empty(down_t_sel.shape[1] * 2, dtype=torch.bfloat16, device=h_sel.device)


def _topk(s, k):
    return K.topk_select(s, k)


def _topk_fake(s, k):
    return torch.empty(k, dtype=torch.int32, device=s.device)


def _ca_fused(res_qw, res_sc, str_qw, str_sc, x, src, row):
    return K.ca_fused_gemv(res_qw, res_sc, str_qw, str_sc, x, src, row)


def _ca_fused_fake(res_qw, res_sc, str_qw, str_sc, x, src, row):
    return torch.empty(src.shape[0], dtype=torch.bfloat16, device=x.device)


_define("int4_ops", "int4_gemv(Tensor qweight, Tensor scales, Tensor x) -> Tensor",
        _int4_gemv, _int4_gemv_fake)
_define("int4_gather_ops",
        "int4_gather_gemv(Tensor qweight, Tensor scales, Tensor x, Tensor indices) -> Tensor",
        _gather_gemv, _gather_gemv_fake)
_define("int4_down_ops",
        "int4_gather_down(Tensor down_t_sel, Tensor scales, Tensor h_sel) -> Tensor",
        _gather_down, _gather_down_fake)
_define("topk_ops", "topk_select(Tensor s, int k) -> Tensor", _topk, _topk_fake)
_define("ca_fused_ops",
        "ca_fused_gemv(Tensor res_qw, Tensor res_sc, Tensor str_qw, Tensor str_sc, Tensor x, "
        "Tensor src, Tensor row) -> Tensor", _ca_fused, _ca_fused_fake)
