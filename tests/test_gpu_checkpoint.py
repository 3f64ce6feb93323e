"""GPU: an int4 checkpoint in the reference's format read into resident
MLPs (dip_checkpoint) - gate/up bytes as stored, down transposed on the GPU
bit-identically to the oracle's CPU route, and a decode step of the loaded
stack at the oracle's parity bars; the StreamingDIPMlp modules built from
the same file give the same y."""
import numpy as np
import pytest
import torch

import dip_oracle as O
from gpu_util import dev_bf16, host_bf16, rel_err

pytestmark = pytest.mark.gpu


def _state(H, I, n, seed):
    g = torch.Generator().manual_seed(seed)
    sd = {"model.embed_tokens.weight": torch.randn(32, H, generator=g)}
    for i in range(n):
        p = f"model.layers.{i}.mlp"
        sd[f"{p}.gate_proj.weight"] = torch.randn(I, H, generator=g) * 0.02
        sd[f"{p}.up_proj.weight"] = torch.randn(I, H, generator=g) * 0.02
        sd[f"{p}.down_proj.weight"] = torch.randn(H, I, generator=g) * 0.02
    return sd


def test_checkpoint_to_resident_stack(tmp_path):
    import dip_checkpoint as C
    from dip_stack import DIPStack
    H, I, n = 1024, 3072, 2
    sd = _state(H, I, n, seed=3)
    C.save_int4_checkpoint(tmp_path, sd)
    layers = C.load_mlp_layers(tmp_path, "cuda")
    assert [L["name"] for L in layers] == [f"model.layers.{i}.mlp" for i in range(n)]
    ref = []
    for i, L in enumerate(layers):
        p = f"model.layers.{i}.mlp"
        gq, gs = O.quantize_int4_groupwise(sd[f"{p}.gate_proj.weight"].numpy())
        uq, us = O.quantize_int4_groupwise(sd[f"{p}.up_proj.weight"].numpy())
        dq, ds = O.quantize_int4_groupwise(sd[f"{p}.down_proj.weight"].numpy())
        dtq, dts = O.transpose_down_to_int4(dq, ds)
        assert np.array_equal(L["gate_qw"].cpu().numpy(), gq)
        assert np.array_equal(host_bf16(L["up_sc"]), us)
        assert np.array_equal(L["down_t_qw"].cpu().numpy(), dtq)      # GPU transpose
        assert np.array_equal(host_bf16(L["down_t_sc"]), dts)
        ref.append((gq, gs, uq, us, dtq, dts))

    import _dip_hip as K
    stack = DIPStack.from_checkpoint(tmp_path, 0.6, "cuda")
    x = O.make_x(H, seed=4)
    stack.x.copy_(dev_bf16(x))
    stack.run_token()
    torch.cuda.synchronize()
    for i, (L, (gq, gs, uq, us, dtq, dts)) in enumerate(zip(layers, ref)):
        # the stage-by-stage step on the loaded weights, checked stage by
        # stage against the oracle, and the stack's (speculative) y equal to it
        y, g, idx, _ = K.mlp_decode(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"],
                                    L["down_t_qw"], L["down_t_sc"], dev_bf16(x), stack.k)
        g_h, idx_h = host_bf16(g), idx.cpu().numpy()
        assert np.array_equal(idx_h, O.topk_select(g_h, stack.k)), i
        tail = O.dip_forward(gq, gs, uq, us, dtq, dts, x, stack.k, idx=idx_h)
        assert rel_err(host_bf16(y), tail["y_f64"]) < 1e-2, i
        # the stack's speculative step: the same sum in another fp32 grouping
        assert rel_err(host_bf16(stack.y[i]), tail["y_f64"]) < 1e-2, i

    names, mods, _ = C.load_streaming_mlps(tmp_path, 0.6, "cuda")
    xin = dev_bf16(x).reshape(1, 1, H)
    for i, mod in enumerate(mods):
        y = mod(xin).reshape(-1)
        assert torch.equal(y.view(torch.int16), stack.y[i].view(torch.int16)), names[i]
