"""Writes the regression fixtures in this directory from the CPU oracle.

The reference stores no golden vectors for this path (its tests draw seeded
random inputs and compute their references at run time), so these fixtures
are the oracle's outputs on fixed inputs chosen for their edge cases.  The
oracle itself is pinned by tests/test_oracle.py (known-answer bytes, closed
forms, brute force, the reference-literal PyTorch route); the fixtures freeze
that pinned behaviour so a later change to the oracle or to the HIP path
shows up as a diff against data, not against a recomputation.

    python tests/golden/make_golden.py      # rewrites the three .npz files

Every file is written with numpy.savez_compressed and read back with
numpy.load(allow_pickle=False).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "oracle"))
import dip_oracle as O  # noqa: E402


def topk_cases():
    """(name, g bits, k) covering the threshold top-k's edge cases
    (kernels/topk_select/topk_select.cu:30-164)."""
    rng = np.random.default_rng(20)
    cases = []
    cases.append(("normal", O.f32_to_bf16(rng.standard_normal(3000).astype(np.float32)), 1800))
    ties = rng.choice(np.array([-2, -1, -0.5, 0.5, 1, 2], np.float32), 2048)
    cases.append(("ties", O.f32_to_bf16(ties), 700))
    special = rng.standard_normal(1024).astype(np.float32)
    special[::37] = np.nan
    special[5::53] = np.inf
    special[7::61] = -np.inf
    special[11::17] = 0.0
    special[13::19] = np.float32(1e-40)   # bf16 subnormals: 0 under the reference's flush
    cases.append(("special", O.f32_to_bf16(special), 300))
    g = O.f32_to_bf16(rng.standard_normal(1000).astype(np.float32))
    cases.append(("k_all", g, 1000))
    cases.append(("k_one", g, 1))
    cases.append(("k_nminus1", g, 999))
    return cases


def quant_input():
    """A [6, 256] fp32 matrix: N(0, 0.02) rows, a zero row (scale floor
    1e-8), a row of exact half-steps (round half to even), a row with -8."""
    rng = np.random.default_rng(21)
    w = (rng.standard_normal((6, 256)) * 0.02).astype(np.float32)
    w[3] = 0.0
    w[4, :128] = np.float32(7.0) * np.tile(np.array([0.5, 1.5, 2.5, -0.5, -1.5, 7.0, -7.0, 3.5],
                                                      np.float32), 16) / np.float32(7.0)
    w[4, 128:] = np.linspace(-1, 1, 128, dtype=np.float32)
    w[5, :128] = np.float32(-8.0 / 7.0) * 0.1
    w[5, 0] = np.float32(0.1)
    return w


def main():
    names, gs, ks, idxs = [], [], [], []
    for name, g, k in topk_cases():
        names.append(name)
        gs.append(g)
        ks.append(k)
        idxs.append(O.topk_select(g, k).astype(np.int32))
    np.savez_compressed(HERE / "topk_cases.npz", names=np.array(names), ks=np.array(ks),
                        **{f"g_{n}": g for n, g in zip(names, gs)},
                        **{f"idx_{n}": i for n, i in zip(names, idxs)})

    w = quant_input()
    qw, sc = O.quantize_int4_groupwise(w)
    np.savez_compressed(HERE / "quant_cases.npz", w=w, qweight=qw, scales=sc,
                        dequant=O.dequantize(qw, sc))

    H, I, keep = 256, 384, 0.6
    L = O.make_layer(H, I, seed=3)
    x = O.make_x(H, seed=4)
    k = O.keep_count(I, keep)
    ref = O.dip_forward(L["gate_qw"], L["gate_sc"], L["up_qw"], L["up_sc"], L["down_t_qw"],
                        L["down_t_sc"], x, k)
    np.savez_compressed(HERE / "mlp_small.npz", hidden=H, inter=I, k=k, x=x,
                        **{n: L[n] for n in ("gate_qw", "gate_sc", "up_qw", "up_sc",
                                             "down_t_qw", "down_t_sc")},
                        g=ref["g"], idx=ref["idx"], h=ref["h"], y=ref["y"], y_f64=ref["y_f64"])
    for f in sorted(HERE.glob("*.npz")):
        print(f"{f.name}: {f.stat().st_size} bytes")


if __name__ == "__main__":
    main()
