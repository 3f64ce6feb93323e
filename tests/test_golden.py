"""The committed regression fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the CPU oracle) against the oracle as it is
now, plus the fixtures' own known answers: a change to the oracle's top-k,
quantizer or forward shows up here as a diff against data."""
from pathlib import Path

import numpy as np

import dip_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def test_topk_fixtures():
    z = _load("topk_cases.npz")
    for name, k in zip(z["names"], z["ks"]):
        g, idx = z[f"g_{name}"], z[f"idx_{name}"]
        assert idx.shape == (int(k),) and len(np.unique(idx)) == int(k), name
        assert np.array_equal(O.topk_select(g, int(k)), idx), name
        # on finite inputs the selected set is the top-k by (|g| desc, id
        # asc); with NaN and infinities the reference's bisection (hi = max|g|
        # = inf) is followed literally instead
        if name != "special":
            assert np.array_equal(np.sort(idx), np.sort(O.topk_key_order(g, int(k)))), name


def test_quant_fixtures():
    z = _load("quant_cases.npz")
    qw, sc = O.quantize_int4_groupwise(z["w"])
    assert np.array_equal(qw, z["qweight"]) and np.array_equal(sc, z["scales"])
    assert np.array_equal(O.dequantize(qw, sc), z["dequant"])
    q = O.unpack_int4(z["qweight"])
    # row 4, group 0: exact half steps with scale 1.0 round half to even
    assert O.bf16_to_f32(z["scales"][4, :1])[0] == 1.0
    assert q[4, :8].tolist() == [0, 2, 2, 0, -2, 7, -7, 4]
    # the zero row keeps the 1e-8 scale floor and quantizes to zeros
    assert not q[3].any() and O.bf16_to_f32(z["scales"][3]).max() > 0


def test_mlp_fixture():
    z = _load("mlp_small.npz")
    k = int(z["k"])
    ref = O.dip_forward(z["gate_qw"], z["gate_sc"], z["up_qw"], z["up_sc"], z["down_t_qw"],
                        z["down_t_sc"], z["x"], k)
    for name in ("g", "idx", "h", "y"):
        assert np.array_equal(ref[name], z[name]), name
    assert np.array_equal(ref["y_f64"], z["y_f64"])
