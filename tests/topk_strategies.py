"""Hypothesis strategies for top-k inputs (bf16 bit patterns): values drawn
from a small pool so that ties are common, with zeros of both signs, bf16
subnormals, infinities and NaN mixed in.  (Imported by tests only.)"""
import numpy as np
from hypothesis import strategies as st

# bit patterns: small tie-prone magnitudes of both signs, +-0, subnormals,
# +-inf, a NaN, and a few large and small normals
POOL = [0x3F80, 0xBF80, 0x4000, 0xC000, 0x3F00, 0xBF00, 0x4040, 0x0000, 0x8000, 0x0001,
        0x8005, 0x007F, 0x7F80, 0xFF80, 0x7FC0, 0x4B00, 0x3A00, 0x0080, 0x8080]


@st.composite
def topk_inputs(draw, max_n=600):
    n = draw(st.integers(1, max_n))
    mode = draw(st.sampled_from(["pool", "random", "mixed"]))
    seed = draw(st.integers(0, 2**31 - 1))
    rng = np.random.default_rng(seed)
    if mode == "pool":
        g = rng.choice(np.array(POOL, np.uint16), n)
    else:
        g = (rng.standard_normal(n).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        if mode == "mixed":
            m = rng.random(n) < 0.3
            g[m] = rng.choice(np.array(POOL, np.uint16), int(m.sum()))
    k = draw(st.integers(0, n))
    return g.astype(np.uint16), k
