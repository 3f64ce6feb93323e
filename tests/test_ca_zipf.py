"""Synthetic cache calibration for the cache-aware module: dip_ca.zipf_counts
(the stand-in for the counts calibrate_cache gathers over generate,
dip_ca.py:272-309) and the hot-set rule applied to its counts
(dip_ca.py:300-308)."""
import itertools

import numpy as np
import torch

import dip_oracle as O


def test_zipf_counts_shape_and_determinism():
    from dip_ca import zipf_counts
    c = zipf_counts(3000, 1800, tokens=64, seed=5)
    assert c.dtype == torch.long and c.shape == (3000,)
    assert int(c.sum()) == 64 * 1800          # k distinct channels per token
    assert 0 <= int(c.min()) and int(c.max()) <= 64
    assert torch.equal(c, zipf_counts(3000, 1800, tokens=64, seed=5))
    assert not torch.equal(c, zipf_counts(3000, 1800, tokens=64, seed=6))


def test_zipf_draw_is_weighted_sampling_without_replacement():
    """Each token's k = 2 of 4 channels: the inclusion frequencies match the
    exact probabilities of drawing one channel after another in proportion
    to w_c = 1 / (rank_c + 1)^s, enumerated over ordered pairs."""
    from dip_ca import zipf_counts
    inter, k, s, seed, tokens = 4, 2, 1.1, 11, 200_000
    rank = torch.randperm(inter, generator=torch.Generator().manual_seed(seed)).numpy()
    w = 1.0 / (rank + 1.0) ** s
    p = np.zeros(inter)
    for a, b in itertools.permutations(range(inter), 2):
        pab = w[a] / w.sum() * w[b] / (w.sum() - w[a])
        p[a] += pab
        p[b] += pab
    assert abs(p.sum() - k) < 1e-12
    c = zipf_counts(inter, k, tokens=tokens, s=s, seed=seed).numpy() / tokens
    sigma = np.sqrt(p * (1 - p) / tokens)
    assert np.all(np.abs(c - p) < 5 * sigma), (c, p)


def test_zipf_counts_follow_popularity():
    from dip_ca import zipf_counts
    inter, k = 25600, 15360
    c = zipf_counts(inter, k, tokens=128, seed=3).numpy()
    rank = torch.randperm(inter, generator=torch.Generator().manual_seed(3)).numpy()
    by_rank = c[np.argsort(rank)]               # counts in popularity order
    assert by_rank[0] == 128                    # the most popular channel: every token
    assert by_rank[:100].mean() > 120 and by_rank[-100:].mean() < by_rank[:100].mean() / 2
    # counts fall with rank (Spearman correlation of rank and count)
    r = np.corrcoef(np.arange(inter), np.argsort(np.argsort(-by_rank, kind="stable")))[0, 1]
    assert r > 0.9


def test_hot_ids_from_counts_matches_oracle_hot_set():
    from dip_ca import hot_ids_from_counts, zipf_counts
    inter, k, cache_n = 6000, 3600, 1800
    c = zipf_counts(inter, k, tokens=128, seed=8)
    hot, _ = O.hot_set(c.numpy(), cache_n)
    got = np.sort(hot_ids_from_counts(c)[:cache_n].numpy())
    assert np.array_equal(got, hot)
    # ties (many channels share a count) are broken by the lower id
    assert len(np.unique(c.numpy())) < inter
