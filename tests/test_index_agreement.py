"""``list_agreement``, the numbering-independent comparison of two builds'
posting lists used for the GPU-vs-CPU index build: identical cells and a
renumbering of the same lists score 1; moving tokens lowers it; two seeds'
clusterings of the same keys score well below 1.  CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from seoulkv_amd import SeoulKV4Index
from seoulkv_amd.index import list_agreement, posting_cosine, posting_pairs
from seoulkv_amd.synthetic import make_cache


@pytest.fixture(scope="module")
def index():
    k, v, _ = make_cache(8192, 64, clustered=True, n_queries=1)
    return k, v, SeoulKV4Index.build(k, v, nprobe=64, n_centroids=512)


def _lists(cell):
    off, vals = cell["offsets"].numpy(), cell["values"].numpy()
    return [vals[off[i]:off[i + 1]].copy() for i in range(len(off) - 1)]


def _cell(lists):
    off = np.concatenate([[0], np.cumsum([len(x) for x in lists])])
    return dict(offsets=torch.from_numpy(off), values=torch.from_numpy(np.concatenate(lists)))


def test_posting_pairs_two_distinct_lists_per_token(index):
    _, _, ix = index
    pp = posting_pairs(ix.cells[0])
    assert pp.shape == (ix.zones.local_begin - ix.zones.sink, 2)
    assert (pp[:, 0] < pp[:, 1]).all()


def test_identical_and_renumbered_lists_agree_fully(index):
    _, _, ix = index
    c = ix.cells[1]
    assert list_agreement(c, c) == 1.0
    lists = _lists(c)
    perm = np.random.default_rng(3).permutation(len(lists))
    assert list_agreement(c, _cell([lists[i] for i in perm])) == 1.0


def test_moved_tokens_lower_the_agreement(index):
    _, _, ix = index
    c = ix.cells[2]
    lists = _lists(c)
    # swap one token between two lists that share neither: 2 of the
    # 2 x tokens memberships move
    a, b = 0, 1
    ta = next(t for t in lists[a] if t not in lists[b])
    tb = next(t for t in lists[b] if t not in lists[a])
    lists[a] = np.sort(np.where(lists[a] == ta, tb, lists[a]))
    lists[b] = np.sort(np.where(lists[b] == tb, ta, lists[b]))
    got = list_agreement(c, _cell(lists))
    n = 2 * len(posting_pairs(c))
    assert 1 - 2 / n <= got < 1


def test_other_seed_clusters_differently_with_equal_quality(index):
    k, v, ix = index
    other = SeoulKV4Index.build(k, v, nprobe=64, n_centroids=512, seed=1)
    got = list_agreement(ix.cells[0], other.cells[0])
    assert 0.5 < got < 0.9
    for h in range(4):
        qa, qb = posting_cosine(ix.cells[h], k[h]), posting_cosine(other.cells[h], k[h])
        assert 0.6 < qa < 0.9 and abs(qa - qb) <= 0.005


def test_posting_cosine_drops_for_scrambled_lists(index):
    k, _, ix = index
    c = ix.cells[3]
    lists = _lists(c)
    rng = np.random.default_rng(7)
    tokens = np.concatenate(lists)
    rng.shuffle(tokens)  # same list sizes, random members
    off = np.concatenate([[0], np.cumsum([len(x) for x in lists])])
    scrambled = dict(c, offsets=torch.from_numpy(off), values=torch.from_numpy(tokens))
    assert posting_cosine(scrambled, k[3]) < posting_cosine(c, k[3]) - 0.2
