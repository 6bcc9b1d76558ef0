"""TokenLayout builders on the host (MinistralModel.cs:703-781).

`forest` -- independent trees laid end to end, each with its own shared
range -- reduces to the reference's Tree for one tree at slot 0, and every
tree of a forest is that tree's Tree shifted by its first slot (positions
unshifted)."""
import numpy as np
import pytest

import jev


def _tree_fields(lay):
    return [lay.slot, lay.position, lay.shared_hi, lay.segment, lay.outputs]


def test_one_tree_forest_is_the_reference_tree():
    trunk, branches = 11, [3, 1, 6]
    offsets = [trunk + sum(branches[:i]) for i in range(len(branches))]
    ref = jev.TokenLayout.tree(0, trunk, offsets, trunk + sum(branches))
    got = jev.TokenLayout.forest([(trunk, branches)])
    for a, b in zip(_tree_fields(ref), _tree_fields(got)):
        assert np.array_equal(a, b)
    assert got.end == ref.end and not got.shared_lo.any()


def test_forest_trees_are_shifted_trees():
    trees = [(7, [2, 5]), (4, [1]), (9, [3, 3, 2])]
    got = jev.TokenLayout.forest(trees)
    t0, o0, b0 = 0, 0, 0
    for trunk, branches in trees:
        n = trunk + sum(branches)
        offsets = [trunk + sum(branches[:i]) for i in range(len(branches))]
        ref = jev.TokenLayout.tree(0, trunk, offsets, n)
        sl = slice(t0, t0 + n)
        assert np.array_equal(got.slot[sl], ref.slot + b0)
        assert np.array_equal(got.position[sl], ref.position)
        assert np.array_equal(got.shared_hi[sl], ref.shared_hi + b0)
        assert np.array_equal(got.segment[sl], ref.segment + b0)
        assert (got.shared_lo[sl] == b0).all()
        assert np.array_equal(got.outputs[o0:o0 + len(branches)], ref.outputs + t0)
        t0, o0, b0 = t0 + n, o0 + len(branches), b0 + n
    assert got.end == b0


def test_forest_rejects_an_empty_branch():
    with pytest.raises(jev.ArgumentError):
        jev.TokenLayout.forest([(3, [2, 0])])
