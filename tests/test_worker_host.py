"""Host-side logic of the worker round helpers (CPU): the one-launch add of a
fused output and its fused delta must equal the reference's per-projection
adds (worker_sync.py:276-284, :346-354)."""

from swarmlora_amd.worker.batched_ops import _add_deltas, _joined
from tests._util import bits_equal, randn


def _pieces(t, dims):
    return list(t.split(dims, dim=-1))


def test_joined_spans_adjacent_pieces_of_one_buffer():
    full = randn((1, 1, 6144), 1)
    parts = _pieces(full, [4096, 1024, 1024])
    j = _joined(parts)
    assert j is not None and j.shape == full.shape and j.data_ptr() == full.data_ptr()
    # pieces of two buffers, or out of order, or rows wider than the pieces: no single view
    other = randn((1, 1, 1024), 2)
    assert _joined([parts[0], parts[1], other]) is None
    assert _joined([parts[1], parts[0]]) is None
    wide = randn((3, 8192), 3)
    assert _joined(_pieces(wide[:, :6144], [4096, 2048])) is None
    assert _joined(_pieces(randn((3, 6144), 4), [4096, 2048])) is not None


def test_one_launch_add_equals_per_projection_adds():
    dims = [4096, 1024, 1024]
    raw = randn((1, 2, 6144), 5)
    delta = randn((1, 2, 6144), 6, std=0.05)
    want = [p + d for p, d in zip(_pieces(raw, dims), _pieces(delta, dims))]
    got = raw.clone()
    parts = _pieces(got, dims)
    _add_deltas(parts, _pieces(delta, dims))
    for g, w in zip(parts, want):
        assert bits_equal(g, w)
    # a missing delta leaves its piece alone and the others are added one by one
    got2 = raw.clone()
    parts2 = _pieces(got2, dims)
    dl = _pieces(delta, dims)
    _add_deltas(parts2, [dl[0], None, dl[2]])
    assert bits_equal(parts2[1], _pieces(raw, dims)[1])
    assert bits_equal(parts2[0], want[0]) and bits_equal(parts2[2], want[2])
