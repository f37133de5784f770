"""Host logic of the drop-in Sampler (no device calls): argument checks,
the penalty window handed to the device, parameter validation."""
from __future__ import annotations

import numpy as np
import pytest

from chenxing_amd import Sampler, SamplingParams
from chenxing_amd.sampler import WINDOW_MAX, _Groups


def test_invalid_params_raise():                       # chenxing tests/test_sampler.py:64-69
    with pytest.raises(ValueError):
        SamplingParams(top_p=1.5)
    with pytest.raises(ValueError):
        SamplingParams(temperature=-1)
    with pytest.raises(ValueError):
        SamplingParams(min_p=-0.1)


def test_window_is_none_without_penalties():
    s = Sampler(10)
    assert s._window(SamplingParams(), [1, 2, 3], 10) is None
    assert s._window(SamplingParams(repetition_penalty=1.2), [], 10) is None


def test_window_follows_n_keep_and_drops_out_of_range_ids():
    s = Sampler(10)
    h = list(range(-3, 200))                            # 203 ids, most out of range
    w = s._window(SamplingParams(repetition_penalty=1.2, n_keep=70), h, 10)
    assert w.size == 70                                 # last max(64, n_keep) ids (sampler.py:67)
    assert np.all(w == -1)                              # 130..199 are >= vocab_size (:68)
    w = s._window(SamplingParams(repetition_penalty=1.2), [-1, 0, 9, 10, 3], 10)
    assert w.tolist() == [-1, 0, 9, -1, 3]
    w = s._window(SamplingParams(repetition_penalty=1.2, n_keep=3), list(range(100)), 10)
    assert w.size == 64                                 # max(64, 3)


def test_window_index_error_like_the_reference():
    # vocab_size larger than the row: the reference indexes the row with the id
    s = Sampler(20)
    with pytest.raises(IndexError):
        s._window(SamplingParams(repetition_penalty=1.2), [15], 10)
    # without the repetition penalty nothing is indexed
    assert s._window(SamplingParams(presence_penalty=0.5), [15], 10).tolist() == [-1]


def test_long_window_deduplicated_when_counts_do_not_matter():
    s = Sampler(100)
    h = [i % 50 for i in range(10_000)]
    w = s._window(SamplingParams(repetition_penalty=1.1, presence_penalty=0.2), h, 100)
    assert sorted(w.tolist()) == list(range(50))


def _check_groups(groups, window, counted):
    """Disjoint id sets, at most 4095 ids each, together the window's ids
    (with their multiplicities when counted)."""
    assert isinstance(groups, _Groups) and len(groups) > 1
    seen = set()
    for g in groups:
        assert g.dtype == np.int32 and 0 < g.size <= WINDOW_MAX
        ids = set(g.tolist())
        assert not ids & seen
        seen |= ids
        if not counted:
            assert len(ids) == g.size
    w = np.asarray([t for t in window if t >= 0])
    if counted:
        assert np.array_equal(np.sort(np.concatenate(groups)), np.sort(w))
    else:
        assert seen == set(w.tolist())


def test_long_windows_split_into_groups():
    """Windows the device index cannot hold in one launch: groups of ids
    applied one after another (each id's penalty depends on its own value
    and count only)."""
    h = [i % 50 for i in range(10_000)]
    _check_groups(Sampler(100)._window(SamplingParams(frequency_penalty=0.1), h, 100), h,
                  True)
    h = list(range(5000)) + [-3, 10**6]
    _check_groups(Sampler(10_000)._window(SamplingParams(repetition_penalty=1.1), h, 10_000),
                  [t if t < 10_000 else -1 for t in h], False)
    rng = np.random.default_rng(3)
    h = rng.integers(0, 20_000, 12_000).tolist()
    _check_groups(Sampler(20_000)._window(SamplingParams(frequency_penalty=0.3,
                                                         presence_penalty=0.1), h, 20_000),
                  h, True)
    # out-of-range ids leave a window that fits: one plain window
    w = Sampler(100)._window(SamplingParams(frequency_penalty=0.1), [5] * 100 + [-1] * 5000, 100)
    assert not isinstance(w, _Groups) and w.tolist() == [5] * 100
    # one id counted more often than one launch can count
    with pytest.raises(ValueError):
        Sampler(100)._window(SamplingParams(frequency_penalty=0.1), [7] * 5000, 100)


def test_batch_argument_checks():
    s = Sampler(8)
    with pytest.raises(ValueError):
        s.sample(np.zeros((2, 8), np.float32), SamplingParams())
    with pytest.raises(ValueError):
        s.sample_batch(np.zeros((2, 8), np.float32), [SamplingParams()] * 3)
    assert s.sample_batch(np.zeros((0, 8), np.float32), []) == []


def test_batch_history_arrays_equal_the_per_row_windows():
    """sample_batch writes plain-int lists through _cxhist's C loop and
    every other window through _window: the arrays must equal the per-row
    windows, whatever the item types (numpy ints, floats, ints beyond 64
    bits fall back), ranges, n_keep and penalty settings."""
    V = 1000
    s = Sampler(V)
    rng = np.random.default_rng(5)
    plist, hists = [], []
    for b in range(40):
        n = int(rng.integers(0, 300))
        ids = [int(t) for t in rng.integers(-5, V + 50, n)]
        kind = b % 8
        if kind == 1:
            ids = tuple(ids)
        elif kind == 2:
            ids = np.asarray(ids, dtype=np.int64)
        elif kind == 3 and ids:
            ids[len(ids) // 2] = np.int64(ids[len(ids) // 2])   # not an exact int
        elif kind == 4 and ids:
            ids[0] = 2 ** 70                                    # beyond 64 bits
        elif kind == 5:
            ids = ids + [2 ** 40, -(2 ** 40), 2 ** 31, V - 1, V, 0]
        pen = [dict(repetition_penalty=1.1), dict(presence_penalty=0.5),
               dict(frequency_penalty=0.3), dict()][b % 4]
        plist.append(SamplingParams(n_keep=[0, 70, 3][b % 3], **pen))
        hists.append(ids)
    wins, lists = s._windows(plist, hists, V)
    assert lists                                                # the C loop takes rows
    hist, hl = s._history_arrays(wins, lists, plist, hists, V)
    for b in range(40):
        w = s._window(plist[b], hists[b], V)
        if w is None:
            assert hl[b] == 0 and np.all(hist[b] == -1)
        else:
            assert hl[b] == w.size
            assert hist[b, :w.size].tolist() == w.tolist()
            assert np.all(hist[b, w.size:] == -1)


def test_cxhist_fill_edge_cases():
    from chenxing_amd import _cxhist
    h = np.full((4, 3), -7, np.int32)
    hl = np.zeros(4, np.int32)
    left = _cxhist.fill([[1, 2, 99], [1.0], [1, 2, 3, 4], (5, 2 ** 70)], [0, 1, 2, 3], h, hl, 50)
    assert left == [1, 2, 3]                     # a float, a row longer than H, 2**70
    assert h[0].tolist() == [1, 2, -1] and hl[0] == 3
    assert hl[1:].tolist() == [0, 0, 0]
    with pytest.raises(IndexError):
        _cxhist.fill([[1]], [4], h, hl, 50)
    with pytest.raises(ValueError):
        _cxhist.fill([[1]], [0], h.astype(np.int64), hl, 50)
