"""The degenerate n-gram guard (oa_detect_degenerate_ngram) on the
known-answer cases of the reference's own tests
(crates/openasr-core/src/models/seq2seq_greedy_decode.rs:1414-1640): the
token tails, the bound functions and the expected (keep_len, ngram_len,
repeats) are the reference's; a flat bound of 4 is the `|_| 4` those cases
pass, `None` the shipped 8/6/4 tiers. Host code only, no GPU.
"""

import pytest

from openasr_amd import decoders as D

FLAT4 = lambda n: 4  # noqa: E731
MAX_NGRAM = 8  # MAX_REPEAT_NGRAM (seq2seq_greedy_decode.rs:11)


def detect(tokens, max_ngram=MAX_NGRAM, bound=FLAT4):
    return D.detect_degenerate_ngram(tokens, max_ngram, bound)


def cycles(ngram, times, prefix=()):
    return list(prefix) + list(ngram) * times


@pytest.mark.parametrize("tokens", [[1, 2, 3, 4, 5], [7, 7], [7, 7, 7], [1, 2, 1, 2, 1, 2],
                                    [1, 2, 1, 2, 1, 2, 1, 2, 9], cycles([21, 22, 23, 24, 25], 2), []])
def test_non_loops_are_left_alone(tokens):
    """:1414-1431 (non-repeating tail, a few cycles), :1502-1507 (a broken
    near-loop), the two-cycle field phrase of :1477-1481"""
    assert detect(tokens) is None


@pytest.mark.parametrize("tokens,want", [
    ([5, 5, 5, 5], (1, 1, 4)),                                    # :1434-1443 single-token stutter
    ([9, 5, 5, 5, 5, 5], (2, 1, 5)),                              # :1445-1452 extra copies truncate to one
    (cycles([11, 12, 13], 5), (3, 3, 5)),                         # :1456-1468 three-token cycle x5
    (cycles([21, 22, 23, 24, 25], 4), (5, 5, 4)),                 # :1471-1476 the field-shape phrase x4
])
def test_loops_trip_and_keep_one_cycle(tokens, want):
    assert detect(tokens) == want


def test_every_ngram_size_trips_at_the_flat_bound():
    """:1484-1500: a distinct n-gram of every size 1..8 repeated exactly four times"""
    for n in range(1, 9):
        ngram = [100 + i for i in range(n)]
        assert detect(cycles(ngram, 4)) == (n, n, 4), n


def test_shipped_tiers_bound_each_cycle_length():
    """:1510-1545: one cycle under each tier survives, exactly at it trips and
    keeps one cycle (8 for n=1, 6 for n=2, 4 for n>=3)"""
    for n, bound in ((1, 8), (2, 6), (3, 4), (5, 4)):
        ngram = [100 + i for i in range(n)]
        assert detect(cycles(ngram, bound - 1), bound=None) is None, n
        assert detect(cycles(ngram, bound), bound=None) == (n, n, bound), n


def test_shipped_tiers_leave_backchannel_alone():
    """:1551-1581: 3..7 identical single tokens and 3..5 two-token cycles are speech"""
    for times in range(3, 8):
        assert detect([42] * times, bound=None) is None
    for times in range(3, 6):
        assert detect(cycles([7, 8], times), bound=None) is None


def test_relaxed_bound_keeps_the_same_prefix_on_an_unbounded_loop():
    """:1590-1614: 64 cycles after a 7-token prefix truncate to the same
    prefix under the flat bound and the tiers"""
    for n in range(1, MAX_NGRAM + 1):
        tokens = cycles([100 + i for i in range(n)], 64, prefix=range(7))
        strict = detect(tokens)
        tiered = detect(tokens, bound=None)
        assert strict is not None and tiered is not None
        assert tokens[:strict[0]] == tokens[:tiered[0]], n
        assert strict[0] == 7 + n


def test_zero_bound_or_zero_ngram_disables_the_guard():
    """:1617-1628"""
    assert detect([5, 5, 5, 5, 5], bound=lambda n: 0) is None
    assert detect([5, 5, 5, 5, 5], max_ngram=0) is None


def test_a_zero_bound_skips_only_its_length():
    """a length whose bound is 0 is skipped, not tripped on every tail
    (:578-585): with n=1 disabled a stutter is still caught as a 2-gram"""
    tokens = [5] * 8
    assert detect(tokens, bound=lambda n: 0 if n == 1 else 4) == (2, 2, 4)
