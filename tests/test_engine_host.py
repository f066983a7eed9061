"""Host logic of speculative decoding (CPU): prompt-lookup drafts and the
acceptance rule of the verify step (engine/engine.py:48-93, 477-484). The
expected drafts are worked out by hand from the lookup's definition: the
latest earlier occurrence of the last 3, else 2, else 1 tokens proposes what
followed it, a continuation that reaches the end reads the draft itself, and no
occurrence repeats the last token."""

from kernel_optim_amd.engine import NgramIndex, accept, draft_len


def test_draft_follows_latest_trigram():
    # (1, 2, 3) occurred at 0..2 and was followed by 4, 1, 2
    assert NgramIndex([1, 2, 3, 4, 1, 2, 3]).draft(3) == [4, 1, 2]


def test_draft_runs_into_itself():
    # only (7,) occurred before, followed by 8, 7 and then the draft's own 8
    assert NgramIndex([7, 8, 7]).draft(3) == [8, 7, 8]
    assert NgramIndex([7, 8, 7]).draft(5) == [8, 7, 8, 7, 8]


def test_draft_latest_occurrence_wins():
    # (1,) occurred at 0 (-> 2) and at 2 (-> 3): the later one proposes 3, 1, then itself
    assert NgramIndex([1, 2, 1, 3, 1]).draft(3) == [3, 1, 3]


def test_draft_prefers_longer_match():
    # bigram (5, 6) was followed by 9; unigram (6,) latest by 7
    seq = [5, 6, 9, 6, 7, 5, 6]
    assert NgramIndex(seq).draft(2) == [9, 6]


def test_draft_without_match_repeats_last():
    assert NgramIndex([42]).draft(4) == [42, 42, 42, 42]
    assert NgramIndex([1, 2, 3]).draft(2) == [3, 3]


def test_extend_is_incremental():
    a = NgramIndex([1, 2, 3, 4])
    a.extend([1, 2, 3])
    b = NgramIndex([1, 2, 3, 4, 1, 2, 3])
    assert a.seq == b.seq and a.after == b.after and a.draft(4) == b.draft(4)


def test_accept_prefix_and_next_token():
    # verify input [last, d1, d2, d3]; greedy ids after each input position
    assert accept([5, 1, 2, 3], [1, 2, 3, 8]) == [1, 2, 3, 8]   # all drafts + the next
    assert accept([5, 1, 2, 3], [1, 2, 9, 4]) == [1, 2, 9]      # stops at the first miss
    assert accept([5, 1, 2, 3], [7, 2, 3, 4]) == [7]            # no draft accepted
    assert accept([5], [6]) == [6]                              # K = 0


def test_draft_len_by_batch():
    assert [draft_len(b) for b in (1, 4, 5, 16, 17, 32, 33)] == [6, 6, 4, 4, 2, 2, 0]
