"""Host logic of the pipelined decode loop (no GPU): ``graph.decode_tokens``
against a stand-in runner that records the order of launches and reads."""
import pytest

from ppu_amd.graph import decode_tokens


class _Runner:
    """Hands out the tokens of ``seq`` in launch order and checks the
    contract ``GreedyDecodeGraph`` enforces: at most two launches
    outstanding, results read in launch order."""

    def __init__(self, seq):
        self.seq, self.log, self.pending, self.launched = list(seq), [], [], 0

    def launch(self):
        assert len(self.pending) < 2, "a third launch before a read"
        slot = self.launched % 2
        self.pending.append((slot, self.seq[self.launched]))
        self.launched += 1
        self.log.append(("launch", slot))
        return slot

    def result(self, slot):
        assert self.pending and self.pending[0][0] == slot, "read out of launch order"
        self.log.append(("result", slot))
        return self.pending.pop(0)[1]


def test_decode_tokens_keeps_one_step_queued():
    r = _Runner([5, 6, 7, 8, 9])
    assert decode_tokens(r, 5) == [5, 6, 7, 8, 9]
    # the next step is always queued before the previous token is read
    assert r.log[:3] == [("launch", 0), ("launch", 1), ("result", 0)]
    assert r.launched == 5 and not r.pending


@pytest.mark.parametrize("count", [0, 1, 2])
def test_decode_tokens_launches_no_step_past_count(count):
    r = _Runner([1, 2, 3, 4])
    assert decode_tokens(r, count) == [1, 2, 3, 4][:count]
    assert r.launched == count and not r.pending


def test_decode_tokens_stops_at_eos_and_drains():
    r = _Runner([3, 4, 99, 5, 6, 7])
    assert decode_tokens(r, 6, eos_ids={99}) == [3, 4, 99]
    # the step queued behind the EOS ran and was read (its token dropped)
    assert r.launched == 4 and not r.pending
    assert r.log[-1] == ("result", 1)
