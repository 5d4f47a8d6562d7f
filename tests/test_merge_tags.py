"""CPU: the one-slot fused merge never accepts a stale partial, across epoch wraps.

The tagged protocol (voltattn_amd/csrc/va_fused.hpp, finish_tagged) stores each
value of a split's partial as a 64-bit word (tag << 32 | value) at word address
mg*S + s of its ticket slot (merge group mg, split s, S splits), and the merging
work-group accepts a word only if its tag is the current call's; a word whose
store has not landed yet still holds whatever was there before. The reference
has no such state: its combine is a second kernel (src/voltattn.cu:651-672).

This emulates that store on the CPU, worst case: the merger always reads the
word before the current store lands, so any previous word with a matching tag
is accepted stale. Tags, epochs and the host's clear policy follow
va_kernels.hpp (TAG_EPOCH_BITS, SLOT_CLEAR_CALLS) and va_runtime.hip
(ticket_slot_for, release_capture_all), at a reduced epoch width so that wraps
happen within a test:

* the former tag, (epoch mod 2^w) << 11 | mg << 1 | 1, accepts a stale word once
  a group's epoch wraps while S changes between calls (planted: it must fail);
* the current tag, (epoch mod 2^w) << 7 | S, with a clear of the slot's store
  every 2^(w-1) eager calls and when a capture's binding is released, never
  does, for adversarial and random call sequences, captures included.
"""
import random
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
KHPP = (ROOT / "voltattn_amd" / "csrc" / "va_kernels.hpp").read_text()


def _const(name):
    return re.search(rf"constexpr\s+\S+(?:\s+\S+)*\s+{name}\s*=\s*([^;]+);", KHPP).group(1)


def test_product_constants_fit_the_tag():
    bits = int(_const("TAG_EPOCH_BITS"))
    assert bits + 7 <= 32                       # epoch field << 7 | S (1..64) in a 32-bit tag
    assert "1ull << (TAG_EPOCH_BITS - 1)" in _const("SLOT_CLEAR_CALLS")


class Slot:
    """One ticket slot's tagged store and epochs, and the host's policy."""

    def __init__(self, width, scheme, clear_every=None):
        self.width, self.scheme, self.clear_every = width, scheme, clear_every
        self.words = {}            # address -> (tag, call id)
        self.epoch = {}            # merge group -> epoch (device counter, unbounded)
        self.counted = 0           # eager calls since the last clear (host)
        self.call = 0
        self.stale = 0

    def tag(self, mg, S):
        e = self.epoch.get(mg, 0) % (1 << self.width)
        if self.scheme == "old":
            return (e << 11) | (mg << 1) | 1
        return (e << 7) | S

    def clear(self):
        self.words.clear()

    def decode(self, H, S, eager=True):
        if eager:                                   # ticket_slot_for: count, clear when due
            self.counted += 1
            if self.clear_every is not None and self.counted >= self.clear_every:
                self.clear()
                self.counted = 0
        self.call += 1
        for mg in range(H):
            t = self.tag(mg, S)
            for s in range(S):
                a = mg * S + s
                old = self.words.get(a)
                if old is not None and old[0] == t:
                    self.stale += 1                 # a word of an earlier call would be merged
                self.words[a] = (t, self.call)
            self.epoch[mg] = self.epoch.get(mg, 0) + 1


def adversarial(slot, between):
    """S = 8 once, `between` calls with S = 4 (addresses 4..7 of group 0 are
    not rewritten), then S = 8 again: its merger reads group 0's old words."""
    slot.decode(1, 8)
    for _ in range(between):
        slot.decode(1, 4)
    slot.decode(1, 8)
    return slot.stale


W = 6


def test_former_tag_accepts_a_stale_word_after_a_wrap():
    # group 0's epoch advances 2^W between the two S = 8 calls: same tag
    assert adversarial(Slot(W, "old"), (1 << W) - 1) > 0


def test_current_tag_without_clears_would_wrap_too():
    # S in the tag alone narrows the case to a group's own old words: the clear is needed
    assert adversarial(Slot(W, "new"), (1 << W) - 1) > 0


@pytest.mark.parametrize("between", [0, 1, (1 << (W - 1)) - 1, (1 << W) - 1, (1 << W), 3 * (1 << W) - 1])
def test_current_tag_with_clears_never_accepts_stale(between):
    assert adversarial(Slot(W, "new", 1 << (W - 1)), between) == 0


def test_random_sequences_with_captures():
    rng = random.Random(20241)
    for trial in range(40):
        slot = Slot(W, "new", 1 << (W - 1))
        graph = None
        for _ in range(600):
            r = rng.random()
            if graph is None and r < 0.02:
                # a captured graph takes the slot: a fixed list of calls, replayed uncounted
                graph = [(rng.randint(1, 6), rng.choice([1, 2, 3, 4, 8, 16, 64])) for _ in range(rng.randint(1, 3))]
            elif graph is not None and r < 0.05:
                slot.clear()                       # release_capture_all clears the slot
                slot.counted = 0
                graph = None
            elif graph is not None:
                for H, S in graph:
                    slot.decode(H, S, eager=False)
            else:
                slot.decode(rng.randint(1, 6), rng.choice([1, 2, 3, 4, 5, 8, 13, 16, 64]))
        assert slot.stale == 0, trial


def test_graph_replays_only_read_their_own_previous_words():
    # a long-lived graph (never released) with calls of different S, replayed
    # far past a wrap without any clear: each call site re-reads its own words
    slot = Slot(W, "new", 1 << (W - 1))
    graph = [(3, 8), (3, 4), (2, 16), (3, 8)]
    for _ in range(5 * (1 << W)):
        for H, S in graph:
            slot.decode(H, S, eager=False)
    assert slot.stale == 0
