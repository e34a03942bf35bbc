"""The arrival-counter protocol of the one-launch EXL3 linear (evamx_device.hpp, arrive_last), run as
a state machine on the CPU over random interleavings of the arriving workgroups' atomic steps.

Each arrival does one atomic add; an add that finds the word in an unknown state (a fresh
workspace) is followed by a compare-and-swap loop. Whatever the word held before the call and
whatever the interleaving, exactly one arrival must see itself last, and the call must leave the
word at rest so that the next call (a graph replay, or another call on the workspace) counts from
zero. The GPU test test_exl3_linear_arrival_counters checks the compiled code on fill patterns;
this one covers interleavings and initial states a GPU run does not choose."""
import random

import pytest

REST = 0x3C6EF372
FIX = 0xA54FF53A
M64 = (1 << 64) - 1


def counting(w, n):
    hi, lo = w >> 32, w & 0xFFFFFFFF
    return hi in (REST, FIX) and lo < n


class Arrival:
    """One workgroup's arrival as a generator of atomic steps on the shared word."""

    def __init__(self, n):
        self.n = n
        self.last = None

    def run(self, mem):
        old = mem["w"]                                   # atomic add: read and write in one step
        mem["w"] = (old + 1) & M64
        yield
        if counting(old, self.n):
            self.last = (old & 0xFFFFFFFF) + 1 == self.n
        else:
            cur = (old + 1) & M64
            while True:
                nxt = (cur + 1) & M64 if counting(cur, self.n) else (FIX << 32) | 1
                actual = mem["w"]                        # compare-and-swap: one atomic step
                if actual == cur:
                    mem["w"] = nxt
                    self.last = (nxt & 0xFFFFFFFF) == self.n
                    yield
                    break
                cur = actual
                yield
        if self.last:
            mem["w"] = REST << 32                        # back to rest
            yield


def run_call(mem, n, rng, sequential=False):
    arrivals = [Arrival(n) for _ in range(n)]
    gens = [a.run(mem) for a in arrivals]
    live = list(range(n))
    while live:
        i = live[0] if sequential else rng.choice(live)
        try:
            next(gens[i])
        except StopIteration:
            live.remove(i)
    return [a.last for a in arrivals]


def initial_words(rng):
    words = [0, M64, 0x7F7F7F7F7F7F7F7F, 0xAAAAAAAAAAAAAAAA, REST << 32, (FIX << 32) | 3, (REST << 32) | 0xFFFFFFFF,
             (FIX << 32) | 0xFFFFFFFF, ((REST - 1) << 32) | 0xFFFFFFFF, ((FIX - 1) << 32) | 0xFFFFFFFF,
             ((REST - 1) << 32) | 0xFFFFFFFE]
    words += [rng.getrandbits(64) for _ in range(24)]
    return words


@pytest.mark.parametrize("n", [1, 2, 3, 4, 7, 14])
def test_one_last_arrival_and_rest_after_every_call(n):
    rng = random.Random(1000 + n)
    for w0 in initial_words(rng):
        # a word that already looks like a counting word with arrivals in flight is the one state
        # the protocol cannot tell from a call in progress; a completed call never leaves one
        if counting(w0, n) and (w0 & 0xFFFFFFFF) != 0:
            continue
        mem = {"w": w0}
        for call in range(6):                            # first use, then replays
            lasts = run_call(mem, n, rng)
            assert lasts.count(True) == 1, (hex(w0), call, lasts)
            assert mem["w"] == REST << 32, (hex(w0), call, hex(mem["w"]))


def test_garbage_counting_word_is_the_documented_limit():
    """A word holding (REST, c) with 0 < c < n is taken for a call in progress: no arrival of a
    fresh call sees itself last. Such a word only arises from a call that never finished, which is
    why the tags exclude one-byte fill patterns (the fill tests use those)."""
    rng = random.Random(7)
    n = 4
    mem = {"w": (REST << 32) | 2}
    lasts = run_call(mem, n, rng, sequential=True)
    assert lasts == [False, True, False, False]    # the count reaches n at the second arrival...
    assert mem["w"] == (REST << 32) + 2            # ...and the last two are counted past the reset
