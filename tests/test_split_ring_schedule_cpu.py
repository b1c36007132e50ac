"""Model of the split ring's LDS schedule (csrc/fp8_gemm_pipe.h, split_loop).

The 256x256 tiles keep two activation slots and three weight slots.  Stage s
sits in activation slot s % 2 and weight slot (s + c) % 3 with c = (1 - KT) mod 3.
Between two barriers the four waves run unsynchronized, so:
  * a DMA into a slot must come in a later barrier interval than every read of
    the slot's previous stage (all waves have passed the barrier between them);
  * a read of a stage must come after a wait that covers that stage's DMAs and a
    barrier (every wave's DMAs have landed).
DMAs of stages past the end still write (zeros), so they count as writes.  The
scale and bias vectors are DMA'd in the last stage's first half into weight
slot 2 and read by the epilogue, whose output staging covers the first 128 KB.
"""

import pytest

HA = HW = 256 * 128  # bytes of one activation / weight stage slot (32 KB)


def a_slot(s):
    return ("A", s % 2)


def w_slot(s, c):
    return ("W", (s + c) % 3)


def schedule(kt_total):
    """Events per barrier interval: ('write', slot, tag) / ('read', slot, tag),
    and the DMA tags each interval's closing wait has landed."""
    c = (1 - kt_total) % 3
    intervals = [[]]
    landed_at_close = []
    issued = []  # DMA tags in issue order (per wave; every wave issues alike)

    def write(slot, tag):
        intervals[-1].append(("write", slot, tag))
        issued.append(tag)

    def read(slot, tag):
        intervals[-1].append(("read", slot, tag))

    def close(outstanding_groups):
        # wait until at most the last `outstanding_groups` DMA groups are in flight
        done = issued[: len(issued) - outstanding_groups] if outstanding_groups else list(issued)
        landed_at_close.append(set(done))
        intervals.append([])

    # prologue: A0 W0 A1 W1, wait for stage 0 (stage 1's two groups in flight)
    write(a_slot(0), ("A", 0)), write(w_slot(0, c), ("W", 0))
    write(a_slot(1), ("A", 1)), write(w_slot(1, c), ("W", 1))
    close(2)
    read(a_slot(0), ("A", 0)), read(w_slot(0, c), ("W", 0))  # substep 0 of stage 0
    for kt in range(kt_total):
        last = kt == kt_total - 1
        read(a_slot(kt), ("A", kt)), read(w_slot(kt, c), ("W", kt))  # substep 1
        if last:
            write(("W", 2), ("V",))
        else:
            write(w_slot(kt + 2, c), ("W", kt + 2))
        close(1)  # stage kt+1 landed; this half's DMA group may be in flight
        write(a_slot(kt + 2), ("A", kt + 2))
        if kt + 1 < kt_total:
            read(a_slot(kt + 1), ("A", kt + 1)), read(w_slot(kt + 1, c), ("W", kt + 1))
    close(0)  # the kernel's final wait for every DMA, then a barrier
    read(("W", 2), ("V",))  # the epilogue reads the vectors
    return intervals, landed_at_close, c


@pytest.mark.parametrize("kt_total", list(range(1, 13)) + [40, 42, 108])
def test_split_ring_has_no_lds_hazard(kt_total):
    intervals, landed, c = schedule(kt_total)
    occupant = {}  # slot -> (tag, interval of its last read)
    last_read = {}
    written_in = {}
    for i, events in enumerate(intervals):
        for kind, slot, tag in events:
            if kind == "write":
                prev = occupant.get(slot)
                if prev is not None and prev in last_read:
                    assert last_read[prev] < i, f"KT={kt_total}: {tag} overwrites {prev} read in the same interval"
                occupant[slot] = tag
                written_in[tag] = i
            else:
                assert occupant.get(slot) == tag, f"KT={kt_total}: {slot} holds {occupant.get(slot)}, not {tag}"
                assert written_in[tag] < i and tag in landed[i - 1], (
                    f"KT={kt_total}: {tag} read before its DMA was waited for")
                last_read[tag] = i
    # The vectors slot is weight slot 2, free in the last stage, and no DMA
    # writes it after the vectors land.
    assert (kt_total + 1 + c) % 3 == 2
    assert occupant[("W", 2)] == ("V",)


def test_vectors_slot_is_outside_the_output_staging():
    staging = 256 * 256 * 2  # bf16 staging tile of the epilogue, from the ring's start
    w_slot2 = 2 * HA + 2 * HW
    assert staging <= w_slot2 and w_slot2 + HW == 160 * 1024
    vec_bytes = 3 * 1024 + 2 * 2048 * 4  # scales, bias and the SwiGLU silu table
    assert vec_bytes <= HW
