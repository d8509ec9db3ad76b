"""The pipelined product's stage schedule, checked on the CPU for every tiling
in the kernels' table and every panel depth it accepts: the steady-state
loop and the drain together multiply every sub-step exactly once, and no
stage is loaded past the last (a stage past it would read a unit beyond the
weights and activations). The rule that a tiling fits a depth is restated
from the kernels' fits(); the test also checks the source still states it."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "libpktito_amd", "csrc", "q8_kernels.hip")


def table():
    s = open(SRC).read()
    a = s.index("static const RingCfg kRing[] = {")
    b = s.index("};", a)
    rows = re.findall(r'\{ "([^"]+)", (\d+), (\d+), (\d+), (\d+), (\d+),', s[a:b])
    return [(n, int(u), int(sl), int(kg)) for (n, _bn, _bm, u, sl, kg) in rows]


def fits(ups, slots, kg, ku):
    """kernels' fits(): ring tilings run whole passes of four stages; pipe
    tilings need their slots' worth of stages and, with one unit a stage, an
    even number of stages past the first fill."""
    if slots == 0:
        return ku % (4 * ups) == 0
    if ku % (kg * ups):
        return False
    ns = ku // (kg * ups)
    return ns >= slots and (ups > 1 or (ns - slots) % 2 == 0)


def schedule(ups, slots, ns):
    """pipe_tile's order: the stages the workgroup loads, and the sub-steps it
    multiplies, in the order its loops visit them."""
    spi = max(2, ups)
    loaded = list(range(slots))                    # the prologue
    done = []
    steady = (ns - slots) * ups
    gi = 0
    while gi < steady:                             # for (gi = 0; gi < steady; gi += SPI)
        for k in range(spi):
            done.append(gi + k)
            if k % ups == ups - 1:                 # the last sub-step of a stage refills
                loaded.append((gi + k) // ups + slots)
        gi += spi
    done += [steady + k for k in range(slots * ups)]   # the drain, unrolled
    return loaded, done


def test_the_source_states_the_rule():
    s = open(SRC).read()
    assert "(c.ups > 1 || (ns - c.slots) % 2 == 0)" in s


def test_every_tiling_loads_in_range_and_multiplies_each_step_once():
    tilings = [t for t in table() if t[2] > 0]
    assert len(tilings) >= 8
    checked = 0
    for name, ups, slots, kg in tilings:
        for ku in range(4, 1028, 4):
            if not fits(ups, slots, kg, ku):
                continue
            ns = ku // (kg * ups)
            loaded, done = schedule(ups, slots, ns)
            assert max(loaded) < ns, (name, ku)
            assert sorted(loaded) == list(range(ns)), (name, ku)
            assert done == list(range(ns * ups)), (name, ku)
            checked += 1
    assert checked > 500


def test_the_rule_rejects_the_odd_tail():
    # four K groups, one unit a stage, two slots, ku = 12: three stages a group,
    # one past the slots' first fill; a steady pass of two would load stage 3
    assert not fits(1, 2, 4, 12)
    loaded, done = schedule(1, 2, 3)
    assert max(loaded) >= 3 or done != list(range(3))
