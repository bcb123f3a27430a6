"""Host logic of the decode state cache (no GPU): slot planning, copy-on-write, refcounts.
These drive the native bookkeeping of libverace_sssd.so (``vmi_state_cache_*``), which
makes no device call until a step is launched.

The planner is checked against a model of the reference's semantics, where every
sequence owns an independent state (``acd_engine.py:85-92`` copies the state lists so
that branches never mutate a shared input): a simulated pool of slots is updated the
way the kernel updates it (item b reads slot in[b] or the identity, writes slot out[b]),
and after every step each handle's slot must hold exactly the state the model says it
has.  The same simulation checks the launch contract of ``vmi_sssd_step_slots``: written
slots are distinct and no slot written in a step is read by another item of that step.
"""
import random

import numpy as np
import pytest

from verace_amd.state_cache import SlotTable


def _simulate(table, pool, model, layer, hs, tag):
    src, dst = table.plan_step(layer, hs)
    assert len(set(dst.tolist())) == len(dst), "written slots must be distinct"
    for b, (s, d) in enumerate(zip(src, dst)):
        assert 0 <= d < table.num_slots
        for b2, s2 in enumerate(src):
            if b2 != b:
                assert s2 != d, "a slot written by one item is read by another"
    reads = [() if s < 0 else pool[layer][s] for s in src]   # all reads before any write
    for h, r, d in zip(hs, reads, dst):
        pool[layer][d] = r + (tag,)
        model[h][layer] = model[h][layer] + (tag,)
    return src, dst


def _check(table, pool, model):
    for h, states in model.items():
        phys = table.phys(h)
        for l, st in enumerate(states):
            if phys[l] < 0:
                assert st == ()
            else:
                assert pool[l][phys[l]] == st, (h, l)
    # refcounts equal the number of holders, free lists hold exactly the unheld slots
    for l in range(table.num_layers):
        held = [table.phys(h)[l] for h in model]
        for s in range(table.num_slots):
            assert table.refs[l, s] == sum(1 for x in held if x == s)
        assert table.free_slots(l) == sum(1 for s in range(table.num_slots) if table.refs[l, s] == 0)


def test_first_step_allocates_then_updates_in_place():
    t = SlotTable(2, 8)
    a, b = t.new(2)
    src, dst = t.plan_step(0, [a, b])
    assert src.tolist() == [-1, -1] and len(set(dst.tolist())) == 2
    src2, dst2 = t.plan_step(0, [b, a])
    assert src2.tolist() == [dst[1], dst[0]] and dst2.tolist() == src2.tolist()
    assert t.phys(a).tolist() == [dst[0], -1]
    assert t.free_slots(0) == 6 and t.free_slots(1) == 8


def test_fork_shares_until_written():
    t = SlotTable(1, 8)
    (p,) = t.new(1)
    _, (s0,) = t.plan_step(0, [p])
    c1, c2 = t.fork(p, 2)
    assert t.refs[0, s0] == 3 and t.phys(c1)[0] == s0
    # one branch steps: it reads the shared slot and writes a fresh one
    src, dst = t.plan_step(0, [c1])
    assert src[0] == s0 and dst[0] != s0 and t.refs[0, s0] == 2
    # the parent and the other branch step together: both still share s0 -> both fresh
    src, dst = t.plan_step(0, [p, c2])
    assert src.tolist() == [s0, s0] and s0 not in dst.tolist()
    assert t.refs[0, s0] == 0 and t.free_slots(0) == 8 - 3
    # now everyone is a sole holder: in place
    src, dst = t.plan_step(0, [c2, p, c1])
    assert src.tolist() == dst.tolist()


def test_release_frees_only_unshared_slots():
    t = SlotTable(2, 4)
    (p,) = t.new(1)
    t.plan_step(0, [p])
    t.plan_step(1, [p])
    (c,) = t.fork(p, 1)
    t.release([p])
    assert t.free_slots(0) == 3 and t.free_slots(1) == 3   # c still holds them
    t.release([c])
    assert t.free_slots(0) == 4 and t.free_slots(1) == 4
    with pytest.raises(ValueError):
        t.plan_step(0, [c])


def test_errors():
    t = SlotTable(1, 2)
    a, b, c = t.new(3)
    with pytest.raises(ValueError):
        t.plan_step(0, [a, a])
    with pytest.raises(ValueError):
        t.plan_step(1, [a])
    t.plan_step(0, [a, b])
    with pytest.raises(RuntimeError, match="full"):
        t.plan_step(0, [c])
    # a failed plan leaves the table unchanged
    assert t.phys(c)[0] == -1 and t.free_slots(0) == 0
    with pytest.raises(ValueError):
        SlotTable(0, 4)


@pytest.mark.parametrize("seed", range(6))
def test_random_tree_search_matches_independent_states(seed):
    """Random prefill / step / fork / release traffic over 3 layers: every handle's slot
    always holds the state an independent copy would have."""
    rng = random.Random(seed)
    L, N = 3, 40
    t = SlotTable(L, N)
    pool = [[None] * N for _ in range(L)]
    model = {}
    tag = 0
    for h in t.new(4):
        model[h] = [()] * L
    for _ in range(200):
        op = rng.random()
        live = list(model)
        if op < 0.5 and live:
            layer = rng.randrange(L)
            hs = rng.sample(live, rng.randint(1, len(live)))
            need = sum(1 for h in hs if t.phys(h)[layer] < 0 or t.refs[layer, t.phys(h)[layer]] > 1)
            if need > t.free_slots(layer):
                with pytest.raises(RuntimeError):
                    t.plan_step(layer, hs)
                continue
            tag += 1
            _simulate(t, pool, model, layer, hs, tag)
        elif op < 0.75 and live and len(live) < 12:
            parent = rng.choice(live)
            for c in t.fork(parent, rng.randint(1, 3)):
                model[c] = list(model[parent])
        elif op < 0.9 and len(live) > 1:
            gone = rng.sample(live, rng.randint(1, len(live) - 1))
            t.release(gone)
            for h in gone:
                del model[h]
        else:
            for h in t.new(1):
                model[h] = [()] * L
        _check(t, pool, model)
