"""Residency policy (host, CPU): the offline replay ``residual_cache`` against
the known answers of the reference's own tests
(tests/test_runpod_v41_routed_precision.py:22-91,117-156,187-230, whose
expected lists are the data here), and the live no-wait policy
``ResidencyPolicy`` (omlx_routed.py:103-260) on scripted call sequences: lagged
harvest, tau, heaviest-first admission into free slots, routing only after a
read lands, LRU eviction down to ``spare``, cooling, and the wait rule."""

import json

import numpy as np
import pytest

from keep_amd.residency import (COOLING, FREE, READING, ResidencyPolicy, plan_pieces, residual_cache, victim_order,
                               wait_stats)


def test_residual_cache_hits_only_after_async_admission():
    ind = np.array([[0, 1], [0, 1], [2, 0]])
    wts = np.array([[0.5, 0.1], [0.5, 0.1], [0.5, 0.5]])
    counts = np.zeros((3, 5))
    hi = residual_cache(ind, wts, k=1, tau=0.3, bounds=[3], warm=None, counts=counts)
    assert hi.tolist() == [[False, False], [True, False], [False, True]]
    assert counts[:, 4].tolist() == [2, 0, 1]


def test_residual_cache_resets_per_record_and_warm_start():
    ind = np.array([[0], [0], [0]])
    wts = np.ones((3, 1))
    counts = np.zeros((1, 5))
    hi = residual_cache(ind, wts, k=1, tau=0.3, bounds=[2, 1], warm=None, counts=counts)
    assert hi[:, 0].tolist() == [False, True, False]
    assert counts[0, 4] == 2
    hi = residual_cache(ind, wts, k=1, tau=0.3, bounds=[3], warm=np.array([0]), counts=np.zeros((1, 5)))
    assert hi.all()


def test_residual_cache_prompt_warm_start():
    ind = np.array([[1], [1], [1], [0]])
    counts = np.zeros((2, 5))
    hi = residual_cache(ind, np.ones((4, 1)), k=1, tau=9.0, bounds=[4], warm=np.array([0]), counts=counts,
                        policy="prompt:2")
    assert hi[:, 0].tolist() == [False, False, True, False]
    assert counts[:, 4].tolist() == [0, 1]
    lru = residual_cache(ind, np.ones((4, 1)), k=1, tau=9.0, bounds=[4], warm=np.array([0]), counts=np.zeros((2, 5)))
    assert lru[:, 0].tolist() == [False, False, False, True]


def test_residual_cache_wait_and_exact_prefill():
    ind = np.array([[1], [1], [0], [1]])
    wts = np.array([[0.2], [0.6], [0.6], [0.6]])
    resident, waited = np.zeros((4, 2), dtype=bool), []
    hi = residual_cache(ind, wts, k=1, tau=0.5, bounds=[4], warm=np.array([0]), counts=np.zeros((2, 5)),
                        policy="wait:0.5", resident=resident, waited=waited)
    assert hi[:, 0].tolist() == [False, True, True, True] and waited == [1, 2, 3]
    assert resident.tolist() == [[True, False], [True, True], [True, True], [True, True]]
    assert wait_stats({0: [1, 2], 3: [2, 5]}, tokens=10, n_layers=4) == {
        "wait_token_share": 0.3, "wait_layer_rerun_share": (4 + 4 + 1) / 40}
    waited = []
    hi = residual_cache(ind, np.full((4, 1), 0.2), k=1, tau=9.0, bounds=[4], warm=np.array([0]),
                        counts=np.zeros((2, 5)), policy="exact:2", waited=waited)
    assert hi[:, 0].tolist() == [True, True, False, True] and waited == []


def test_residual_cache_served_timing():
    ind = np.array([[1], [1], [1], [1], [1]])
    wts = np.ones((5, 1))

    def run(policy):
        return residual_cache(ind, wts, k=1, tau=0.5, bounds=[5], warm=np.array([0]), counts=np.zeros((2, 5)),
                              policy=policy)[:, 0].tolist()
    assert run("lru") == [False, True, True, True, True]
    assert run("lag:3") == [False, False, False, True, True]
    assert run("frozen:4") == [False, False, False, False, True]
    assert run("lag:2+frozen:1") == [False, False, True, True, True]
    counts = np.zeros((2, 5))
    residual_cache(ind, wts, k=1, tau=0.5, bounds=[5], warm=np.array([0]), counts=counts, policy="lag:3")
    assert counts[:, 4].tolist() == [0, 1]


def test_residual_cache_oracle_and_trace():
    ind = np.array([[0, 1], [2, 1], [2, 0], [3, 3]])
    wts = np.array([[0.9, 0.1], [0.5, 0.1], [0.5, 0.2], [0.3, 0.3]])
    counts = np.zeros((4, 5))
    hi = residual_cache(ind, wts, k=2, tau=0.3, bounds=[3, 1], warm=None, counts=counts, policy="oracle")
    assert hi.tolist() == [[True, False], [True, False], [True, True], [True, True]]
    assert counts[:, 4].sum() == 0
    trace: list = []
    residual_cache(ind, wts, k=2, tau=0.3, bounds=[3, 1], warm=None, counts=counts, trace=trace)
    assert trace == [(0, 0, 0), (0, 1, 2), (1, 0, 3)]


def test_residual_cache_reports_the_resident_set():
    ind = np.array([[0, 1], [2, 1], [2, 0]])
    wts = np.array([[0.9, 0.1], [0.5, 0.1], [0.5, 0.2]])
    resident = np.zeros((3, 4), dtype=bool)
    residual_cache(ind, wts, k=2, tau=0.3, bounds=[3], warm=np.array([3, 1]), counts=np.zeros((4, 5)),
                   resident=resident)
    assert resident.tolist() == [[False, True, False, True], [True, True, False, False], [True, False, True, False]]
    resident[:] = False
    residual_cache(ind, wts, k=2, tau=0.3, bounds=[3], warm=None, counts=np.zeros((4, 5)), policy="oracle",
                   resident=resident)
    assert resident.all(axis=0).tolist() == [True, False, True, False]


def test_residual_cache_takes_one_threshold_per_expert():
    ind = np.array([[0, 1], [0, 1], [0, 1]])
    wts = np.array([[0.4, 0.2], [0.4, 0.2], [0.4, 0.2]], dtype=np.float32)
    same = [residual_cache(ind, wts, k=2, tau=tau, bounds=[3], warm=None, counts=np.zeros((2, 5)))
            for tau in (0.3, np.array([0.3, 0.3]))]
    np.testing.assert_array_equal(*same)
    assert same[0].tolist() == [[False, False], [True, False], [True, False]]
    counts = np.zeros((2, 5))
    hi = residual_cache(ind, wts, k=2, tau=np.array([0.5, 0.2]), bounds=[3], warm=None, counts=counts)
    assert hi.tolist() == [[False, False], [False, True], [False, True]] and counts[:, 4].tolist() == [0, 1]


def test_residual_cache_prompt_with_fewer_heavy_experts_than_slots():
    # one expert carries all the prompt's mass: it joins the most recent residents, the rest fill from the
    # old set (most recent first kept), never a negative slice of it
    ind = np.array([[2], [2], [0]])
    hi = residual_cache(ind, np.ones((3, 1)), k=3, tau=9.0, bounds=[3], warm=np.array([0, 1]),
                        counts=np.zeros((3, 5)), policy="prompt:2")
    assert hi[:, 0].tolist() == [False, False, True]


# ----------------------------------------------------------------------------- live policy


class Scripted:
    """Hooks of a policy under test: reads land when released, and every
    route / unroute is logged with the landed state of the read."""

    def __init__(self):
        self.landed, self.log, self.reads = set(), [], []

    def bind(self, **kw):
        return ResidencyPolicy(read=self.read, done=self.done, route=self.route, unroute=self.unroute, **kw)

    def read(self, layer, e, s):
        self.reads.append((e, s) if layer == 0 else (layer, e, s))
        return (layer, e)

    def done(self, h):
        return h[1] in self.landed

    def route(self, layer, e, s):
        assert e in self.landed, "routed before its bytes landed"
        self.log.append(("route", e, s) if layer == 0 else ("route", layer, e, s))

    def unroute(self, layer, e, s):
        self.log.append(("unroute", e, s) if layer == 0 else ("unroute", layer, e, s))


def _call(p, want, score, layer=0):
    p.begin()
    p.observe(np.asarray(want), np.asarray(score, dtype=np.float64), layer)


def _cooling(tab):
    """(slot, call that evicted it) of every cooling slot."""
    return [(s, int(tab.stamp[s])) for s in tab.slots_in(COOLING)]


def test_policy_harvests_lagged_demand_and_routes_only_landed_reads():
    h = Scripted()
    p = h.bind(num_experts=8, slots=4, order=[0, 1, 2, 3, 4, 5, 6, 7], tau=0.3, spare=1, lag=2)
    tab = p.table()
    assert p.resident_mask().tolist() == [True] * 4 + [False] * 4
    _call(p, [[5, 0]], [3.0, 1.0])  # call 1: expert 5 strong (0.75), 0 weak (0.25)
    _call(p, [[0, 1]], [1.0, 1.0])  # call 2: harvests nothing yet (lag 2)
    assert h.reads == [] and p.stats["calls"] == 0
    # call 3 harvests call 1: 5 is wanted but no slot is free; the spare rule evicts the coldest unwanted
    # resident (3: the starting order puts colder experts first) into cooling
    _call(p, [[0, 1]], [1.0, 1.0])
    assert p.stats["no_slot"] == 1 and h.log == [("unroute", 3, 3)] and _cooling(tab) == [(3, 3)]
    # call 4 harvests call 2 (nothing strong beyond residents 0, 1, both 0.5); the cooled slot is free only
    # once the harvested call is at least the eviction's step
    _call(p, [[5, 6]], [1.0, 1.0])
    assert tab.slots_in(FREE) == [] and _cooling(tab) == [(3, 3)]
    # call 5 harvests call 3 (at step 3: slot 3 leaves cooling); 0 and 1 are wanted and resident
    _call(p, [[0, 1]], [1.0, 1.0])
    assert tab.slots_in(FREE) == [3] and _cooling(tab) == []
    # call 6 harvests call 4: 5 and 6 wanted (0.5 each), one free slot: the heavier (ties: higher id) is read
    _call(p, [[0, 1]], [1.0, 1.0])
    assert h.reads == [(6, 3)] and tab.slots_in(READING) == [3] and tab.expert[3] == 6
    assert p.stats["no_slot"] == 2
    # not landed: not routed, even across a harvest
    _call(p, [[0, 1]], [1.0, 1.0])
    assert ("route", 6, 3) not in h.log and 6 not in tab.assignment()
    h.landed.add(6)
    _call(p, [[0, 1]], [1.0, 1.0])
    assert ("route", 6, 3) in h.log and tab.assignment()[6] == 3 and tab.slot_expert()[3] == 6
    assert p.stats["installed"] == 1
    # the spare rule evicted 2 when 6 was admitted (call 6); it thawed once call 6 was harvested (call 8)
    assert tab.describe() == {"free": [2], "reading": [], "routed": [0, 1, 3], "cooling": []}


def test_policy_lru_eviction_protects_the_wanted_and_counts():
    h = Scripted()
    p = h.bind(num_experts=6, slots=3, order=[0, 1, 2, 3, 4, 5], tau=0.4, spare=2, lag=1)
    _call(p, [[2, 1]], [1.0, 1.0])  # call 1
    _call(p, [[0, 4]], [1.0, 0.0])  # call 2 harvests call 1: 2 and 1 wanted (0.5): refreshed; spare 2 -> evict 0
    assert [x for x in h.log if x[0] == "unroute"] == [("unroute", 0, 0)]
    assert p.table().stamp[2] == 1 and p.table().stamp[1] == 1
    # the evicted slot is cooling until a later harvest; call 2's own demand (0 strong, 4 weak) arrives next
    _call(p, [[3, 3]], [1.0, 1.0])  # call 3 harvests call 2: 0 wanted, absent; slot 0 frees (evicted at step 2)
    assert h.reads == [(0, 0)]
    # eviction keeps spare: free + cooling counted; 1 and 2 are the residents, the coldest not wanted goes
    assert p.stats["evicted"] >= 1 and p.stats["admitted"] == 1


def test_policy_frees_slots_last_in_first_out():
    # two slots cool at one harvest, the later-evicted one is reused first
    h = Scripted()
    p = h.bind(num_experts=8, slots=4, order=[0, 1, 2, 3, 4, 5, 6, 7], tau=0.3, spare=2, lag=1)
    _call(p, [[0, 1]], [1.0, 1.0])  # call 1
    _call(p, [[6, 0]], [3.0, 1.0])  # call 2 harvests call 1: evicts 3 then 2 (least recent first)
    assert h.log == [("unroute", 3, 3), ("unroute", 2, 2)]
    _call(p, [[0, 1]], [1.0, 1.0])  # call 3 harvests call 2: both slots thaw (evicted at 2), 6 reads slot 2
    assert h.reads == [(6, 2)]


def test_policy_tau_inf_never_harvests():
    h = Scripted()
    p = h.bind(num_experts=4, slots=2, order=[0, 1, 2, 3], tau=float("inf"), spare=1, lag=1)
    for _ in range(4):
        _call(p, [[2, 3]], [1.0, 1.0])
    assert h.reads == [] and h.log == [] and p.stats["calls"] == 0


def test_policy_wait_rule_fetches_over_the_least_recent():
    h = Scripted()
    h.landed.update(range(8))
    p = h.bind(num_experts=8, slots=3, order=[0, 1, 2, 3, 4, 5, 6, 7], tau=float("inf"), lag=1)
    p.begin()
    p.fetch([5, 1])  # 5 absent: over the least recently used resident not demanded (2: colder start)
    assert p.table().assignment() == {0: 0, 1: 1, 5: 2} and h.log == [("unroute", 2, 2), ("route", 5, 2)]
    p.fetch([6, 7, 5], strong=[6])  # only 6 is fetched: victims are not demanded first (0), then demanded ones
    assert p.table().assignment()[6] == 0 and 5 in p.table().assignment() and p.stats["waits"] == 2
    with pytest.raises(RuntimeError, match="fewer slots"):
        p.fetch([2, 3, 4, 7])


def test_wait_rule_lands_an_inflight_admission_instead_of_reading_twice():
    h = Scripted()
    p = h.bind(num_experts=8, slots=4, order=[0, 1, 2, 3, 4, 5, 6, 7], tau=0.3, spare=1, lag=1)
    _call(p, [[0, 1]], [1.0, 1.0])
    _call(p, [[6, 0]], [3.0, 1.0])  # harvest of call 1 evicts 3 (spare 1)
    _call(p, [[0, 1]], [1.0, 1.0])  # harvest of call 2 reads 6 into the thawed slot 3; not landed
    assert h.reads == [(6, 3)]
    h.landed.add(6)
    p.fetch([6, 0])
    assert h.reads == [(6, 3)] and p.table().assignment()[6] == 3 and p.stats["installed"] == 1


def test_policy_layers_share_one_clock():
    h = Scripted()
    p = ResidencyPolicy.layers([(8, 4, range(8)), (6, 3, [5, 4, 3, 2, 1, 0])], tau=0.3, spare=1, lag=1,
                               read=h.read, done=h.done, route=h.route, unroute=h.unroute)
    h.landed.update(range(8))

    def call():
        p.begin()
        p.observe(np.array([[6, 0]]), np.array([[3.0, 1.0]]), 0)
        p.observe(np.array([[0, 1]]), np.array([[3.0, 1.0]]), 1)
    call()
    call()  # harvests call 1 in both layers: no free slot; each evicts its coldest unwanted resident
    assert h.log == [("unroute", 3, 3), ("unroute", 1, 3, 2)] and h.reads == [] and p.stats["calls"] == 1
    call()  # harvests call 2: the slots evicted at call 2 thaw and take each layer's wanted expert
    assert h.reads == [(6, 3), (1, 0, 2)]
    call()  # the reads have landed: routed at the next harvest, in each layer's own table
    assert [x for x in h.log if x[0] == "route"] == [("route", 6, 3), ("route", 1, 0, 2)]
    assert p.table(0).assignment()[6] == 3 and p.table(1).assignment()[0] == 2
    # layer 1 kept one spare: its coldest unwanted resident (4) went when 0 was admitted
    assert p.resident_mask(1).tolist() == [True, False, False, False, False, True]


def test_prefill_pieces_fit_the_slots():
    index = np.array([[0, 1], [2, 3], [0, 4], [5, 6], [7, 0]])
    share = np.array([[0.6, 0.4], [0.5, 0.5], [0.9, 0.1], [0.5, 0.5], [0.7, 0.3]])
    # 0.2: all but expert 4 at token 2 (0.1) must be resident; 4 slots: tokens 0-2 hold {0,1,2,3}, token 3 overflows
    assert plan_pieces(index, share, 4, 0.2) == [(0, 3, [0, 1, 2, 3]), (3, 5, [0, 5, 6, 7])]
    # 0.45: the weak routes (1: 0.4, 4: 0.1, 0: 0.3) need no slot
    assert plan_pieces(index, share, 4, 0.45) == [(0, 3, [0, 2, 3]), (3, 5, [5, 6, 7])]
    # a token that alone needs more than the slots is a piece of its own (no empty piece before it)
    assert plan_pieces(index, share, 1, 0.2) == [(0, 1, [0, 1]), (1, 2, [2, 3]), (2, 3, [0]), (3, 4, [5, 6]),
                                                 (4, 5, [0, 7])]
    assert plan_pieces(index, share, 8, 0.2) == [(0, 5, [0, 1, 2, 3, 5, 6, 7])]
    assert plan_pieces(np.zeros((0, 2), int), np.zeros((0, 2)), 4, 0.2) == [(0, 0, [])]


def test_run_pieces_fetches_each_piece_before_running_it():
    h = Scripted()
    h.landed.update(range(8))
    p = h.bind(num_experts=8, slots=4, order=[0, 1, 2, 3, 4, 5, 6, 7], tau=float("inf"), lag=1)
    index = np.array([[0, 1], [2, 3], [0, 4], [5, 6], [7, 0]])
    score = np.array([[3.0, 2.0], [1.0, 1.0], [9.0, 1.0], [1.0, 1.0], [7.0, 3.0]])  # raw: normalised per token
    seen = []

    def run(a, b):
        seen.append((a, b, sorted(p.table().assignment())))
    assert p.run_pieces(index, score, 0.2, run) == 2
    # piece 2 fetches 5, 6, 7 over 1, 2, 3 (least recent, not demanded by it); 0 stays
    assert seen == [(0, 3, [0, 1, 2, 3]), (3, 5, [0, 5, 6, 7])]
    assert p.stats["waits"] == 1 and p.stats["tokens"] == 5


def test_stats_log_rows(tmp_path):
    h = Scripted()
    p = h.bind(num_experts=4, slots=2, order=[0, 1, 2, 3], tau=0.3, spare=1, lag=1)
    _call(p, [[2, 3]], [1.0, 1.0])
    _call(p, [[0, 1]], [1.0, 1.0])
    path = tmp_path / "stats.jsonl"
    p.write_log(path)
    row = p.write_log(path, verify=True)
    lines = [json.loads(x) for x in path.read_text().splitlines()]
    assert len(lines) == 2 and lines[1] == row and row["mismatched"] == 0
    assert row["step"] == 2 and row["calls"] == 1 and row["tokens"] == 1 and row["demand"] == 2
    assert set(ResidencyPolicy.STATS) <= set(row)


def test_victim_order():
    last = np.array([3.0, 1.0, 2.0, 0.0])
    slot_expert = np.array([10, 11, 12, 13])
    assert victim_order(last, slot_expert, fetched={13}, demanded={13, 11}) == [2, 0, 1]
    # ties in recency: lower slot first; slots holding nothing (recency inf) after the residents of their group
    assert victim_order([1.0, 1.0, np.inf, 0.0], [4, 5, -1, 6], fetched=set(), demanded={6}) == [0, 1, 2, 3]


def test_policy_rejects_bad_setups():
    with pytest.raises(ValueError):
        ResidencyPolicy(4, 5, [0, 1, 2, 3])
    with pytest.raises(ValueError):
        ResidencyPolicy(4, 2, [0, 0, 1])
    with pytest.raises(ValueError):
        ResidencyPolicy(4, 2, [0, 1], lag=0)
    with pytest.raises(ValueError, match="unknown replay option"):
        residual_cache(np.zeros((1, 1), int), np.ones((1, 1)), 1, 0.5, [1], None, np.zeros((1, 5)), policy="fifo")
