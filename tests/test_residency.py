"""Residency policy (host, CPU): the offline replay ``residual_cache`` against
the known answers of the reference's own tests
(tests/test_runpod_v41_routed_precision.py:22-91,117-156,187-230, whose
expected lists are the data here), and the live no-wait policy
``ResidencyPolicy`` (omlx_routed.py:103-260) on scripted call sequences: lagged
harvest, tau, heaviest-first admission into free slots, routing only after a
read lands, LRU eviction down to ``spare``, cooling, and the wait rule."""

import numpy as np
import pytest

from keep_amd.residency import ResidencyPolicy, residual_cache, victim_order, wait_stats


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

    def read(self, e, s):
        self.reads.append((e, s))
        return e

    def done(self, h):
        return h in self.landed

    def route(self, e, s):
        assert e in self.landed, "routed before its bytes landed"
        self.log.append(("route", e, s))

    def unroute(self, e, s):
        self.log.append(("unroute", e, s))


def _call(p, want, score):
    p.begin()
    p.observe(np.asarray(want), np.asarray(score, dtype=np.float64))


def test_policy_harvests_lagged_demand_and_routes_only_landed_reads():
    h = Scripted()
    p = h.bind(num_experts=8, slots=4, order=[0, 1, 2, 3, 4, 5, 6, 7], tau=0.3, spare=1, lag=2)
    assert p.resident_mask().tolist() == [True] * 4 + [False] * 4
    _call(p, [[5, 0]], [3.0, 1.0])  # call 1: expert 5 strong (0.75), 0 weak (0.25)
    _call(p, [[0, 1]], [1.0, 1.0])  # call 2: harvests nothing yet (lag 2)
    assert h.reads == [] and p.stats["calls"] == 0
    # call 3 harvests call 1: 5 is wanted but no slot is free; the spare rule evicts the coldest unwanted
    # resident (3: the starting order puts colder experts first) into cooling
    _call(p, [[0, 1]], [1.0, 1.0])
    assert p.stats["no_slot"] == 1 and h.log == [("unroute", 3, 3)] and p.cooling == [(3, 3)]
    # call 4 harvests call 2 (nothing strong beyond residents 0, 1, both 0.5); the cooled slot is free only
    # once the harvested call is at least the eviction's step
    _call(p, [[5, 6]], [1.0, 1.0])
    assert p.free == [] and p.cooling == [(3, 3)]
    # call 5 harvests call 3 (at step 3: slot 3 leaves cooling); 0 and 1 are wanted and resident
    _call(p, [[0, 1]], [1.0, 1.0])
    assert p.free == [3] and p.cooling == []
    # call 6 harvests call 4: 5 and 6 wanted (0.5 each), one free slot: the heavier (ties: higher id) is read
    _call(p, [[0, 1]], [1.0, 1.0])
    assert h.reads == [(6, 3)] and p.reading.keys() == {6}
    assert p.stats["no_slot"] == 2
    # not landed: not routed, even across a harvest
    _call(p, [[0, 1]], [1.0, 1.0])
    assert ("route", 6, 3) not in h.log and 6 not in p.slot_of
    h.landed.add(6)
    _call(p, [[0, 1]], [1.0, 1.0])
    assert ("route", 6, 3) in h.log and p.slot_of[6] == 3 and p.slot_expert[3] == 6
    assert p.stats["installed"] == 1


def test_policy_lru_eviction_protects_the_wanted_and_counts():
    h = Scripted()
    p = h.bind(num_experts=6, slots=3, order=[0, 1, 2, 3, 4, 5], tau=0.4, spare=2, lag=1)
    _call(p, [[2, 1]], [1.0, 1.0])  # call 1
    _call(p, [[0, 4]], [1.0, 0.0])  # call 2 harvests call 1: 2 and 1 wanted (0.5): refreshed; spare 2 -> evict 0
    assert [x for x in h.log if x[0] == "unroute"] == [("unroute", 0, 0)]
    assert p.last_use[2] == 1 and p.last_use[1] == 1
    # the evicted slot is cooling until a later harvest; call 2's own demand (0 strong, 4 weak) arrives next
    _call(p, [[3, 3]], [1.0, 1.0])  # call 3 harvests call 2: 0 wanted, absent; slot 0 frees (evicted at step 2)
    assert h.reads == [(0, 0)]
    # eviction keeps spare: free + cooling counted; 1 and 2 are the residents, the coldest not wanted goes
    assert p.stats["evicted"] >= 1 and p.stats["admitted"] == 1


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
    assert p.slot_of == {0: 0, 1: 1, 5: 2} and h.log == [("unroute", 2, 2), ("route", 5, 2)]
    p.fetch([6, 7, 5], strong=[6])  # only 6 is fetched: victims are not demanded first (0), then demanded ones
    assert p.slot_of[6] == 0 and 5 in p.slot_of and p.stats["waits"] == 2
    with pytest.raises(RuntimeError, match="fewer slots"):
        p.fetch([2, 3, 4, 7])


def test_victim_order():
    last = np.array([3.0, 1.0, 2.0, 0.0])
    slot_expert = np.array([10, 11, 12, 13])
    assert victim_order(last, slot_expert, fetched={13}, demanded={13, 11}) == [2, 0, 1]


def test_policy_rejects_bad_setups():
    with pytest.raises(ValueError):
        ResidencyPolicy(4, 5, [0, 1, 2, 3])
    with pytest.raises(ValueError):
        ResidencyPolicy(4, 2, [0, 0, 1])
    with pytest.raises(ValueError):
        ResidencyPolicy(4, 2, [0, 1], lag=0)
