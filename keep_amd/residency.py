"""Expert residency: which experts of a layer's pool sit in its device slots.

The routed layers serve only resident experts (the router's served bias is
``OFF`` for the others) and read an expert's codes at its slot's row of the
pool (``slot_map[e]``). This module keeps that state on the host.

Design. Every slot of a layer's pool is in one of four states, held in
numpy arrays (``SlotTable``):

    FREE --read--> READING --landed--> ROUTED --evict--> COOLING --later call--> FREE

A ROUTED slot carries the call that last demanded its expert (its recency);
a COOLING slot the call that evicted it, since calls issued before the
eviction may still read it; a FREE slot the order in which it was freed (the
most recently freed is reused first). One ``ResidencyPolicy`` holds the
tables of every layer of a model behind one clock: ``begin()`` once per
forward call, then each layer's demand is recorded with ``observe``.

The rules are the serving cache's (behaviour of the reference's routed
cache, ``scripts/v41_build/omlx_routed.py:103-260``, and its wait rule,
``scripts/v41_build/omlx_lattice.py:283-324,427-449``):

- no-wait: ``lag`` calls after a call ran, its demand (the router's demand
  top-k and raw scores) is harvested. Every demanded slot whose normalised
  weight reaches ``tau`` wants its expert; a wanted resident's recency is
  refreshed, a wanted absent expert is read into a free slot (heaviest
  first) and routed only once its bytes have landed, and residents nobody
  wanted are evicted, least recent first, until ``spare`` slots are free or
  cooling;
- wait: ``fetch`` reads a call's demand in before the call runs, over the
  least recently demanded residents; ``plan_pieces`` splits a prefill into
  pieces whose demand fits the slots, each fetched and run before the next
  overwrites slots.

``ResidencyCache`` binds a policy to a device: slot pools written by
``loaders.ExpertInstaller`` on its own stream, the router's ``bias_served``
and ``slot_map`` tensors (changed between calls, in stream order), and the
nested tier's slot rows (``HotTier.route_slot``) rewritten as experts move.
``replay`` / ``wait_stats`` simulate the policy offline over recorded
routings (behaviour of ``scripts/runpod/v41_reap/local_eval.py:184-286``).
"""

from __future__ import annotations

import json
import time
from dataclasses import dataclass
from typing import Callable, Sequence

import numpy as np
import torch

from keep_amd.router import OFF

FREE, READING, ROUTED, COOLING = 0, 1, 2, 3
_NAMES = ("free", "reading", "routed", "cooling")


# ----------------------------------------------------------------------------- offline replay


@dataclass
class ReplayOptions:
    """A replay policy string, options joined by ``+``: ``lru`` (default),
    ``oracle``, ``lag:N`` (an admission serves from N tokens on),
    ``frozen:P`` (nothing lands in a record's first P tokens), ``prompt:P``
    (after P tokens the record's own heaviest experts replace the residents),
    ``exact:P`` (as prompt, and those P tokens are served whatever they ask),
    ``wait:W`` (an absent expert asked with gate >= W is served by waiting)."""

    oracle: bool = False
    lag: int = 1
    frozen: int = 0
    prompt: int = 0
    exact: int = 0
    wait: float = float("inf")

    @classmethod
    def parse(cls, policy: str) -> "ReplayOptions":
        opt = cls()
        for part in filter(None, policy.split("+")):
            name, _, value = part.partition(":")
            if name == "oracle":
                opt.oracle = True
            elif name in ("lag", "frozen", "prompt", "exact"):
                setattr(opt, name, int(value or 0))
            elif name == "wait":
                opt.wait = float(value)
            elif name != "lru":
                raise ValueError(f"unknown replay option {name!r}")
        opt.lag = max(opt.lag, 1)
        opt.prompt = opt.prompt or opt.exact
        return opt

    @property
    def delayed(self) -> bool:
        return self.lag > 1 or self.frozen > 0


class _Recency:
    """At most ``capacity`` experts, least recent first: a dict keyed by
    expert whose values are insertion ticks, so order = sorted ticks."""

    def __init__(self, capacity: int, start=()):
        self.capacity, self.tick, self.at = capacity, 0, {}
        for e in start:
            self.touch(int(e))

    def __contains__(self, e: int) -> bool:
        return e in self.at

    def order(self) -> list[int]:
        return sorted(self.at, key=self.at.__getitem__)

    def touch(self, e: int) -> None:
        self.tick += 1
        self.at[e] = self.tick

    def add(self, e: int) -> None:
        self.touch(e)
        if len(self.at) > self.capacity:
            del self.at[min(self.at, key=self.at.__getitem__)]

    def replace(self, experts: Sequence[int]) -> None:
        self.at = {}
        for e in experts:
            self.touch(int(e))


def replay(ind: np.ndarray, wts: np.ndarray, k: int, tau, bounds: Sequence[int], warm, counts: np.ndarray,
           policy: str = "lru", trace: list | None = None, resident: np.ndarray | None = None,
           waited: list | None = None) -> np.ndarray:
    """Replay of a cache of ``k`` resident experts over routings ``ind`` /
    ``wts`` ``[T, top_k]`` (records of ``bounds`` tokens back to back). Returns
    ``hit[t, s]``: slot ``s`` of token ``t`` found its expert served. After each
    token every slot whose gate reaches its expert's threshold (``tau``: one
    value or one per expert) admits or refreshes the expert, resident from the
    next token (``ReplayOptions`` for the others). Each record starts from
    ``warm`` (or empty). ``counts[e, 4]`` counts the admissions (reads) of
    expert ``e``; ``trace`` collects them as (record, token in record,
    expert); ``resident[t]`` receives the experts token ``t`` is served from;
    ``waited`` the tokens that waited."""

    opt = ReplayOptions.parse(policy)
    n_exp = counts.shape[0]
    thr = np.broadcast_to(np.asarray(tau, dtype=np.float64), (n_exp,))
    hit = np.zeros(ind.shape, dtype=bool)
    edges = np.concatenate([[0], np.cumsum(bounds)]).astype(int)
    for rec in range(len(bounds)):
        lo, hi = edges[rec], edges[rec + 1]
        if opt.oracle:
            _replay_oracle(ind, wts, k, n_exp, lo, hi, hit, resident)
        else:
            _ReplayRecord(ind, wts, k, thr, opt, rec, lo, hi, warm, counts, trace, resident, waited).run(hit)
    return hit


def _mass(ind: np.ndarray, wts: np.ndarray, lo: int, hi: int, n: int) -> np.ndarray:
    return np.bincount(ind[lo:hi].ravel(), weights=wts[lo:hi].ravel(), minlength=n)


def _replay_oracle(ind, wts, k, n_exp, lo, hi, hit, resident) -> None:
    """A record's ``k`` heaviest experts, fixed in advance (no admissions)."""
    mass = _mass(ind, wts, lo, hi, n_exp)
    top = np.argsort(-mass, kind="stable")[:k]
    hit[lo:hi] = np.isin(ind[lo:hi], top[mass[top] > 0])
    if resident is not None:
        resident[lo:hi, top] = True


class _ReplayRecord:
    """One record of the ``lru`` replay and its options."""

    def __init__(self, ind, wts, k, thr, opt, rec, lo, hi, warm, counts, trace, resident, waited):
        self.ind, self.wts, self.k, self.thr, self.opt = ind, wts, k, thr, opt
        self.rec, self.lo, self.hi = rec, lo, hi
        self.counts, self.trace, self.resident, self.waited = counts, trace, resident, waited
        self.cache = _Recency(k, [] if warm is None else list(warm))
        self.due: list[tuple[int, int]] = []  # (first token served, expert), in admission order
        self.flight: set[int] = set()

    def admit(self, e: int, t: int) -> None:
        self.counts[e, 4] += 1
        if self.trace is not None:
            self.trace.append((self.rec, t - self.lo, e))
        self.cache.add(e)

    def warm_start(self, t: int) -> None:
        """After the prompt: its heaviest experts (up to k) become the most
        recent residents, heaviest last; the most recent of the old ones fill
        the remaining places."""
        mass = _mass(self.ind, self.wts, self.lo, t, self.counts.shape[0])
        top = [int(e) for e in np.argsort(-mass, kind="stable")[:self.k] if mass[e] > 0]
        for e in top:
            if e not in self.cache:
                self.counts[e, 4] += 1
        old = [e for e in self.cache.order() if e not in top]
        room = self.k - len(top)
        self.cache.replace((old[max(0, len(old) - room):] if room > 0 else []) + top[::-1])

    def run(self, hit: np.ndarray) -> None:
        o = self.opt
        for t in range(self.lo, self.hi):
            if o.prompt and t == self.lo + o.prompt:
                self.warm_start(t)
            while self.due and self.due[0][0] <= t:
                e = self.due.pop(0)[1]
                self.flight.discard(e)
                if e not in self.cache:
                    self.admit(e, t)
            row = self.ind[t].astype(int)
            gate = self.wts[t]
            in_exact = t < self.lo + o.exact
            absent = np.array([e not in self.cache for e in row])
            late = absent & (in_exact | (gate >= o.wait))
            if late.any() and self.waited is not None and not in_exact:
                self.waited.append(t)
            hit[t] = ~absent | np.isin(row, row[late])  # one waited read serves every slot of its expert
            if self.resident is not None:
                self.resident[t, self.cache.order() + row[late].tolist()] = True
            for e in row[gate >= self.thr[row]].tolist():
                if e in self.cache:
                    self.cache.touch(e)
                elif not o.delayed:
                    self.admit(e, t)
                elif e not in self.flight:
                    self.flight.add(e)
                    self.due.append((max(t + o.lag, self.lo + o.frozen), e))


def wait_stats(log: dict[int, list], tokens: int, n_layers: int) -> dict[str, float]:
    """Share of tokens that waited in some layer, and of all layer work that a
    replay from each such token's first waiting layer repeats. ``log`` maps a
    layer to the tokens that waited in it."""

    first: dict[int, int] = {}
    for layer in sorted(log):
        for t in log[layer]:
            first[t] = min(first.get(t, layer), layer)
    rerun = np.asarray([n_layers - layer for layer in first.values()], dtype=np.int64)
    return {"wait_token_share": len(first) / max(tokens, 1),
            "wait_layer_rerun_share": float(rerun.sum()) / max(tokens * n_layers, 1)}


# kept under the name the replay has in the reference's evaluation script
residual_cache = replay


def victim_order(recency, slot_expert, fetched: set, demanded: set) -> list[int]:
    """Slots the wait rule overwrites, first to last: slots holding no
    fetched expert, those whose expert is not demanded at all first, each
    group least recent first (ties by slot)."""

    recency = np.asarray(recency, dtype=np.float64)
    held = np.asarray(slot_expert, dtype=np.int64)
    ok = ~np.isin(held, np.fromiter(fetched, np.int64, len(fetched)))
    in_demand = np.isin(held, np.fromiter(demanded, np.int64, len(demanded)))
    idx = np.arange(held.size)
    order = np.lexsort((idx, recency, in_demand))
    return [int(s) for s in order if ok[s]]


# ----------------------------------------------------------------------------- live policy


class SlotTable:
    """One layer's pool of ``slots`` rows over ``num_experts`` experts. ``order``
    lists experts hottest first; the first ``slots`` start routed, colder ones
    less recent."""

    def __init__(self, num_experts: int, slots: int, order):
        if not 1 <= slots <= num_experts:
            raise ValueError(f"slots must be in 1..{num_experts}")
        order = np.asarray([int(e) for e in order], dtype=np.int64)
        if (len(np.unique(order)) != len(order) or len(order) < slots or order.min() < 0
                or order.max() >= num_experts):
            raise ValueError("order must list at least `slots` distinct experts of the pool")
        self.num_experts, self.slots = num_experts, slots
        self.state = np.full(slots, ROUTED, dtype=np.int8)
        self.expert = order[:slots].copy()             # -1 when the slot holds no routed expert
        self.stamp = -1.0 - np.arange(slots)           # recency (routed) / eviction call (cooling)
        self.seq = np.zeros(slots, dtype=np.int64)     # free: order of freeing; reading: order of admission
        self.handle: list = [None] * slots
        self.where = np.full(num_experts, -1, dtype=np.int64)  # expert -> routed slot
        self.where[self.expert] = np.arange(slots)
        self.read_at = np.full(num_experts, -1, dtype=np.int64)  # expert -> slot being read into
        self.counter = 0

    # views
    def routed(self) -> np.ndarray:
        return self.where >= 0

    def slots_in(self, state: int) -> list[int]:
        return np.flatnonzero(self.state == state).tolist()

    def describe(self) -> dict:
        return {name: self.slots_in(s) for s, name in enumerate(_NAMES)}

    def slot_expert(self) -> np.ndarray:
        """Expert routed at every slot (-1 for the others)."""
        return np.where(self.state == ROUTED, self.expert, -1)

    def assignment(self) -> dict[int, int]:
        """Routed expert -> its slot."""
        s = np.flatnonzero(self.state == ROUTED)
        return dict(zip(self.expert[s].tolist(), s.tolist()))

    def _next(self) -> int:
        self.counter += 1
        return self.counter


class ResidencyPolicy:
    """The serving cache's policy over the ``SlotTable`` of every layer, IO-free.

    Hooks (``ResidencyCache`` binds them to a device): ``read(layer, expert,
    slot)`` starts a read and returns a handle, ``done(handle)`` says whether
    it has landed, ``wait(handle)`` blocks until it has, ``route(layer, expert,
    slot)`` / ``unroute(layer, expert, slot)`` switch an expert on and off in
    the router. ``ResidencyPolicy(num_experts, slots, order)`` is a one-layer
    policy; ``ResidencyPolicy.layers([...])`` takes one ``(num_experts, slots,
    order)`` per layer."""

    STATS = ("calls", "tokens", "demand", "resident", "wanted", "admitted", "installed", "evicted", "no_slot",
             "waits", "policy_s", "wait_s")

    def __init__(self, num_experts: int | None = None, slots: int | None = None, order=None, *,
                 tables: Sequence[SlotTable] | None = None, tau: float = 0.2, spare: int = 4, lag: int = 2,
                 route_scale: float = 1.0, read: Callable | None = None, done: Callable | None = None,
                 wait: Callable | None = None, route: Callable | None = None, unroute: Callable | None = None):
        if lag < 1:
            raise ValueError("lag must be >= 1: a call's demand is read once it has run")
        self.tables = list(tables) if tables is not None else [SlotTable(num_experts, slots, order)]
        self.tau, self.spare, self.lag, self.route_scale = float(tau), int(spare), int(lag), float(route_scale)
        self._hooks = {"read": read, "done": done, "wait": wait, "route": route, "unroute": unroute}
        self.step = 0
        self.pending: dict[int, dict[int, list]] = {}  # call -> layer -> demand arrays
        self.stats = dict.fromkeys(self.STATS, 0)
        self.started = time.time()

    @classmethod
    def layers(cls, shapes: Sequence[tuple[int, int, Sequence[int]]], **kw) -> "ResidencyPolicy":
        return cls(tables=[SlotTable(*s) for s in shapes], **kw)

    # hooks
    def read(self, layer: int, expert: int, slot: int):
        f = self._hooks["read"]
        return f(layer, expert, slot) if f else None

    def done(self, handle) -> bool:
        f = self._hooks["done"]
        return f(handle) if f else True

    def wait(self, handle) -> None:
        f = self._hooks["wait"]
        if f:
            f(handle)
        else:
            while not self.done(handle):
                time.sleep(0)

    def route(self, layer: int, expert: int, slot: int) -> None:
        if self._hooks["route"]:
            self._hooks["route"](layer, expert, slot)

    def unroute(self, layer: int, expert: int, slot: int) -> None:
        if self._hooks["unroute"]:
            self._hooks["unroute"](layer, expert, slot)

    # state
    def table(self, layer: int = 0) -> SlotTable:
        return self.tables[layer]

    def resident_mask(self, layer: int = 0) -> np.ndarray:
        return self.tables[layer].routed()

    # --- demand, recorded as a call is issued ------------------------------------

    def observe(self, want, want_score, layer: int = 0) -> None:
        """Record this call's demand in ``layer``: ``want`` / ``want_score``
        ``[T, k]`` (host arrays, or anything ``_host`` turns into them later)."""
        self.pending.setdefault(self.step, {}).setdefault(layer, []).append((want, want_score))

    def _host(self, a) -> np.ndarray:
        return np.asarray(a)

    # --- the no-wait policy, run before each call ----------------------------------

    def begin(self) -> None:
        """Start a forward call: harvest, in every layer, the demand of the call
        ``lag`` calls back (it has run: its demand is on the host)."""
        self.step += 1
        ready = self.step - self.lag
        demand = self.pending.pop(ready, None)
        for old in [c for c in self.pending if c < ready]:
            del self.pending[old]
        if demand is None or self.tau == float("inf"):
            return
        t0 = time.perf_counter()
        self.stats["calls"] += 1
        for layer in sorted(demand):
            for want, score in demand[layer]:
                self.harvest(layer, ready, self._host(want), self._host(score))
        self.stats["policy_s"] += time.perf_counter() - t0

    def harvest(self, layer: int, call: int, index: np.ndarray, weight: np.ndarray) -> None:
        """One call's demand in one layer."""
        tab = self.tables[layer]
        index = np.asarray(index, dtype=np.int64)
        index = index.reshape(-1, index.shape[-1])
        share = np.asarray(weight, dtype=np.float64).reshape(index.shape)
        share = share / (share.sum(-1, keepdims=True) + 1e-20) * self.route_scale
        if layer == 0:
            self.stats["tokens"] += index.shape[0]
        self.stats["demand"] += index.size
        valid = (index >= 0) & (index < tab.num_experts)
        self.stats["resident"] += int(tab.routed()[index[valid]].sum())
        strong = valid & (share >= self.tau)
        best = np.full(tab.num_experts, -1.0)
        np.maximum.at(best, index[strong], share[strong])
        wanted = np.flatnonzero(best >= 0)
        self.install(layer)
        hit = tab.where[wanted]
        tab.stamp[hit[hit >= 0]] = call
        missing = wanted[(hit < 0) & (tab.read_at[wanted] < 0)]
        self.stats["wanted"] += int(missing.size)
        # slots evicted at or before the harvested call can be reused: every call that could route there has run
        thawed = np.flatnonzero((tab.state == COOLING) & (tab.stamp <= call))
        for s in thawed[np.argsort(tab.seq[thawed], kind="stable")]:
            tab.state[s], tab.seq[s] = FREE, tab._next()
        for e in missing[np.lexsort((-missing, -best[missing]))]:  # heaviest first, ties by higher expert
            free = np.flatnonzero(tab.state == FREE)
            if free.size == 0:
                self.stats["no_slot"] += 1
                continue
            s = int(free[np.argmax(tab.seq[free])])  # the most recently freed slot
            tab.state[s], tab.expert[s], tab.seq[s] = READING, e, tab._next()
            tab.read_at[e] = s
            tab.handle[s] = self.read(layer, int(e), s)
            self.stats["admitted"] += 1
        self.evict(layer, wanted)

    def install(self, layer: int) -> None:
        """Route the experts whose bytes have landed, in admission order."""
        tab = self.tables[layer]
        reading = np.flatnonzero(tab.state == READING)
        for s in reading[np.argsort(tab.seq[reading], kind="stable")]:
            if not self.done(tab.handle[s]):
                continue
            self._land(layer, int(s))
            self.stats["installed"] += 1

    def _land(self, layer: int, s: int) -> None:
        tab = self.tables[layer]
        e = int(tab.expert[s])
        self.route(layer, e, s)
        tab.state[s], tab.handle[s], tab.stamp[s] = ROUTED, None, self.step
        tab.where[e], tab.read_at[e] = s, -1

    def evict(self, layer: int, protected: np.ndarray) -> None:
        """Unroute the least recent residents not in ``protected`` until
        ``spare`` slots are free or cooling."""
        tab = self.tables[layer]
        short = self.spare - int(np.isin(tab.state, (FREE, COOLING)).sum())
        if short <= 0:
            return
        cand = np.flatnonzero((tab.state == ROUTED) & ~np.isin(tab.expert, protected))
        cand = cand[np.lexsort((cand, tab.stamp[cand]))][:short]
        for s in cand:
            self._drop(layer, int(s))
            tab.state[s], tab.stamp[s], tab.seq[s] = COOLING, self.step, tab._next()
            self.stats["evicted"] += 1

    def _drop(self, layer: int, s: int) -> None:
        tab = self.tables[layer]
        e = int(tab.expert[s])
        tab.where[e], tab.expert[s] = -1, -1
        self.unroute(layer, e, s)

    # --- the wait rule -------------------------------------------------------------

    def fetch(self, want, strong=None, layer: int = 0) -> None:
        """Read every demanded absent expert of ``layer`` (or only those in
        ``strong``) now, over the least recently demanded residents, and route
        each once read. No fetched expert is overwritten; a demanded one only
        when no other slot is left."""
        tab = self.tables[layer]
        t0 = time.perf_counter()
        want = np.asarray(want, dtype=np.int64).ravel()
        self.stats["demand"] += int(want.size)
        self.stats["resident"] += int(tab.routed()[want].sum())
        demanded = np.unique(want)
        fetched = demanded if strong is None else np.unique(np.asarray(strong, dtype=np.int64).ravel())
        here = tab.where[fetched]
        tab.stamp[here[here >= 0]] = self.step
        for s in tab.read_at[fetched[here < 0]]:  # admitted by the no-wait rule and still in flight: wait for it
            if s >= 0:
                self.wait(tab.handle[s])
                self._land(layer, int(s))
                self.stats["installed"] += 1
        missing = fetched[tab.where[fetched] < 0]
        if missing.size == 0:
            self.stats["wait_s"] += time.perf_counter() - t0
            return
        recency = np.where(tab.state == ROUTED, tab.stamp, np.inf)
        victims = [s for s in victim_order(recency, tab.slot_expert(), set(fetched.tolist()),
                                           set(demanded.tolist())) if tab.state[s] != READING]
        if len(victims) < missing.size:
            raise RuntimeError("fewer slots than one call's demand")
        reads = []
        for e, s in zip(missing.tolist(), victims):
            if tab.state[s] == ROUTED:
                self._drop(layer, s)
                self.stats["evicted"] += 1
            tab.state[s], tab.expert[s] = READING, e
            tab.read_at[e] = s
            reads.append((s, self.read(layer, e, s)))
        for s, h in reads:
            self.wait(h)
            self._land(layer, s)
            self.stats["installed"] += 1
        self.stats["waits"] += 1
        self.stats["wait_s"] += time.perf_counter() - t0

    def run_pieces(self, index, score, wait_min: float, run: Callable[[int, int], None], layer: int = 0) -> int:
        """Prefill of ``layer`` under the wait rule (behaviour of
        ``omlx_lattice.py:427-449``): the demand ``index`` / raw ``score``
        ``[T, k]`` is normalised per token (times ``route_scale``) and split by
        ``plan_pieces``; for each piece its experts of share >= ``wait_min`` are
        fetched, then ``run(start, end)`` runs the layer on its tokens. On a
        device the next piece's copies queue behind that run on the caller's
        stream, so they never overwrite slots it still reads. Returns the
        number of pieces."""
        index = np.asarray(index, dtype=np.int64)
        index = index.reshape(-1, index.shape[-1])
        score = np.asarray(score, dtype=np.float64).reshape(index.shape)
        share = score / (score.sum(-1, keepdims=True) + 1e-20) * self.route_scale
        pieces = plan_pieces(index, share, self.tables[layer].slots, wait_min)
        if layer == 0:
            self.stats["tokens"] += index.shape[0]
        for a, b, held in pieces:
            self.fetch(index[a:b].ravel(), held, layer)
            run(a, b)
        return len(pieces)

    def row(self) -> dict:
        """One line of the stats log."""
        return {"t": round(time.time() - self.started, 2), "step": self.step, **self.stats,
                "reading": int(sum(int((t.state == READING).sum()) for t in self.tables))}

    def write_log(self, path, verify: bool = False) -> dict:
        """Append ``row()`` (and, with ``verify``, the count of routed slots
        whose device bytes differ from their expert's stored bytes) to a JSONL
        file; returns the row."""
        row = self.row()
        if verify:
            row["mismatched"] = self.mismatched()
        with open(path, "a") as f:
            f.write(json.dumps(row) + "\n")
        return row

    def mismatched(self) -> int:
        return 0  # a policy without a device holds no bytes


def plan_pieces(index: np.ndarray, share: np.ndarray, slots: int, wait_min: float) -> list[tuple[int, int, list]]:
    """Prefill under the wait rule: split ``T`` tokens (``index`` / normalised
    ``share`` ``[T, k]``) into consecutive pieces ``(start, end, held)`` whose
    experts of share >= ``wait_min`` (``held``, sorted) fit ``slots``; a token
    that alone needs more than ``slots`` is a piece of its own (whose fetch
    then raises).

    Behaviour of ``omlx_lattice.py:432-441``, without its empty first piece
    when the first token alone overflows."""
    index = np.asarray(index, dtype=np.int64).reshape(-1, np.asarray(index).shape[-1])
    need = np.asarray(share, dtype=np.float64).reshape(index.shape) >= wait_min
    pieces, start, held = [], 0, set()
    for t in range(index.shape[0]):
        mine = set(index[t][need[t]].tolist())
        if t > start and len(held | mine) > slots:
            pieces.append((start, t, sorted(held)))
            start, held = t, set()
        held |= mine
    pieces.append((start, index.shape[0], sorted(held)))
    return pieces


# ----------------------------------------------------------------------------- on a device


@dataclass
class LayerBinding:
    """The device side of one layer: its installer (slot pools and layer
    file), the router's served bias of every expert when resident, and an
    optional nested tier whose slot rows follow the residents."""

    installer: object
    pool_bias: np.ndarray
    hot_tier: object = None
    hot_row_of: dict | None = None  # expert -> residual row of the nested tier


class ResidencyCache(ResidencyPolicy):
    """``ResidencyPolicy`` on a device, over one layer or many.

    ``ResidencyCache(installer, num_experts, order, ...)`` binds one layer;
    ``ResidencyCache.for_layers([(installer, num_experts, order), ...])`` one
    policy over several. Per layer: ``installer`` is a
    ``loaders.ExpertInstaller`` over the slot pools (``{w1, w3, w2}: (codes
    [S, ...], scales [S, ...])``); ``pool_bias`` the router's served bias of
    every expert when resident (the correction bias, or zeros);
    ``bias_served[layer]`` (float32 ``[E]``, ``OFF`` for absent experts) and
    ``slot_map[layer]`` (int32 ``[E]``) the device tensors the routed layer
    reads, changed only between calls and in the current stream's order; a
    ``hot_tier`` (``nn.HotTier`` over the slots, with ``hot_row_of`` mapping
    its experts to residual rows) gets the new slot row of every expert routed.
    The starting residents are read in at construction unless ``load`` is False.
    A decode step is ``begin()``, the layers' calls with ``bias(layer)`` and
    ``slots(layer)``, and ``observe(router_output, layer)`` after each.
    """

    def __init__(self, installer=None, num_experts: int | None = None, order=None, *, pool_bias=None,
                 hot_tier=None, hot_row_of: dict | None = None, load: bool = True,
                 layers: Sequence[tuple] | None = None, **kw):
        if layers is None:
            layers = [(installer, num_experts, order, pool_bias, hot_tier, hot_row_of)]
        specs = [tuple(spec) + (None,) * (6 - len(spec)) for spec in layers]
        tables = []
        self.bindings: list[LayerBinding] = []
        for inst, n_exp, order_i, bias_i, tier, rows in specs:
            slots = int(next(iter(inst.pools.values()))[0].shape[0])
            tables.append(SlotTable(n_exp, slots, order_i))
            bias = np.zeros(n_exp, np.float32) if bias_i is None else np.asarray(bias_i, np.float32).reshape(n_exp)
            if tier is not None and rows is None:
                raise ValueError("a hot tier needs hot_row_of: the residual row of each of its experts")
            if tier is not None and tier.hot_of_slot.numel() != slots:
                raise ValueError(f"the hot tier must have one row entry per slot ({slots})")
            self.bindings.append(LayerBinding(inst, bias.copy(), tier, None if rows is None else dict(rows)))
        super().__init__(tables=tables, **kw)
        self.device = self.bindings[0].installer.device
        self._bias = [np.where(t.routed(), b.pool_bias, OFF).astype(np.float32) for t, b in zip(tables, self.bindings)]
        self._map = [np.where(t.routed(), t.where, 0).astype(np.int32) for t in tables]  # absent: row 0, weight 0
        self.bias_served = [torch.from_numpy(b.copy()).to(self.device) for b in self._bias]
        self.slot_map = [torch.from_numpy(m.copy()).to(self.device) for m in self._map]
        self._dirty = [False] * len(tables)
        for layer, (t, b) in enumerate(zip(tables, self.bindings)):
            if b.hot_tier is not None:
                for s, e in enumerate(t.slot_expert().tolist()):
                    b.hot_tier.route_slot(s, b.hot_row_of.get(e))
                b.hot_tier.publish()
        if load:  # the starting residents' bytes, before the first call
            for t, b in zip(tables, self.bindings):
                for ev in [b.installer.submit(int(e), s) for s, e in enumerate(t.slot_expert().tolist())]:
                    ev.synchronize()

    @classmethod
    def for_layers(cls, layers: Sequence[tuple], **kw) -> "ResidencyCache":
        """``layers``: ``(installer, num_experts, order[, pool_bias[, hot_tier, hot_row_of]])`` per layer."""
        return cls(layers=layers, **kw)

    def bias(self, layer: int = 0) -> torch.Tensor:
        return self.bias_served[layer]

    def slots(self, layer: int = 0) -> torch.Tensor:
        return self.slot_map[layer]

    # hooks
    def read(self, layer: int, expert: int, slot: int):
        return self.bindings[layer].installer.submit(expert, slot)

    def done(self, handle) -> bool:
        return handle is None or self.bindings[0].installer.ready(handle)

    def wait(self, handle) -> None:
        if handle is not None:
            handle.synchronize()

    def route(self, layer: int, expert: int, slot: int) -> None:
        b = self.bindings[layer]
        self._bias[layer][expert], self._map[layer][expert] = b.pool_bias[expert], slot
        self._dirty[layer] = True
        if b.hot_tier is not None:  # the slot's residual row is now this expert's (or none)
            b.hot_tier.route_slot(slot, b.hot_row_of.get(expert))

    def unroute(self, layer: int, expert: int, slot: int) -> None:
        self._bias[layer][expert] = OFF
        self._dirty[layer] = True

    def _publish(self) -> None:
        """Queue the router tensors' new values on the current stream (pinned
        staging, so the host may change them again at once)."""
        for layer, dirty in enumerate(self._dirty):
            if not dirty:
                continue
            self.bias_served[layer].copy_(torch.from_numpy(self._bias[layer].copy()).pin_memory(), non_blocking=True)
            self.slot_map[layer].copy_(torch.from_numpy(self._map[layer].copy()).pin_memory(), non_blocking=True)
            self._dirty[layer] = False
        for b in self.bindings:
            if b.hot_tier is not None:
                b.hot_tier.publish()

    def begin(self) -> None:
        super().begin()
        self._publish()

    def fetch(self, want, strong=None, layer: int = 0) -> None:
        super().fetch(want, strong, layer)
        self._publish()

    def observe(self, router_output, layer: int = 0) -> None:
        """Record the demand (``want``, ``want_score``) of a call just issued,
        with no host sync (pinned copies and an event, read ``lag`` calls later)."""
        want = torch.empty(router_output.want.shape, dtype=torch.int32, pin_memory=True)
        score = torch.empty(router_output.want_score.shape, dtype=torch.float32, pin_memory=True)
        want.copy_(router_output.want, non_blocking=True)
        score.copy_(router_output.want_score, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        super().observe((want, ev), score, layer)

    def _host(self, a) -> np.ndarray:
        if isinstance(a, tuple):  # (pinned demand, its event)
            a[1].synchronize()
            return a[0].numpy()
        return a.numpy() if isinstance(a, torch.Tensor) else np.asarray(a)

    def differing(self, layer: int, slot: int) -> int:
        """Tensors of a routed slot whose device bytes differ from its
        expert's bytes in the layer file."""
        tab, inst = self.tables[layer], self.bindings[layer].installer
        e = int(tab.slot_expert()[slot])
        if e < 0:
            return 0
        bad = 0
        for proj, (codes, scales) in inst.pools.items():
            for name, dst in ((f"{proj}_codes", codes), (f"{proj}_scales", scales)):
                stored = np.ascontiguousarray(inst.layer.read(name, [e])[0]).reshape(-1).view(np.uint8)
                here = dst[slot].contiguous().reshape(-1).view(torch.uint8).cpu().numpy()
                bad += not np.array_equal(stored, here)
        return bad

    def mismatched(self) -> int:
        """Routed slots of the first and last layer whose bytes differ from their experts' stored bytes."""
        torch.cuda.synchronize(self.device)
        layers = sorted({0, len(self.tables) - 1})
        return sum(self.differing(layer, s) for layer in layers for s in self.tables[layer].slots_in(ROUTED))
