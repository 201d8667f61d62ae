"""Expert residency: which experts of a layer's pool sit in its device slots.

The routed layers serve only resident experts (the router's served bias is
``OFF`` for the others) and read an expert's codes at its slot's row of the
pool (``slot_map[e]``). This module is the host side that keeps that state:

- ``ResidencyPolicy``: the no-wait policy of the serving cache
  (``scripts/v41_build/omlx_routed.py:103-260``). Each forward call records
  its demand (the demand top-k and raw scores the router already returns);
  ``lag`` calls later that demand is harvested: every demanded slot whose
  normalised weight reaches ``tau`` is wanted; a wanted resident is refreshed
  (least-recently-used order), a wanted absent expert is read into a free slot
  (heaviest first) and routed only once its bytes have landed; residents that
  nobody wants are evicted until ``spare`` slots are free or cooling, and an
  evicted slot cools for one call before it is reused. ``fetch`` is the wait
  rule (``omlx_lattice.py:260-325``): the demand is read in before the call
  runs, over the least recently demanded residents (``victim_order``).
- ``ResidencyCache``: the policy on a device: the pool arrays, the router's
  ``bias_served`` and ``slot_map`` device tensors (changed only between calls,
  in stream order), reads and copies through ``loaders.ExpertInstaller`` on
  its own stream, an expert routed only after its copy event completes.
- ``residual_cache`` / ``wait_stats``: the offline replay of the policy over
  recorded routings (``scripts/runpod/v41_reap/local_eval.py:184-286``), with
  its options (lag, frozen prompt, prompt warm start, exact prefill, wait,
  oracle), for choosing ``tau`` and the slot count.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Callable

import numpy as np
import torch

from keep_amd.router import OFF

# ----------------------------------------------------------------------------- replay


def residual_cache(ind: np.ndarray, wts: np.ndarray, k: int, tau, bounds: list[int], warm, counts: np.ndarray,
                   policy: str = "lru", trace: list | None = None, resident: np.ndarray | None = None,
                   waited: list | None = None) -> np.ndarray:
    """Replay of a cache of ``k`` resident experts over routings ``ind``/``wts``
    ``[T, top_k]`` (records of ``bounds`` back to back): ``hi[t, s]`` says
    whether slot ``s`` of token ``t`` found its expert resident. After each
    token every slot with gate >= ``tau`` (one value or one per expert) admits
    or refreshes its expert, resident from the next token on (``lag:N``: N
    tokens on; ``frozen:P``: nothing lands in a record's first P tokens).
    Each record starts from ``warm`` (or empty). ``prompt:P``: after P tokens
    the record's own top ``k`` by gate mass replace the residents;
    ``exact:P``: the same, and those tokens are served whatever they ask;
    ``wait:W``: an absent expert asked with gate >= W is served anyway (the
    token waits; ``waited`` collects it). ``oracle``: each record's top ``k``
    by mass, fixed in advance, no admissions. ``counts[e, 4]`` counts the
    admissions (fetches) of expert ``e``; ``trace`` collects them as (record,
    token in record, expert); ``resident[t]`` receives the set token t sees.
    (``local_eval.py:184-275``.)"""

    n_exp = counts.shape[0]
    hi = np.zeros(ind.shape, dtype=bool)
    thr = np.broadcast_to(np.asarray(tau, dtype=np.float64), (n_exp,))
    opts = {}
    for part in policy.split("+"):
        key, _, val = part.partition(":")
        opts[key] = val
    exact = int(opts.get("exact") or 0)
    prompt = int(opts.get("prompt") or 0) or exact
    wait = float(opts["wait"]) if "wait" in opts else float("inf")
    lag = int(opts.get("lag") or 1)
    frozen = int(opts.get("frozen") or 0)
    delayed = lag > 1 or frozen > 0

    def mass_order(lo: int, hi_: int) -> tuple[np.ndarray, np.ndarray]:
        mass = np.bincount(ind[lo:hi_].ravel(), weights=wts[lo:hi_].ravel(), minlength=n_exp)
        return mass, np.argsort(-mass, kind="stable")

    start = 0
    for rec, n in enumerate(bounds):
        end = start + n
        if policy == "oracle":
            mass, order = mass_order(start, end)
            hot = order[:k]
            hi[start:end] = np.isin(ind[start:end], hot[mass[hot] > 0])
            if resident is not None:
                resident[start:end, hot] = True
            start = end
            continue
        lru: OrderedDict[int, None] = OrderedDict((int(e), None) for e in (warm if warm is not None else []))

        def admit(e: int, t: int) -> None:
            counts[e, 4] += 1
            if trace is not None:
                trace.append((rec, t - start, e))
            lru[e] = None
            if len(lru) > k:
                lru.popitem(last=False)

        arrivals: list[tuple[int, int]] = []  # (first token it serves, expert), in admission order
        in_flight: set[int] = set()
        for t in range(start, end):
            if prompt and t == start + prompt:
                mass, order = mass_order(start, t)
                top = [int(e) for e in order[:k] if mass[e] > 0]
                counts[[e for e in top if e not in lru], 4] += 1
                rest = [e for e in lru if e not in top]
                keep = rest[max(0, len(rest) - (k - len(top))):] if len(top) < k else []
                lru = OrderedDict((e, None) for e in keep + top[::-1])  # the heaviest most recent
            while arrivals and arrivals[0][0] <= t:
                e = arrivals.pop(0)[1]
                in_flight.discard(e)
                if e not in lru:
                    admit(e, t)
            row = [int(e) for e in ind[t]]
            late = [e for s, e in enumerate(row) if e not in lru and (t < start + exact or wts[t, s] >= wait)]
            if late and waited is not None and t >= start + exact:
                waited.append(t)
            hi[t] = [e in lru or e in late for e in row]
            if resident is not None:
                resident[t, list(lru) + late] = True
            for s, e in enumerate(row):
                if wts[t, s] < thr[e]:
                    continue
                if e in lru:
                    lru.move_to_end(e)
                elif not delayed:
                    admit(e, t)
                elif e not in in_flight:
                    in_flight.add(e)
                    arrivals.append((max(t + lag, start + frozen), e))
        start = end
    return hi


def wait_stats(log: dict[int, list], tokens: int, n_layers: int) -> dict[str, float]:
    """Share of tokens that waited in some layer, and of all layer work that a
    replay from each such token's first waiting layer repeats
    (``local_eval.py:278-286``)."""

    first: dict[int, int] = {}
    for layer in sorted(log):
        for t in log[layer]:
            first.setdefault(t, layer)
    return {"wait_token_share": len(first) / max(tokens, 1),
            "wait_layer_rerun_share": sum(n_layers - layer for layer in first.values()) / max(tokens * n_layers, 1)}


def victim_order(last_use, slot_expert, fetched: set, demanded: set) -> list[int]:
    """Slots to overwrite, first to last: least recently demanded first, the
    residents this call demands but does not fetch after all others, fetched
    ones never (``omlx_lattice.py:320-324``)."""

    free = [int(s) for s in np.argsort(np.asarray(last_use), kind="stable") if int(slot_expert[s]) not in fetched]
    return sorted(free, key=lambda s: int(slot_expert[s]) in demanded)


# ----------------------------------------------------------------------------- live policy


class ResidencyPolicy:
    """The serving cache's policy for one layer's pool of ``slots`` rows over
    ``num_experts`` experts, IO-free: ``read(expert, slot)`` starts a read and
    returns a handle, ``done(handle)`` says whether it has landed, ``route`` /
    ``unroute`` switch an expert on and off in the router. ``order`` lists the
    experts hottest first; the first ``slots`` start resident."""

    STATS = ("calls", "tokens", "demand", "resident", "wanted", "admitted", "installed", "evicted", "no_slot", "waits")

    def __init__(self, num_experts: int, slots: int, order, *, tau: float = 0.2, spare: int = 4, lag: int = 2,
                 route_scale: float = 1.0, read: Callable | None = None, done: Callable | None = None,
                 route: Callable | None = None, unroute: Callable | None = None):
        if not 1 <= slots <= num_experts:
            raise ValueError(f"slots must be in 1..{num_experts}")
        if lag < 1:
            raise ValueError("lag must be >= 1: a call's demand is read once it has run")
        order = [int(e) for e in order]
        if sorted(order) != sorted(set(order)) or len(order) < slots or min(order) < 0 or max(order) >= num_experts:
            raise ValueError("order must list at least `slots` distinct experts of the pool")
        self.num_experts, self.slots = num_experts, slots
        self.tau, self.spare, self.lag, self.route_scale = float(tau), int(spare), int(lag), float(route_scale)
        self._read, self._done = read, done
        self._route, self._unroute = route, unroute
        self.slot_expert = np.array(order[:slots], dtype=np.int64)  # -1: unrouted
        self.slot_of = {e: s for s, e in enumerate(order[:slots])}
        self.last_use = -1.0 - np.arange(slots, dtype=np.float64)  # colder starting experts go first
        self.cooling: list[tuple[int, int]] = []
        self.free: list[int] = []
        self.reading: dict[int, tuple[int, object]] = {}
        self.pending: dict[int, list] = {}
        self.step = 0
        self.stats = dict.fromkeys(self.STATS, 0)

    # hooks; ResidencyCache binds them to the device
    def read(self, expert: int, slot: int):
        return self._read(expert, slot) if self._read else None

    def done(self, handle) -> bool:
        return self._done(handle) if self._done else True

    def wait(self, handle) -> None:
        while not self.done(handle):
            pass

    def route(self, expert: int, slot: int) -> None:
        if self._route:
            self._route(expert, slot)

    def unroute(self, expert: int, slot: int) -> None:
        if self._unroute:
            self._unroute(expert, slot)

    def resident_mask(self) -> np.ndarray:
        m = np.zeros(self.num_experts, dtype=bool)
        m[list(self.slot_of)] = True
        return m

    # --- demand, recorded as a call is issued ------------------------------------

    def observe(self, want, want_score) -> None:
        """Record this call's demand: ``want``/``want_score`` ``[T, k]`` (host
        arrays, or anything ``harvest`` can turn into them later)."""
        self.pending.setdefault(self.step, []).append((want, want_score))

    def _host(self, a) -> np.ndarray:
        return np.asarray(a)

    # --- the policy, run before each call -----------------------------------------

    def begin(self) -> None:
        """Start a call: harvest the demand of the call ``lag`` calls back."""
        self.step += 1
        ready = self.step - self.lag
        if self.tau != float("inf") and ready in self.pending:
            for want, score in self.pending.pop(ready):
                self.harvest(ready, self._host(want), self._host(score))
        for old in [s for s in self.pending if s < ready]:
            del self.pending[old]

    def harvest(self, call: int, index: np.ndarray, weight: np.ndarray) -> None:
        """One call's demand (``omlx_routed.py:177-216``)."""
        index = np.asarray(index).reshape(-1, np.asarray(index).shape[-1])
        weight = np.asarray(weight, dtype=np.float64).reshape(index.shape)
        weight = weight / (weight.sum(-1, keepdims=True) + 1e-20) * self.route_scale
        self.stats["calls"] += 1
        self.stats["tokens"] += index.shape[0]
        self.stats["demand"] += index.size
        wanted: dict[int, float] = {}
        for e, w in zip(index[weight >= self.tau].tolist(), weight[weight >= self.tau].tolist()):
            wanted[int(e)] = max(w, wanted.get(int(e), 0.0))
        self.stats["resident"] += sum(int(e) in self.slot_of for e in index.ravel().tolist())
        self.install()
        missing = []
        for e, w in wanted.items():
            slot = self.slot_of.get(e)
            if slot is not None:
                self.last_use[slot] = call
            elif e not in self.reading:
                missing.append((w, e))
        self.stats["wanted"] += len(missing)
        self.free += [s for s, since in self.cooling if since <= call]
        self.cooling = [(s, since) for s, since in self.cooling if since > call]
        for _, e in sorted(missing, reverse=True):  # heaviest first
            if not self.free:
                self.stats["no_slot"] += 1
                continue
            slot = self.free.pop()
            self.reading[e] = (slot, self.read(e, slot))
            self.stats["admitted"] += 1
        self.evict(set(wanted))

    def install(self) -> None:
        """Route the experts whose bytes have landed (``omlx_routed.py:218-229``)."""
        for e in [e for e, (_, h) in self.reading.items() if self.done(h)]:
            slot, _ = self.reading.pop(e)
            self.route(e, slot)
            self.slot_expert[slot], self.slot_of[e] = e, slot
            self.last_use[slot] = self.step
            self.stats["installed"] += 1

    def evict(self, protected: set) -> None:
        """Unroute the least recently demanded residents until ``spare`` slots
        are free or cooling (``omlx_routed.py:231-247``)."""
        short = self.spare - len(self.free) - len(self.cooling)
        if short <= 0:
            return
        order = np.argsort(self.last_use, kind="stable")
        victims = [int(s) for s in order if self.slot_expert[s] >= 0 and int(self.slot_expert[s]) not in protected]
        for slot in victims[:short]:
            e = int(self.slot_expert[slot])
            del self.slot_of[e]
            self.slot_expert[slot] = -1
            self.last_use[slot] = np.inf
            self.unroute(e, slot)
            self.cooling.append((slot, self.step))  # calls built before may still route here
            self.stats["evicted"] += 1

    def fetch(self, want, strong=None) -> None:
        """The wait rule: read every demanded absent expert (or only ``strong``)
        now, over the least recently demanded residents, and route it once read;
        no fetched expert is evicted (``omlx_lattice.py:283-317``)."""
        want = [int(e) for e in np.asarray(want).ravel().tolist()]
        demanded = set(want)
        self.stats["demand"] += len(want)
        self.stats["resident"] += sum(e in self.slot_of for e in want)
        fetched = demanded if strong is None else {int(e) for e in np.asarray(strong).ravel().tolist()}
        for e in fetched & self.slot_of.keys():
            self.last_use[self.slot_of[e]] = self.step
        missing = sorted(fetched - self.slot_of.keys())
        if not missing:
            return
        victims = victim_order(self.last_use, self.slot_expert, fetched, demanded)
        if len(victims) < len(missing):
            raise RuntimeError("fewer slots than one call's demand")
        reads = []
        for e, slot in zip(missing, victims):
            old = int(self.slot_expert[slot])
            if old >= 0:
                del self.slot_of[old]
                self.unroute(old, slot)
                self.stats["evicted"] += 1
            reads.append((e, slot, self.read(e, slot)))
        for e, slot, h in reads:
            self.wait(h)
            self.route(e, slot)
            self.slot_expert[slot], self.slot_of[e] = e, slot
            self.last_use[slot] = self.step
            self.stats["installed"] += 1
        self.stats["waits"] += 1


class ResidencyCache(ResidencyPolicy):
    """``ResidencyPolicy`` on a device for one layer.

    ``installer`` is a ``loaders.ExpertInstaller`` over the layer's slot pools
    (``{w1, w3, w2}: (codes [S, ...], scales [S, ...])``); ``pool_bias`` is
    the router's served bias of every expert when resident (the correction
    bias, or zeros). ``bias_served`` (float32 ``[E]``, ``OFF`` for absent
    experts) and ``slot_map`` (int32 ``[E]``) are the device tensors the
    routed layer reads; they change only between calls and in the order of
    the current stream. ``observe(router_output)`` records a call's demand
    without a host sync (pinned copies and an event, read ``lag`` calls later).
    The starting residents (``order[:S]``) are read in at construction unless
    ``load`` is False. A decode step is ``begin()``, the layer call with
    ``bias_served`` and ``slot_map``, then ``observe`` of its router output.
    """

    def __init__(self, installer, num_experts: int, order, *, pool_bias=None, load: bool = True, **kw):
        self.installer = installer
        self.device = installer.device
        pools = installer.pools
        slots = int(next(iter(pools.values()))[0].shape[0])
        super().__init__(num_experts, slots, order, **kw)
        self.pool_bias = (np.zeros(num_experts, np.float32) if pool_bias is None
                          else np.asarray(pool_bias, dtype=np.float32).reshape(num_experts).copy())
        self._bias = np.full(num_experts, OFF, np.float32)
        self._map = np.zeros(num_experts, np.int32)  # an absent expert reads row 0 with weight 0
        for e, s in self.slot_of.items():
            self._bias[e], self._map[e] = self.pool_bias[e], s
        self.bias_served = torch.from_numpy(self._bias.copy()).to(self.device)
        self.slot_map = torch.from_numpy(self._map.copy()).to(self.device)
        self._dirty = False
        if load:  # the starting residents' bytes, before the first call
            for ev in [installer.submit(e, s) for e, s in self.slot_of.items()]:
                ev.synchronize()

    def read(self, expert: int, slot: int):
        return self.installer.submit(expert, slot)

    def done(self, handle) -> bool:
        return self.installer.ready(handle)

    def wait(self, handle) -> None:
        handle.synchronize()

    def route(self, expert: int, slot: int) -> None:
        self._bias[expert], self._map[expert] = self.pool_bias[expert], slot
        self._dirty = True

    def unroute(self, expert: int, slot: int) -> None:
        self._bias[expert] = OFF
        self._dirty = True

    def _publish(self) -> None:
        """Queue the router tensors' new values on the current stream (pinned
        staging, so the host may change them again at once)."""
        if not self._dirty:
            return
        self.bias_served.copy_(torch.from_numpy(self._bias.copy()).pin_memory(), non_blocking=True)
        self.slot_map.copy_(torch.from_numpy(self._map.copy()).pin_memory(), non_blocking=True)
        self._dirty = False

    def begin(self) -> None:
        super().begin()
        self._publish()

    def fetch(self, want, strong=None) -> None:
        super().fetch(want, strong)
        self._publish()

    def observe(self, router_output) -> None:
        """Record the demand (``want``, ``want_score``) of a call just issued."""
        want = torch.empty(router_output.want.shape, dtype=torch.int32, pin_memory=True)
        score = torch.empty(router_output.want_score.shape, dtype=torch.float32, pin_memory=True)
        want.copy_(router_output.want, non_blocking=True)
        score.copy_(router_output.want_score, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        super().observe((want, ev), score)

    def _host(self, a) -> np.ndarray:
        if isinstance(a, tuple):  # (pinned demand, its event)
            a[1].synchronize()
            return a[0].numpy()
        return a.numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
