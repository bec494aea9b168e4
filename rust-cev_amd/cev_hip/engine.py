"""The packed-pass engine over the device stack and the device prefix store.

Host mirror of Engine::run_many / plan / pass (crates/cev-model/src/engine.rs:
242-306, :327-363, :365-472) with the PrefixCache (engine.rs:474-503) replaced
by a cev_prefix_store over the stack's slot-addressed K/V caches:
  - plan(): PrefixCache::get -> a hit's slots are held for this call;
  - an uncached prefix reserves slots for its whole length; its head is
    prefilled there in 512-token chunks and its tail is computed by the
    first pass right after it, so the cached prefix is contiguous with no
    cat (engine.rs:247-256, :445-461);
  - the packing loop fills passes under the token budget exactly as the
    reference does (tails first, questions greedily, engine.rs:259-287);
  - a pass reserves scratch slots for its question tokens, builds the
    slot-addressed block table (cev_table_from_slots), runs the stack,
    reads the code-head logits at the gather rows, then puts every plan
    whose tail it computed into the store (engine.rs:445-462);
  - every held range is released when the call returns.
Requests are (prefix token ids, [question token ids]) after tokenisation
and the LCP split, which stay the engine's (engine.rs:327-363).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

from . import BlockTable, PrefixStore


@dataclass
class _Plan:
    prefix: np.ndarray
    suffixes: List[np.ndarray]
    begin: int = -1        # first cache slot of the prefix
    done: int = 0          # prefix tokens computed (in the cache)
    cached: bool = False   # whole prefix was a store hit
    held: List[int] = field(default_factory=list)


class DeviceEngine:
    def __init__(self, stack, budget: int, code_ids, pass_tokens: int = 2048, prefill_chunk: int = 512):
        self.stack = stack
        self.store = PrefixStore(stack.capacity, budget)
        self.code_ids = np.asarray(code_ids, np.int64)
        self.pass_tokens = int(pass_tokens)
        self.prefill_chunk = int(prefill_chunk)
        self.passes = 0

    def run_many(self, requests: Sequence):
        """requests: [(prefix ids, [question ids])].  Returns per request
        dict(logits (questions, n_codes) f32, hidden (questions, H) f32,
        prefix_cached), the Readout fields of engine.rs:463-469."""
        plans = [self._plan(p, qs) for p, qs in requests]
        try:
            for p in plans:
                if p.cached:
                    continue
                tail = min(len(p.prefix), max(1, self.prefill_chunk))
                head = len(p.prefix) - tail
                p.begin = self.store.reserve(len(p.prefix))
                p.held.append(p.begin)
                if head > 0:
                    self.stack.prefill(p.begin, p.prefix[:head], self.prefill_chunk)
                p.done = head
            items = [(pi, qi) for pi, p in enumerate(plans) for qi in range(len(p.suffixes))]
            out = [np.zeros((len(p.suffixes), len(self.code_ids)), np.float32) for p in plans]
            hid = [np.zeros((len(p.suffixes), self.stack.w.hidden), np.float32) for p in plans]
            rest = items
            while rest:
                budget = self.pass_tokens
                for p in plans:  # pending tails go first and count against the budget
                    budget = max(0, budget - (len(p.prefix) - p.done))
                n = 0
                while n < len(rest):
                    pi, qi = rest[n]
                    ln = len(plans[pi].suffixes[qi])
                    if n > 0 and ln > budget:
                        break
                    budget = max(0, budget - ln)
                    n += 1
                batch, rest = rest[:n], rest[n:]
                self._pass(plans, batch, out, hid)
            return [dict(logits=out[i], hidden=hid[i], prefix_cached=p.cached) for i, p in enumerate(plans)]
        finally:
            for p in plans:
                for b in p.held:
                    self.store.release(b)

    def _plan(self, prefix, suffixes) -> _Plan:
        prefix = np.asarray(prefix, np.int64)
        p = _Plan(prefix, [np.asarray(s, np.int64) for s in suffixes])
        hit = self.store.get(prefix)
        if hit is not None:
            p.begin, p.done, p.cached = hit, len(prefix), True
            p.held.append(hit)
        return p

    def _pass(self, plans, batch, out, hid):
        import torch
        n_q = sum(len(plans[pi].suffixes[qi]) for pi, qi in batch)
        scratch = self.store.reserve(n_q)
        try:
            items, tokens, slot = [], [], scratch
            for p in plans:
                if p.done < len(p.prefix):
                    tokens.append(p.prefix[p.done:])
            for pi, qi in batch:
                s = plans[pi].suffixes[qi]
                items.append((pi, len(s), slot))
                tokens.append(s)
                slot += len(s)
            table, pos, slots, gather = BlockTable.from_slots([(p.begin, len(p.prefix), p.done) for p in plans], items,
                                                              self.stack.capacity)
            hidden = self.stack.hidden(self.stack.run(np.concatenate(tokens), pos, slots, table), gather)
            logits = self.stack.code_logits(hidden, self.code_ids).cpu().numpy()
            hidden = hidden.cpu().numpy()
            for k, (pi, qi) in enumerate(batch):
                out[pi][qi] = logits[k]
                hid[pi][qi] = hidden[k]
            # tails are now computed: the prefix is cached (engine.rs:445-462)
            for p in plans:
                if p.done < len(p.prefix):
                    p.done = len(p.prefix)
                    self.store.put(p.prefix, p.begin)
            self.passes += 1
        finally:
            self.store.release(scratch)
        torch.cuda.current_stream().synchronize()
