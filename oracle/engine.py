"""CPU oracle of the packed-pass engine (test infrastructure: loaded by
tests/ only, never by the product path).

Restates Engine::run_many, plan and pass (crates/cev-model/src/engine.rs:
242-306, :327-363, :365-472) and PrefixCache (engine.rs:474-503) over the
Qwen3 oracle: per-plan pasts are numpy K/V concatenated in plan order for a
pass (engine.rs:367-387), tails extend their plan's past and the prefix is
put into the LRU cache (engine.rs:445-462), logits are the f32 code head at
the gather rows (engine.rs:463).  Requests are (prefix ids, [question ids]).
"""
from __future__ import annotations

import numpy as np

from . import engine_pass, rms_norm


class PrefixCache:
    """engine.rs:474-503: entries in LRU order, bounded by total key length."""

    def __init__(self, budget: int):
        self.budget, self.entries = budget, []

    def get(self, key):
        for i, (k, _) in enumerate(self.entries):
            if k == key:
                e = self.entries.pop(i)
                self.entries.append(e)
                return e[1]
        return None

    def put(self, key, kv):
        if len(key) > self.budget:
            return
        self.entries = [e for e in self.entries if e[0] != key]
        self.entries.append((key, kv))
        while sum(len(k) for k, _ in self.entries) > self.budget:
            self.entries.pop(0)


class OracleEngine:
    def __init__(self, oracle, budget: int, code_ids, pass_tokens: int = 2048, prefill_chunk: int = 512):
        self.o = oracle
        self.cache = PrefixCache(budget)
        self.code_ids = np.asarray(code_ids, np.int64)
        self.pass_tokens, self.prefill_chunk = pass_tokens, prefill_chunk
        self.passes = 0

    def run_many(self, requests):
        plans = []
        for prefix, qs in requests:
            key = tuple(int(x) for x in prefix)
            hit = self.cache.get(key)
            plans.append(dict(prefix=np.asarray(prefix, np.int64), key=key, qs=[np.asarray(q, np.int64) for q in qs],
                              past=hit, cached=hit is not None, tail=(len(prefix), len(prefix))))
        for p in plans:
            if p["cached"]:
                continue
            n = len(p["prefix"])
            tail = min(n, max(1, self.prefill_chunk))
            head = n - tail
            p["past"] = self.o.prefill_kv(p["prefix"][:head], self.prefill_chunk) if head > 0 else None
            p["tail"] = (head, n)
        items = [(pi, qi) for pi, p in enumerate(plans) for qi in range(len(p["qs"]))]
        out = [np.zeros((len(p["qs"]), len(self.code_ids)), np.float32) for p in plans]
        hid = [np.zeros((len(p["qs"]), self.o.w.hidden), np.float32) for p in plans]
        rest = items
        while rest:
            budget = self.pass_tokens
            for p in plans:
                budget = max(0, budget - (p["tail"][1] - p["tail"][0]))
            n = 0
            while n < len(rest):
                pi, qi = rest[n]
                ln = len(plans[pi]["qs"][qi])
                if n > 0 and ln > budget:
                    break
                budget = max(0, budget - ln)
                n += 1
            batch, rest = rest[:n], rest[n:]
            self._pass(plans, batch, out, hid)
        return [dict(logits=out[i], hidden=hid[i], prefix_cached=p["cached"]) for i, p in enumerate(plans)]

    def _past_len(self, p):
        return 0 if p["past"] is None else p["past"][0][0].shape[1]

    def _pass(self, plans, batch, out, hid):
        w = self.o.w
        pasts = [p["past"] for p in plans if p["past"] is not None]
        if pasts:
            past = [(np.concatenate([pp[i][0] for pp in pasts], 1), np.concatenate([pp[i][1] for pp in pasts], 1))
                    for i in range(w.n_layers)]
        else:
            past = [(np.zeros((w.hkv, 0, w.d), np.float32),) * 2 for _ in range(w.n_layers)]
        specs = [(self._past_len(p), len(p["prefix"]), p["tail"][0]) for p in plans]
        ep = engine_pass(specs, [(pi, len(plans[pi]["qs"][qi])) for pi, qi in batch])
        tokens = [p["prefix"][p["tail"][0]:p["tail"][1]] for p in plans if p["tail"][1] > p["tail"][0]]
        tokens += [plans[pi]["qs"][qi] for pi, qi in batch]
        x, kv = self.o._layers(np.concatenate(tokens), ep["pos"], ep["mask"], past=past)
        h_rows = rms_norm(x[ep["gather"]], self.o.W["norm"], w.eps, self.o.bf).astype(np.float32)
        logits = self.o.code_logits(h_rows, self.code_ids).astype(np.float32)
        for k, (pi, qi) in enumerate(batch):
            out[pi][qi] = logits[k]
            hid[pi][qi] = h_rows[k]
        at = 0
        for p in plans:
            tl = p["tail"][1] - p["tail"][0]
            if tl == 0:
                continue
            new = [(k[:, at:at + tl], v[:, at:at + tl]) for k, v in kv]
            at += tl
            if p["past"] is None:
                p["past"] = new
            else:
                p["past"] = [(np.concatenate([pk, k], 1), np.concatenate([pv, v], 1)) for (pk, pv), (k, v) in zip(p["past"], new)]
            self.cache.put(p["key"], p["past"])
            p["tail"] = (len(p["prefix"]), len(p["prefix"]))
        self.passes += 1
