"""Radix tree (litelang/models/radix_cache.py:19-203): the CPU oracle
(oracle/radix.py) and the product (lite_lang_amd/models/radix_cache.py) against

  * the reference's scripted sequence radix_cache.py:217-269 with every
    intermediate value derived by hand (tests/golden/radix_script_kat.json);
  * operation traces recorded from the reference module itself under
    serving-like interleavings with splits, shared-prefix inserts and
    evictions (tests/golden/radix_traces.json, written by
    tests/golden/make_radix_golden.py);
  * each other, plus invariants, on fresh random interleavings.
Bit-exact: returned lengths, slot ids, taken-token counts, final trees.
"""
import json
import os
import random

import pytest
import torch

from oracle.radix import RadixOracle

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _product():
    from lite_lang_amd.models.radix_cache import RadixTree
    return RadixTree()


def _norm(tree):
    """Nested [tokens, slots, ref, children] lists for either implementation."""
    def rec(n):
        return [list(n[0]), list(n[1]), int(n[2]), [rec(c) for c in n[3]]]
    return rec(tree.snapshot())


class _Adapter:
    """Common call surface: lists in, lists out."""

    def __init__(self, tree, is_product):
        self.t, self.p = tree, is_product

    def insert(self, key, value, shared=0):
        if self.p:
            k = torch.tensor(key, dtype=torch.int64)
            return self.t.insert(k, torch.tensor(value, dtype=torch.int64), k[:shared] if shared else None)
        return self.t.insert(key, value, key[:shared])

    def match(self, key):
        got, n = self.t.match_prefix(torch.tensor(key, dtype=torch.int64) if self.p else key)
        return ([] if got is None else [int(x) for x in got]), n

    def evict(self, need):
        got = self.t.evict_node(need)
        return [] if got is None else [int(x) for x in got]

    @property
    def taken(self):
        return self.t.all_taken_tokens_ if self.p else self.t.all_taken


def _replay(ad, ops):
    for i, o in enumerate(ops):
        if o["op"] == "insert":
            ret = ad.insert(o["key"], o["value"], o.get("shared", 0))
            assert ret == o["ret"], f"op {i}: insert returned {ret}, expected {o['ret']}"
            assert ad.taken == o["all_taken"], f"op {i}: all_taken {ad.taken} != {o['all_taken']}"
        elif o["op"] == "match":
            slots, n = ad.match(o["key"])
            assert (slots, n) == (o["slots"], o["len"]), f"op {i}: match {(slots, n)} != {(o['slots'], o['len'])}"
        else:
            slots = ad.evict(o["need"])
            assert slots == o["slots"], f"op {i}: evicted {slots} != {o['slots']}"
            assert ad.taken == o["all_taken"], f"op {i}: all_taken {ad.taken} != {o['all_taken']}"


@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_script_kat(impl):
    kat = json.load(open(os.path.join(GOLD, "radix_script_kat.json")))
    ad = _Adapter(_product(), True) if impl == "product" else _Adapter(RadixOracle(), False)
    _replay(ad, kat["ops"])
    assert _norm(ad.t) == kat["final_tree"]


@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_reference_traces(impl):
    data = json.load(open(os.path.join(GOLD, "radix_traces.json")))
    assert len(data["traces"]) >= 8
    n_evict = 0
    for tr in data["traces"]:
        ad = _Adapter(_product(), True) if impl == "product" else _Adapter(RadixOracle(), False)
        _replay(ad, tr["ops"])
        assert _norm(ad.t) == tr["final_tree"], f"seed {tr['seed']}: final tree differs"
        n_evict += sum(o["op"] == "evict" for o in tr["ops"])
    assert n_evict > 100  # the traces exercise eviction


def test_evict_more_than_taken_raises():
    for t in (_product(), RadixOracle()):
        ad = _Adapter(t, isinstance(t, type(_product())))
        ad.insert([5, 6, 7], [0, 1, 2])
        with pytest.raises(ValueError):
            t.evict_node(4)
        assert t.evict_node(0) is None


@pytest.mark.parametrize("seed", range(6))
def test_product_equals_oracle_random(seed):
    """Fresh interleavings (different vocabulary and lengths from the recorded
    ones), checked step by step, with invariants on every match."""
    rng = random.Random(1000 + seed)
    prod, orc = _Adapter(_product(), True), _Adapter(RadixOracle(), False)
    inserted = []
    free = list(range(64))
    live = []
    for _ in range(300):
        if live and rng.random() < 0.5:
            toks, slots, shared = live.pop(rng.randrange(len(live)))
            a = prod.insert(toks, slots, shared)
            b = orc.insert(toks, slots, shared)
            assert a == b and prod.taken == orc.taken
            free += slots[shared:a]
            inserted.append(toks)
        else:
            toks = [rng.randrange(4) for _ in range(rng.randint(1, 12))]
            (sa, na), (sb, nb) = prod.match(toks), orc.match(toks)
            assert (sa, na) == (sb, nb)
            assert len(sa) == na
            # the matched length is the longest prefix shared with a cached key
            best = max([0] + [sum(1 for _ in __import__("itertools").takewhile(
                lambda p: p[0] == p[1], zip(toks, k))) for k in inserted])
            assert na <= best
            need = len(toks) - na
            if need > len(free):
                want = need - len(free)
                if want <= orc.taken:
                    ea, eb = prod.evict(want), orc.evict(want)
                    assert ea == eb and prod.taken == orc.taken
                    free += ea
            if need > len(free):
                if na:
                    prod.insert(toks[:na], sa, na)
                    orc.insert(toks[:na], sb, na)
                continue
            rng.shuffle(free)
            live.append((toks, sa + [free.pop() for _ in range(need)], na))
        assert _norm(prod.t) == _norm(orc.t)
