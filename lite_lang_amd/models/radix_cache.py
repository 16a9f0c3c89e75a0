"""Radix tree of token-id runs -> KV slot runs, with reference counts and LRU
eviction of unreferenced leaves.

Counterpart of litelang/models/radix_cache.py (TreeNode :19-53, RadixTree
:65-203); the observable behaviour (matched lengths, returned slot ids, which
node is split, ref-count bookkeeping, LRU eviction order by last-touch stamp,
evicted token count) is the reference's. Token and slot runs are held as
numpy int64 arrays; the public methods take and return torch CPU tensors
like the reference.
"""
from __future__ import annotations

import itertools

import numpy as np
import torch
from sortedcontainers import SortedKeyList


def _np(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().numpy().astype(np.int64, copy=False)
    return np.asarray(x, dtype=np.int64)


def common_prefix_len(a: np.ndarray, b: np.ndarray) -> int:
    n = min(a.shape[0], b.shape[0])
    if n == 0:
        return 0
    neq = np.nonzero(a[:n] != b[:n])[0]
    return int(neq[0]) if neq.size else n


class TreeNode:
    __slots__ = ("token_ids", "page_cache_token_idxs", "ref_count", "child", "parent_node", "time")

    def __init__(self, tree, token_ids, slot_ids, ref_count=0):
        self.token_ids = token_ids
        self.page_cache_token_idxs = slot_ids
        self.ref_count = ref_count
        self.child = {}
        self.parent_node = None
        self.time = next(tree._clock)

    def split_node(self, tree, match_len: int) -> "TreeNode":
        """Keep the first match_len tokens here; move the rest (and all
        children) into a new child that inherits the reference count."""
        tail = TreeNode(tree, self.token_ids[match_len:], self.page_cache_token_idxs[match_len:],
                        self.ref_count)
        tail.child = self.child
        for c in tail.child.values():
            c.parent_node = tail
        tail.parent_node = self
        self.child = {int(tail.token_ids[0]): tail}
        self.token_ids = self.token_ids[:match_len]
        self.page_cache_token_idxs = self.page_cache_token_idxs[:match_len]
        return tail

    def can_evict(self) -> bool:
        return not self.child and self.ref_count == 0


class RadixTree:
    def __init__(self):
        self._clock = itertools.count(1)
        self.root = TreeNode(self, np.zeros(0, np.int64), np.zeros(0, np.int64), 1)
        self.evict_node_set_ = SortedKeyList(key=lambda n: n.time)
        self._in_set = set()
        self.all_taken_tokens_ = 0

    # ------------------------------------------------------------ evict set
    def _add(self, node):
        if id(node) not in self._in_set:
            self._in_set.add(id(node))
            self.evict_node_set_.add(node)

    def _discard(self, node):
        if id(node) in self._in_set:
            self._in_set.discard(id(node))
            self.evict_node_set_.remove(node)

    # ------------------------------------------------------------ insert
    def insert(self, key, value, shared_key=None) -> int:
        """Insert a finished request's tokens (all but the last generated one)
        with their slots; releases the refs taken on the shared prefix at
        admission. Returns the length already present in the tree."""
        key, value = _np(key), _np(value)
        shared = _np(shared_key) if shared_key is not None else np.zeros(0, np.int64)
        parent, has, ml = self._find_parent(self.root, key, 0, shared)
        if ml > 0:
            tail = parent.split_node(self, ml)
            if tail.can_evict():
                self._discard(parent)
                self._add(tail)
        if has >= key.shape[0]:
            return has
        self.all_taken_tokens_ += key.shape[0] - has
        node = TreeNode(self, key[has:], value[has:])
        parent.child[int(key[has])] = node
        node.parent_node = parent
        if node.can_evict():
            self._discard(parent)
            self._add(node)
        return has

    def _find_parent(self, node, key, has, shared):
        while True:
            if key.shape[0] <= 0:
                return node, has, 0
            c = node.child.get(int(key[0]))
            if c is None:
                return node, has, 0
            ml = common_prefix_len(key, c.token_ids)
            has += ml
            if ml != c.token_ids.shape[0]:
                if shared.shape[0] > 0:
                    raise RuntimeError("radix insert: shared prefix ends inside a node")
                return c, has, ml
            if shared.shape[0] > 0:
                c.ref_count -= 1
                if c.can_evict():
                    self._add(c)
            node, key, shared = c, key[ml:], shared[ml:]

    # ------------------------------------------------------------ match
    def match_prefix(self, key):
        """Longest cached prefix of `key`: returns (slot ids or None, length).
        Every node on the matched path gets a reference and a fresh stamp."""
        key = _np(key)
        node, has, values, ml = self.root, 0, [], 0
        while key.shape[0] > 0:
            c = node.child.get(int(key[0]))
            if c is None:
                ml = 0
                break
            ml = common_prefix_len(key, c.token_ids)
            has += ml
            values.append(c.page_cache_token_idxs[:ml])
            self._discard(c)
            c.ref_count += 1
            c.time = next(self._clock)
            node = c
            if ml != c.token_ids.shape[0]:
                break
            key = key[ml:]
            ml = 0
        if ml > 0:
            tail = node.split_node(self, ml)
            tail.ref_count -= 1
            if tail.can_evict():
                self._add(tail)
        if not values:
            return None, has
        return torch.from_numpy(np.concatenate(values)), has

    # ------------------------------------------------------------ evict
    def evict_node(self, need_token_nums):
        """Evict least-recently-stamped unreferenced leaves until more than
        `need_token_nums` tokens are released; returns their slots or None."""
        if need_token_nums <= 0:
            return None
        if need_token_nums > self.all_taken_tokens_:
            raise ValueError(f"cannot evict {need_token_nums} tokens: the tree holds "
                             f"{self.all_taken_tokens_}")
        freed, out = 0, []
        while len(self.evict_node_set_):
            node = self.evict_node_set_.pop(0)
            self._in_set.discard(id(node))
            freed += self._del_node(node, out)
            if freed > need_token_nums:
                break
        self.all_taken_tokens_ -= freed
        if not out:
            return None
        return torch.from_numpy(np.concatenate(out))

    def _del_node(self, node, out) -> int:
        assert node.ref_count == 0, f"evicting a node still referenced {node.ref_count} time(s)"
        out.append(node.page_cache_token_idxs)
        parent = node.parent_node
        del parent.child[int(node.token_ids[0])]
        if parent.can_evict():
            self._add(parent)
        return node.token_ids.shape[0]

    # ------------------------------------------------------------ inspection
    def snapshot(self):
        """Nested (tokens, slots, ref_count, children) tuples, children sorted
        by first token; used by tests to compare tree states."""
        def rec(n):
            return (n.token_ids.tolist(), n.page_cache_token_idxs.tolist(), n.ref_count,
                    [rec(n.child[k]) for k in sorted(n.child)])
        return rec(self.root)

    def evict_order(self):
        """First tokens of the evictable leaves, oldest stamp first."""
        return [n.token_ids.tolist() for n in self.evict_node_set_]
