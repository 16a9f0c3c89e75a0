"""CPU restatement of the reference radix tree (test infrastructure only).

Follows litelang/models/radix_cache.py step by step with plain Python lists:
  * TreeNode :19-53 (split_node :31-47 -- the tail inherits the ref count and
    the children and gets a fresh stamp; can_evict :49-50; touch :52-53);
  * the stamp is one counter per tree (the reference's module-global counter
    :7-16 orders the nodes of one tree the same way);
  * RadixTree.insert :72-98 with find_parent_node :100-128 (a shared prefix
    gives back the refs taken at admission, node by node);
  * match_prefix :130-145 with find_prefix_token_idxs :147-169 (discard from
    the evict set before the stamp changes, ref += 1, touch; a partial match
    splits the node and the unused tail drops the ref again);
  * evict_node :171-191 with try_del_node :193-203 (pop the oldest stamp,
    stop once strictly more than the need is freed).
The evict set is a list kept sorted by stamp. Slot ids are returned as lists.
"""
from __future__ import annotations


class Node:
    def __init__(self, tree, tokens, slots, ref=0):
        self.tokens = list(tokens)
        self.slots = list(slots)
        self.ref = ref
        self.child = {}
        self.parent = None
        tree.clock += 1
        self.time = tree.clock

    def can_evict(self):
        return not self.child and self.ref == 0


def _match(a, b):
    i = 0
    for x, y in zip(a, b):
        if x != y:
            break
        i += 1
    return i


class RadixOracle:
    def __init__(self):
        self.clock = 0
        self.root = Node(self, [], [], 1)
        self.evict = []  # nodes, ascending stamp
        self.all_taken = 0

    # evict-set operations of a set ordered by stamp
    def _add(self, n):
        if n not in self.evict:
            self.evict.append(n)
            self.evict.sort(key=lambda x: x.time)

    def _discard(self, n):
        if n in self.evict:
            self.evict.remove(n)

    def _split(self, n, k):
        tail = Node(self, n.tokens[k:], n.slots[k:], n.ref)
        tail.child = n.child
        for c in tail.child.values():
            c.parent = tail
        n.child = {tail.tokens[0]: tail}
        tail.parent = n
        n.tokens, n.slots = n.tokens[:k], n.slots[:k]
        return tail

    def insert(self, key, value, shared=()):
        full_key, full_val = list(key), list(value)
        key, shared = list(key), list(shared)
        node, has, ml = self.root, 0, 0
        while key and key[0] in node.child:
            c = node.child[key[0]]
            ml = _match(key, c.tokens)
            has += ml
            if ml != len(c.tokens):
                node = c
                break
            if shared:
                c.ref -= 1
                if c.can_evict():
                    self._add(c)
            node, key, shared, ml = c, key[ml:], shared[ml:], 0
        if ml > 0:
            tail = self._split(node, ml)
            if tail.can_evict():
                self._discard(node)
                self._add(tail)
        if has >= len(full_key):
            return has
        self.all_taken += len(full_key) - has
        new = Node(self, full_key[has:], full_val[has:])
        node.child[new.tokens[0]] = new
        new.parent = node
        if new.can_evict():
            self._discard(node)
            self._add(new)
        return has

    def match_prefix(self, key):
        key = list(key)
        node, has, vals, ml = self.root, 0, [], 0
        while key and key[0] in node.child:
            c = node.child[key[0]]
            ml = _match(key, c.tokens)
            has += ml
            vals += c.slots[:ml]
            self._discard(c)
            c.ref += 1
            self.clock += 1
            c.time = self.clock
            node = c
            if ml != len(c.tokens):
                break
            key, ml = key[ml:], 0
        if ml > 0:
            tail = self._split(node, ml)
            tail.ref -= 1
            if tail.can_evict():
                self._add(tail)
        return (vals if vals else None), has

    def evict_node(self, need):
        if need <= 0:
            return None
        if need > self.all_taken:
            raise ValueError("eviction request exceeds the tokens held by the tree")
        freed, out = 0, []
        while self.evict:
            n = self.evict.pop(0)
            assert n.ref == 0
            out += n.slots
            freed += len(n.tokens)
            p = n.parent
            del p.child[n.tokens[0]]
            if p.can_evict():
                self._add(p)
            if freed > need:
                break
        self.all_taken -= freed
        return out if out else None

    def snapshot(self):
        def rec(n):
            return [n.tokens, n.slots, n.ref, [rec(n.child[k]) for k in sorted(n.child)]]
        return rec(self.root)
