"""CPU restatement of the slot / request-row allocator (test infrastructure only).

Follows litelang/models/cache.py: FreeReq (:105-135) and PageCache
(:140-347), minus the device pool itself. Pure Python lists and numpy; the
slot table is a numpy int32 array.
"""
from __future__ import annotations

import numpy as np


class FreeReq:
    """LIFO request-row allocator (cache.py:105-135).

    The reference keeps a linked list headed by a sentinel: allocation pops
    the head, freeing pushes the freed row in front. A Python list used as a
    stack (top = end) gives the same order.
    """

    def __init__(self, max_batch_size: int):
        self.stack = list(range(max_batch_size - 1, -1, -1))

    def alloc_new_req(self):
        return self.stack.pop() if self.stack else None

    def free_req(self, rid: int) -> bool:
        self.stack.append(int(rid))
        return True


class PageCache:
    """Token-granular slot allocator (cache.py:140-347).

    Free slots are the window free[start:end] of a stack that starts as
    arange(P); allocation takes the next `total` entries in order
    (cache.py:225-249), freeing writes the freed slots back just below
    `start` (cache.py:287-295).
    """

    def __init__(self, max_batch_size: int, max_length: int, kv_max_size: int):
        self.kv_max_size_ = kv_max_size
        self.free = np.arange(kv_max_size, dtype=np.int32)
        self.start = 0
        self.end = kv_max_size
        self.req_to_tokens_ = np.zeros((max_batch_size, max_length), dtype=np.int32)
        self.free_req_ = FreeReq(max_batch_size)

    def alloc_token_idxs(self, b_rids, b_length, b_new):
        """Take sum(b_new) slots; request r receives the next b_new[r] of them
        at columns b_length[r] .. b_length[r] + b_new[r] - 1 of its row
        (the bucketize mapping of cache.py:238-248)."""
        total = int(sum(int(n) for n in b_new))
        assert self.start + total <= self.end, "KV pool exhausted"
        idxs = self.free[self.start:self.start + total].copy()
        self.start += total
        g = 0
        for rid, length, new in zip(b_rids, b_length, b_new):
            for c in range(int(new)):
                self.req_to_tokens_[int(rid), int(length) + c] = idxs[g]
                g += 1
        return idxs

    def alloc_req(self):
        return self.free_req_.alloc_new_req()

    def free_rid(self, rid):
        self.free_req_.free_req(rid)

    def add_refs(self, rid, token_idxs):
        token_idxs = np.asarray(token_idxs, dtype=np.int32)
        self.req_to_tokens_[int(rid), : token_idxs.shape[0]] = token_idxs

    def free_token_idxs(self, token_idxs):
        token_idxs = np.asarray(token_idxs, dtype=np.int32)
        n = token_idxs.shape[0]
        assert self.start - n >= 0, "free-slot stack overfilled"
        self.free[self.start - n:self.start] = token_idxs
        self.start -= n

    def get_token_index(self, reqs):
        """Concatenated slot rows req_to_tokens[rid, :length-1] (cache.py:277-282)."""
        return np.concatenate([self.req_to_tokens_[r.rid, : r.length - 1] for r in reqs])

    def free_req(self, req):
        self.free_token_idxs(self.req_to_tokens_[req.rid, : req.length - 1].copy())
        self.free_rid(req.rid)
        return True

    def dealloc_reqs(self, reqs):
        for r in reqs:
            self.free_req(r)

    def can_allocated(self, length):
        return self.start + length <= self.end

    def if_need_more_tokens(self, length):
        return self.start + length - self.end
