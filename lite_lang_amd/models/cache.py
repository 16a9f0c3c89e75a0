"""Paged (token-granular) KV pool and slot allocator.

Counterpart of litelang/models/cache.py (FreeReq :105-135, PageCache
:140-347). The pool is one device tensor kv_cache_[L, P, 2*KVH, D] (K heads
then V heads, the reference layout), addressed through the int32 slot table
req_to_tokens_[max_batch, max_length]. The free-slot stack and the request
rows stay on the host, so slot ids are decided exactly as in the reference
(LIFO reuse, contiguous pops); only the resulting slot-table writes go to the
device, through the ll_assign_slots kernel, in one upload per call.
"""
from __future__ import annotations

import numpy as np
import torch

from lite_lang_amd import ops


def get_dtype_size(dtype: torch.dtype) -> int:
    if dtype == torch.bool:
        return 1
    if dtype.is_floating_point:
        return torch.finfo(dtype).bits // 8
    return torch.iinfo(dtype).bits // 8


class FreeReq:
    """LIFO request-row allocator: alloc_new_req pops the most recently freed
    row (rows 0, 1, 2, ... on a fresh allocator); free_req pushes."""

    def __init__(self, max_batch_size: int):
        self._stack = list(range(max_batch_size - 1, -1, -1))

    def alloc_new_req(self):
        return self._stack.pop() if self._stack else None

    def free_req(self, rid) -> bool:
        self._stack.append(int(rid))
        return True

    def num_free(self) -> int:
        return len(self._stack)


def _host_ints(x):
    if isinstance(x, torch.Tensor):
        return x.tolist()
    return [int(v) for v in x]


class PageCache:
    def __init__(
        self,
        max_batch_size,
        max_length,
        mem_usage,
        num_layers,
        head_dim,
        num_key_value_heads,
        torch_dtype=torch.bfloat16,
        tp_rank=0,
        tp_world_size=1,
        kv_max_size=None,
        device=None,
    ):
        assert tp_world_size == 1, "this build runs tp=1 (one GPU, no collectives)"
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.num_key_value_heads_ = num_key_value_heads
        self.torch_dtype_ = torch_dtype
        self.dtype_size_ = get_dtype_size(torch_dtype)
        self.num_layers_ = num_layers
        self.head_dim_ = head_dim
        self.max_batch_size_ = max_batch_size
        self.max_length_ = max_length
        self.memory_usage_ = mem_usage
        # KiB per token slot over all layers (cache.py:185-194)
        self.token_size_ = head_dim * num_key_value_heads * 2 * self.dtype_size_ * num_layers / 1024
        if kv_max_size is None:
            free_b, _ = torch.cuda.mem_get_info(self.device)
            # cache.py:218-223: available MiB * mem_usage / 2, in slots
            kv_max_size = int((free_b / 1024**2 * mem_usage) / 2 * 1024**2 // 1024 // self.token_size_)
        assert kv_max_size > 0, (f"no KV token slot fits the memory budget "
                                 f"(mem_usage {mem_usage}, {self.token_size_:.1f} KiB per slot)")
        self.kv_max_size_ = int(kv_max_size)
        self.kv_cache_ = torch.empty(
            (num_layers, self.kv_max_size_, 2 * num_key_value_heads, head_dim),
            dtype=torch_dtype, device=self.device)
        self.req_to_tokens_ = torch.zeros((max_batch_size, max_length), dtype=torch.int32,
                                          device=self.device)
        self.physical_free_token_ = np.arange(self.kv_max_size_, dtype=np.int32)
        self.physical_free_token_start_ = 0
        self.physical_free_token_end_ = self.kv_max_size_
        self.free_req_ = FreeReq(max_batch_size)
        # host mirror of the slot table (kept in step with every device write)
        self._r2t_host = np.zeros((max_batch_size, max_length), dtype=np.int32)

    # ------------------------------------------------------------ slots
    def _check_and_mirror(self, slots, rows, cols):
        if slots.shape[0] == 0:
            return
        if rows.min() < 0 or rows.max() >= self.max_batch_size_ or cols.min() < 0 \
                or cols.max() >= self.max_length_:
            raise IndexError(f"slot-table write outside [{self.max_batch_size_}, "
                             f"{self.max_length_}] (request longer than max_length?)")
        self._r2t_host[rows, cols] = slots

    def _upload_assign(self, slots: np.ndarray, rows: np.ndarray, cols: np.ndarray):
        n = slots.shape[0]
        if n == 0:
            return torch.empty((0,), dtype=torch.int32, device=self.device)
        packed = np.stack([slots, rows, cols]).astype(np.int32)
        dev = torch.from_numpy(packed).pin_memory().to(self.device, non_blocking=True)
        ops.assign_slots(self.req_to_tokens_, dev, n)
        return dev[0]

    def alloc_token_idxs(self, b_rids, b_length, b_new_add_token_length):
        """Pop sum(b_new) slots; request r gets the next b_new[r] of them at
        columns b_length[r] .. of its row (cache.py:225-249). Returns the
        device int32 slot ids in batch order."""
        slots, rows, cols = self.plan_token_idxs(b_rids, b_length, b_new_add_token_length)
        return self._upload_assign(slots, rows, cols)

    def plan_token_idxs(self, b_rids, b_length, b_new_add_token_length):
        """Host half of alloc_token_idxs: pops the slots, updates the host
        mirror of the slot table and returns (slots, rows, cols) int32 arrays;
        the caller writes them to the device table (ll_assign_slots)."""
        rids = _host_ints(b_rids)
        lens = _host_ints(b_length)
        new = _host_ints(b_new_add_token_length)
        total = int(sum(new))
        free = self.physical_free_token_end_ - self.physical_free_token_start_
        assert total <= free, f"KV pool exhausted: {total} slots requested, {free} free"
        s0 = self.physical_free_token_start_
        slots = self.physical_free_token_[s0:s0 + total].copy()
        self.physical_free_token_start_ += total
        if all(v == 1 for v in new):  # one slot per request (a decode step)
            rows = np.array(rids, dtype=np.int32)
            cols = np.array(lens, dtype=np.int32)
        else:
            rows = np.repeat(np.asarray(rids, dtype=np.int32), new)
            offs = np.arange(total, dtype=np.int32) - np.repeat(
                np.cumsum([0] + new[:-1], dtype=np.int64).astype(np.int32), new)
            cols = np.repeat(np.asarray(lens, dtype=np.int32), new) + offs
        self._check_and_mirror(slots, rows, cols)
        return slots, rows, cols

    def alloc_req(self):
        return self.free_req_.alloc_new_req()

    def free_req(self, req):
        rid, length = req.rid, req.length - 1
        self.free_token_idxs(self._r2t_host[rid, :length].copy())
        self.free_rid(rid)
        return True

    def get_token_index(self, reqs):
        """Host copy of the concatenated slot rows [rid, :length-1] (cache.py:277-282)."""
        return np.concatenate([self._r2t_host[r.rid, : r.length - 1] for r in reqs])

    def add_refs(self, rid, token_idxs):
        """req_to_tokens[rid, :n] = token_idxs (cache.py:284-285)."""
        t = np.asarray(_host_ints(token_idxs), dtype=np.int32)
        n = t.shape[0]
        rows, cols = np.full(n, rid, dtype=np.int32), np.arange(n, dtype=np.int32)
        self._check_and_mirror(t, rows, cols)
        self._upload_assign(t, rows, cols)

    def free_token_idxs(self, token_idxs):
        """Push slots back just below the stack window (cache.py:287-295)."""
        t = np.asarray(_host_ints(token_idxs), dtype=np.int32)
        n = t.shape[0]
        assert self.physical_free_token_start_ - n >= 0, (
            f"returning {n} slots would overfill the free-slot stack (double free?)")
        s = self.physical_free_token_start_
        self.physical_free_token_[s - n:s] = t
        self.physical_free_token_start_ -= n

    def free_rid(self, rid):
        self.free_req_.free_req(rid)

    def dealloc_reqs(self, reqs):
        for req in reqs:
            self.free_req(req)

    def can_allocated(self, length):
        return self.physical_free_token_start_ + length <= self.physical_free_token_end_

    def if_need_more_tokens(self, length):
        return self.physical_free_token_start_ + length - self.physical_free_token_end_

    def slot_table_host(self) -> np.ndarray:
        return self._r2t_host
