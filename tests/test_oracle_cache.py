"""Pins of the oracle allocator (oracle/cache.py) and batch metadata.

Golden vectors: the expected slot rows of the reference's own allocator test
(test/test_page_atten.py:86-102, tests/golden/page_cache_kat.json).
Invariants: LIFO reuse of freed slots and request rows (cache.py:114-135,
287-295), per-request contiguity of a batch allocation (cache.py:238-248).
"""
import json
import os

import numpy as np
import pytest

from oracle.cache import FreeReq, PageCache
from oracle.runner_batch import Req, no_padding_messages

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _rows(pc, rids, lens):
    return np.concatenate([pc.req_to_tokens_[r, :l] for r, l in zip(rids, lens)]).tolist()


def test_page_cache_kat_from_reference_test():
    kat = json.load(open(os.path.join(GOLD, "page_cache_kat.json")))
    pc = PageCache(kat["max_batch_size"], kat["max_length"], 4096)
    rids = [pc.alloc_req(), pc.alloc_req()]
    assert rids == [0, 1]
    lens = kat["prefill"]["seq_lens"]
    pc.alloc_token_idxs(rids, [0, 0], lens)
    assert _rows(pc, rids, lens) == kat["prefill"]["expected_rows_concat"]
    pc.alloc_token_idxs(rids, lens, kat["decode"]["new_tokens"])
    lens2 = [l + n for l, n in zip(lens, kat["decode"]["new_tokens"])]
    assert _rows(pc, rids, lens2) == kat["decode"]["expected_rows_concat"]


def test_free_req_is_lifo():
    fr = FreeReq(4)
    a, b, c = fr.alloc_new_req(), fr.alloc_new_req(), fr.alloc_new_req()
    assert (a, b, c) == (0, 1, 2)
    fr.free_req(1)
    fr.free_req(0)
    assert fr.alloc_new_req() == 0 and fr.alloc_new_req() == 1 and fr.alloc_new_req() == 3
    assert fr.alloc_new_req() is None


def test_freed_slots_are_reused_first_in_order():
    pc = PageCache(4, 64, 100)
    pc.alloc_token_idxs([0, 1], [0, 0], [3, 4])  # slots 0..6
    pc.free_token_idxs(np.array([5, 2, 4], dtype=np.int32))
    assert pc.start == 4
    got = pc.alloc_token_idxs([2], [0], [5])
    # the freed run [5, 2, 4] sits just below `start`, then 7, 8
    assert got.tolist() == [5, 2, 4, 7, 8]
    assert pc.req_to_tokens_[2, :5].tolist() == [5, 2, 4, 7, 8]
    with pytest.raises(AssertionError):
        pc.alloc_token_idxs([3], [0], [200])


def test_alloc_with_zero_length_requests_and_offsets():
    pc = PageCache(4, 64, 100)
    got = pc.alloc_token_idxs([3, 1, 2], [10, 0, 4], [2, 0, 3])
    assert got.tolist() == [0, 1, 2, 3, 4]
    assert pc.req_to_tokens_[3, 10:12].tolist() == [0, 1]
    assert pc.req_to_tokens_[2, 4:7].tolist() == [2, 3, 4]
    assert pc.if_need_more_tokens(96) == 1 and pc.can_allocated(95)


def test_no_padding_messages():
    r0 = Req(rid=3, input_tokens=[7, 8, 9], shared_tokens=[1, 2])
    r1 = Req(rid=0, input_tokens=[5])
    ids, pos, st, lens, sh, rids = no_padding_messages([r0, r1], True)
    assert ids == [7, 8, 9, 5] and pos == [2, 3, 4, 0] and st == [0, 3]
    assert lens == [5, 1] and sh == [2, 0] and rids == [3, 0]
    r0.output_tokens.append(11)
    r1.output_tokens.append(12)
    ids, pos, st, lens, sh, rids = no_padding_messages([r0, r1], False)
    assert pos == [5, 1] and st == [0, 1] and lens == [6, 2]
