"""CPU oracle of the lite_lang Qwen2 token loop -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference semantics of every function
on the hot path (ops, slot allocator, radix prefix cache, NoPad batch
metadata, Qwen2 forward). It is the checker the GPU path is compared against
and the CPU baseline timed beside it. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it; the product package ``lite_lang_amd`` never does, and has no CPU path.

Each function cites the reference file:line it follows (paths relative to
the lite_lang repository root). How each function is pinned (golden vectors,
known-answer tests, closed forms, invariants) is listed in
tests/test_oracle_*.py; a function without such a check says
"parity unpinned" in its docstring.

Modules:
  ops           kernels: rmsnorm, rope, silu_and_mul, decode / prefill
                attention over the slot table, linear, argmax, int8 W8A8
  cache         PageCache / FreeReq slot and request-row allocator
  radix         RadixTree prefix cache
  runner_batch  NoPad batch metadata
  qwen2         Qwen2 forward and greedy generation
"""
