"""Writes tests/golden/radix_traces.json: operation traces of the reference
RadixTree (litelang/models/radix_cache.py), recorded by running that module in
the build container (CPU only; it is pure Python over torch CPU tensors).

Only the tree's outputs under long interleavings are taken from it -- the
eviction order there depends on split stamps and ref counts that no closed
form fixes. The traces follow the serving protocol of runner_batch.py:118-147
and :184-204: admission matches input[:-1] and holds the refs; finish inserts
the request's tokens with its slots and the matched prefix as shared_key;
eviction asks for what a new admission lacks.

Run from the repository root with the reference checked out at
/root/reference:  python tests/golden/make_radix_golden.py
The reference's evict_node moves a single evicted run to the GPU with
.cuda(); in this GPU-less container that call is made an identity so the
returned slot ids can be recorded (the move does not change them).
"""
import importlib.util
import json
import os
import random

import torch

REF = "/root/reference/litelang/models/radix_cache.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "radix_traces.json")


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_radix_cache", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def snapshot(node):
    toks = [] if node.token_ids is None else node.token_ids.tolist()
    slots = [] if node.page_cache_token_idxs is None else node.page_cache_token_idxs.tolist()
    return [toks, slots, node.ref_count, [snapshot(node.child[k]) for k in sorted(node.child)]]


def trace(mod, seed, n_req=40, vocab=6, slots_total=48):
    """One serving-like interleaving over a small vocabulary (many shared
    prefixes, frequent splits)."""
    rng = random.Random(seed)
    tree = mod.RadixTree()
    free = list(range(slots_total))
    ops = []
    live = []  # (tokens, slots, shared_len)
    for step in range(n_req * 3):
        if live and (rng.random() < 0.45 or len(live) > 6):
            # finish a request: insert tokens[:-1] with their slots, shared prefix given back
            toks, slots, shared = live.pop(rng.randrange(len(live)))
            key = torch.tensor(toks[:-1], dtype=torch.int64)
            val = torch.tensor(slots[:-1], dtype=torch.int64)
            ret = tree.insert(key, val, key[:shared])
            dup = slots[shared:ret]  # already cached beyond the shared prefix: freed by the caller
            free += dup + [slots[-1]]
            ops.append({"op": "insert", "key": toks[:-1], "value": slots[:-1], "shared": shared,
                        "ret": ret, "all_taken": tree.all_taken_tokens_})
        else:
            plen = rng.randint(2, 9)
            base = rng.choice([[], [0], [0, 1], [1, 2, 3], [0, 1, 2]])
            toks = (base + [rng.randrange(vocab) for _ in range(plen)])[:max(plen, 2)]
            key = torch.tensor(toks[:-1], dtype=torch.int64)
            got, has = tree.match_prefix(key)
            got = [] if got is None else got.tolist()
            ops.append({"op": "match", "key": toks[:-1], "slots": got, "len": has})
            need = len(toks) - has + rng.randint(0, 3)  # new tokens plus a few decode slots
            if need > len(free):
                want = need - len(free)
                if want <= tree.all_taken_tokens_:
                    ev = tree.evict_node(want)
                    ev = [] if ev is None else ev.tolist()
                    free += ev
                    ops.append({"op": "evict", "need": want, "slots": ev,
                                "all_taken": tree.all_taken_tokens_})
            if need > len(free):
                # cannot admit: give the refs back as the runner would on a failed admission
                k = torch.tensor(got and toks[:has] or [], dtype=torch.int64)
                ret = tree.insert(k, torch.tensor(got, dtype=torch.int64), k) if has else 0
                ops.append({"op": "insert", "key": toks[:has], "value": got, "shared": has,
                            "ret": ret, "all_taken": tree.all_taken_tokens_})
                continue
            rng.shuffle(free)
            new = [free.pop() for _ in range(len(toks) - has)]
            live.append((toks, got + new, has))
    return {"seed": seed, "ops": ops, "final_tree": snapshot(tree.root)}


def main():
    mod = load_reference()
    torch.Tensor.cuda = lambda self, *a, **k: self  # see the module docstring
    traces = [trace(mod, seed) for seed in range(12)]
    json.dump({"source": REF.replace("/root/reference/", ""), "generator": os.path.basename(__file__),
               "traces": traces}, open(OUT, "w"))
    print(f"wrote {OUT}: {sum(len(t['ops']) for t in traces)} operations")


if __name__ == "__main__":
    main()
