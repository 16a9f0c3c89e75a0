"""Which running requests to swap out when the KV budget is exceeded
(litelang/scheduler/pause_strategy.py:1-55)."""
from __future__ import annotations

STRATEGY_REGISTRY = {}


def register_strategy(cls):
    STRATEGY_REGISTRY[cls.__name__] = cls
    return cls


class Strategy:
    def ordering(self, reqs):
        raise NotImplementedError


@register_strategy
class FIFOStrategy(Strategy):
    def ordering(self, reqs):
        return sorted(reqs, key=lambda r: r.id)


@register_strategy
class ShortestFirstStrategy(Strategy):
    # the reference orders longest first under this name (:28-31); kept
    def ordering(self, reqs):
        return sorted(reqs, key=lambda r: r.length, reverse=True)


@register_strategy
class LongestFirstStrategy(Strategy):
    # and shortest first under this one (:34-37); kept
    def ordering(self, reqs):
        return sorted(reqs, key=lambda r: r.length)


@register_strategy
class LIFOStrategy(Strategy):
    def ordering(self, reqs):
        return sorted(reqs, key=lambda r: r.id, reverse=True)


def select_swapped_reqs(reqs, strategy, need_tokens):
    """Take requests in the strategy's order until their lengths add up to
    strictly more than need_tokens (pause_strategy.py:43-55)."""
    chosen, used = [], 0
    for req in strategy.ordering(reqs):
        used += req.length
        chosen.append(req)
        if used > need_tokens:
            break
    return chosen
