"""Host side of the token loop: Qwen2 runner, paged KV pool, radix prefix
cache and NoPad batch metadata (counterparts of litelang/models/*)."""
