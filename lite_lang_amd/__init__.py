"""lite_lang_amd: MI355X-native (gfx950) Qwen2 token loop with the lite_lang API.

Kernels live in ``liblitelang_amd.so`` (HIP C++, C ABI in include/litelang_amd.h);
``lite_lang_amd.kernel`` mirrors ``litelang.kernel`` signature for signature,
``lite_lang_amd.models`` holds the host side (Qwen2 runner, paged KV pool,
radix prefix cache, NoPad batch metadata).
"""
__version__ = "0.1.0"
