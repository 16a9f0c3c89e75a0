"""SiLU_and_Mul, drop-in for litelang/kernel/develop_silu_and_mul/silu_and_mul.py:54-78."""
from lite_lang_amd import ops


def silu_and_mul_fwd(input):
    """input [M, 2N]: writes up * silu(gate) over the gate half in place and
    returns the view input[:, :N] (row stride 2N), as the reference does."""
    return ops.silu_and_mul(input, input[:, : input.shape[-1] // 2])
