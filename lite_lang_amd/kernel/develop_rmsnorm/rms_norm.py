"""RMSNorm, drop-in for litelang/kernel/develop_rmsnorm/rms_norm.py:71-98."""
from lite_lang_amd import ops


def rmsnorm(x, gamma, variance_epsilon):
    """out = (x / sqrt(mean(x^2) + eps)) * gamma, computed in fp32, cast to x.dtype.

    Same contract as the reference: x is 2-D [M, N], gamma [N], returns a new
    tensor (rms_norm.py:72-79).
    """
    assert x.shape[1] == gamma.shape[0], (
        f"gamma shape 0: {gamma.shape[0]} not match x shape 1: {x.shape[1]}")
    assert x.ndim == 2, "shapesize shoule equal to 2"
    if x.stride(1) != 1:
        x = x.contiguous()
    return ops.rmsnorm(x, gamma.contiguous(), variance_epsilon)
