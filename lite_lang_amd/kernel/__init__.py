"""Drop-in counterparts of ``litelang.kernel.*`` backed by HIP kernels."""
