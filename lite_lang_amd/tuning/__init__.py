"""Vendor-library GEMM solution selection for the prefill projections."""
import os

_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "prefill_gemm_mi355x.csv")
_loaded = False


def use_prefill_gemm_solutions(path: str = _FILE) -> bool:
    """Make torch's bf16/fp16 GEMMs use the solutions recorded in `path` (a
    TunableOp results file written by tune_prefill_gemms.py) for the shapes it
    lists; every other shape keeps the library's own choice, and nothing is
    tuned at run time. torch ignores the file when its recorded library
    versions or GPU architecture differ from the running ones. Returns whether
    the file was loaded."""
    global _loaded
    if _loaded:
        return True
    if not os.path.exists(path):
        return False
    import torch
    import torch.cuda.tunable as tunable
    if not torch.cuda.is_available():
        return False
    tunable.enable(True)
    tunable.tuning_enable(False)
    _loaded = bool(tunable.read_file(path))
    if not _loaded:
        tunable.enable(False)
    return _loaded
