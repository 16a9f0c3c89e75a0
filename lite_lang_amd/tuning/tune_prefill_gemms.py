"""Select the vendor-library GEMM solutions of the prefill projections.

Runs PyTorch's TunableOp (it benchmarks every hipBLASLt and rocBLAS solution
for a GEMM shape and keeps the fastest) on the prefill projection shapes of
the benchmark configurations and writes the results file that
`lite_lang_amd.tuning.use_prefill_gemm_solutions()` loads. Run on an MI355X
with the deployment image (the file records the PyTorch, HIP, hipBLASLt and
rocBLAS versions and the GPU architecture; torch ignores it on a mismatch):

    python -m lite_lang_amd.tuning.tune_prefill_gemms [out.csv]

The projections run as torch.matmul(x, w.t()) with x [M, K] and the weight
[N, K], M = prompt tokens of the prefill batch.
"""
import os
import sys

import torch
import torch.cuda.tunable as tunable

# (name, N, K) of the bf16 prefill projections; M = 40 prompts x 600 tokens
SHAPES = {
    "qwen2.5-3b": [("qkv", 2560, 2048), ("o", 2048, 2048), ("gate_up", 22016, 2048),
                   ("down", 2048, 11008)],
    "qwen2-1.5b": [("qkv", 2048, 1536), ("o", 1536, 1536), ("gate_up", 17920, 1536),
                   ("down", 1536, 8960)],
}
M_VALUES = (24000,)
DEFAULT_OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "prefill_gemm_mi355x.csv")


def main(out=DEFAULT_OUT):
    dev = torch.device("cuda:0")
    tunable.enable(True)
    tunable.tuning_enable(True)
    tunable.set_rotating_buffer_size(512)  # MB cycled between trials: operands not all cache-hot
    tunable.set_max_tuning_duration(200)  # ms per solution
    tunable.set_max_tuning_iterations(50)
    tunable.set_filename(out)  # the results are written there when the process exits
    for model, shapes in SHAPES.items():
        for M in M_VALUES:
            for name, N, K in shapes:
                x = torch.randn(M, K, device=dev).bfloat16()
                w = (torch.randn(N, K, device=dev) * 0.02).bfloat16()
                torch.matmul(x, w.t())
                torch.cuda.synchronize()
                print(f"tuned {model} {name} M={M} N={N} K={K}", flush=True)
    print(f"results go to {out} at exit")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else DEFAULT_OUT)
