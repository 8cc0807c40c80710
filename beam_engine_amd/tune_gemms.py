"""Tunes the library GEMM solutions of the e2e decode step with PyTorch TunableOp.

The e2e benchmark's decode step runs five bf16 weight GEMMs with M = 128
candidates (8 requests x beam 16) on a Llama-3-8B-shaped decoder: fused QKV,
output projection, fused gate/up, down projection and the LM head.  They are
library calls (hipBLASLt / rocBLAS through ``torch.nn.functional.linear``),
outside this build's attention path.  ``python -m beam_engine_amd.tune_gemms
[--out FILE]`` times every candidate solution of each shape with TunableOp,
rotating over more weight copies than the 256 MB Infinity Cache holds (each
decode GEMM streams its weights from HBM once per step), and writes the
winners to a TunableOp results file; ``e2e.use_tuned_gemms`` loads that file
(tuning off) before the benchmark runs.
"""

from __future__ import annotations

import argparse
import os
import sys

DEFAULT_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tunableop_e2e_decode.csv")

# (N, K) of y[M, N] = x[M, K] W[N, K]^T
SHAPES = {"qkv": (6144, 4096), "o_proj": (4096, 4096), "gate_up": (28672, 4096), "down": (4096, 14336),
          "lm_head": (128256, 4096)}


def main(argv=None) -> int:
    import torch
    import torch.nn.functional as F
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--out", default=DEFAULT_FILE)
    ap.add_argument("--m", type=int, default=128, help="GEMM rows (decode candidates per step)")
    args = ap.parse_args(argv)
    tun = torch.cuda.tunable
    tun.enable(True)
    tun.tuning_enable(True)
    tun.record_untuned_enable(False)
    tun.set_rotating_buffer_size(1024)            # MB: weights come from HBM, as in the decode step
    tun.set_max_tuning_duration(200)              # ms per solution
    tun.set_filename(args.out)
    dev = torch.device("cuda")
    for name, (n, k) in SHAPES.items():
        x = torch.randn(args.m, k, device=dev, dtype=torch.bfloat16)
        w = torch.randn(n, k, device=dev, dtype=torch.bfloat16) * 0.02
        F.linear(x, w)
        torch.cuda.synchronize()
        print(f"tuned {name}: [{args.m}, {k}] x [{n}, {k}]^T", flush=True)
    for r in tun.get_results():
        print(r)
    write = getattr(torch._C, "_cuda_tunableop_write_file", None)
    if write is not None:
        write(args.out)
    print(f"results go to {args.out} (written at exit)", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
